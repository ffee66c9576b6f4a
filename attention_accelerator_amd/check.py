#!/usr/bin/env python3
"""Compare BF16 output rows against golden rows (the check of
pyfiles/check_gqa_output.py, same flags, same PASS/FAIL text, vectorised).

Per element: fail when the BF16 code distance (pyfiles/gqa_reference.py:49-53)
exceeds --max-ulp (64), unless both BF16 exponent fields are <= 0x3d, i.e. both
|x| < 2^-65 (pyfiles/check_gqa_output.py:57-64).
"""
from __future__ import annotations

import argparse
from pathlib import Path
from typing import Tuple

import numpy as np

from .memfmt import read_mem


def ordered(codes: np.ndarray) -> np.ndarray:
    c = np.asarray(codes, dtype=np.int32)
    return np.where(c & 0x8000, 0x8000 - (c & 0x7FFF), 0x8000 + c)


def ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return np.abs(ordered(a) - ordered(b))


def failures(golden: np.ndarray, actual: np.ndarray, max_ulp: int = 64) -> np.ndarray:
    """Boolean mask of failing elements under the checker's policy."""
    g = np.asarray(golden, dtype=np.int32)
    a = np.asarray(actual, dtype=np.int32)
    dist = ulp_distance(g, a)
    tiny = (((g >> 7) & 0xFF) <= 0x3D) & (((a >> 7) & 0xFF) <= 0x3D)
    return (dist > max_ulp) & ~tiny


def worst(golden: np.ndarray, actual: np.ndarray) -> Tuple[int, int, int]:
    """(distance, row, col) of the largest distance (first one on ties)."""
    dist = ulp_distance(golden, actual).reshape(np.asarray(golden).shape[0], -1)
    if dist.size == 0:
        return 0, 0, 0
    idx = int(np.argmax(dist))
    r, c = divmod(idx, dist.shape[1])
    return int(dist[r, c]), r, c


def _f(code: int) -> float:
    return float(np.array([code << 16], dtype=np.uint32).view(np.float32)[0])


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--golden", type=Path, default=Path("tests/data/gqa_golden.mem"))
    ap.add_argument("--rtl", "--actual", dest="actual", type=Path,
                    default=Path("tests/data/gqa_rtl_out.mem"), help="output .mem file")
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--max-ulp", type=int, default=64)
    ap.add_argument("--show-rows", type=int, default=2)
    ap.add_argument("--show-elements", type=int, default=8)
    ap.add_argument("--max-mismatches", type=int, default=10)
    args = ap.parse_args(argv)
    golden = read_mem(args.golden, args.head_dim)
    actual = read_mem(args.actual, args.head_dim)
    if golden.shape[0] != actual.shape[0]:
        raise SystemExit(f"FAIL: golden has {golden.shape[0]} rows, actual has {actual.shape[0]}")
    shown = args.head_dim if args.show_elements < 0 else args.show_elements
    for row in range(min(args.show_rows, golden.shape[0])):
        n = min(shown, golden.shape[1])
        print(f"row {row:02d} golden: " + " ".join(f"{v:04x}" for v in golden[row, :n]))
        print(f"row {row:02d} actual: " + " ".join(f"{v:04x}" for v in actual[row, :n]))
    bad = failures(golden, actual, args.max_ulp)
    w = worst(golden, actual)
    rows, cols = np.nonzero(bad)
    for r, c in list(zip(rows.tolist(), cols.tolist()))[:args.max_mismatches]:
        g, a = int(golden[r, c]), int(actual[r, c])
        print(f"mismatch row={r} col={c}: golden=0x{g:04x} ({_f(g):.7g}) rtl=0x{a:04x} "
              f"({_f(a):.7g}) ulp={int(ulp_distance(g, a))}")
    n_bad = int(bad.sum())
    if n_bad:
        raise SystemExit(f"FAIL: {n_bad} elements exceed {args.max_ulp} ULP; "
                         f"worst={w[0]} at row={w[1]}, col={w[2]}")
    print(f"PASS: all {actual.shape[0]} output rows ({actual.size} BF16 values) "
          f"matched golden within {args.max_ulp} ULP; worst ULP={w[0]} at row={w[1]}, col={w[2]}")


if __name__ == "__main__":
    main()
