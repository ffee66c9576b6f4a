#!/usr/bin/env python3
"""Stimulus + golden vector generator (test infrastructure only).

Same command line and same output files as pyfiles/gen_gqa_wrapper_vectors.py:38-155
(gqa_q.mem, gqa_k.mem, gqa_v.mem, gqa_golden.mem, gqa_config.txt), built on the
restatement in oracle/golden_model.py; for the reference's modes the files are
byte-identical to what the reference script writes.  One extra mode, "normal",
draws N(0,1) (random.gauss) in the same order.  Rows past ~2K positions use the
compiled restatement (oracle/oracle.py) for the golden loop.
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))

import numpy as np  # noqa: E402

from oracle import golden_model as gm  # noqa: E402


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--out-dir", type=Path, default=Path("tests/data"))
    ap.add_argument("--seq-len", type=int, default=None)
    ap.add_argument("--target-input-vectors", type=int, default=None)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--tile-dim", type=int, default=16)
    ap.add_argument("--kv-block-len", type=int, default=16)
    ap.add_argument("--q-heads", type=int, default=32)
    ap.add_argument("--kv-heads", type=int, default=8)
    ap.add_argument("--query-position", type=int, default=None)
    ap.add_argument("--seed", type=int, default=20260731)
    ap.add_argument("--mode", choices=("smoke", "random", "normal"), default="smoke")
    args = ap.parse_args(argv)
    # Validation of pyfiles/gen_gqa_wrapper_vectors.py:57-78.
    if args.q_heads % args.kv_heads or args.head_dim % args.tile_dim:
        ap.error("q-heads must be divisible by kv-heads and head-dim by tile-dim")
    if args.kv_block_len <= 0:
        ap.error("kv-block-len must be positive")
    if args.seq_len is not None and args.target_input_vectors is not None:
        ap.error("--seq-len and --target-input-vectors are mutually exclusive")
    if args.target_input_vectors is not None:
        q_elements = args.q_heads * args.head_dim
        per_pos = 2 * args.kv_heads * args.head_dim
        rem = args.target_input_vectors - q_elements
        if rem <= 0 or rem % per_pos:
            ap.error("target-input-vectors must equal q-heads*head-dim + "
                     "N*(2*kv-heads*head-dim), for a positive integer N")
        args.seq_len = rem // per_pos
    if args.seq_len is None:
        args.seq_len = 16
    if args.seq_len <= 0:
        ap.error("seq-len must be positive")
    qpos = args.seq_len - 1 if args.query_position is None else args.query_position
    if not 0 <= qpos < args.seq_len:
        ap.error("query-position must be in [0, seq-len)")

    q, k, v = gm.stimulus(args.mode, args.seq_len, args.seed, q_heads=args.q_heads,
                          kv_heads=args.kv_heads, head_dim=args.head_dim,
                          kv_block_len=args.kv_block_len)
    qb, kb, vb = gm.beats(q, k, v, args.tile_dim)
    if args.seq_len <= 2048:
        golden = gm.golden_attention(q, k, v, args.seq_len, qpos)
    else:
        from oracle import oracle as orc
        golden = orc.decode(np.array(q, dtype=np.uint16), np.array(k, dtype=np.uint16),
                            np.array(v, dtype=np.uint16), args.seq_len, qpos,
                            rope_q=True, rope_k=True, sum_mode=gm.python_sum_mode()).tolist()
    out = args.out_dir
    gm.write_mem(out / "gqa_q.mem", qb)
    gm.write_mem(out / "gqa_k.mem", kb)
    gm.write_mem(out / "gqa_v.mem", vb)
    gm.write_mem(out / "gqa_golden.mem", golden)
    (out / "gqa_config.txt").write_text(gm.config_text(
        seq_len=args.seq_len, head_dim=args.head_dim, tile_dim=args.tile_dim,
        q_heads=args.q_heads, kv_heads=args.kv_heads, kv_block_len=args.kv_block_len,
        query_position=qpos, mode=args.mode, seed=args.seed))
    n_pos = gm.kv_input_len(args.seq_len, args.kv_block_len)
    print(f"Wrote {args.q_heads * args.head_dim + 2 * args.kv_heads * args.seq_len * args.head_dim} "
          f"valid BF16 input-vector elements ({n_pos - args.seq_len} masked K/V pad rows) "
          f"and golden output to {out}")


if __name__ == "__main__":
    main()
