"""Compiled restatement of the golden attention (test infrastructure only).

numpy + ctypes over liboracle.so (oracle/gqa_oracle.c, built by oracle/Makefile).
Only tests/, the smoke check and the benchmark's CPU-baseline leg import this
module, and only as the checker.  It extends the one-token golden of
pyfiles/gen_gqa_wrapper_vectors.py:121-139 to the shapes this build runs:

* decode:  a batch of independent sequences, each with its own seq_len and
  query_position (mask p < seq_len and p <= query_position,
  gqa_attention_wrapper.v:279);
* prefill: several new query tokens per sequence appended after a cache, query
  t at position start+t seeing keys p <= start+t (the same mask per row).

Per query token and head the arithmetic is the reference loop itself (double,
libm, Python's sum() order), so on single-sequence inputs it reproduces
golden_model.golden_attention bit for bit.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
from pathlib import Path
from typing import Optional, Sequence, Union

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_lib = None

SUM_SEQUENTIAL = 0
SUM_NEUMAIER = 1


def build() -> Path:
    """Compile liboracle.so with oracle/Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        dp = ctypes.POINTER(ctypes.c_double)
        u16p = ctypes.POINTER(ctypes.c_uint16)
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_double]
        L.oracle_f32_to_bf16.restype = ctypes.c_int32
        L.oracle_rope_half_split.argtypes = [dp, ctypes.c_int, ctypes.c_int64, ctypes.c_double, dp]
        L.oracle_rope_half_split.restype = None
        L.oracle_prepare_rows.argtypes = [u16p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int64, ctypes.c_double, dp]
        L.oracle_prepare_rows.restype = None
        L.oracle_attend.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, dp, dp, dp,
                                    ctypes.c_int64, ctypes.c_int64, ctypes.c_double, ctypes.c_int,
                                    u16p, dp]
        L.oracle_attend.restype = ctypes.c_int
        _lib = L
    return _lib


def _dp(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def _u16p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


def f32_to_bf16(x: float) -> int:
    return int(lib().oracle_f32_to_bf16(float(x)))


def rope_row(row: np.ndarray, position: int, theta: float = 500000.0) -> np.ndarray:
    """pyfiles/gen_gqa_wrapper_vectors.py:25-35 on a float64 row."""
    src = np.ascontiguousarray(row, dtype=np.float64)
    out = np.empty_like(src)
    lib().oracle_rope_half_split(_dp(src), src.shape[0], int(position), float(theta), _dp(out))
    return out


def prepare_rows(rows_bf16: np.ndarray, rotate: bool, pos0: int = 0,
                 theta: float = 500000.0) -> np.ndarray:
    """BF16 codes [n, d] -> float64 [n, d], rotating row r at position pos0 + r."""
    src = np.ascontiguousarray(rows_bf16, dtype=np.uint16)
    n, d = src.shape
    if not rotate:
        # Exact widening BF16 -> f32 -> f64 (pyfiles/gqa_reference.py:22-23).
        return (src.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    out = np.empty((n, d), dtype=np.float64)
    if n:
        lib().oracle_prepare_rows(_u16p(src), n, d, d, 1, int(pos0), float(theta), _dp(out))
    return out


def attend(q_ref: np.ndarray, k_ref: np.ndarray, v_ref: np.ndarray, n_keys: int,
           scale: float, sum_mode: int = SUM_SEQUENTIAL, want_f64: bool = False):
    """The golden loop for one query token on prepared float64 operands.
    q_ref [Hq, d]; k_ref, v_ref [Hkv, S, d] with S >= n_keys."""
    q_ref = np.ascontiguousarray(q_ref, dtype=np.float64)
    k_ref = np.ascontiguousarray(k_ref, dtype=np.float64)
    v_ref = np.ascontiguousarray(v_ref, dtype=np.float64)
    hq, d = q_ref.shape
    hkv, s, _ = k_ref.shape
    if not 1 <= n_keys <= s:
        raise ValueError("n_keys out of range")
    out = np.empty((hq, d), dtype=np.uint16)
    out64 = np.empty((hq, d), dtype=np.float64) if want_f64 else None
    rc = lib().oracle_attend(hq, hkv, d, _dp(q_ref), _dp(k_ref), _dp(v_ref), s, int(n_keys),
                             float(scale), int(sum_mode), _u16p(out),
                             _dp(out64) if want_f64 else ctypes.POINTER(ctypes.c_double)())
    if rc != 0:
        raise OverflowError("golden output beyond the f32 range")
    return (out, out64) if want_f64 else out


IntOrSeq = Union[int, Sequence[int], np.ndarray]


def decode(q: np.ndarray, k: np.ndarray, v: np.ndarray, seq_len: IntOrSeq,
           query_position: IntOrSeq, *, rope_q: bool = True, rope_k: bool = False,
           theta: float = 500000.0, scale: Optional[float] = None,
           sum_mode: int = SUM_SEQUENTIAL, want_f64: bool = False,
           kv_heads: Optional[Sequence[int]] = None):
    """Golden decode over a batch.

    q [B, Hq, d] (or [Hq, d]); k, v [B, Hkv, S, d] (or [Hkv, S, d]) BF16 codes in
    position order; seq_len / query_position per sequence.  Rows at positions
    >= min(seq_len, query_position + 1) are never read (they may hold NaN).
    kv_heads restricts the work to those KV heads (and their Q heads); the other
    output rows are left zero.
    Returns out [B, Hq, d] BF16 codes (and float64 values with want_f64)."""
    single = q.ndim == 2
    if single:
        q, k, v = q[None], k[None], v[None]
    bsz, hq, d = q.shape
    _, hkv, cap, _ = k.shape
    sl = np.broadcast_to(np.asarray(seq_len, dtype=np.int64), (bsz,))
    qp = np.broadcast_to(np.asarray(query_position, dtype=np.int64), (bsz,))
    sc = 1.0 / math.sqrt(d) if scale is None else float(scale)
    out = np.zeros((bsz, hq, d), dtype=np.uint16)
    out64 = np.zeros((bsz, hq, d), dtype=np.float64) if want_f64 else None
    for b in range(bsz):
        if not (1 <= sl[b] <= cap and 0 <= qp[b] < sl[b]):
            raise ValueError(f"sequence {b}: need 1 <= seq_len <= {cap} and 0 <= qpos < seq_len")
        n_keys = int(qp[b]) + 1
        group = hq // hkv
        sel = list(range(hkv)) if kv_heads is None else [int(x) for x in kv_heads]
        qsel = [h for g in sel for h in range(g * group, (g + 1) * group)]
        q_ref = np.stack([prepare_rows(q[b, h][None], rope_q, int(qp[b]), theta)[0]
                          for h in qsel])
        k_ref = np.stack([prepare_rows(k[b, h, :n_keys], rope_k, 0, theta) for h in sel])
        v_ref = np.stack([prepare_rows(v[b, h, :n_keys], False) for h in sel])
        r = attend(q_ref, k_ref, v_ref, n_keys, sc, sum_mode, want_f64)
        if want_f64:
            out[b, qsel], out64[b, qsel] = r
        else:
            out[b, qsel] = r
    if single:
        out = out[0]
        out64 = out64[0] if want_f64 else None
    return (out, out64) if want_f64 else out


def prefill(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, k_new: np.ndarray,
            v_new: np.ndarray, start: IntOrSeq, *, rope_q: bool = True, rope_k_new: bool = True,
            rope_k_cache: bool = False, theta: float = 500000.0, scale: Optional[float] = None,
            sum_mode: int = SUM_SEQUENTIAL, rows: Optional[Sequence[int]] = None,
            want_f64: bool = False, threads: int = 1):
    """Golden chunked prefill: the one-token golden applied per new query token.

    q [B, T, Hq, d], k_new / v_new [B, T, Hkv, d] BF16 codes; k_cache / v_cache
    [B, Hkv, S, d] with positions < start[b] valid.  Query t of sequence b sits at
    position start[b]+t and sees keys p <= start[b]+t: cached rows for p < start,
    new row p-start otherwise (rotated at p when rope_k_new, unrounded, as the
    golden rotates K).  rows selects which t to compute (default all).
    threads > 1 runs the tokens of a sequence on that many threads (the C loop
    releases the GIL; each token's arithmetic is unchanged, so the result is too).
    Returns out [B, len(rows), Hq, d] BF16 codes (and float64 with want_f64)."""
    bsz, t_new, hq, d = q.shape
    hkv = k_new.shape[2]
    st = np.broadcast_to(np.asarray(start, dtype=np.int64), (bsz,))
    sc = 1.0 / math.sqrt(d) if scale is None else float(scale)
    rows = list(range(t_new)) if rows is None else list(rows)
    out = np.zeros((bsz, len(rows), hq, d), dtype=np.uint16)
    out64 = np.zeros((bsz, len(rows), hq, d), dtype=np.float64) if want_f64 else None
    for b in range(bsz):
        s0 = int(st[b])
        total = s0 + t_new
        k_ref = np.empty((hkv, total, d), dtype=np.float64)
        v_ref = np.empty((hkv, total, d), dtype=np.float64)
        for h in range(hkv):
            k_ref[h, :s0] = prepare_rows(k_cache[b, h, :s0], rope_k_cache, 0, theta)
            v_ref[h, :s0] = prepare_rows(v_cache[b, h, :s0], False)
            k_ref[h, s0:] = prepare_rows(k_new[b, :, h], rope_k_new, s0, theta)
            v_ref[h, s0:] = prepare_rows(v_new[b, :, h], False)
        def one(i, t, b=b, s0=s0, k_ref=k_ref, v_ref=v_ref):
            pos = s0 + t
            q_ref = np.stack([prepare_rows(q[b, t, h][None], rope_q, pos, theta)[0]
                              for h in range(hq)])
            r = attend(q_ref, k_ref, v_ref, pos + 1, sc, sum_mode, want_f64)
            if want_f64:
                out[b, i], out64[b, i] = r
            else:
                out[b, i] = r

        if threads > 1 and len(rows) > 1:
            from concurrent.futures import ThreadPoolExecutor
            with ThreadPoolExecutor(max_workers=threads) as ex:
                list(ex.map(lambda it: one(*it), enumerate(rows)))
        else:
            for i, t in enumerate(rows):
                one(i, t)
    return (out, out64) if want_f64 else out


def host_threads(cap: int = 16) -> int:
    """Threads for the oracle on this host: the cores this process may run on, at most cap."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        n = os.cpu_count() or 1
    return max(1, min(cap, n))


if os.environ.get("GQA_ORACLE_AUTOBUILD", "1") == "1" and not _LIB_PATH.exists():
    try:
        build()
    except Exception:  # pragma: no cover - lib() retries and reports
        pass
