#!/usr/bin/env python3
"""Run one GQA attention step from .mem stimulus on the GPU: the stand-in for the
Vivado/XSim step of pyfiles/run_gqa_regression.py:53-62.

Inputs, as scripts/run_gqa_wrapper_sim.tcl and tests/tb_gqa_attention_wrapper.sv
take them:
  $VECTORS_DIR (or --vectors)  gqa_config.txt, gqa_q.mem, gqa_k.mem, gqa_v.mem
                               [, gqa_golden.mem for the self-check]
  $INVALID_CONFIG=1            program N_Q_HEADS=31 (tb_gqa_attention_wrapper.sv:323)
                               and expect the call to be rejected
  $MAX_ULP / --max-ulp         self-check tolerance (default 64)
Output: gqa_rtl_out.mem (32 rows x 128 BF16; --out / $RTL_OUT to redirect).

Like the testbench it prints "PASS: ..." when the output matches gqa_golden.mem
within the tolerance (tb_gqa_attention_wrapper.sv:221-245), and
"PASS: invalid configuration rejected" for the rejection case (:330-336).  Both
operands are rotated (Q at QUERY_POSITION, K at each position) as the core does.
"""
from __future__ import annotations

import argparse
import math
import os
import sys
from pathlib import Path

import numpy as np


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--vectors", type=Path, default=Path(os.environ.get("VECTORS_DIR", "tests/data")))
    ap.add_argument("--out", type=Path, default=None)
    ap.add_argument("--max-ulp", type=int, default=int(os.environ.get("MAX_ULP", "64")))
    ap.add_argument("--invalid-config", action="store_true",
                    default=os.environ.get("INVALID_CONFIG", "0") not in ("", "0"))
    args = ap.parse_args(argv)

    import torch

    from . import attention as A
    from ._lib import GQA_ERR_INVALID_CONFIG, GQA_OK, GqaConfigError, lib
    from .check import failures, worst
    from .memfmt import config_int, read_config, read_mem, write_mem

    vec = args.vectors
    cfg = read_config(vec / "gqa_config.txt")
    seq_len = config_int(cfg, "SEQ_LEN")
    head_dim = config_int(cfg, "HEAD_DIM", 128)
    tile_dim = config_int(cfg, "TILE_DIM", 16)
    n_q = config_int(cfg, "N_Q_HEADS", 32)
    n_kv = config_int(cfg, "N_KV_HEADS", 8)
    blk = config_int(cfg, "KV_BLOCK_LEN", 16)
    qpos = config_int(cfg, "QUERY_POSITION", seq_len - 1)
    kv_len = config_int(cfg, "KV_INPUT_SEQ_LEN", (seq_len + blk - 1) // blk * blk)
    scale_bf16 = config_int(cfg, "SCALE_BF16", 0x3DB5)
    if args.invalid_config:
        n_q = 31
    out_path = args.out or Path(os.environ.get("RTL_OUT", vec / "gqa_rtl_out.mem"))

    # The register write sequence of tests/tb_gqa_attention_wrapper.sv:323-329 and
    # the start-time check of gqa_attention_wrapper.v:230-237.
    n_kv_tiles = (seq_len + blk - 1) // blk
    reg_status = lib().gqa_validate_registers(n_q, n_kv, head_dim, tile_dim, seq_len, n_kv_tiles,
                                              blk, scale_bf16)
    # The stimulus always carries the fixed geometry; only the programmed registers vary.
    q = read_mem(vec / "gqa_q.mem", tile_dim).reshape(A.N_Q_HEADS, A.HEAD_DIM)
    k = read_mem(vec / "gqa_k.mem", tile_dim).reshape(A.N_KV_HEADS, kv_len, A.HEAD_DIM)
    v = read_mem(vec / "gqa_v.mem", tile_dim).reshape(A.N_KV_HEADS, kv_len, A.HEAD_DIM)
    dev = torch.device("cuda", 0)
    tq = torch.from_numpy(q.view(np.int16)).view(torch.bfloat16).to(dev)
    tk = torch.from_numpy(k.view(np.int16)).view(torch.bfloat16).to(dev)
    tv = torch.from_numpy(v.view(np.int16)).view(torch.bfloat16).to(dev)
    sentinel = torch.full((1, A.N_Q_HEADS, A.HEAD_DIM), -1, dtype=torch.int16, device=dev)
    out = sentinel.clone().view(torch.bfloat16)
    params = A.make_params(rope_q=True, rope_k=True, scale=1.0 / math.sqrt(A.HEAD_DIM),
                           n_q_heads=n_q, n_kv_heads=n_kv, head_dim=head_dim)
    status = GQA_OK
    try:
        A.gqa_attention(tq[None], tk[None], tv[None], qpos, seq_len, out=out, params=params)
    except GqaConfigError:
        status = GQA_ERR_INVALID_CONFIG
    torch.cuda.synchronize()
    if status == GQA_OK and reg_status != GQA_OK:
        status = reg_status
    if status != GQA_OK and not torch.equal(out.view(torch.int16), sentinel):
        print("FAIL: rejected call wrote output")
        return 1
    if status != GQA_OK:
        if args.invalid_config:
            print("PASS: invalid configuration rejected")
            return 0
        print(f"FAIL: configuration rejected (status {status})")
        return 1
    if args.invalid_config:
        print("FAIL: invalid configuration accepted")
        return 1
    rows = out[0].view(torch.int16).cpu().numpy().view(np.uint16)
    write_mem(out_path, rows)
    golden_path = vec / "gqa_golden.mem"
    if golden_path.exists():
        golden = read_mem(golden_path, head_dim)
        if golden.shape != rows.shape:
            print(f"FAIL: golden has {golden.shape[0]} rows, output has {rows.shape[0]}")
            return 1
        bad = failures(golden, rows, args.max_ulp)
        w = worst(golden, rows)
        if bad.any():
            print(f"FAIL: {int(bad.sum())} elements exceed {args.max_ulp} ULP; "
                  f"worst={w[0]} at row={w[1]}, col={w[2]}")
            return 1
        print(f"PASS: {rows.shape[0]} output rows within {args.max_ulp} ULP "
              f"(worst {w[0]} at row={w[1]}, col={w[2]})")
    else:
        print(f"wrote {out_path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
