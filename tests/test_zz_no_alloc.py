"""gqa_decode_bf16_noalloc (the decode entry point that allocates nothing) against
gqa_decode_bf16 through the C ABI: two calls in a row on the library's own device
array, the second with a smaller batch that takes the one-launch path (whose counters
live in that array), then the first shape again; outputs bit-identical to the
workspace entry point's (the same kernels and plan) and within 64 BF16 ULP of the
oracle.  A batch whose workspace does not fit the array is rejected before launch."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import attention_accelerator_amd as gqa
from attention_accelerator_amd import stimulus
from attention_accelerator_amd._lib import GqaKvLayout, lib
from oracle import oracle as orc
from _util import assert_within_ulp, to_codes

pytestmark = pytest.mark.gpu


def _noalloc(b: stimulus.DecodeBatch, dev) -> np.ndarray:
    q, k, v = b.q.to(dev).contiguous(), b.k.to(dev), b.v.to(dev)
    sl, qp = b.seq_len.to(dev), b.query_pos.to(dev)
    out = torch.full((q.shape[0], 32, 128), float("nan"), dtype=torch.bfloat16, device=dev)
    p = gqa.make_params()
    lay = GqaKvLayout(k.stride(0), k.stride(1), k.stride(2), k.shape[2])
    print(f"noalloc call: batch {q.shape[0]}, capacity {k.shape[2]}", flush=True)
    st = lib().gqa_decode_bf16_noalloc(ctypes.byref(p), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                       ctypes.byref(lay), sl.data_ptr(), qp.data_ptr(), q.shape[0],
                                       out.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    assert st == 0, f"status {st}"
    torch.cuda.synchronize()
    return to_codes(out)


def _workspace(b: stimulus.DecodeBatch, dev) -> np.ndarray:
    out = gqa.gqa_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.query_pos, b.seq_len)
    torch.cuda.synchronize()
    return to_codes(out)


def test_noalloc_matches_workspace_entry_point(dev):
    big = stimulus.decode_batch(64, 8192, min_len=512, max_len=8192, seed=41, gen_device="cuda", device=dev)
    small = stimulus.decode_batch(2, 4096, min_len=1, max_len=4096, seed=42)
    for name, b in (("B=64 ragged (stream-K)", big), ("B=2 (one launch)", small),
                    ("B=64 ragged again", big)):
        got = _noalloc(b, dev)
        want = _workspace(b, dev)
        assert np.array_equal(got, want), f"{name}: no-alloc output differs from gqa_decode_bf16"
    # oracle parity on the smaller batch (all rows) and on two sequences of the larger one
    ref = orc.decode(to_codes(small.q), to_codes(small.k), to_codes(small.v), small.seq_len.numpy(),
                     small.query_pos.numpy())
    assert_within_ulp(ref, _noalloc(small, dev), 64, "no-alloc B=2")
    sub = stimulus.DecodeBatch(big.q[:2].cpu(), big.k[:2].cpu(), big.v[:2].cpu(), big.seq_len[:2].cpu(),
                               big.query_pos[:2].cpu())
    ref = orc.decode(to_codes(sub.q), to_codes(sub.k), to_codes(sub.v), sub.seq_len.numpy(),
                     sub.query_pos.numpy())
    assert_within_ulp(ref, _noalloc(big, dev)[:2], 64, "no-alloc B=64 sequences 0, 1")


def test_noalloc_rejects_batch_beyond_its_array(dev):
    """1000 sequences of capacity 8192 need more than the 32 MiB array: rejected with
    GQA_ERR_WORKSPACE, nothing launched (the output keeps its contents)."""
    n, cap = 1000, 8192
    q = torch.zeros((n, 32, 128), dtype=torch.bfloat16, device=dev)
    kv = torch.zeros((1, 8, cap, 128), dtype=torch.bfloat16, device=dev).expand(n, 8, cap, 128)
    sl = torch.full((n,), 16, dtype=torch.int32, device=dev)
    qp = sl - 1
    out = torch.full((n, 32, 128), 7.0, dtype=torch.bfloat16, device=dev)
    p = gqa.make_params()
    lay = GqaKvLayout(kv.stride(0), kv.stride(1), kv.stride(2), cap)
    st = lib().gqa_decode_bf16_noalloc(ctypes.byref(p), q.data_ptr(), kv.data_ptr(), kv.data_ptr(),
                                       ctypes.byref(lay), sl.data_ptr(), qp.data_ptr(), n, out.data_ptr(),
                                       torch.cuda.current_stream(dev).cuda_stream)
    assert st == 3
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
