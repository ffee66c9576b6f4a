"""Rows whose golden value is NaN: Q heads scaled by 2^126 with one element +inf (the BF16
overflow of a larger scale), so that the dot products meet inf - inf.

The golden's f32_to_bf16 keeps a NaN's sign (pyfiles/gqa_reference.py:17-19), and the NaN an
invalid operation creates on x86 (the default NaN) has its sign bit set, so those rows come
out 0xffc0 in the golden -- and in the oracle, compiled C on the same kind of host.  Every
path must give the same codes there (the reference checker compares raw codes,
pyfiles/check_gqa_output.py:55-69) and stay within 64 BF16 ULP everywhere else."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import attention_accelerator_amd as gqa
from oracle import oracle as orc
from _util import assert_within_ulp, to_codes

pytestmark = pytest.mark.gpu

_F = 2.0 ** 126


def _nan_rows(want) -> int:
    w = np.asarray(want).reshape(-1, 128)
    nan = (w & 0x7FFF) > 0x7F80
    assert (w[nan] == 0xFFC0).all(), "the golden's NaN rows carry the x86 default NaN"
    return int(nan.any(axis=1).sum())


@pytest.mark.parametrize("single", [True, False])
def test_decode_rows_of_infinite_q(dev, single):
    g = torch.Generator("cpu").manual_seed(61)
    lens = [300, 1000, 37, 2048]
    q = torch.randn((4, 32, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((4, 8, 2048, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((4, 8, 2048, 128), generator=g).to(torch.bfloat16)
    for b, h in ((0, 5), (1, 20), (3, 31)):
        q[b, h] = (q[b, h].float() * _F).to(torch.bfloat16)
        q[b, h, 3] = float("inf")
    sl = np.asarray(lens)
    want = orc.decode(to_codes(q), to_codes(k), to_codes(v), sl, sl - 1)
    assert _nan_rows(want) >= 3
    got = to_codes(gqa.gqa_attention(q.to(dev), k.to(dev), v.to(dev), sl - 1, sl,
                                     params=gqa.make_params(stream_k=not single)))
    torch.cuda.synchronize()
    assert_within_ulp(want, got, 64, f"decode, Q heads x 2^126 ({'one launch' if single else 'three'})")


@pytest.mark.parametrize("n_new", [8, 40])
def test_chunk_rows_of_infinite_q(dev, n_new):
    """Multi-token decode (8 new tokens: the stream-K path) and a 40-token chunk (the
    prefill attention kernel): the rows of the scaled heads go to the fp64 rescore."""
    g = torch.Generator("cpu").manual_seed(62 + n_new)
    starts = [500, 77]
    cap = max(starts) + n_new
    q = torch.randn((2, n_new, 32, 128), generator=g).to(torch.bfloat16)
    kn = torch.randn((2, n_new, 8, 128), generator=g).to(torch.bfloat16)
    vn = torch.randn((2, n_new, 8, 128), generator=g).to(torch.bfloat16)
    k = torch.full((2, 8, cap, 128), float("nan"), dtype=torch.bfloat16)
    v = torch.full((2, 8, cap, 128), float("nan"), dtype=torch.bfloat16)
    for b, s in enumerate(starts):
        k[b, :, :s] = torch.randn((8, s, 128), generator=g).to(torch.bfloat16)
        v[b, :, :s] = torch.randn((8, s, 128), generator=g).to(torch.bfloat16)
    q[0, :, 9] = (q[0, :, 9].float() * _F).to(torch.bfloat16)
    q[0, :, 9, 40] = float("inf")
    q[1, 2, 30] = (q[1, 2, 30].float() * _F).to(torch.bfloat16)
    q[1, 2, 30, 100] = -float("inf")
    want = orc.prefill(to_codes(q), to_codes(k), to_codes(v), to_codes(kn), to_codes(vn), np.asarray(starts))
    assert _nan_rows(want) >= 2
    out = gqa.gqa_prefill(q.to(dev), kn.to(dev), vn.to(dev), k.to(dev), v.to(dev), starts)
    torch.cuda.synchronize()
    assert_within_ulp(want.reshape(-1, 128), to_codes(out).reshape(-1, 128), 64, f"T={n_new}, Q heads x 2^126")


@pytest.mark.parametrize("stream_k", [False, True])
def test_decode_infinite_v_beside_masked_keys(dev, stream_k):
    """V of the last key a query sees holds +inf in one dim, and the keys after it (inside the
    sequence, past the query position) are masked.  The golden never reads a masked key, so
    that dim comes out +inf.  The kernels load a masked key's V as a clamped copy of the last
    valid row; weighted by p = 0 it gave 0 * inf = NaN until masked rows were left out of the
    weighted sum.  Both launch shapes, every element against the oracle."""
    from attention_accelerator_amd import stimulus
    b = stimulus.decode_batch(3, 64, lengths=torch.tensor([40, 33, 64]), seed=71)
    qp = torch.tensor([20, 32, 50])
    for s, p in enumerate(qp.tolist()):
        b.v[s, s % 8, p, 5] = float("inf")
    want = orc.decode(to_codes(b.q), to_codes(b.k), to_codes(b.v), b.seq_len.numpy(), qp.numpy())
    got = to_codes(gqa.gqa_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), qp, b.seq_len,
                                     params=gqa.make_params(stream_k=stream_k)))
    torch.cuda.synchronize()
    w = np.asarray(want).reshape(-1, 128)
    assert (w[:, 5] == 0x7F80).sum() == 12          # 3 sequences x 4 heads: +inf in the golden
    assert_within_ulp(want, got, 64, f"decode, +inf V beside masked keys, stream_k={stream_k}")


@pytest.mark.parametrize("stream_k", [False, True])
def test_decode_nan_score_makes_the_row_nan(dev, stream_k):
    """A key whose score is NaN (K +inf in a dim where every Q head of the group is 0 after
    RoPE -- both dims of the pair zeroed -- so 0 * inf):
    the golden's max() and exp(s - max) make every weight, and so the whole row, NaN.  The fp64
    kernels clamped exp2's argument with fmax, which turned the NaN into p = 0 and left the row
    finite, until the clamp kept NaN."""
    from attention_accelerator_amd import stimulus
    b = stimulus.decode_batch(2, 300, lengths=torch.tensor([300, 170]), seed=72)
    b.q[0, 4:8, 9] = 0.0
    b.q[0, 4:8, 9 + 64] = 0.0
    b.k[0, 1, 123, 9] = float("inf")
    want = orc.decode(to_codes(b.q), to_codes(b.k), to_codes(b.v), b.seq_len.numpy(), b.query_pos.numpy())
    got = to_codes(gqa.gqa_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.query_pos, b.seq_len,
                                     params=gqa.make_params(stream_k=stream_k)))
    torch.cuda.synchronize()
    assert _nan_rows(want) == 4                      # heads 4..7 of sequence 0
    assert_within_ulp(want, got, 64, f"decode, NaN score, stream_k={stream_k}")
