"""Inputs shaped against the MFMA paths' fp64-rescore flag, every output row against the oracle.

The prefill and multi-token kernels form scores and P.V with split-operand MFMAs and fp32
accumulation; an output row goes to the fp64 rescore when one of its elements lies closer to
zero than the kernel's error estimate for it.  That estimate has to follow the two things
the error scales with:

* the magnitude of the products q_i k_i summed into each score, not the score itself:
  Q and K of large norm whose products cancel (RoPE off; 56 dim pairs (i, i + 64) with Q's
  two dims equal and K's opposite, x 2^6, N(0,1) in the other dims) give scores of N(0,1)
  size whose fp32 partial sums are ~10^4 times larger.  Variants: every product of the
  first dims positive (the largest partial sums the accumulation can carry), and pairs
  (i, i + 16) that cancel inside one 32-dim MFMA step;
* each output dimension's own V scale: V with 1, 4 or 16 channels scaled by 2^6, 2^10 or
  2^14 over every key, the other channels N(0,1).

Shapes: the chunked-prefill workload (B=4, 512 new tokens after 8192 cached positions) and
the multi-token decode workload (B=64, 16 new tokens after U[512, 8192] cached positions).
Every element within 64 BF16 ULP of the oracle (the reference checker's policy,
pyfiles/check_gqa_output.py:57-64, on the per-token golden of
pyfiles/gen_gqa_wrapper_vectors.py:121-139).  The oracle runs on the host's cores in
threads (its C loop releases the GIL)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import attention_accelerator_amd as gqa
from oracle import oracle as orc
from _util import assert_within_ulp, to_codes

pytestmark = pytest.mark.gpu

# 56 dim pairs (i, i + shift) carry the cancelling products; the rest stay N(0,1)
_NC = 56


def _inputs(starts, n_new, seed, dev):
    """N(0,1) BF16 inputs drawn on the device; cache rows >= start hold NaN."""
    g = torch.Generator(device=dev.type).manual_seed(seed)
    bsz, cap = len(starts), max(starts) + n_new
    q = torch.randn((bsz, n_new, 32, 128), generator=g, device=dev).to(torch.bfloat16)
    kn = torch.randn((bsz, n_new, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    vn = torch.randn((bsz, n_new, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((bsz, 8, cap, 128), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((bsz, 8, cap, 128), generator=g, device=dev).to(torch.bfloat16)
    for b, s in enumerate(starts):
        k[b, :, s:] = float("nan")
        v[b, :, s:] = float("nan")
    return q, kn, vn, k, v


def _outlier_channels(v, vn, n_ch, exp, seed):
    """Scale n_ch V channels (chosen from seed) by 2^exp over every key, cached and new."""
    ch = torch.from_numpy(np.random.default_rng(seed).choice(128, n_ch, replace=False))
    ch = ch.to(v.device)
    f = 2.0 ** exp
    v[..., ch] = (v[..., ch].float() * f).to(torch.bfloat16)
    vn[..., ch] = (vn[..., ch].float() * f).to(torch.bfloat16)
    return ch.tolist()


def _cancelling(q, kn, k, shift=64, aligned=False):
    """56 dims i of Q and K scaled by 2^6 (aligned: made positive), dims i + shift of Q equal
    to dim i and of K its negation: those products cancel pairwise in exact arithmetic, so
    the scores are the other dims' N(0,1) sum while the fp32 partial sums reach
    ~sqrt(56) * 2^12 (aligned: ~56 * 2^12)."""
    lo_dims = [i for i in range(128) if (i // shift) % 2 == 0][:_NC]
    lo_idx = torch.tensor(lo_dims, device=q.device)
    hi_idx = lo_idx + shift
    for t, sign in ((q, 1.0), (kn, -1.0), (k, -1.0)):
        lo = t[..., lo_idx].float() * 64.0
        if aligned:
            lo = lo.abs()
        lo = lo.to(torch.bfloat16)
        t[..., lo_idx] = lo
        t[..., hi_idx] = lo if sign > 0 else -lo


def _run_and_check(q, kn, vn, k, v, starts, what, rope=True):
    bsz, n_new, cap = q.shape[0], q.shape[1], k.shape[2]
    ws = torch.empty(gqa.prefill_workspace_bytes(bsz, n_new, cap), dtype=torch.uint8, device=q.device)
    out = gqa.gqa_prefill(q, kn, vn, k, v, starts, rope_q=rope, rope_k=rope, workspace=ws)
    torch.cuda.synchronize()
    n_rs = gqa.prefill_rescored_rows(ws, bsz, n_new, cap)
    print(f"{what}: {n_rs} of {bsz * n_new * 32} rows rescored in fp64", flush=True)
    got = to_codes(out)
    qc, knc, vnc = to_codes(q), to_codes(kn), to_codes(vn)
    # the cache as the call left it: rows < start as given (the chunk's rows are the
    # append's, which the oracle forms from the new rows itself)
    kc, vc = to_codes(k), to_codes(v)
    want, want64 = orc.prefill(qc, kc, vc, knc, vnc, np.asarray(starts), rope_q=rope,
                               rope_k_new=rope, want_f64=True, threads=orc.host_threads())
    return assert_within_ulp(want.reshape(-1, 128), got.reshape(-1, 128), 64, what,
                             ref64=want64.reshape(-1, 128))


_PREFILL_STARTS = [8192] * 4


def _ragged_starts(seed=20260805):
    return [int(x) for x in np.random.default_rng(seed).integers(512, 8193, size=64)]


def test_prefill_config5_all_rows(dev):
    """B=4, 512 new tokens over 8192 cached positions, N(0,1): all 2,048 query rows (65,536
    output rows of 128) against the oracle."""
    q, kn, vn, k, v = _inputs(_PREFILL_STARTS, 512, 20260805, dev)
    w = _run_and_check(q, kn, vn, k, v, _PREFILL_STARTS, "config 5, all rows")
    print(f"config 5 all rows: worst {w} ULP")


@pytest.mark.parametrize("n_ch,exp", [(1, 14), (4, 10), (16, 6)])
def test_prefill_outlier_v_channels(dev, n_ch, exp):
    q, kn, vn, k, v = _inputs(_PREFILL_STARTS, 512, 100 + n_ch, dev)
    ch = _outlier_channels(v, vn, n_ch, exp, n_ch)
    _run_and_check(q, kn, vn, k, v, _PREFILL_STARTS, f"prefill, V channels {ch} x 2^{exp}")


_CANCEL = [(64, False), (64, True), (16, False)]


@pytest.mark.parametrize("shift,aligned", _CANCEL)
def test_prefill_cancelling_scores(dev, shift, aligned):
    q, kn, vn, k, v = _inputs(_PREFILL_STARTS, 512, 7 + shift, dev)
    _cancelling(q, kn, k, shift, aligned)
    _run_and_check(q, kn, vn, k, v, _PREFILL_STARTS,
                   f"prefill, cancelling products (i, i+{shift}){' aligned' if aligned else ''}", rope=False)


@pytest.mark.parametrize("n_ch", [1, 4, 16])
@pytest.mark.parametrize("exp", [6, 10, 14])
def test_multi_outlier_v_channels(dev, n_ch, exp):
    starts = _ragged_starts()
    q, kn, vn, k, v = _inputs(starts, 16, 200 + n_ch + exp, dev)
    ch = _outlier_channels(v, vn, n_ch, exp, n_ch + exp)
    _run_and_check(q, kn, vn, k, v, starts, f"multi-token T=16, V channels {ch} x 2^{exp}")


@pytest.mark.parametrize("n_new,shift,aligned", [(4, 64, False), (16, 64, False), (16, 64, True),
                                                 (8, 16, False)])
def test_multi_cancelling_scores(dev, n_new, shift, aligned):
    starts = _ragged_starts()
    q, kn, vn, k, v = _inputs(starts, n_new, 9 + n_new + shift, dev)
    _cancelling(q, kn, k, shift, aligned)
    _run_and_check(q, kn, vn, k, v, starts, f"multi-token T={n_new}, cancelling products "
                   f"(i, i+{shift}){' aligned' if aligned else ''}", rope=False)


def test_decode_cancelling_and_outliers(dev):
    """The decode path (fp64 throughout) on both shapes at once, B=64 ragged."""
    starts = _ragged_starts()
    q, kn, vn, k, v = _inputs(starts, 1, 11, dev)
    _cancelling(q, kn, k)
    _outlier_channels(v, vn, 4, 14, 3)
    qd = q[:, 0].contiguous()
    sl = torch.tensor(starts, dtype=torch.int32)
    got = to_codes(gqa.gqa_attention(qd, k, v, sl - 1, sl, rope_q=False))
    torch.cuda.synchronize()
    want = orc.decode(to_codes(qd), to_codes(k), to_codes(v), np.asarray(starts),
                      np.asarray(starts) - 1, rope_q=False)
    assert_within_ulp(want, got, 64, "decode, cancelling products + V channels x 2^14")


@pytest.mark.parametrize("n_new,huge", [(16, "chunk"), (32, "cached")])
def test_zero_weight_huge_v(dev, n_new, huge):
    """V rows the softmax gives no weight set each dim's largest |V| far above the outputs:
    Q x 2^10 (scores ~3000 in natural-log units, the softmax peaked on a cached key or two)
    and keys that score ~0 (weight exactly 0) with huge V -- the chunk's own rows, K x 2^-100
    and V x 2^100 (T=16, the multi-token merge's decision), or cached positions 0..63, K x
    2^-40 and V x 2^90, one staging block of their own that stays inside the staging range
    (T=32, the prefill kernel's decision; in the chunk's block, or past 2^100, they would mark
    their block unstageable and every row would be rescored anyway).  Each element in units
    of its dim's largest |V| is then ~2^-90 or less, and the flag decision has to form its
    squares without underflow: in fp32 every square was zero, no row was flagged, and rows
    whose output cancels between two near-tied keys missed 64 ULP (found by a wider run of
    the random-shape draw, multi-token seed 66941)."""
    starts = [int(x) for x in np.random.default_rng(77).integers(135, 1104, size=8)]
    q, kn, vn, k, v = _inputs(starts, n_new, 77 + n_new, dev)
    q = (q.float() * 2.0 ** 10).to(torch.bfloat16)
    if huge == "chunk":
        kn = (kn.float() * 2.0 ** -100).to(torch.bfloat16)
        vn = (vn.float() * 2.0 ** 100).to(torch.bfloat16)
    else:
        k[:, :, :64] = (k[:, :, :64].float() * 2.0 ** -40).to(torch.bfloat16)
        v[:, :, :64] = (v[:, :, :64].float() * 2.0 ** 90).to(torch.bfloat16)
    _run_and_check(q, kn, vn, k, v, starts, f"T={n_new}, zero-weight huge V ({huge} keys)")


def test_prefill_tiny_weight_huge_v(dev):
    """Keys of tiny weight and huge V (prefill, T=64): Q x 2^4 (scores up to ~50 in natural-log
    units) and the chunk's V x 2^40.  The chunk keys' weights reach down to ~1e-13, yet times V
    ~1e12 they add ~0.1 to O(1) outputs; in the kernel's fp16 split such a p lies below 2^-25
    and is dropped.  The attention loop bounds what fp16's subnormal quantum can add to each
    element and the row is rescored where that bound reaches its smallest element (found by a
    wider run of the random-shape draw, prefill seed 87509: 776 elements off by up to 3 %)."""
    starts = [320, 700]
    q, kn, vn, k, v = _inputs(starts, 64, 87, dev)
    q = (q.float() * 2.0 ** 4).to(torch.bfloat16)
    vn = (vn.float() * 2.0 ** 40).to(torch.bfloat16)
    _run_and_check(q, kn, vn, k, v, starts, "prefill T=64, Q x 2^4, chunk V x 2^40")


def test_multi_tiny_weight_huge_v(dev):
    """Multi-token, T=16: Q x 2^6 (scores up to ~300 in log2 units) and the chunk's V x 2^120,
    near the BF16 maximum.  Chunk keys whose p lies below fp32's normal range are lost (to
    v_exp_f32's flush or the BF16 split), yet times V ~2^121 they add ~0.01 to the outputs.
    The merge bounds that loss per element (capacity * 2^-123 of D_j) and rescores the rows
    where it reaches an element (found by a run of the random-shape draw with scales 2^+-2 ..
    2^+-120: nine multi-token draws off by up to 30,911 ULP)."""
    starts = [int(x) for x in np.random.default_rng(134).integers(256, 700, size=4)]
    q, kn, vn, k, v = _inputs(starts, 16, 134, dev)
    q = (q.float() * 2.0 ** 6).to(torch.bfloat16)
    vn = (vn.float() * 2.0 ** 120).to(torch.bfloat16)
    _run_and_check(q, kn, vn, k, v, starts, "multi-token T=16, Q x 2^6, chunk V x 2^120")
