"""Multi-token decode (chunks of 1..16 new tokens per sequence: speculative drafts, a few
steps of one sequence at once) through gqa_prefill, which sends chunks of up to 16 tokens
down the stream-K path (key ranges split over all CUs, per-range partials merged; one wave
per 16 query columns, 1, 2 or 4 waves per workgroup) and longer ones through the prefill
attention kernel.  Every output row is checked against the compiled oracle's
per-token reference step (the one-token golden of pyfiles/gen_gqa_wrapper_vectors.py:
121-139 per new token, new K rotated at its position, not re-rounded), within 64 BF16 ULP
with the reference checker's tiny-value exemption (pyfiles/check_gqa_output.py:33-34,57-64).
Cache rows past the chunk hold NaN, so a read of one would poison the output."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import attention_accelerator_amd as gqa
from oracle import oracle as orc
from _util import assert_within_ulp, to_codes

pytestmark = pytest.mark.gpu


def _chunk(starts, n_new, capacity, seed):
    """N(0,1) BF16 inputs; cache rows < start random, rows >= start NaN."""
    g = torch.Generator("cpu").manual_seed(seed)
    batch = len(starts)
    q = torch.randn((batch, n_new, 32, 128), generator=g).to(torch.bfloat16)
    kn = torch.randn((batch, n_new, 8, 128), generator=g).to(torch.bfloat16)
    vn = torch.randn((batch, n_new, 8, 128), generator=g).to(torch.bfloat16)
    k = torch.full((batch, 8, capacity, 128), float("nan"), dtype=torch.bfloat16)
    v = torch.full((batch, 8, capacity, 128), float("nan"), dtype=torch.bfloat16)
    for b, s in enumerate(starts):
        k[b, :, :s] = torch.randn((8, s, 128), generator=g).to(torch.bfloat16)
        v[b, :, :s] = torch.randn((8, s, 128), generator=g).to(torch.bfloat16)
    return q, kn, vn, k, v


def _oracle(q, kn, vn, k, v, starts, rope_q=True, rope_k=True):
    """The oracle's BF16 rows and their double-precision values."""
    return orc.prefill(to_codes(q), to_codes(k), to_codes(v), to_codes(kn), to_codes(vn),
                       np.asarray(starts), rope_q=rope_q, rope_k_new=rope_k, want_f64=True)


def _check(want, got, what):
    """64 BF16 ULP per element (an output row that cancels to near zero is rescored in fp64
    by the library); returns the worst distance."""
    return assert_within_ulp(want[0], got, 64, what, ref64=want[1])


def _run(q, kn, vn, k, v, starts, dev, **kw):
    kd, vd = k.to(dev), v.to(dev)
    out = gqa.gqa_prefill(q.to(dev), kn.to(dev), vn.to(dev), kd, vd, starts, **kw)
    torch.cuda.synchronize()
    return to_codes(out), kd, vd


# Starts at 0 (the chunk sees only itself), inside the first 16-key range, on and off
# range boundaries, and long enough to span several workgroups' ranges.
_STARTS = [0, 1, 15, 16, 33, 700, 2047, 4100]


@pytest.mark.parametrize("n_new", [1, 2, 3, 4, 5, 8, 11, 16])
def test_multi_all_rows_against_oracle(dev, n_new):
    """Every output row (up to 8 x 16 x 32 x 128 = 524,288 elements) within 64 ULP of the
    oracle.  At T=16 one element of these inputs cancels to 2.0e-9 (10^7 times smaller than
    its neighbours): the MFMA kernels' fp32 scores put it at -5.8e-9, so its row is flagged
    and rescored in fp64."""
    starts = _STARTS
    q, kn, vn, k, v = _chunk(starts, n_new, max(starts) + n_new + 5, 30 + n_new)
    want = _oracle(q, kn, vn, k, v, starts)
    got, kd, vd = _run(q, kn, vn, k, v, starts, dev)
    _check(want, got, f"multi T={n_new}")
    kc, vc = to_codes(kd), to_codes(vd)
    for b, s in enumerate(starts):
        assert np.array_equal(vc[b, :, s:s + n_new], to_codes(vn[b]).transpose(1, 0, 2))
        assert (kc[b, :, s + n_new:] == to_codes(k[b, :, s + n_new:])).all()


@pytest.mark.parametrize("q_scale,seed", [(16.0, 7), (64.0, 8)])
def test_multi_peaked_scores(dev, q_scale, seed):
    """Q scaled up by a power of two (a peaked softmax): the fp32 score sums err in
    proportion to the scores, and the rows sent to the fp64 rescore follow the row's max;
    every element within 64 ULP of the oracle (T = 16, four sequences)."""
    starts = [900, 2100, 3000, 1777]
    q, kn, vn, k, v = _chunk(starts, 16, 3100, seed)
    q = (q.float() * q_scale).to(torch.bfloat16)
    want = _oracle(q, kn, vn, k, v, starts)
    got, _, _ = _run(q, kn, vn, k, v, starts, dev)
    _check(want, got, f"T=16, Q x{q_scale:g}")


@pytest.mark.parametrize("q_exp,k_exp", [(100, 40), (64, 64)])
def test_multi_scores_past_fp32_range(dev, q_exp, k_exp):
    """One Q head scaled by 2^q_exp and one KV head's keys (cached and new) by 2^k_exp: their
    dot products pass the fp32 range, so the MFMA kernels' rows for them are not finite, and
    those rows go to the fp64 rescore, which matches the double golden; every row within
    64 ULP of the oracle."""
    starts = [500, 300]
    q, kn, vn, k, v = _chunk(starts, 8, 700, 3)
    q[0, :, 5] = (q[0, :, 5].float() * 2.0 ** q_exp).to(torch.bfloat16)
    k[0, 1, :500] = (k[0, 1, :500].float() * 2.0 ** k_exp).to(torch.bfloat16)
    kn[0, :, 1] = (kn[0, :, 1].float() * 2.0 ** k_exp).to(torch.bfloat16)
    want = _oracle(q, kn, vn, k, v, starts)
    got, _, _ = _run(q, kn, vn, k, v, starts, dev)
    _check(want, got, f"T=8, Q x2^{q_exp}, K x2^{k_exp}")


def test_multi_no_rope(dev):
    starts = [3, 260, 1500]
    q, kn, vn, k, v = _chunk(starts, 3, 1510, 40)
    want = _oracle(q, kn, vn, k, v, starts, rope_q=False, rope_k=False)
    got, kd, _ = _run(q, kn, vn, k, v, starts, dev, rope_q=False, rope_k=False)
    _check(want, got, "multi no rope")
    assert np.array_equal(to_codes(kd)[1, 5, 260:263], to_codes(kn[1, :, 5]))


def test_multi_long_sequences(dev):
    """8192 cached positions (the longest of the decode workloads) beside short ones."""
    starts = [8188, 3001, 9]
    q, kn, vn, k, v = _chunk(starts, 4, 8192, 41)
    want = _oracle(q, kn, vn, k, v, starts)
    got, _, _ = _run(q, kn, vn, k, v, starts, dev)
    _check(want, got, "multi long")


@pytest.mark.parametrize("n_new,bsz", [(4, 150), (9, 70), (16, 130)])
def test_multi_many_sequences(dev, n_new, bsz):
    """More than 64 sequences: the plan, each workgroup's search for its first piece and the
    merge take the batch 64 sequences at a time, so the second and third windows of 64 are
    used here.  Ragged starts 0..600 (short segments, many pieces per workgroup range):
    every output row within the tolerance of the oracle."""
    rng = np.random.default_rng(60 + n_new)
    starts = [int(x) for x in rng.integers(0, 601, size=bsz)]
    q, kn, vn, k, v = _chunk(starts, n_new, max(starts) + n_new, 60 + n_new)
    want = _oracle(q, kn, vn, k, v, starts)
    got, _, _ = _run(q, kn, vn, k, v, starts, dev)
    _check(want, got, f"multi T={n_new} B={bsz}")


@pytest.mark.parametrize("n_new,n_wgs", [(4, "1"), (4, "7"), (4, "64"), (4, "333"), (4, "4096"),
                                         (7, "2"), (7, "130"), (12, "4"), (12, "37"), (16, "1024")])
def test_multi_partition_counts(dev, n_new, n_wgs):
    """The split of the keys over workgroups (params.stream_wgs: that many one-wave
    workgroups for T <= 4, twice as many waves in workgroups of 2 or 4 for longer chunks)
    changes the order of the partial sums only: every split stays within the tolerance of
    the oracle."""
    starts = [5, 1200, 64, 2999, 0, 17]
    q, kn, vn, k, v = _chunk(starts, n_new, 3016, 42)
    want = _oracle(q, kn, vn, k, v, starts)
    got, _, _ = _run(q, kn, vn, k, v, starts, dev, params=gqa.make_params(rope_k=True, stream_wgs=int(n_wgs)))
    _check(want, got, f"multi T={n_new} wgs={n_wgs}")


@pytest.mark.parametrize("n_new", [4, 16])
def test_multi_and_prefill_kernel_agree(dev, n_new):
    """The same chunk through the stream-K path and through the prefill attention kernel
    (params without the multi-token plan): both within the tolerance of the oracle, caches
    bit-identical."""
    starts = [77, 1024, 300]
    q, kn, vn, k, v = _chunk(starts, n_new, 1100, 43)
    want = _oracle(q, kn, vn, k, v, starts)
    a, ka, va = _run(q, kn, vn, k, v, starts, dev)
    b, kb, vb = _run(q, kn, vn, k, v, starts, dev, params=gqa.make_params(rope_k=True, multi_token=False))
    _check(want, a, "stream-K path")
    _check(want, b, "prefill kernel path")
    assert np.array_equal(to_codes(ka), to_codes(kb)) and np.array_equal(to_codes(va), to_codes(vb))


@pytest.mark.parametrize("n_new,t", [(4, 3), (16, 9), (16, 15)])
def test_multi_causal_independence(dev, n_new, t):
    """Token t's row does not depend on the chunk's later tokens: perturbing the Q, K and V
    of tokens t.. leaves rows 0..t-1 bit-identical."""
    starts = [400, 31]
    q, kn, vn, k, v = _chunk(starts, n_new, 420, 44)
    ref, _, _ = _run(q, kn, vn, k, v, starts, dev)
    q2, kn2, vn2 = q.clone(), kn.clone(), vn.clone()
    q2[:, t:] = torch.randn(q2[:, t:].shape).to(torch.bfloat16) * 3
    kn2[:, t:] = torch.randn(kn2[:, t:].shape).to(torch.bfloat16) * 4
    vn2[:, t:] = torch.randn(vn2[:, t:].shape).to(torch.bfloat16) * 4
    got, _, _ = _run(q2, kn2, vn2, k, v, starts, dev)
    assert np.array_equal(got[:, :t], ref[:, :t])
    assert not np.array_equal(got[:, t], ref[:, t])


def test_multi_position_major_cache(dev):
    """Cache stored [B][S][8][128]: the same bits as head-major."""
    starts = [45, 130, 0]
    q, kn, vn, k, v = _chunk(starts, 2, 140, 45)
    want, kd_ref, _ = _run(q, kn, vn, k, v, starts, dev)
    kp = k.permute(0, 2, 1, 3).contiguous().to(dev).permute(0, 2, 1, 3)
    vp = v.permute(0, 2, 1, 3).contiguous().to(dev).permute(0, 2, 1, 3)
    got = to_codes(gqa.gqa_prefill(q.to(dev), kn.to(dev), vn.to(dev), kp, vp, starts))
    torch.cuda.synchronize()
    assert np.array_equal(got, want)
    assert np.array_equal(to_codes(kp), to_codes(kd_ref))


@pytest.mark.parametrize("n_new", [3, 7, 10])
def test_multi_invalid_device_start_gives_nan_rows(dev, n_new):
    """A device start past capacity - T: NaN rows for that sequence, its cache untouched,
    the other sequences unaffected (one- and two-wave stream-K kernels, prefill kernel)."""
    starts = torch.tensor([40, 98, 7], dtype=torch.int32)   # sequence 1: 98 + T > 100
    q, kn, vn, k, v = _chunk([40, 0, 7], n_new, 100, 46)
    kd, vd = k.to(dev), v.to(dev)
    out = gqa.gqa_prefill(q.to(dev), kn.to(dev), vn.to(dev), kd, vd, starts.to(dev))
    torch.cuda.synchronize()
    got = to_codes(out)
    assert (got[1] == 0x7FC0).all()
    assert np.array_equal(to_codes(kd)[1], to_codes(k)[1])
    idx = [0, 2]
    want = _oracle(q[idx], kn[idx], vn[idx], k[idx], v[idx], [40, 7])
    _check(want, got[idx], "valid beside invalid")


def test_multi_workspace_garbage_and_repeat(dev):
    """A workspace full of 0xFF gives the same bits (the plan, partials and Q operands are
    all written before they are read), and a PreparedPrefill repeats them call after call."""
    starts = [128, 0, 777, 5]
    q, kn, vn, k, v = _chunk(starts, 4, 790, 47)
    a, _, _ = _run(q, kn, vn, k, v, starts, dev)
    ws = torch.empty(gqa.prefill_workspace_bytes(4, 4, k.shape[2]), dtype=torch.uint8, device=dev)
    ws.fill_(0xFF)
    b, _, _ = _run(q, kn, vn, k, v, starts, dev, workspace=ws)
    assert np.array_equal(a, b)
    kd, vd = k.to(dev), v.to(dev)
    call = gqa.PreparedPrefill(q.to(dev), kn.to(dev), vn.to(dev), kd, vd,
                               torch.tensor(starts, dtype=torch.int32, device=dev))
    for _ in range(3):
        got = to_codes(call())
        torch.cuda.synchronize()
        assert np.array_equal(got, a)


def test_multi_two_byte_aligned_inputs(dev):
    """Q and the new K/V rows at 2-byte (not 16-byte) aligned addresses take the preparation
    kernel's element-wise loads: the same bits as aligned inputs."""
    starts = [300, 9]
    q, kn, vn, k, v = _chunk(starts, 3, 320, 48)
    want, _, _ = _run(q, kn, vn, k, v, starts, dev)

    def shifted(x):
        flat = torch.empty(x.numel() + 1, dtype=x.dtype, device=dev)
        view = flat[1:].view(x.shape)
        view.copy_(x.to(dev))
        return view

    qs, kns, vns = shifted(q), shifted(kn), shifted(vn)
    assert qs.data_ptr() % 16 != 0 and kns.data_ptr() % 16 != 0
    kd, vd = k.to(dev), v.to(dev)
    got = to_codes(gqa.gqa_prefill(qs, kns, vns, kd, vd, starts))
    torch.cuda.synchronize()
    assert np.array_equal(got, want)


@pytest.mark.parametrize("skew", ["0", "250"])
def test_multi_xcd_skew_bounds(dev, monkeypatch, skew):
    """Equal ranges (skew 0) and the largest XCD weighting (odd ranges 3/4 of the size, even
    ones 5/4) over a short and a long batch: every row within the tolerance of the oracle."""
    monkeypatch.setenv("GQA_XCD_SKEW", skew)
    starts = [5, 1200, 64, 2999, 0, 17, 640]
    q, kn, vn, k, v = _chunk(starts, 4, 3010, 49)
    want = _oracle(q, kn, vn, k, v, starts)
    got, _, _ = _run(q, kn, vn, k, v, starts, dev, params=gqa.make_params(rope_k=True, stream_wgs=96))
    _check(want, got, f"multi skew={skew}")


def test_multi_long_context_sampled_rows(dev):
    """131,064 cached positions (the longest decode workload's capacity) and 8 new tokens:
    the first and last token's rows against the oracle (each sees 131,065 .. 131,072 keys)."""
    st, n_new, cap = 131064, 8, 131072
    g = torch.Generator("cpu").manual_seed(50)
    q = torch.randn((1, n_new, 32, 128), generator=g).to(torch.bfloat16)
    kn = torch.randn((1, n_new, 8, 128), generator=g).to(torch.bfloat16)
    vn = torch.randn((1, n_new, 8, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((1, 8, cap, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((1, 8, cap, 128), generator=g).to(torch.bfloat16)
    got, _, _ = _run(q, kn, vn, k, v, [st], dev)
    rows = [0, n_new - 1]
    want, want64 = orc.prefill(to_codes(q), to_codes(k), to_codes(v), to_codes(kn), to_codes(vn),
                               np.asarray([st]), rows=rows, want_f64=True)
    assert_within_ulp(want, got[:, rows], 64, "multi 131072", ref64=want64)


@pytest.mark.parametrize("n_wgs", ["1", "7", "64", "1024"])
@pytest.mark.parametrize("heads", ["all", "one per kv head"])
def test_rescore_pieces(dev, n_wgs, heads):
    """Rows forced to the fp64 rescore.  Every head: Q scaled by 2^100 and K by 2^40, so
    every dot product passes the fp32 range and all 64 rows (2 sequences x 1 token x 32
    heads, 4 per (sequence, KV head)) of the MFMA kernels come out not finite -- the tiles
    path, four rows as the columns of one fp64 MFMA chunk.  One head per KV head: those Q
    rows scaled by 2^100 (scores ~2^100, far past the flag's bound), 16 rows, one per pair --
    the rows path, each row's keys cut into pieces in proportion to its length (a row of 3001
    keys gets about 30 times the pieces of one of 91).  Rescore grids of 1 (fewer workgroups
    than rows), 7, 64 and 1024 workgroups (params.stream_wgs sets the grid).  Every row must
    match the oracle, and V dimension 5, zero in every key, exactly."""
    p = gqa.make_params(rope_k=True, stream_wgs=int(n_wgs))
    starts = [90, 3000]
    q, kn, vn, k, v = _chunk(starts, 1, 3001, 77)
    vn[..., 5] = 0.0
    for b, s in enumerate(starts):
        v[b, :, :s, 5] = 0.0
    hs = list(range(32)) if heads == "all" else list(range(0, 32, 4))
    q[:, :, hs] = (q[:, :, hs].float() * 2.0 ** 100).to(torch.bfloat16)
    if heads == "all":
        kn = (kn.float() * 2.0 ** 40).to(torch.bfloat16)
        k = (k.float() * 2.0 ** 40).to(torch.bfloat16)
    want = _oracle(q, kn, vn, k, v, starts)
    ws = torch.empty(gqa.prefill_workspace_bytes(2, 1, 3001, params=p), dtype=torch.uint8, device=dev)
    got, _, _ = _run(q, kn, vn, k, v, starts, dev, workspace=ws, params=p)
    n_rs = gqa.prefill_rescored_rows(ws, 2, 1, 3001, params=p)
    assert n_rs == 64 if heads == "all" else 16 <= n_rs < 32
    assert np.all(got[..., 5] == 0)
    _check(want, got.reshape(-1, 128), f"{n_rs} flagged rows ({heads}), {n_wgs} rescore workgroups")


@pytest.mark.parametrize("n_new,rope_q,rope_k", [
    (4, True, True),      # stream-K path, every row flagged: more rows than rescore workgroups
    (16, True, False),    # Q rotated with the cos/sin rows, the chunk's keys read as stored
    (40, True, True),     # prefill attention kernel path
    (24, False, False),   # no RoPE at all
])
def test_every_row_rescored(dev, n_new, rope_q, rope_k):
    """V dimension 5 is exactly zero in every row, so every output row holds an exact zero
    and is flagged for the fp64 rescore (min |x| = 0 < 2^-17 rms): the rescore runs with
    one piece per row (more flagged rows than workgroups) and must reproduce every row of
    the oracle, the zero dimension exactly."""
    starts = [37, 300, 1000, 8, 513, 64, 2049, 129][: 8 if n_new <= 16 else 3]
    cap = max(starts) + n_new
    q, kn, vn, k, v = _chunk(starts, n_new, cap, 40 + n_new)
    vn[..., 5] = 0.0
    for b, s in enumerate(starts):
        v[b, :, :s, 5] = 0.0
    want = _oracle(q, kn, vn, k, v, starts, rope_q=rope_q, rope_k=rope_k)
    got, _, _ = _run(q, kn, vn, k, v, starts, dev, rope_q=rope_q, rope_k=rope_k)
    assert np.all(got[..., 5] == 0)
    w = _check(want, got.reshape(-1, 128), f"T={n_new} rope_q={rope_q} rope_k={rope_k}, all rows rescored")
    print("worst ULP", w)
