"""Decode kernel parity against the compiled oracle (oracle/oracle.py) on N(0,1)
BF16 inputs, the masking rules, and size-independent properties.

Tolerance: 64 BF16 ULP per element with the reference checker's tiny-value
exemption (pyfiles/check_gqa_output.py:33-34,57-64).  Cache rows that the mask
excludes hold NaN, so any read of one would poison the output."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import attention_accelerator_amd as gqa
from attention_accelerator_amd import stimulus
from oracle import golden_model as gm
from oracle import oracle as orc
from _util import assert_within_ulp, to_codes, to_dev

pytestmark = pytest.mark.gpu


def _codes(t: torch.Tensor) -> np.ndarray:
    return to_codes(t)


def _oracle(batch: stimulus.DecodeBatch, rope_k=False, kv_heads=None, want_f64=False):
    return orc.decode(_codes(batch.q), _codes(batch.k), _codes(batch.v),
                      batch.seq_len.numpy(), batch.query_pos.numpy(), rope_k=rope_k,
                      kv_heads=kv_heads, want_f64=want_f64)


def _run(batch: stimulus.DecodeBatch, dev, **kw):
    out = gqa.gqa_attention(batch.q.to(dev), batch.k.to(dev), batch.v.to(dev),
                            batch.query_pos, batch.seq_len, **kw)
    torch.cuda.synchronize()
    return _codes(out)


def test_golden_smoke_normal_len30(dev):
    """The golden smoke case: N(0,1), SEQ_LEN=30, qpos 29, RoPE on Q and K."""
    q, k, v = gm.stimulus("normal", 30, 20260805)
    want = np.array(gm.golden_attention(q, k, v, 30, 29), dtype=np.uint16)
    got = _codes(gqa.gqa_attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), 29, 30,
                                   rope_q=True, rope_k=True))
    assert_within_ulp(want, got, 64, "normal L=30")


def test_single_sequence_4096(dev):
    """B=1, L=4096, qpos 4095, K cache post-RoPE (only Q rotated)."""
    b = stimulus.decode_batch(1, 4096, seed=11)
    want, want64 = _oracle(b, want_f64=True)
    w = assert_within_ulp(want, _run(b, dev), 64, "L=4096", ref64=want64)
    print("worst ULP", w)


@pytest.mark.parametrize("seed", [1, 2])
def test_ragged_batch(dev, seed):
    b = stimulus.decode_batch(12, 1536, min_len=1, max_len=1536, seed=seed)
    assert_within_ulp(_oracle(b), _run(b, dev), 64, f"ragged seed {seed}")


def test_causal_mask_differs_from_padding(dev):
    """query_position < seq_len - 1: rows qpos+1 .. seq_len-1 are valid cache rows that
    the causal mask excludes; they hold NaN here and must not be read."""
    g = torch.Generator().manual_seed(5)
    lengths = torch.randint(2, 700, (6,), generator=g).to(torch.int32)
    b = stimulus.decode_batch(6, 704, lengths=lengths, seed=6)
    qpos = torch.tensor([int(torch.randint(0, int(x) - 1, (1,), generator=g)) for x in lengths],
                        dtype=torch.int32)
    k, v = b.k.clone(), b.v.clone()
    for i in range(6):
        k[i, :, int(qpos[i]) + 1:] = float("nan")
        v[i, :, int(qpos[i]) + 1:] = float("nan")
    b = stimulus.DecodeBatch(b.q, k, v, b.seq_len, qpos)
    got = _run(b, dev)
    assert np.isfinite(got.view(np.int16).astype(np.float32)).all()
    assert_within_ulp(_oracle(b), got, 64, "causal")


def test_seq_len_one_is_v0_exactly(dev):
    """One visible key: weight 1, output = V[0] bit for bit."""
    b = stimulus.decode_batch(3, 64, lengths=torch.tensor([1, 1, 1]), seed=7)
    got = _run(b, dev)
    v0 = _codes(b.v[:, :, 0])                      # [B, 8, 128]
    want = np.repeat(v0, 4, axis=1)                # Q head h uses KV head h // 4
    assert np.array_equal(got, want)


def test_equal_scores_give_mean_of_v(dev):
    """Smoke mode of the reference generator: Q = K = 0, every visible score equal,
    output = BF16(mean of V rows 0..qpos) (pyfiles/gen_gqa_wrapper_vectors.py:4-7)."""
    q, k, v = gm.stimulus("smoke", 45, 1)
    got = _codes(gqa.gqa_attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), 40, 45,
                                   rope_q=True, rope_k=True))
    vv = (np.array(v, dtype=np.uint32) << 16).view(np.float32).astype(np.float64)
    mean = vv[:, :41].mean(axis=1)                              # [8, 128]
    want = np.array([[gm.f32_to_bf16(x) for x in mean[h // 4]] for h in range(32)],
                    dtype=np.uint16)
    assert_within_ulp(want, got, 2, "mean of V")


def test_deterministic(dev):
    b = stimulus.decode_batch(8, 2048, min_len=100, max_len=2048, seed=8)
    assert np.array_equal(_run(b, dev), _run(b, dev))


@pytest.mark.parametrize("wgs", ["1", "7", "333", "2048", "6000"])
def test_stream_partition_invariance(dev, wgs):
    """The key space cut into 1 .. 6000 workgroup ranges (pieces start and end at
    arbitrary keys, ranges span several sequences and heads, up to 47 pieces per
    segment): same parity."""
    b = stimulus.decode_batch(5, 3000, min_len=1, max_len=3000, seed=9)
    got = _run(b, dev, params=gqa.make_params(stream_k=True, stream_wgs=int(wgs)))
    assert_within_ulp(_oracle(b), got, 64, f"{wgs} workgroups")


@pytest.mark.parametrize("skew", ["0", "250"])
@pytest.mark.parametrize("wgs", ["7", "333", "2048"])
def test_stream_xcd_skew_bounds(dev, wgs, skew, monkeypatch):
    """Equal ranges (skew 0) and the largest XCD weighting (odd ranges 3/4 of the range
    size, even ones 5/4): the same parity on the stream and paged-free path."""
    b = stimulus.decode_batch(5, 3000, min_len=1, max_len=3000, seed=10)
    monkeypatch.setenv("GQA_XCD_SKEW", skew)
    got = _run(b, dev, params=gqa.make_params(stream_k=True, stream_wgs=int(wgs)))
    assert_within_ulp(_oracle(b), got, 64, f"{wgs} workgroups, skew={skew}")


@pytest.mark.parametrize("wgs", ["16", "200", "1024", "5000"])
def test_single_launch_pieces(dev, wgs):
    """Small batches run as one launch whose pieces (256 keys and up, here 256 .. 18432)
    merge in-kernel: parity for every piece size, and the stream-K path agrees to 1 BF16
    ULP (both carry every step in fp64; only the order of the sums differs)."""
    b = stimulus.decode_batch(4, 2300, min_len=1, max_len=2300, seed=19)
    single = _run(b, dev, params=gqa.make_params(stream_wgs=int(wgs)))
    want = _oracle(b)
    assert_within_ulp(want, single, 64, f"single launch, {wgs}")
    stream = _run(b, dev, params=gqa.make_params(stream_k=True, stream_wgs=int(wgs)))
    assert_within_ulp(stream, single, 1, "single launch vs stream-K")


def test_single_launch_workspace_init_and_reuse(dev):
    """The single-launch path counts finished pieces in the workspace: after
    gqa_decode_workspace_init (here over garbage) one workspace serves many calls in a row,
    each leaving the counters at zero (same bits every time)."""
    import ctypes
    from attention_accelerator_amd._lib import lib
    b = stimulus.decode_batch(2, 4096, seed=20)
    want = _oracle(b)
    nbytes = gqa.decode_workspace_bytes(2, 4096)
    ref = None
    for fill in (0xFF, 0x5A):
        ws = torch.full((nbytes,), fill, dtype=torch.uint8, device=dev)
        p = gqa.make_params()
        assert lib().gqa_decode_workspace_init(ctypes.byref(p), 2, 4096, ws.data_ptr(), nbytes,
                                               torch.cuda.current_stream().cuda_stream) == 0
        for _ in range(4):
            got = _codes(gqa.gqa_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.query_pos,
                                           b.seq_len, workspace=ws))
            if ref is None:
                assert_within_ulp(want, got, 64, "single launch")
                ref = got
            assert np.array_equal(got, ref)


def test_workspace_reuse_across_calls(dev):
    """A prepared call reuses one workspace: repeated calls give identical bits, and
    the same workspace then serves other inputs."""
    from attention_accelerator_amd.attention import PreparedDecode
    sk = gqa.make_params(stream_k=True)
    b = stimulus.decode_batch(6, 2500, min_len=1, max_len=2500, seed=17)
    ref = _run(b, dev, params=sk)
    call = PreparedDecode(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.query_pos.to(dev),
                          b.seq_len.to(dev), params=sk)
    for _ in range(3):
        out = call()
        torch.cuda.synchronize()
        assert np.array_equal(_codes(out), ref)
    # same workspace, other contents
    b2 = stimulus.decode_batch(6, 2500, min_len=1, max_len=2500, seed=18)
    out2 = gqa.gqa_attention(b2.q.to(dev), b2.k.to(dev), b2.v.to(dev), b2.query_pos, b2.seq_len,
                             workspace=call.workspace, params=sk)
    assert_within_ulp(_oracle(b2), _codes(out2), 64, "reused workspace")


def test_position_major_cache_layout(dev):
    """Cache stored [B][S][8][128] (position-major) gives the same bits as [B][8][S][128]."""
    b = stimulus.decode_batch(3, 500, min_len=200, max_len=500, seed=10)
    ref = _run(b, dev)
    kp = b.k.permute(0, 2, 1, 3).contiguous().to(dev).permute(0, 2, 1, 3)
    vp = b.v.permute(0, 2, 1, 3).contiguous().to(dev).permute(0, 2, 1, 3)
    out = gqa.gqa_attention(b.q.to(dev), kp, vp, b.query_pos, b.seq_len)
    assert np.array_equal(_codes(out), ref)


def test_no_rope(dev):
    b = stimulus.decode_batch(2, 300, min_len=100, max_len=300, seed=12)
    want = orc.decode(_codes(b.q), _codes(b.k), _codes(b.v), b.seq_len.numpy(),
                      b.query_pos.numpy(), rope_q=False, rope_k=False)
    got = _run(b, dev, rope_q=False, rope_k=False)
    assert_within_ulp(want, got, 64, "no rope")


def test_rope_on_k_long(dev):
    """RoPE on K inside the kernel (the reference's unrotated cache) at 2K positions."""
    b = stimulus.decode_batch(2, 2048, min_len=1500, max_len=2048, seed=13)
    want = _oracle(b, rope_k=True)
    got = _run(b, dev, rope_q=True, rope_k=True)
    assert_within_ulp(want, got, 64, "rope_k")


def test_device_resident_lengths(dev):
    b = stimulus.decode_batch(5, 900, min_len=10, max_len=900, seed=14)
    ref = _run(b, dev)
    out = gqa.gqa_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev),
                            b.query_pos.to(dev), b.seq_len.to(dev))
    assert np.array_equal(_codes(out), ref)


@pytest.mark.parametrize("path", ["single", "three"])
def test_invalid_device_lengths_give_nan_rows(dev, path):
    p = gqa.make_params(stream_k=path != "single")
    b = stimulus.decode_batch(3, 256, lengths=torch.tensor([100, 50, 200]), seed=15)
    qpos = torch.tensor([99, 50, 199], dtype=torch.int32)      # sequence 1: qpos == seq_len
    out = _codes(gqa.gqa_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), qpos.to(dev),
                                   b.seq_len.to(dev), params=p))
    assert (out[1] == 0x7FC0).all()
    good = stimulus.DecodeBatch(b.q[[0, 2]], b.k[[0, 2]], b.v[[0, 2]], b.seq_len[[0, 2]],
                                qpos[[0, 2]])
    assert_within_ulp(_oracle(good), out[[0, 2]], 64, "valid rows next to an invalid one")


@pytest.mark.parametrize("path", ["single", "three"])
def test_huge_scores(dev, path):
    """Q heads scaled by 2^40 and 2^100 (scores far beyond 2^24 in log2 units, a one-hot
    softmax in the double golden): the running max and the pieces' (m, l) are doubles, so
    the largest key keeps p = 1 in every piece and the merge weights stay exact; every row,
    the scaled heads' and the others', within 64 ULP of the oracle."""
    b = stimulus.decode_batch(4, 700, min_len=300, max_len=700, seed=41)
    q = b.q.clone()
    q[0, 3] = (q[0, 3].float() * 2.0 ** 100).to(torch.bfloat16)
    q[2, 17] = (q[2, 17].float() * 2.0 ** 40).to(torch.bfloat16)
    b = stimulus.DecodeBatch(q, b.k, b.v, b.seq_len, b.query_pos)
    got = _run(b, dev, params=gqa.make_params(stream_k=path != "single"))
    assert_within_ulp(_oracle(b), got, 64, f"huge scores ({path})")


def test_host_validation_rejects(dev):
    b = stimulus.decode_batch(2, 64, lengths=torch.tensor([10, 20]), seed=16)
    q, k, v = b.q.to(dev), b.k.to(dev), b.v.to(dev)
    out = torch.full((2, 32, 128), 7.0, dtype=torch.bfloat16, device=dev)
    for qpos, sl in (([10, 5], [10, 20]), ([-1, 5], [10, 20]), ([5, 5], [0, 20]),
                     ([5, 5], [65, 20])):
        with pytest.raises(gqa.GqaConfigError):
            gqa.gqa_attention(q, k, v, qpos, sl, out=out)
    torch.cuda.synchronize()
    assert (out.float() == 7.0).all()      # a rejected call writes nothing


def test_batch64_ragged_512_8192(dev):
    """B=64, lengths U[512, 8192], capacity 8192, NaN in unused rows: every output
    against the oracle."""
    b = stimulus.decode_batch(64, 8192, min_len=512, max_len=8192, seed=20260805,
                              gen_device="cuda", device=dev)
    got = _codes(gqa.gqa_attention(b.q, b.k, b.v, b.query_pos, b.seq_len))
    want, want64 = _oracle(b, want_f64=True)
    w = assert_within_ulp(want, got, 64, "B=64 ragged", ref64=want64)
    print("worst ULP", w)


@pytest.mark.parametrize("bsz,hi,seed", [(300, 600, 31), (1000, 48, 32)])
def test_many_sequences(dev, bsz, hi, seed):
    """Batches spanning many 64-sequence windows of the plan (300 sequences up to 600 keys;
    1000 sequences of 1..48 keys, many segments per workgroup range): every output against
    the oracle.  N(0,1) V: with a few dozen keys
    the outputs are sums of a few large terms, and 1 in ~10^6 of them cancels to within
    1e-7 of zero, where 64 BF16 ULP is an absolute error of a few 1e-8 -- scores carried
    in fp32 once missed it here (72 ULP); carried in fp64 they meet it."""
    b = stimulus.decode_batch(bsz, hi, min_len=1, max_len=hi, seed=seed)
    want, want64 = _oracle(b, want_f64=True)
    sk = gqa.make_params(stream_k=True)
    got = _run(b, dev, params=sk)
    assert_within_ulp(want, got, 64, f"B={bsz}", ref64=want64)
    assert np.array_equal(_run(b, dev, params=sk), got)


def test_long_context_131072(dev):
    """B=8, L=131072 (multi-split combine, 4 GB of K/V): every sequence against the oracle
    on two KV heads -- sequence s on heads s and (s + 3) % 8, so each of the 8 KV heads is
    checked on two sequences and sequence 7, at the highest cache addresses, is covered;
    the whole batch finite and deterministic."""
    b = stimulus.decode_batch(8, 131072, seed=20260805, gen_device="cuda", device=dev)
    out1 = _codes(gqa.gqa_attention(b.q, b.k, b.v, b.query_pos, b.seq_len))
    out2 = _codes(gqa.gqa_attention(b.q, b.k, b.v, b.query_pos, b.seq_len))
    assert np.array_equal(out1, out2)
    assert np.isfinite(out1.view(np.int16).astype(np.float32)).all()
    for s in range(8):
        heads = [s, (s + 3) % 8]
        sub = stimulus.DecodeBatch(b.q[s:s + 1], b.k[s:s + 1], b.v[s:s + 1], b.seq_len[s:s + 1],
                                   b.query_pos[s:s + 1])
        want, want64 = _oracle(sub, kv_heads=heads, want_f64=True)
        rows = [h for kvh in heads for h in range(4 * kvh, 4 * kvh + 4)]
        assert_within_ulp(want[0, rows], out1[s, rows], 64, f"L=131072 seq {s} heads {heads}",
                          ref64=want64[0, rows])


def test_workspace_plan_mismatch_rejected(dev):
    """A workspace from new_workspace(B, S) serves (B, S) only: another capacity or batch
    is rejected on the host before any launch."""
    b = stimulus.decode_batch(2, 1024, seed=21)
    ws = gqa.new_workspace(2, 2048, dev)
    with pytest.raises(ValueError, match="prepared for"):
        gqa.gqa_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.query_pos, b.seq_len, workspace=ws)
    ws = gqa.new_workspace(2, 1024, dev)
    got = _codes(gqa.gqa_attention(b.q.to(dev), b.k.to(dev), b.v.to(dev), b.query_pos, b.seq_len,
                                   workspace=ws))
    assert_within_ulp(_oracle(b), got, 64, "tagged workspace")
