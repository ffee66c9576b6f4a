"""Pin the oracle where the reference's own files leave it open: closed forms,
invariants, a textbook routine (torch fp64 softmax attention) and brute force --
and show that plausible mistakes planted in the oracle fail these pins."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import golden_model as gm
from oracle import oracle as orc


def rand_codes(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)
    return x.view(torch.int16).numpy().view(np.uint16)


def widen(codes):
    return (np.asarray(codes, dtype=np.uint32) << 16).view(np.float32).astype(np.float64)


# ---------------------------------------------------------------- BF16 codec

@pytest.mark.parametrize("x,code", [
    (1.0, 0x3F80), (-2.0, 0xC000), (0.0, 0x0000), (-0.0, 0x8000),
    (1.0 / math.sqrt(128), 0x3DB5),                  # SCALE default, axi_lite_regs.v:116
    (1.0 + 2 ** -8, 0x3F80),                          # exact tie -> even
    (1.0 + 3 * 2 ** -8, 0x3F82),                      # exact tie -> even (up)
    (1.0 + 2 ** -8 + 2 ** -30, 0x3F80),               # double rounding: f32 first, then tie
    (1.0 + 2 ** -8 + 2 ** -20, 0x3F81),               # above the tie after f32 rounding
    (float("inf"), 0x7F80), (float("nan"), 0x7FC0),
])
def test_f32_to_bf16_known_values(x, code):
    assert gm.f32_to_bf16(x) == code
    assert orc.f32_to_bf16(x) == code


def test_f32_to_bf16_overflow_raises():
    with pytest.raises(OverflowError):
        gm.f32_to_bf16(1e39)


def test_bf16_widening_exact():
    for code in (0x0001, 0x3F80, 0x7F7F, 0x8001, 0xFF7F, 0x3DB5):
        assert gm.f32_to_bf16(gm.bf16_to_f32(code)) == code


@pytest.mark.parametrize("a,b,d", [
    (0x3F80, 0x3F81, 1), (0x0000, 0x8000, 0), (0x0001, 0x8001, 2),
    (0x3F80, 0xBF80, 2 * 0x3F80), (0x7F7F, 0x7F80, 1),
])
def test_ulp_distance(a, b, d):
    assert gm.ulp_distance(a, b) == d


def test_checker_tiny_exemption():
    # both exponents <= 0x3d (|x| < 2^-65): exempt however far apart
    assert not gm.element_fails(0x1E80, 0x0001, 64)
    # one side larger: not exempt
    assert gm.element_fails(0x1F00, 0x0001, 64)
    assert not gm.element_fails(0x3F80, 0x3F80 + 64, 64)
    assert gm.element_fails(0x3F80, 0x3F80 + 65, 64)


def test_mem_packing_element0_rightmost():
    assert gm.pack_bf16([0x1111, 0x2222, 0x3333]) == "333322221111"
    assert gm.unpack_bf16("3333_2222_1111", 3) == [0x1111, 0x2222, 0x3333]
    with pytest.raises(ValueError):
        gm.unpack_bf16("12345", 2)


# ---------------------------------------------------------------- RoPE

def test_rope_identity_at_position_zero():
    row = list(widen(rand_codes(128, 1)))
    assert gm.rope_half_split(row, 0) == row


def test_rope_matches_complex_rotation():
    """rotate_half pairs (i, i+64): (x + iy) * exp(i * pos * theta^(-2i/128))."""
    row = widen(rand_codes(128, 2))
    for pos in (1, 29, 4095, 131071):
        got = np.array(gm.rope_half_split(list(row), pos))
        z = (row[:64] + 1j * row[64:]) * np.exp(1j * pos * 500000.0 ** (-2.0 * np.arange(64) / 128))
        assert np.allclose(got[:64], z.real, atol=1e-12) and np.allclose(got[64:], z.imag, atol=1e-12)
        # each pair keeps its norm
        assert np.allclose(got[:64] ** 2 + got[64:] ** 2, row[:64] ** 2 + row[64:] ** 2)


# ---------------------------------------------------------------- attention

def _textbook(q, k, v, n_keys, qpos, rope_q=True, rope_k=False):
    """softmax(q k^T / sqrt(d)) v in float64 with torch, GQA by repeat_interleave(4)."""
    qd = torch.tensor(np.stack([gm.rope_half_split(list(r), qpos) if rope_q else r
                                for r in widen(q)]), dtype=torch.float64)
    kd = widen(k[:, :n_keys])
    if rope_k:
        kd = np.stack([[gm.rope_half_split(list(kd[h, p]), p) for p in range(n_keys)]
                       for h in range(kd.shape[0])])
    kd = torch.tensor(kd, dtype=torch.float64).repeat_interleave(4, dim=0)
    vd = torch.tensor(widen(v[:, :n_keys]), dtype=torch.float64).repeat_interleave(4, dim=0)
    s = torch.einsum("hd,hpd->hp", qd, kd) / math.sqrt(128)
    return torch.einsum("hp,hpd->hd", torch.softmax(s, dim=-1), vd).numpy()


@pytest.mark.parametrize("n,qpos,rope_k", [(1, 0, False), (37, 36, True), (300, 200, False)])
def test_attention_matches_textbook_fp64(n, qpos, rope_k):
    q = rand_codes((32, 128), 3)
    k = rand_codes((8, n, 128), 4)
    v = rand_codes((8, n, 128), 5)
    _, f64 = orc.decode(q, k, v, n, qpos, rope_k=rope_k, want_f64=True)
    want = _textbook(q, k, v, qpos + 1, qpos, rope_k=rope_k)
    assert np.allclose(f64, want, rtol=1e-11, atol=1e-13)


def test_equal_scores_give_mean_of_v():
    """smoke mode (pyfiles/gen_gqa_wrapper_vectors.py:4-7): Q = K = 0 -> mean of V."""
    q, k, v = gm.stimulus("smoke", 30, 0)
    out = gm.golden_attention(q, k, v, 30, 20)
    mean = widen(np.array(v))[:, :21].mean(axis=1)
    for h in range(32):
        assert out[h] == [gm.f32_to_bf16(x) for x in mean[h // 4]]


def test_single_key_returns_v0():
    q, k, v = rand_codes((32, 128), 6), rand_codes((8, 1, 128), 7), rand_codes((8, 1, 128), 8)
    out = orc.decode(q, k, v, 1, 0, rope_k=True)
    assert np.array_equal(out, np.repeat(v[:, 0], 4, axis=0))


def test_brute_force_two_keys():
    """Two keys by hand: out = (e^s0 v0 + e^s1 v1) / (e^s0 + e^s1)."""
    q, k, v = rand_codes((32, 128), 9), rand_codes((8, 2, 128), 10), rand_codes((8, 2, 128), 11)
    _, f64 = orc.decode(q, k, v, 2, 1, rope_q=False, want_f64=True)
    qd, kd, vd = widen(q), widen(k), widen(v)
    for h in (0, 13, 31):
        s = [float(qd[h] @ kd[h // 4, p]) / math.sqrt(128) for p in (0, 1)]
        w = [math.exp(x - max(s)) for x in s]
        want = (w[0] * vd[h // 4, 0] + w[1] * vd[h // 4, 1]) / (w[0] + w[1])
        assert np.allclose(f64[h], want, rtol=1e-13)


def test_head_grouping():
    """Q heads 4g..4g+3 read KV head g only."""
    q, k, v = rand_codes((32, 128), 12), rand_codes((8, 40, 128), 13), rand_codes((8, 40, 128), 14)
    base = orc.decode(q, k, v, 40, 39)
    k2, v2 = k.copy(), v.copy()
    k2[5] = rand_codes((40, 128), 15)
    v2[5] = rand_codes((40, 128), 16)
    out = orc.decode(q, k2, v2, 40, 39)
    changed = np.any(out != base, axis=1)
    assert changed[20:24].all() and not changed[:20].any() and not changed[24:].any()


def test_key_permutation_invariance_without_rope():
    q, k, v = rand_codes((32, 128), 17), rand_codes((8, 64, 128), 18), rand_codes((8, 64, 128), 19)
    perm = np.random.default_rng(0).permutation(64)
    a = orc.decode(q, k, v, 64, 63, rope_q=False)
    b = orc.decode(q, k[:, perm], v[:, perm], 64, 63, rope_q=False)
    assert max(gm.ulp_distance(int(x), int(y)) for x, y in zip(a.ravel(), b.ravel())) <= 1


def test_masked_rows_never_read():
    q, k, v = rand_codes((32, 128), 20), rand_codes((8, 50, 128), 21), rand_codes((8, 50, 128), 22)
    base = orc.decode(q, k, v, 50, 30)
    k2, v2 = k.copy(), v.copy()
    k2[:, 31:] = 0x7FC0
    v2[:, 31:] = 0x7FC0
    assert np.array_equal(orc.decode(q, k2, v2, 50, 30), base)


def test_output_is_convex_combination():
    q, k, v = rand_codes((32, 128), 23), rand_codes((8, 90, 128), 24), rand_codes((8, 90, 128), 25)
    _, f64 = orc.decode(q, k, v, 90, 89, want_f64=True)
    vd = widen(v)
    for h in range(32):
        assert (f64[h] <= vd[h // 4].max(axis=0) + 1e-12).all()
        assert (f64[h] >= vd[h // 4].min(axis=0) - 1e-12).all()


def test_sum_modes_agree_within_one_ulp():
    """CPython <= 3.11 sums left to right, >= 3.12 compensates; outputs differ by <= 1 ULP."""
    q, k, v = rand_codes((32, 128), 26), rand_codes((8, 700, 128), 27), rand_codes((8, 700, 128), 28)
    a = orc.decode(q, k, v, 700, 699, sum_mode=orc.SUM_SEQUENTIAL)
    b = orc.decode(q, k, v, 700, 699, sum_mode=orc.SUM_NEUMAIER)
    assert max(gm.ulp_distance(int(x), int(y)) for x, y in zip(a.ravel(), b.ravel())) <= 1


def test_prefill_rows_equal_decode_rows():
    """A prefill query row t is the one-token golden at position start+t over the cache
    plus the first t+1 new rows."""
    start, t_new = 20, 6
    q = rand_codes((1, t_new, 32, 128), 29)
    kc, vc = rand_codes((1, 8, start, 128), 30), rand_codes((1, 8, start, 128), 31)
    kn, vn = rand_codes((1, t_new, 8, 128), 32), rand_codes((1, t_new, 8, 128), 33)
    out = orc.prefill(q, kc, vc, kn, vn, start)
    for t in (0, 3, 5):
        pos = start + t
        kk = np.concatenate([kc[0], kn[0, :t + 1].transpose(1, 0, 2)], axis=1)
        vv = np.concatenate([vc[0], vn[0, :t + 1].transpose(1, 0, 2)], axis=1)
        q_ref = np.stack([orc.prepare_rows(q[0, t, h][None], True, pos)[0] for h in range(32)])
        k_ref = np.stack([np.concatenate([orc.prepare_rows(kc[0, h], False),
                                          orc.prepare_rows(kn[0, :t + 1, h], True, start)])
                          for h in range(8)])
        v_ref = widen(vv)
        want = orc.attend(q_ref, k_ref, v_ref, pos + 1, 1 / math.sqrt(128))
        assert np.array_equal(out[0, t], want)
        assert kk.shape[1] == pos + 1


# ---------------------------------------------------------------- planted mistakes

def _fixture_case():
    q, k, v = gm.stimulus("random", 30, 20260805)
    want = gm.read_mem(GOLDEN / "random_len30" / "gqa_golden.mem", 128)
    return q, k, v, want


@pytest.mark.parametrize("mistake", ["interleaved_pairs", "sign", "no_scale", "head_map",
                                     "off_by_one_mask", "bf16_direct_rounding"])
def test_planted_mistakes_fail_the_pins(mistake, monkeypatch):
    """Each plausible mistake in the oracle changes the golden rows the reference wrote."""
    q, k, v, want = _fixture_case()
    real_rope = gm.rope_half_split
    if mistake == "interleaved_pairs":
        def rope(row, pos, theta=500000.0):
            out = list(row)
            for i in range(len(row) // 2):
                a = pos * theta ** (-2.0 * i / len(row))
                c, s = math.cos(a), math.sin(a)
                x, y = row[2 * i], row[2 * i + 1]
                out[2 * i], out[2 * i + 1] = x * c - y * s, x * s + y * c
            return out
        monkeypatch.setattr(gm, "rope_half_split", rope)
        got = gm.golden_attention(q, k, v, 30, 29)
    elif mistake == "sign":
        monkeypatch.setattr(gm, "rope_half_split",
                            lambda row, pos, theta=500000.0: real_rope(row, -pos, theta))
        got = gm.golden_attention(q, k, v, 30, 29)
    elif mistake == "no_scale":
        got = gm.golden_attention(q, k, v, 30, 29, scale=1.0)
    elif mistake == "head_map":
        # Q head h read KV head h % 8 instead of h // 4
        slot = [(h % 8) * 4 + h // 8 for h in range(32)]
        q_perm = [None] * 32
        for h in range(32):
            q_perm[slot[h]] = q[h]
        out_perm = gm.golden_attention(q_perm, k, v, 30, 29)
        got = [out_perm[slot[h]] for h in range(32)]
    elif mistake == "off_by_one_mask":
        got = gm.golden_attention(q, k, v, 30, 28)
    else:
        monkeypatch.setattr(gm, "f32_to_bf16", lambda x: int(np.float64(x).view(np.uint64) >> 48) & 0xFFFF)
        got = gm.golden_attention(q, k, v, 30, 29)
    assert got != want
