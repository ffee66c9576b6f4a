"""Seeded random cases over every path -- decode (one and three launches), paged decode,
multi-token (T <= 16), prefill (T > 16) and chunks with no cache -- with random batch sizes,
lengths, query positions, RoPE flags and power-of-two scales on whole tensors or single heads
of Q, K and V (2^-100 .. 2^100: peaked and flat softmax, tiny and huge values).  Every output
element within 64 BF16 ULP of the compiled oracle (the reference checker's policy,
pyfiles/check_gqa_output.py:57-64).  A wider run of the same draw found a peaked prefill row
missing 64 ULP unflagged, rows with scores past 2^33 coming out NaN on the fp64 paths, and
multi-token rows with dot products past the fp32 range coming out NaN; each has a test of
its own as well."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import attention_accelerator_amd as gqa
from oracle import oracle as orc
from _util import assert_within_ulp, to_codes

pytestmark = pytest.mark.gpu

_SCALES = [1.0, 1.0, 2.0 ** 4, 2.0 ** 10, 2.0 ** 40, 2.0 ** 100, 2.0 ** -10, 2.0 ** -40, 2.0 ** -100]


def _bf(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16)


def _perturb(rng, t: torch.Tensor, head_axis: int):
    """t scaled by a random power of two, whole or on one head; returns (tensor, label)."""
    f = float(rng.choice(_SCALES))
    if f == 1.0:
        return t, "1"
    if rng.random() < 0.5:
        t = t.clone()
        idx = [slice(None)] * t.dim()
        h = int(rng.integers(t.shape[head_axis]))
        idx[head_axis] = h
        t[tuple(idx)] = _bf(t[tuple(idx)].float() * f)
        return t, f"head {h} x 2^{int(np.log2(f))}"
    return _bf(t.float() * f), f"x 2^{int(np.log2(f))}"


def _decode_case(rng, g, dev, paged: bool, single: bool):
    batch = int(rng.integers(1, 25))
    cap = int(rng.integers(1, 1500))
    if paged:
        cap = (cap + 15) // 16 * 16
    sl = rng.integers(1, cap + 1, size=batch)
    qp = np.array([int(rng.integers(0, s)) if rng.random() < 0.3 else int(s) - 1 for s in sl])
    rope_k = bool(rng.random() < 0.3)
    q = _bf(torch.randn((batch, 32, 128), generator=g))
    k = _bf(torch.randn((batch, 8, cap, 128), generator=g))
    v = _bf(torch.randn((batch, 8, cap, 128), generator=g))
    q, dq = _perturb(rng, q, 1)
    k, dk = _perturb(rng, k, 1)
    v, dv = _perturb(rng, v, 1)
    for b in range(batch):
        k[b, :, sl[b]:] = float("nan")
        v[b, :, sl[b]:] = float("nan")
    what = f"{'paged' if paged else 'decode'} B={batch} cap={cap} rope_k={rope_k} q {dq}, k {dk}, v {dv}"
    print(what, flush=True)
    if paged:
        nb = cap // 16
        table = torch.from_numpy(rng.permutation(batch * nb).astype(np.int32)).reshape(batch, nb)
        kp = torch.empty((batch * nb, 8, 16, 128), dtype=torch.bfloat16)
        vp = torch.empty_like(kp)
        for b in range(batch):
            for j in range(nb):
                kp[table[b, j]] = k[b, :, 16 * j:16 * j + 16]
                vp[table[b, j]] = v[b, :, 16 * j:16 * j + 16]
        out = gqa.gqa_decode_paged(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), [int(x) for x in qp],
                                   [int(x) for x in sl], rope_k=rope_k)
    else:
        out = gqa.gqa_attention(q.to(dev), k.to(dev), v.to(dev), [int(x) for x in qp], [int(x) for x in sl],
                                params=gqa.make_params(rope_k=rope_k, stream_k=not single))
    torch.cuda.synchronize()
    want = orc.decode(to_codes(q), to_codes(k), to_codes(v), sl, qp, rope_k=rope_k)
    return want, to_codes(out), what


def _chunk_case(rng, g, dev, kind: str):
    if kind == "multi":
        batch, n_new = int(rng.integers(1, 9)), int(rng.integers(1, 17))
    elif kind == "chunk0":
        batch, n_new = int(rng.integers(1, 4)), int(rng.choice([1, 3, 8, 16, 17, 40]))
    else:
        batch, n_new = int(rng.integers(1, 3)), int(rng.choice([17, 33, 64]))
    cap = int(rng.integers(n_new, 1200 + n_new))
    starts = np.zeros(batch, dtype=np.int64) if kind == "chunk0" else rng.integers(0, cap - n_new + 1, size=batch)
    rope_q, rope_k = bool(rng.random() < 0.9), bool(rng.random() < 0.8)
    q = _bf(torch.randn((batch, n_new, 32, 128), generator=g))
    kn = _bf(torch.randn((batch, n_new, 8, 128), generator=g))
    vn = _bf(torch.randn((batch, n_new, 8, 128), generator=g))
    k = torch.full((batch, 8, cap, 128), float("nan"), dtype=torch.bfloat16)
    v = k.clone()
    for b in range(batch):
        s = int(starts[b])
        k[b, :, :s] = _bf(torch.randn((8, s, 128), generator=g))
        v[b, :, :s] = _bf(torch.randn((8, s, 128), generator=g))
    q, dq = _perturb(rng, q, 2)
    kn, dk = _perturb(rng, kn, 2)
    vn, dv = _perturb(rng, vn, 2)
    what = (f"{kind} B={batch} T={n_new} cap={cap} starts={starts.tolist()} rope_q={rope_q} rope_k={rope_k} "
            f"q {dq}, k_new {dk}, v_new {dv}")
    print(what, flush=True)
    out = gqa.gqa_prefill(q.to(dev), kn.to(dev), vn.to(dev), k.to(dev), v.to(dev), [int(x) for x in starts],
                          rope_q=rope_q, rope_k=rope_k)
    torch.cuda.synchronize()
    want = orc.prefill(to_codes(q), to_codes(k), to_codes(v), to_codes(kn), to_codes(vn), starts,
                       rope_q=rope_q, rope_k_new=rope_k)
    return want, to_codes(out), what


@pytest.mark.parametrize("seed,kind", [(66941, "multi"), (87509, "prefill"), (92115, "prefill")])
def test_random_case_regression(dev, seed, kind):
    """Draws of the wider runs that once missed 64 ULP for a reason of this library's own:
    66941 (multi-token B=8 T=16, Q x 2^10, the chunk's K x 2^-100 and V x 2^100) had two rows
    that cancel between near-tied keys left unflagged, the flag's squares underflowing fp32;
    87509 and 92115 (prefill T=64 and 17, Q or one head x 2^4, the chunk's V x 2^40) had
    hundreds of elements off by up to 3 %: chunk keys of weight ~1e-13 and V ~1e12 fell below
    the fp16 split's subnormal quantum, an error the flag did not bound."""
    rng = np.random.default_rng(seed)
    g = torch.Generator("cpu").manual_seed(seed)
    want, got, what = _chunk_case(rng, g, dev, kind)
    assert_within_ulp(want.reshape(-1, 128), got.reshape(-1, 128), 64, what)


@pytest.mark.parametrize("seed", range(24))
def test_random_case(dev, seed):
    rng = np.random.default_rng(9100 + seed)
    g = torch.Generator("cpu").manual_seed(9100 + seed)
    kind = ["decode", "decode1", "paged", "multi", "multi", "prefill", "chunk0"][seed % 7]
    if kind in ("decode", "decode1", "paged"):
        want, got, what = _decode_case(rng, g, dev, kind == "paged", kind == "decode1")
    else:
        want, got, what = _chunk_case(rng, g, dev, kind)
    assert_within_ulp(want.reshape(-1, 128), got.reshape(-1, 128), 64, what)
