"""The reference's two mask known-answer tests, restated at the level of a whole
attention step on every path (decode single launch, decode stream-K, paged decode,
multi-token and prefill).

- tests/tb_flash_softmax_mask.v:27-45: a block of four keys of which only key 0 is
  valid, scores 0, 16, 50, 100 (0x0000, 0x4180, 0x4248, 0x42c8).  The masked keys'
  probabilities must be exact zeros, so the output is V[0] bit for bit although the
  masked scores would dominate the softmax.
- tests/tb_score_tile_mask.v:30-41: scores 1, 2, 3, 4 (0x3f80, 0x4000, 0x4040, 0x4080)
  with valid mask 0011.  Here the block is a 16-key block and the mask is causal
  (query position 1, sequence length 16): the output must equal the padding case
  (sequence length 2) bit for bit and the closed form
  BF16(f32((e V0 + e^2 V1) / (e + e^2))) of the reference's double arithmetic
  (pyfiles/gen_gqa_wrapper_vectors.py:121-139, pyfiles/gqa_reference.py:15-19).

Scores are set exactly: scale 1.0, no RoPE, Q = 1.0 in dimension 0 of every head and
K = the score in dimension 0 of every KV head, zeros elsewhere."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import attention_accelerator_amd as gqa
from _util import assert_within_ulp, to_codes

pytestmark = pytest.mark.gpu

SOFTMAX_SCORES = (0.0, 16.0, 50.0, 100.0)       # tb_flash_softmax_mask.v:35
TILE_SCORES = (1.0, 2.0, 3.0, 4.0)              # tb_score_tile_mask.v:31-34


def _bf16_rne(x64: np.ndarray) -> np.ndarray:
    """double -> f32 (RNE) -> BF16 code (RNE): pyfiles/gqa_reference.py:15-19."""
    u = np.asarray(x64, dtype=np.float64).astype(np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def _bf16_values(t: torch.Tensor) -> np.ndarray:
    return t.float().numpy().astype(np.float64)


def _kv(scores, capacity, seed, batch=1):
    """K rows with the given dimension-0 scores (later rows repeat the last score, so a
    masked key always outscores the valid ones), N(0,1) BF16 V rows."""
    g = torch.Generator("cpu").manual_seed(seed)
    k = torch.zeros((batch, 8, capacity, 128), dtype=torch.bfloat16)
    for p in range(capacity):
        k[:, :, p, 0] = scores[min(p, len(scores) - 1)]
    v = torch.randn((batch, 8, capacity, 128), generator=g).to(torch.bfloat16)
    return k, v


def _q(batch, tokens=None):
    shape = (batch, 32, 128) if tokens is None else (batch, tokens, 32, 128)
    q = torch.zeros(shape, dtype=torch.bfloat16)
    q[..., 0] = 1.0
    return q


def _decode(q, k, v, qpos, seq_len, dev, path):
    if path == "paged":
        # one 16-position block per sequence, blocks in reverse order in the pool
        b, _, cap, _ = k.shape
        n_blk = cap // 16
        kp = k.reshape(b, 8, n_blk, 16, 128).permute(0, 2, 1, 3, 4).reshape(b * n_blk, 8, 16, 128)
        vp = v.reshape(b, 8, n_blk, 16, 128).permute(0, 2, 1, 3, 4).reshape(b * n_blk, 8, 16, 128)
        perm = torch.arange(b * n_blk - 1, -1, -1)
        table = torch.empty(b * n_blk, dtype=torch.int32)
        table[perm] = torch.arange(b * n_blk, dtype=torch.int32)
        out = gqa.gqa_decode_paged(q.to(dev), kp[perm].contiguous().to(dev), vp[perm].contiguous().to(dev),
                                   table.reshape(b, n_blk).to(dev), qpos, seq_len,
                                   rope_q=False, rope_k=False, scale=1.0)
    else:
        p = gqa.make_params(rope_q=False, rope_k=False, scale=1.0, stream_k=path == "stream")
        out = gqa.gqa_attention(q.to(dev), k.to(dev), v.to(dev), qpos, seq_len, params=p)
    torch.cuda.synchronize()
    return to_codes(out)


@pytest.fixture(params=["single", "stream", "paged"])
def decode_path(request):
    return request.param


def _v0_rows(v, pos=0):
    """[B, 32, 128] codes: V[pos] of KV head h // 4 for every Q head h."""
    return np.repeat(to_codes(v[:, :, pos]), 4, axis=1)


@pytest.mark.parametrize("qpos,seq_len", [(0, 1), (0, 4), (0, 16)])
def test_one_valid_key_of_four(dev, decode_path, qpos, seq_len):
    """Padding (seq_len 1) and causal (query position 0 of 4 or 16 keys) masks: exact
    zeros for the masked keys, output V[0] bit for bit."""
    k, v = _kv(SOFTMAX_SCORES, 16, seed=1)
    got = _decode(_q(1), k, v, qpos, seq_len, dev, decode_path)
    assert np.array_equal(got, _v0_rows(v)), f"{decode_path}: masked keys leaked into the output"


def _tile_closed_form(v):
    """BF16 of (e^1 V0 + e^2 V1) / (e^1 + e^2) in double, [B, 32, 128] codes."""
    vv = _bf16_values(v)                                           # [B, 8, S, 128]
    w0, w1 = math.exp(1.0 - 2.0), 1.0                              # max-subtracted as the golden
    x = (w0 * vv[:, :, 0] + w1 * vv[:, :, 1]) / (w0 + w1)
    return np.repeat(_bf16_rne(x), 4, axis=1)


def test_score_tile_mask_causal_equals_padding(dev, decode_path):
    """Valid mask 0011 inside a 16-key block: causal (qpos 1 of 16) == padding (length 2)
    bit for bit, both within 1 BF16 ULP of the closed form."""
    k, v = _kv(TILE_SCORES, 16, seed=2)
    causal = _decode(_q(1), k, v, 1, 16, dev, decode_path)
    padding = _decode(_q(1), k, v, 1, 2, dev, decode_path)
    assert np.array_equal(causal, padding)
    assert_within_ulp(_tile_closed_form(v), causal, 1, f"{decode_path} tile mask")


@pytest.mark.parametrize("n_new", [4, 16, 40])
def test_chunk_first_token_sees_one_key(dev, n_new):
    """Multi-token (4, 16 new tokens) and prefill (40) paths, empty cache: token 0
    attends to key 0 only, although keys 1.. score 16, 50, 100: its rows are V[0] bit
    for bit.  Token 1 sees keys 0 and 1 only (scores 1, 2 in a second call, mask 0011 of
    the tile test): within the 64-ULP policy of the closed form (these paths score in fp32
    on MFMA)."""
    k_new, v_new = _kv(SOFTMAX_SCORES, n_new, seed=3)                 # [1, 8, T, 128]
    kn = k_new.permute(0, 2, 1, 3).contiguous()                      # [1, T, 8, 128]
    vn = v_new.permute(0, 2, 1, 3).contiguous()
    cap = max(64, n_new)
    kc = torch.zeros((1, 8, cap, 128), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    out = gqa.gqa_prefill(_q(1, n_new).to(dev), kn.to(dev), vn.to(dev), kc, vc, 0,
                          rope_q=False, rope_k=False, scale=1.0)
    torch.cuda.synchronize()
    got = to_codes(out)                                              # [1, T, 32, 128]
    assert np.array_equal(got[:, 0], _v0_rows(v_new)), f"T={n_new}: masked keys leaked into token 0"

    k_new, v_new = _kv(TILE_SCORES, n_new, seed=4)
    kn = k_new.permute(0, 2, 1, 3).contiguous()
    vn = v_new.permute(0, 2, 1, 3).contiguous()
    out = gqa.gqa_prefill(_q(1, n_new).to(dev), kn.to(dev), vn.to(dev), kc, vc, 0,
                          rope_q=False, rope_k=False, scale=1.0)
    torch.cuda.synchronize()
    got = to_codes(out)
    assert_within_ulp(_tile_closed_form(v_new), got[:, 1], 64, f"T={n_new} token 1")
