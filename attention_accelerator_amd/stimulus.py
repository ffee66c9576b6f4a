"""Synthetic inputs for the measured workloads: BF16 N(0,1) Q/K/V.

Values come from torch.Generator('cpu').manual_seed(seed).randn in fp32, rounded
to BF16 with round-to-nearest-even (the reference rounds through f32 the same way,
pyfiles/gqa_reference.py:15-19).  Ragged lengths are drawn from the same
generator.  Unused cache rows are filled with NaN so that any read of a masked
row would poison the output.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

N_Q_HEADS, N_KV_HEADS, HEAD_DIM = 32, 8, 128
DEFAULT_SEED = 20260805


@dataclass
class DecodeBatch:
    q: torch.Tensor          # [B, 32, 128] bf16
    k: torch.Tensor          # [B, 8, capacity, 128] bf16 (post-RoPE cache)
    v: torch.Tensor          # [B, 8, capacity, 128] bf16
    seq_len: torch.Tensor    # [B] int32 (host)
    query_pos: torch.Tensor  # [B] int32 (host)

    @property
    def capacity(self) -> int:
        return self.k.shape[2]


def _randn_bf16(g: torch.Generator, shape, device) -> torch.Tensor:
    x = torch.randn(shape, generator=g, dtype=torch.float32, device=g.device)
    return x.to(torch.bfloat16).to(device)


def decode_batch(batch: int, capacity: int, *, lengths: Optional[torch.Tensor] = None,
                 min_len: Optional[int] = None, max_len: Optional[int] = None,
                 seed: int = DEFAULT_SEED, device="cpu", pad_nan: bool = True,
                 gen_device: str = "cpu") -> DecodeBatch:
    """B sequences with a [B, 8, capacity, 128] cache.  Lengths: given, drawn
    uniformly from [min_len, max_len] (inclusive), or all = capacity.
    query_position = length - 1 (decode of the next token).
    gen_device "cpu" reproduces the same values on any machine; "cuda" draws the
    values on the GPU (fast for multi-GB caches; reproducible for a given
    torch build).  Lengths are always drawn on the CPU."""
    g_len = torch.Generator("cpu").manual_seed(seed)
    g = g_len if gen_device == "cpu" else torch.Generator(gen_device).manual_seed(seed)
    if lengths is None:
        if min_len is None:
            lengths = torch.full((batch,), capacity, dtype=torch.int32)
        else:
            hi = capacity if max_len is None else max_len
            lengths = torch.randint(min_len, hi + 1, (batch,), generator=g_len, dtype=torch.int64)
    lengths = torch.as_tensor(lengths, dtype=torch.int32).reshape(batch)
    if int(lengths.max()) > capacity or int(lengths.min()) < 1:
        raise ValueError("lengths must lie in [1, capacity]")
    q = _randn_bf16(g, (batch, N_Q_HEADS, HEAD_DIM), device)
    k = torch.empty((batch, N_KV_HEADS, capacity, HEAD_DIM), dtype=torch.bfloat16, device=device)
    v = torch.empty_like(k)
    for b in range(batch):
        n = int(lengths[b])
        k[b, :, :n] = _randn_bf16(g, (N_KV_HEADS, n, HEAD_DIM), device)
        v[b, :, :n] = _randn_bf16(g, (N_KV_HEADS, n, HEAD_DIM), device)
        fill = float("nan") if pad_nan else 0.0
        k[b, :, n:] = fill
        v[b, :, n:] = fill
    return DecodeBatch(q, k, v, lengths.clone(), (lengths - 1).to(torch.int32))


def algorithmic_bytes_decode(lengths, q_heads: int = N_Q_HEADS, kv_heads: int = N_KV_HEADS,
                             head_dim: int = HEAD_DIM) -> int:
    """HBM bytes one decode step must move: every valid K and V row once, the Q rows
    in, the output rows out, and two int32 per sequence."""
    lengths = [int(x) for x in lengths]
    n = len(lengths)
    kv = sum(2 * kv_heads * head_dim * 2 * x for x in lengths)
    return kv + 2 * n * q_heads * head_dim * 2 + 8 * n


def decode_flops(lengths, q_heads: int = N_Q_HEADS, head_dim: int = HEAD_DIM) -> int:
    """QK^T and PV multiply-adds, 2 flops each."""
    return sum(q_heads * int(x) * head_dim * 4 for x in lengths)
