"""Helpers shared by the tests: BF16 code arrays <-> torch tensors, ULP summaries."""
from __future__ import annotations

import numpy as np
import torch

from attention_accelerator_amd.check import failures, ulp_distance, worst


def to_dev(codes, device) -> torch.Tensor:
    """uint16 BF16 codes (numpy or nested lists) -> bfloat16 tensor on device."""
    arr = np.ascontiguousarray(np.asarray(codes, dtype=np.uint16))
    return torch.from_numpy(arr.view(np.int16)).view(torch.bfloat16).to(device)


def to_codes(t: torch.Tensor) -> np.ndarray:
    """bfloat16 tensor -> uint16 BF16 codes (numpy, host)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def assert_within_ulp(want, got, max_ulp: int = 64, what: str = "") -> int:
    """The reference checker's policy (64 BF16 ULP, tiny-value exemption); returns worst ULP."""
    want = np.asarray(want, dtype=np.uint16).reshape(-1, 128)
    got = np.asarray(got, dtype=np.uint16).reshape(-1, 128)
    assert want.shape == got.shape
    bad = failures(want, got, max_ulp)
    w = worst(want, got)
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements exceed {max_ulp} ULP; "
                           f"worst={w[0]} at row={w[1]}, col={w[2]}")
    return w[0]


__all__ = ["to_dev", "to_codes", "assert_within_ulp", "ulp_distance"]
