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


def bf16_value(codes) -> np.ndarray:
    return (np.asarray(codes, dtype=np.uint32) << 16).view(np.float32).astype(np.float64)


def error_report(want, got, ref64=None, limit: int = 8) -> str:
    """Worst elements by ULP with their values (and the float64 golden when given)."""
    want = np.asarray(want, dtype=np.uint16).reshape(-1)
    got = np.asarray(got, dtype=np.uint16).reshape(-1)
    dist = ulp_distance(want, got).reshape(-1)
    order = np.argsort(-dist, kind="stable")[:limit]
    lines = []
    gv, wv = bf16_value(got), bf16_value(want)
    for i in order:
        extra = ""
        if ref64 is not None:
            r = np.asarray(ref64).reshape(-1)[i]
            extra = f" golden64={r:.6e} abs_err={abs(gv[i] - r):.3e}"
        lines.append(f"  elem {i} (row {i // 128}, col {i % 128}): want 0x{int(want[i]):04x}"
                     f" ({wv[i]:.6e}) got 0x{int(got[i]):04x} ({gv[i]:.6e}) ulp={int(dist[i])}{extra}")
    if ref64 is not None:
        err = np.abs(gv - np.asarray(ref64).reshape(-1))
        lines.append(f"  max |got - golden64| = {err.max():.3e}, rms = {np.sqrt((err ** 2).mean()):.3e},"
                     f" rms(golden64) = {np.sqrt((np.asarray(ref64) ** 2).mean()):.3e}")
    return "\n".join(lines)


def assert_within_ulp(want, got, max_ulp: int = 64, what: str = "", ref64=None) -> int:
    """The reference checker's policy (64 BF16 ULP, tiny-value exemption); returns worst ULP."""
    want = np.asarray(want, dtype=np.uint16).reshape(-1, 128)
    got = np.asarray(got, dtype=np.uint16).reshape(-1, 128)
    assert want.shape == got.shape
    bad = failures(want, got, max_ulp)
    w = worst(want, got)
    if bad.any() or ref64 is not None:
        print(f"{what}: worst {w[0]} ULP, {int(bad.sum())} over {max_ulp}\n"
              + error_report(want, got, ref64))
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements exceed {max_ulp} ULP; "
                           f"worst={w[0]} at row={w[1]}, col={w[2]}")
    return w[0]


__all__ = ["to_dev", "to_codes", "assert_within_ulp", "ulp_distance"]

