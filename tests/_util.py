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


# Absolute error floor of the MFMA paths: scores accumulate in fp32 (Q in three BF16 parts
# against BF16 K), about 1e-7 in the log2 domain, which moves an N(0,1)-input output by up
# to ~1e-8.  An output that cancels to within ~4e-8 of zero can therefore exceed 64 BF16
# ULP of its own tiny value while being as accurate as its neighbours.
MFMA_FLOOR_ABS = 2e-8


def assert_within_ulp_or_floor(want, got, ref64, max_ulp: int = 64, floor_abs: float = MFMA_FLOOR_ABS,
                               what: str = "") -> int:
    """64 BF16 ULP per element (the reference checker's policy), except elements whose
    absolute error against the double-precision golden is within floor_abs; returns the
    number of such floor elements."""
    want = np.asarray(want, dtype=np.uint16).reshape(-1)
    got = np.asarray(got, dtype=np.uint16).reshape(-1)
    ref = np.asarray(ref64, dtype=np.float64).reshape(-1)
    bad = failures(want.reshape(-1, 128), got.reshape(-1, 128), max_ulp).reshape(-1)
    err = np.abs(bf16_value(got) - ref)
    floor = bad & (err <= floor_abs)
    real = bad & ~floor
    if bad.any():
        idx = np.nonzero(bad)[0][:8]
        print(f"{what}: {int(bad.sum())} elements over {max_ulp} ULP, {int(floor.sum())} within the "
              f"{floor_abs:.0e} floor: " + ", ".join(f"{i}: golden {ref[i]:.3e} got {bf16_value(got[i:i+1])[0]:.3e}"
                                                      for i in idx))
    assert not real.any(), (f"{what}: {int(real.sum())} elements exceed {max_ulp} ULP and the "
                            f"{floor_abs:.0e} absolute floor")
    return int(floor.sum())
