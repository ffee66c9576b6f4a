"""The RoPE kernel against the reference's RoPE set (pyfiles/gen_rope_test_vectors.py,
512 rows, row r at position r; tests/tb_rope_unit.sv checks <= 64 ULP) and against
the oracle at large positions."""
from __future__ import annotations

import hashlib
import random

import numpy as np
import pytest
import torch

import attention_accelerator_amd as gqa
from conftest import GOLDEN
from oracle import golden_model as gm
from oracle import oracle as orc
from _util import assert_within_ulp, to_codes, to_dev

pytestmark = pytest.mark.gpu


def _rope_inputs():
    rng = random.Random(20260805)
    rows = [[rng.uniform(-0.25, 0.25) for _ in range(128)] for _ in range(512)]
    return np.array([[gm.f32_to_bf16(x) for x in row] for row in rows], dtype=np.uint16)


def test_rope_set_512_rows(dev):
    inp = _rope_inputs()
    got = to_codes(gqa.rope_half_split(to_dev(inp, dev), 0))
    want = np.array([[gm.f32_to_bf16(x) for x in
                      gm.rope_half_split([gm.bf16_to_f32(v) for v in row], pos)]
                     for pos, row in enumerate(inp.tolist())], dtype=np.uint16)
    # the restated golden is the reference's file, byte for byte
    text = "\n".join(gm.pack_bf16(b) for row in want.tolist() for b in gm.chunks(row, 16)) + "\n"
    digest = dict(ln.split()[::-1] for ln in (GOLDEN / "rope" / "rope.sha256").read_text().splitlines())
    assert hashlib.sha256(text.encode()).hexdigest() == digest["golden.mem"]
    assert_within_ulp(want, got, 64, "rope 512")
    # every one of the 65,536 elements bit for bit: the kernel rotates in double and rounds
    # double -> f32 -> BF16 as the golden does
    bad = np.argwhere(want != got)
    assert bad.size == 0, f"{len(bad)} elements differ from the golden, first at (row, dim) {bad[0].tolist()}"


def test_rope_positions_tensor_and_large_positions(dev):
    inp = _rope_inputs()[:64]
    pos = np.array([0, 1, 4095, 8191, 131071, 65536, 12345, 99999] * 8, dtype=np.int32)
    got = to_codes(gqa.rope_half_split(to_dev(inp, dev),
                                       torch.from_numpy(pos).to(dev)))
    want = np.stack([[orc.f32_to_bf16(x) for x in orc.rope_row(orc.prepare_rows(r[None], False)[0], int(p))]
                     for r, p in zip(inp, pos)]).astype(np.uint16)
    assert_within_ulp(want, got, 1, "rope positions")


def test_rope_pos0_offset(dev):
    inp = _rope_inputs()[:10]
    a = to_codes(gqa.rope_half_split(to_dev(inp, dev), 1000))
    b = to_codes(gqa.rope_half_split(to_dev(inp, dev),
                                     torch.arange(1000, 1010, dtype=torch.int32, device=dev)))
    assert np.array_equal(a, b)
