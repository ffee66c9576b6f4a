"""The product checker (attention_accelerator_amd/check.py) and .mem codec
(attention_accelerator_amd/memfmt.py) pinned against the oracle's restatement of the
reference (oracle/golden_model.py, itself pinned bit for bit against the reference's
own generator output in test_oracle_golden.py).

Every GPU parity verdict runs through check.failures, so a loosened exemption there
would weaken every GPU test at once: here it must agree with the reference policy
(pyfiles/check_gqa_output.py:57-64 over pyfiles/gqa_reference.py:49-53) on every
BF16 code against a spread of neighbours, and the codec must read and write the
reference's files exactly as the reference does (pyfiles/gqa_reference.py:26-46)."""
from __future__ import annotations

import numpy as np
import pytest

from attention_accelerator_amd import check, memfmt
from conftest import GOLDEN, REFERENCE_CASES
from oracle import golden_model as gm

# Offsets around the 64-ULP boundary, small and large moves, and moves across zero.
OFFSETS = (0, 1, -1, 2, 63, -63, 64, -64, 65, -65, 66, 127, -128, 300, -300, 0x4000, 0x7FFF,
           0x8000, 0x8001, -0x8001)


def _pairs():
    a = np.arange(0x10000, dtype=np.int64)
    cols = []
    for off in OFFSETS:
        cols.append((a + off) & 0xFFFF)
    cols.append(a ^ 0x8000)                     # same magnitude, other sign
    b = np.stack(cols, axis=1)
    return np.broadcast_to(a[:, None], b.shape).reshape(-1), b.reshape(-1)


def test_ulp_distance_matches_reference_on_all_codes():
    a, b = _pairs()
    got = check.ulp_distance(a, b)
    want = np.fromiter((gm.ulp_distance(int(x), int(y)) for x, y in zip(a, b)), dtype=np.int64,
                       count=a.size)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("max_ulp", [0, 1, 64])
def test_failures_match_reference_policy_on_all_codes(max_ulp):
    a, b = _pairs()
    got = check.failures(a, b, max_ulp)
    want = np.fromiter((gm.element_fails(int(x), int(y), max_ulp) for x, y in zip(a, b)), dtype=bool,
                       count=a.size)
    assert np.array_equal(got, want)


def test_tiny_value_exemption_boundary():
    """Both exponent fields <= 0x3d are exempt; one side at 0x3e is not."""
    exp = np.arange(0, 0x100, dtype=np.int64)
    mant = np.array([0, 1, 0x40, 0x7F], dtype=np.int64)
    codes = ((exp[:, None] << 7) | mant[None, :]).reshape(-1)
    codes = np.concatenate([codes, codes | 0x8000])
    a = np.repeat(codes, codes.size)
    b = np.tile(codes, codes.size)
    got = check.failures(a, b, 64)
    want = np.fromiter((gm.element_fails(int(x), int(y), 64) for x, y in zip(a, b)), dtype=bool,
                       count=a.size)
    assert np.array_equal(got, want)
    # a pair far apart, both below 2^-65: exempt; one of them at exponent 0x3e: not
    assert not check.failures(np.array([0x3D << 7]), np.array([0x8000 | (0x3D << 7) | 0x7F]), 64)[0]
    assert check.failures(np.array([0x3E << 7]), np.array([0x8000 | (0x3D << 7) | 0x7F]), 64)[0]


def _mem_files():
    files = sorted(GOLDEN.glob("*/gqa_golden.mem"))
    assert len(files) == len(REFERENCE_CASES)
    return files


@pytest.mark.parametrize("path", _mem_files(), ids=lambda p: p.parent.name)
def test_mem_codec_matches_reference_reader_and_writer(path, tmp_path):
    want = np.array(gm.read_mem(path, 128), dtype=np.uint16)
    got = memfmt.read_mem(path, 128)
    assert got.shape == (32, 128)
    assert np.array_equal(got, want)
    # format_mem writes exactly the reference's text (which is the committed file's text)
    assert memfmt.format_mem(got) == path.read_text()
    out = tmp_path / "rows.mem"
    memfmt.write_mem(out, got)
    assert np.array_equal(np.array(gm.read_mem(out, 128), dtype=np.uint16), want)


def test_mem_codec_beats_and_comments(tmp_path):
    """16-element beats (the stimulus files), // comments, blank lines and '_' separators."""
    rng = np.random.default_rng(3)
    rows = rng.integers(0, 0x10000, size=(10, 16), dtype=np.uint16)
    path = tmp_path / "beats.mem"
    gm.write_mem(path, rows.tolist())
    text = path.read_text().splitlines()
    text.insert(3, "// a comment line")
    text.insert(5, "")
    text[0] = text[0][:32] + "_" + text[0][32:]
    path.write_text("\n".join(text) + "\n")
    assert np.array_equal(memfmt.read_mem(path, 16), np.array(gm.read_mem(path, 16), dtype=np.uint16))
    assert np.array_equal(memfmt.read_mem(path, 16), rows)
    # element 0 is the rightmost four hex digits
    one = np.arange(16, dtype=np.uint16)[None]
    assert memfmt.format_mem(one).strip() == gm.pack_bf16(range(16))
    assert memfmt.format_mem(one).strip().endswith("0000")
    with pytest.raises(ValueError):
        bad = tmp_path / "bad.mem"
        bad.write_text("abcd\n")
        memfmt.read_mem(bad, 16)
