"""Pin the oracle against the reference's own outputs (tests/golden/, written by
tests/golden/make_fixtures.py from pyfiles/gen_gqa_wrapper_vectors.py,
pyfiles/gen_rope_test_vectors.py and pyfiles/gen_bf16_primitive_vectors.py).

Bit-exact: the stimulus files (draw order + .mem packing + BF16 rounding), the
golden output rows (RoPE + attention loop + output rounding), gqa_config.txt, the
RoPE set and the BF16 add/mul conformance words."""
from __future__ import annotations

import hashlib
import random
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from conftest import DEFAULT_SEED, GOLDEN, REFERENCE_CASES, ROOT
from oracle import golden_model as gm
from oracle import oracle as orc

CASE_IDS = [c[0] for c in REFERENCE_CASES]


def _sha_text(text: str) -> str:
    return hashlib.sha256(text.encode()).hexdigest()


def _mem_text(rows) -> str:
    return "\n".join(gm.pack_bf16(r) for r in rows) + "\n"


def _digests(path: Path) -> dict:
    out = {}
    for line in path.read_text().splitlines():
        h, name = line.split()
        out[name] = h
    return out


def _case(case):
    name, mode, seq_len, seed, qpos, blk = case
    return name, mode, seq_len, DEFAULT_SEED if seed is None else seed, \
        seq_len - 1 if qpos is None else qpos, blk


@pytest.mark.parametrize("case", REFERENCE_CASES, ids=CASE_IDS)
def test_stimulus_files_bit_exact(case):
    name, mode, seq_len, seed, qpos, blk = _case(case)
    q, k, v = gm.stimulus(mode, seq_len, seed, kv_block_len=blk)
    qb, kb, vb = gm.beats(q, k, v, 16)
    want = _digests(GOLDEN / name / "stimulus.sha256")
    assert _sha_text(_mem_text(qb)) == want["gqa_q.mem"]
    assert _sha_text(_mem_text(kb)) == want["gqa_k.mem"]
    assert _sha_text(_mem_text(vb)) == want["gqa_v.mem"]


@pytest.mark.parametrize("case", REFERENCE_CASES, ids=CASE_IDS)
def test_golden_rows_python_restatement(case):
    name, mode, seq_len, seed, qpos, blk = _case(case)
    q, k, v = gm.stimulus(mode, seq_len, seed, kv_block_len=blk)
    got = gm.golden_attention(q, k, v, seq_len, qpos)
    assert got == gm.read_mem(GOLDEN / name / "gqa_golden.mem", 128)


@pytest.mark.parametrize("case", REFERENCE_CASES, ids=CASE_IDS)
def test_golden_rows_compiled_restatement(case):
    name, mode, seq_len, seed, qpos, blk = _case(case)
    q, k, v = gm.stimulus(mode, seq_len, seed, kv_block_len=blk)
    got = orc.decode(np.array(q, dtype=np.uint16), np.array(k, dtype=np.uint16),
                     np.array(v, dtype=np.uint16), seq_len, qpos, rope_q=True, rope_k=True)
    want = np.array(gm.read_mem(GOLDEN / name / "gqa_golden.mem", 128), dtype=np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("case", REFERENCE_CASES, ids=CASE_IDS)
def test_config_text(case):
    name, mode, seq_len, seed, qpos, blk = _case(case)
    text = gm.config_text(seq_len=seq_len, head_dim=128, tile_dim=16, q_heads=32, kv_heads=8,
                          kv_block_len=blk, query_position=qpos, mode=mode, seed=seed)
    assert text == (GOLDEN / name / "gqa_config.txt").read_text()


def test_reference_committed_config_record():
    """tests/data/gqa_config.txt of the reference pins the accuracy corpus: SEQ_LEN=30,
    qpos 29, seed 20260805, 65536 valid / 69632 transported elements."""
    cfg = dict(ln.split("=", 1) for ln in (GOLDEN / "random_len30" / "gqa_config.txt")
               .read_text().splitlines())
    assert cfg["SEQ_LEN"] == "30" and cfg["QUERY_POSITION"] == "29"
    assert cfg["SEED"] == "20260805" and cfg["SCALE_BF16"] == "0x3db5"
    assert cfg["VALID_INPUT_BF16_VECTORS"] == "65536"
    assert cfg["TRANSPORT_BF16_VECTORS"] == "69632"


def test_generator_cli_writes_reference_files(tmp_path):
    """oracle/gen_vectors.py takes the reference generator's flags and writes the same
    five files byte for byte."""
    for name, mode, seq_len, seed, qpos, blk in [_case(REFERENCE_CASES[i]) for i in (0, 3, 8, 12)]:
        out = tmp_path / name
        cmd = [sys.executable, str(ROOT / "oracle" / "gen_vectors.py"), "--out-dir", str(out),
               "--mode", mode, "--seq-len", str(seq_len), "--seed", str(seed),
               "--query-position", str(qpos), "--kv-block-len", str(blk)]
        subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
        want = _digests(GOLDEN / name / "stimulus.sha256")
        for f in ("gqa_q.mem", "gqa_k.mem", "gqa_v.mem"):
            assert hashlib.sha256((out / f).read_bytes()).hexdigest() == want[f], (name, f)
        assert (out / "gqa_golden.mem").read_bytes() == (GOLDEN / name / "gqa_golden.mem").read_bytes()
        assert (out / "gqa_config.txt").read_text() == (GOLDEN / name / "gqa_config.txt").read_text()


def test_generator_cli_target_input_vectors(tmp_path):
    """--target-input-vectors 65536 selects SEQ_LEN=30 (README.md:121-140)."""
    subprocess.run([sys.executable, str(ROOT / "oracle" / "gen_vectors.py"), "--out-dir",
                    str(tmp_path), "--mode", "random", "--seed", "20260805",
                    "--target-input-vectors", "65536"], check=True, stdout=subprocess.DEVNULL)
    assert (tmp_path / "gqa_golden.mem").read_bytes() == \
        (GOLDEN / "random_len30" / "gqa_golden.mem").read_bytes()


def _rope_set():
    """pyfiles/gen_rope_test_vectors.py:16-20 restated: 512 rows, uniform(-0.25,0.25),
    seed 20260805, row r rotated at position r."""
    rng = random.Random(20260805)
    rows = [[rng.uniform(-0.25, 0.25) for _ in range(128)] for _ in range(512)]
    inp = [[gm.f32_to_bf16(x) for x in row] for row in rows]
    golden = [[gm.f32_to_bf16(x) for x in gm.rope_half_split([gm.bf16_to_f32(v) for v in row], pos)]
              for pos, row in enumerate(inp)]
    return inp, golden


def test_rope_vectors_bit_exact():
    inp, golden = _rope_set()
    want = _digests(GOLDEN / "rope" / "rope.sha256")
    in_beats = [b for row in inp for b in gm.chunks(row, 16)]
    gold_beats = [b for row in golden for b in gm.chunks(row, 16)]
    assert _sha_text(_mem_text(in_beats)) == want["in.mem"]
    assert _sha_text(_mem_text(gold_beats)) == want["golden.mem"]
    head = gm.read_mem(GOLDEN / "rope" / "golden_rows0_31.mem", 16)
    assert head == gold_beats[:len(head)]


def test_compiled_rope_matches_python_rope():
    inp, _ = _rope_set()
    for pos in (0, 1, 17, 300, 511, 131071):
        row = [gm.bf16_to_f32(v) for v in inp[pos % 512]]
        want = gm.rope_half_split(row, pos)
        got = orc.rope_row(np.array(row), pos)
        assert np.array_equal(np.array(want), got), pos


def test_bf16_primitive_words_bit_exact():
    """pyfiles/gen_bf16_primitive_vectors.py:26-36 restated; its add/mul goldens pin
    f32_to_bf16's double -> f32 -> BF16 path on 131072 roundings."""
    rng = random.Random(20260805)
    a = [gm.f32_to_bf16(rng.uniform(-0.25, 0.25)) for _ in range(65536)]
    b = [gm.f32_to_bf16(rng.uniform(-0.25, 0.25)) for _ in range(65536)]
    add = [gm.f32_to_bf16(gm.bf16_to_f32(x) + gm.bf16_to_f32(y)) for x, y in zip(a, b)]
    mul = [gm.f32_to_bf16(gm.bf16_to_f32(x) * gm.bf16_to_f32(y)) for x, y in zip(a, b)]
    want = _digests(GOLDEN / "bf16_primitives" / "bf16_primitives.sha256")

    def words(ws):
        return "\n".join(f"{w:04x}" for w in ws) + "\n"

    assert _sha_text(words(a)) == want["a.mem"]
    assert _sha_text(words(b)) == want["b.mem"]
    assert _sha_text(words(add)) == want["add_golden.mem"]
    assert _sha_text(words(mul)) == want["mul_golden.mem"]
    # the compiled rounding agrees with the Python one on the same values
    for x, y in list(zip(a, b))[:2000]:
        s = gm.bf16_to_f32(x) + gm.bf16_to_f32(y)
        assert orc.f32_to_bf16(s) == gm.f32_to_bf16(s)
