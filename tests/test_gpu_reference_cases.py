"""The reference's regression cases on the GPU kernel, against the golden rows its
own generator wrote (tests/golden/, pyfiles/run_gqa_regression.py:13-20 + extras).

Both operands rotated (Q at QUERY_POSITION, K at each position), scale 1/sqrt(128),
output within 64 BF16 ULP per element (pyfiles/check_gqa_output.py:33-34,57-64)."""
from __future__ import annotations

import pytest

from attention_accelerator_amd import gqa_attention
from attention_accelerator_amd.memfmt import read_mem
from conftest import DEFAULT_SEED, GOLDEN, REFERENCE_CASES
from oracle import golden_model as gm
from _util import assert_within_ulp, to_codes, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", REFERENCE_CASES, ids=[c[0] for c in REFERENCE_CASES])
def test_reference_case(case, dev):
    name, mode, seq_len, seed, qpos, blk = case
    qpos = seq_len - 1 if qpos is None else qpos
    q, k, v = gm.stimulus(mode, seq_len, DEFAULT_SEED if seed is None else seed, kv_block_len=blk)
    out = gqa_attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), qpos, seq_len,
                        rope_q=True, rope_k=True)
    golden = read_mem(GOLDEN / name / "gqa_golden.mem", 128)
    w = assert_within_ulp(golden, to_codes(out), 64, name)
    print(f"{name}: worst {w} ULP")
