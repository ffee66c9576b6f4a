"""The ctypes stub that INTEGRATION.md gives a maintainer (its sections 2, 4 and 5), run as
written: the Python blocks are taken from the document, the library path filled in, and the
stub's functions called.

* gqa_step (the golden-model call surface) on the reference's regression case random_len30
  against the golden rows its generator wrote (64 BF16 ULP, pyfiles/check_gqa_output.py:57-64);
* gqa_prefill_step and gqa_decode_paged_step against the package's tensor calls on the same
  inputs, bit for bit (same library, same kernels)."""
from __future__ import annotations

import re

import numpy as np
import pytest
import torch

import attention_accelerator_amd as gqa
from attention_accelerator_amd import _lib
from attention_accelerator_amd.memfmt import read_mem
from conftest import GOLDEN, ROOT
from oracle import golden_model as gm
from _util import assert_within_ulp, to_codes

pytestmark = pytest.mark.gpu


def _stub() -> dict:
    text = (ROOT / "INTEGRATION.md").read_text()
    blocks = []
    for sec in ("## 2.", "## 4.", "## 5."):
        start = text.index(sec)
        end = text.find("\n## ", start + 4)
        part = text[start:end if end > 0 else len(text)]
        blocks += re.findall(r"```python\n(.*?)```", part, flags=re.S)
    assert len(blocks) == 3, "one Python block per section"
    src = "\n".join(blocks)
    assert '"/path/to/attention_accelerator_amd/libgqa.so"' in src
    src = src.replace('"/path/to/attention_accelerator_amd/libgqa.so"', repr(str(_lib.LIB_PATH)))
    ns: dict = {}
    exec(compile(src, "INTEGRATION.md", "exec"), ns)
    return ns


def test_golden_call_surface(dev):
    ns = _stub()
    q, k, v = gm.stimulus("random", 30, 20260805)
    got = np.asarray(ns["gqa_step"](q, k, v, 30, 29), dtype=np.uint16)
    golden = read_mem(GOLDEN / "random_len30" / "gqa_golden.mem", 128)
    w = assert_within_ulp(golden, got, 64, "INTEGRATION.md gqa_step, random_len30")
    print(f"gqa_step random_len30: worst {w} ULP", flush=True)


def test_prefill_and_paged_stubs(dev):
    ns = _stub()
    g = torch.Generator("cpu").manual_seed(5)
    starts, n_new, cap = [100, 37], 8, 160
    q = torch.randn((2, n_new, 32, 128), generator=g).to(torch.bfloat16).to(dev)
    kn = torch.randn((2, n_new, 8, 128), generator=g).to(torch.bfloat16).to(dev)
    vn = torch.randn((2, n_new, 8, 128), generator=g).to(torch.bfloat16).to(dev)
    k0 = torch.randn((2, 8, cap, 128), generator=g).to(torch.bfloat16).to(dev)
    v0 = torch.randn((2, 8, cap, 128), generator=g).to(torch.bfloat16).to(dev)
    k1, v1, k2, v2 = k0.clone(), v0.clone(), k0.clone(), v0.clone()
    a = ns["gqa_prefill_step"](q, kn, vn, k1, v1, starts)
    b = gqa.gqa_prefill(q, kn, vn, k2, v2, starts)
    torch.cuda.synchronize()
    assert np.array_equal(to_codes(a), to_codes(b))
    assert torch.equal(k1, k2) and torch.equal(v1, v2)

    # paged decode over the prefilled cache: blocks of 16 positions in reverse pool order
    nb = cap // 16
    perm = torch.arange(2 * nb - 1, -1, -1)
    kp = k1.reshape(2, 8, nb, 16, 128).permute(0, 2, 1, 3, 4).reshape(2 * nb, 8, 16, 128)[perm].contiguous()
    vp = v1.reshape(2, 8, nb, 16, 128).permute(0, 2, 1, 3, 4).reshape(2 * nb, 8, 16, 128)[perm].contiguous()
    table = torch.empty(2 * nb, dtype=torch.int32)
    table[perm] = torch.arange(2 * nb, dtype=torch.int32)
    table = table.reshape(2, nb).to(dev)
    sl = torch.tensor([s + n_new for s in starts], dtype=torch.int32, device=dev)
    qp = (sl - 1).contiguous()
    qd = torch.randn((2, 32, 128), generator=g).to(torch.bfloat16).to(dev)
    c = ns["gqa_decode_paged_step"](qd, kp, vp, table, sl, qp)
    d = gqa.gqa_decode_paged(qd, kp, vp, table, qp, sl)
    torch.cuda.synchronize()
    assert np.array_equal(to_codes(c), to_codes(d))
    e = gqa.gqa_attention(qd, k1, v1, qp, sl)
    torch.cuda.synchronize()
    assert_within_ulp(to_codes(e), to_codes(c), 1, "paged stub vs contiguous decode")
