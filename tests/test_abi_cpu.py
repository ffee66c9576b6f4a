"""C-ABI checks that need no GPU: the library loads, exports every function
include/gqa.h declares, and rejects bad configurations before any launch
(gqa_attention_wrapper.v:230-244: start suppressed, error flag raised)."""
from __future__ import annotations

import ctypes
import math
import re

import pytest

from attention_accelerator_amd import _lib
from attention_accelerator_amd._lib import GqaKvLayout, GqaParams
from conftest import ROOT

OK, BAD_CFG, BAD_PTR, BAD_WS = 0, 1, 2, 3


def header_functions():
    text = (ROOT / "include" / "gqa.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gqa_[a-z0-9_]+)\s*\(", text)))


def test_exports_match_header():
    declared = header_functions()
    assert declared == sorted(_lib.EXPORTS)
    L = _lib.lib()
    for name in declared:
        assert hasattr(L, name), name


def test_status_strings_and_version():
    assert _lib.status_string(0) == "ok"
    assert "invalid" in _lib.status_string(1)
    assert _lib.lib().gqa_abi_version() >> 16 == 4


@pytest.mark.parametrize("regs,ok", [
    ((32, 8, 128, 16, 30, 2, 16, 0x3DB5), True),
    ((32, 8, 128, 16, 13, 4, 4, 0x3DB5), True),      # PYNQ-Z2 KV_BLOCK_LEN=4
    ((31, 8, 128, 16, 30, 2, 16, 0x3DB5), False),    # N_Q_HEADS (tb_gqa_attention_wrapper.sv:323)
    ((32, 4, 128, 16, 30, 2, 16, 0x3DB5), False),    # N_KV_HEADS
    ((32, 8, 64, 16, 30, 2, 16, 0x3DB5), False),     # HEAD_DIM
    ((32, 8, 128, 8, 30, 2, 16, 0x3DB5), False),     # TILE_DIM
    ((32, 8, 128, 16, 0, 0, 16, 0x3DB5), False),     # SEQ_LEN == 0
    ((32, 8, 128, 16, 30, 1, 16, 0x3DB5), False),    # N_KV_TILES != ceil(30/16)
    ((32, 8, 128, 16, 32, 3, 16, 0x3DB5), False),
    ((32, 8, 128, 16, 30, 2, 16, 0x0000), False),    # SCALE == 0
])
def test_validate_registers(regs, ok):
    st = _lib.lib().gqa_validate_registers(*regs)
    assert st == (OK if ok else BAD_CFG)


def _lens(vals):
    arr = (ctypes.c_int32 * len(vals))(*vals)
    return arr


@pytest.mark.parametrize("sl,qp,cap,want", [
    ([30], [29], 32, OK), ([1], [0], 1, OK), ([30, 17], [10, 16], 32, OK),
    ([30], [30], 32, BAD_CFG), ([30], [-1], 32, BAD_CFG), ([0], [0], 32, BAD_CFG),
    ([33], [0], 32, BAD_CFG),
])
def test_validate_lengths(sl, qp, cap, want):
    assert _lib.lib().gqa_validate_lengths(_lens(sl), _lens(qp), len(sl), cap) == want


def _params(**kw):
    base = dict(n_q_heads=32, n_kv_heads=8, head_dim=128, scale=1 / math.sqrt(128),
                rope_theta=500000.0, flags=1)
    base.update(kw)
    return GqaParams(**base)


def test_workspace_bytes():
    L = _lib.lib()
    p = _params()
    n = L.gqa_decode_workspace_bytes(ctypes.byref(p), 64, 8192)
    assert n > 0 and n % 256 == 0
    assert L.gqa_decode_workspace_bytes(ctypes.byref(_params(n_q_heads=31)), 64, 8192) == 0
    assert L.gqa_decode_workspace_bytes(ctypes.byref(p), 0, 8192) == 0


def _decode(p, *, q=256, k=256, v=256, layout=None, sl=256, qp=256, batch=1, out=256,
            ws=256, ws_bytes=1 << 30):
    L = _lib.lib()
    layout = layout or GqaKvLayout(8 * 64 * 128, 64 * 128, 128, 64)
    return L.gqa_decode_bf16(ctypes.byref(p) if p is not None else None, q, k, v,
                             ctypes.byref(layout), sl, qp, batch, out, ws, ws_bytes, None)


@pytest.mark.parametrize("kw,want", [
    (dict(p=_params(n_q_heads=31)), BAD_CFG),
    (dict(p=_params(n_kv_heads=4)), BAD_CFG),
    (dict(p=_params(head_dim=64)), BAD_CFG),
    (dict(p=_params(scale=0.0)), BAD_CFG),
    (dict(p=_params(scale=float("nan"))), BAD_CFG),
    (dict(p=_params(rope_theta=0.0)), BAD_CFG),
    (dict(p=_params(flags=16)), BAD_CFG),
    (dict(p=_params(stream_wgs=-1)), BAD_CFG),
    (dict(p=_params(stream_wgs=65537)), BAD_CFG),
    (dict(p=_params(), batch=0), BAD_CFG),
    (dict(p=_params(), layout=GqaKvLayout(0, 0, 64, 64)), BAD_CFG),
    (dict(p=_params(), layout=GqaKvLayout(0, 0, 128, 0)), BAD_CFG),
    (dict(p=None), BAD_PTR),
    (dict(p=_params(), q=None), BAD_PTR),
    (dict(p=_params(), k=None), BAD_PTR),
    (dict(p=_params(), out=None), BAD_PTR),
    (dict(p=_params(), sl=None), BAD_PTR),
    (dict(p=_params(), k=264), BAD_PTR),                        # K not 16-byte aligned
    (dict(p=_params(), layout=GqaKvLayout(8, 0, 132, 64)), BAD_PTR),   # stride % 8
    (dict(p=_params(), ws=None), BAD_WS),
    (dict(p=_params(), ws_bytes=16), BAD_WS),
])
def test_decode_rejects_before_launch(kw, want):
    """Every rejection returns before touching the device (the fake pointers here
    would fault if anything were launched)."""
    assert _decode(**kw) == want


def test_rope_rejects():
    L = _lib.lib()
    assert L.gqa_rope_rows_bf16(256, 256, 4, 64, None, 0, 500000.0, None) == BAD_CFG
    assert L.gqa_rope_rows_bf16(256, 256, 4, 128, None, 0, -1.0, None) == BAD_CFG
    assert L.gqa_rope_rows_bf16(None, 256, 4, 128, None, 0, 500000.0, None) == BAD_PTR
    assert L.gqa_rope_rows_bf16(None, None, 0, 128, None, 0, 500000.0, None) == OK


def test_profile_read_empty():
    p = _lib.GqaProfile()
    assert _lib.lib().gqa_profile_read(ctypes.byref(p)) == OK
    assert p.calls == 0


def test_profile_read_stages_empty_and_bounds():
    L = _lib.lib()
    ms = (ctypes.c_double * 4)(-1.0, -1.0, -1.0, -1.0)
    n = ctypes.c_int32(-1)
    assert L.gqa_profile_read_stages(ms, 4, ctypes.byref(n)) == OK
    assert n.value == 0 and list(ms) == [0.0, 0.0, 0.0, 0.0]
    assert L.gqa_profile_read_stages(ms, 5, ctypes.byref(n)) == BAD_PTR       # at most four stages
    assert L.gqa_profile_read_stages(None, 2, ctypes.byref(n)) == BAD_PTR
    assert L.gqa_profile_read_stages(ms, 2, None) == OK                       # the count is optional
    assert L.gqa_abi_version() == (4 << 16) | 1


def test_workspace_init_rejects():
    L = _lib.lib()
    p = _params()
    n = L.gqa_decode_workspace_bytes(ctypes.byref(p), 4, 1000)
    assert L.gqa_decode_workspace_init(ctypes.byref(_params(n_q_heads=31)), 4, 1000, 256, n, None) == BAD_CFG
    assert L.gqa_decode_workspace_init(ctypes.byref(p), 0, 1000, 256, n, None) == BAD_CFG
    assert L.gqa_decode_workspace_init(ctypes.byref(p), 4, 1000, None, n, None) == BAD_WS
    assert L.gqa_decode_workspace_init(ctypes.byref(p), 4, 1000, 256, n - 1, None) == BAD_WS
    assert L.gqa_decode_workspace_init(ctypes.byref(p), 4, 1000, 260, n, None) == BAD_WS
    assert L.gqa_decode_workspace_init(None, 4, 1000, 256, n, None) == BAD_PTR


def test_prefill_workspace_bytes():
    L = _lib.lib()
    p = _params(flags=3)
    n = L.gqa_prefill_workspace_bytes(ctypes.byref(p), 4, 512, 8704)
    # at least the fp16 K and V staging planes (8704 positions of 32 (sequence, KV head) pairs)
    # and the fp32 rotated new K rows
    assert n >= 2 * 4 * 8 * 8704 * 128 * 2 + 4 * 512 * 8 * 128 * 4 and n % 256 == 0
    # the staging planes (and per pair one block scale word and the block's key and V maxima
    # for the rescore flag, 8 + 64 words) follow the capacity, rounded up to 64 positions
    grow = L.gqa_prefill_workspace_bytes(ctypes.byref(p), 4, 512, 8705) - n
    assert 2 * 4 * 8 * 64 * 128 * 2 <= grow <= 2 * 4 * 8 * 64 * 128 * 2 + 4 * 8 * (1 + 8 + 64) * 4 + 768
    assert L.gqa_prefill_workspace_bytes(ctypes.byref(_params(head_dim=64)), 4, 512, 8704) == 0
    assert L.gqa_prefill_workspace_bytes(ctypes.byref(p), 4, 0, 8704) == 0
    assert L.gqa_prefill_workspace_bytes(ctypes.byref(p), 4, 512, 511) == 0


def _prefill(p, *, q=256, kn=256, vn=256, k=256, v=256, layout=None, start=256, batch=1,
             n_new=8, out=256, ws=256, ws_bytes=1 << 30):
    L = _lib.lib()
    layout = layout or GqaKvLayout(8 * 64 * 128, 64 * 128, 128, 64)
    return L.gqa_prefill_bf16(ctypes.byref(p) if p is not None else None, q, kn, vn, k, v,
                              ctypes.byref(layout), start, batch, n_new, out, ws, ws_bytes, None)


@pytest.mark.parametrize("kw,want", [
    (dict(p=_params(n_q_heads=31)), BAD_CFG),
    (dict(p=_params(scale=0.0)), BAD_CFG),
    (dict(p=_params(flags=3, rope_theta=-5.0)), BAD_CFG),
    (dict(p=_params(), batch=0), BAD_CFG),
    (dict(p=_params(), n_new=0), BAD_CFG),
    (dict(p=_params(), n_new=65), BAD_CFG),                      # chunk longer than the cache
    (dict(p=_params(), layout=GqaKvLayout(0, 0, 64, 64)), BAD_CFG),
    (dict(p=_params(), layout=GqaKvLayout(0, 0, 1 << 25, 64)), BAD_CFG),   # rows span >= 4 GiB
    (dict(p=None), BAD_PTR),
    (dict(p=_params(), q=None), BAD_PTR),
    (dict(p=_params(), kn=None), BAD_PTR),
    (dict(p=_params(), start=None), BAD_PTR),
    (dict(p=_params(), out=None), BAD_PTR),
    (dict(p=_params(), k=264), BAD_PTR),
    (dict(p=_params(), out=260), BAD_PTR),
    (dict(p=_params(), ws=None), BAD_WS),
    (dict(p=_params(), ws_bytes=16), BAD_WS),
])
def test_prefill_rejects_before_launch(kw, want):
    assert _prefill(**kw) == want


def test_kv_append_rejects_before_launch():
    L = _lib.lib()
    lay = GqaKvLayout(8 * 64 * 128, 64 * 128, 128, 64)
    p = _params(flags=2)
    assert L.gqa_kv_append_bf16(None, 256, 256, 256, 256, ctypes.byref(lay), 256, 1, 1, None) == BAD_PTR
    assert L.gqa_kv_append_bf16(ctypes.byref(p), 256, 256, 256, 256, ctypes.byref(lay), 256, 0, 1, None) == BAD_CFG
    assert L.gqa_kv_append_bf16(ctypes.byref(p), 256, 256, 256, 256, ctypes.byref(lay), 256, 1, 65, None) == BAD_CFG
    assert L.gqa_kv_append_bf16(ctypes.byref(p), 256, None, 256, 256, ctypes.byref(lay), 256, 1, 1, None) == BAD_PTR
    assert L.gqa_kv_append_bf16(ctypes.byref(p), 256, 256, 264, 256, ctypes.byref(lay), 256, 1, 1, None) == BAD_PTR


def test_workspace_plan_tag():
    """A workspace tagged with its plan (batch, capacity, plan flags, stream_wgs) is rejected
    for another plan (the single-launch counters sit at a plan-dependent offset); untagged
    buffers pass."""
    import torch
    from attention_accelerator_amd.attention import _check_workspace_plan, _plan_key, make_params
    p = make_params()
    ws = torch.empty(16, dtype=torch.uint8)
    _check_workspace_plan(ws, p, 4, 1000)                 # untagged: the caller's contract
    ws.gqa_decode_plan = _plan_key(p, 4, 1000)
    _check_workspace_plan(ws, p, 4, 1000)
    _check_workspace_plan(ws, make_params(rope_k=True), 4, 1000)      # RoPE flags do not move it
    for args in ((p, 4, 2000), (p, 3, 1000), (make_params(stream_k=True), 4, 1000),
                 (make_params(stream_wgs=96), 4, 1000)):
        with pytest.raises(ValueError, match="prepared for"):
            _check_workspace_plan(ws, *args)


_SIZES_SCRIPT = r"""
import ctypes, json
from attention_accelerator_amd import _lib
from attention_accelerator_amd.attention import make_params
L = _lib.lib()
out = []
for kw in ({}, {"stream_wgs": 96}, {"stream_k": True}, {"multi_token": False}):
    p = make_params(rope_k=True, **kw)
    out.append([L.gqa_decode_workspace_bytes(ctypes.byref(p), b, c) for b, c in ((4, 2048), (64, 8192))]
               + [L.gqa_decode_paged_workspace_bytes(ctypes.byref(p), 64, 512)]
               + [L.gqa_prefill_workspace_bytes(ctypes.byref(p), b, t, c)
                  for b, t, c in ((64, 16, 8208), (64, 8, 8200), (4, 512, 8704))]
               + [L.gqa_prefill_rescored_rows_offset(ctypes.byref(p), 64, 16, 8208)])
print(json.dumps(out))
"""


def test_workspace_sizes_ignore_the_environment():
    """Workspace sizes (and the rescored-row offset) follow the arguments only: the same
    numbers in processes whose environments set the variables that once chose the plan and
    the XCD weighting of the ranges (which moves no buffer)."""
    import json
    import os
    import subprocess
    import sys
    envs = [{}, {"GQA_STREAM_WGS": "96", "GQA_PREFILL_MULTI": "0", "GQA_SINGLE_LAUNCH_MAX_KEYS": "0",
                 "GQA_XCD_SKEW": "250"}]
    runs = []
    for extra in envs:
        env = dict(os.environ)
        for k in ("GQA_STREAM_WGS", "GQA_PREFILL_MULTI", "GQA_SINGLE_LAUNCH_MAX_KEYS", "GQA_XCD_SKEW"):
            env.pop(k, None)
        env.update(extra)
        env["PYTHONPATH"] = str(ROOT) + os.pathsep + env.get("PYTHONPATH", "")
        r = subprocess.run([sys.executable, "-c", _SIZES_SCRIPT], env=env, cwd=str(ROOT),
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        runs.append(json.loads(r.stdout.strip().splitlines()[-1]))
    assert runs[0] == runs[1]
    sizes = runs[0]
    assert all(n > 0 for row in sizes for n in row)
    # the params fields do choose the plan: stream_wgs moves the stream-K buffers, stream_k
    # the small decode batch's plan, multi_token the short chunks' path
    assert sizes[1][1] != sizes[0][1] and sizes[1][3] != sizes[0][3]
    assert sizes[2][0] != sizes[0][0]
    assert sizes[3][3] != sizes[0][3] and sizes[3][5] == sizes[0][5]


def test_python_shape_checks_before_any_launch():
    """Host-side shape checks of the paged entry point reject wrong geometry on the CPU
    (tensors not on a GPU are rejected before any library call)."""
    import torch
    import attention_accelerator_amd as gqa
    q = torch.zeros((2, 32, 128), dtype=torch.bfloat16)
    pool = torch.zeros((4, 8, 16, 128), dtype=torch.bfloat16)
    table = torch.zeros((2, 2), dtype=torch.int32)
    with pytest.raises(ValueError):
        gqa.gqa_decode_paged(q, pool, pool, table, [0, 0], [1, 1])
    with pytest.raises(ValueError):
        gqa.gqa_decode_paged(q[:, :16], pool, pool, table, [0, 0], [1, 1])
