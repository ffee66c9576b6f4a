"""HIP graph capture of the prepared calls (launch amortisation: a serving loop replays one
captured step instead of issuing its launches from the host).  The library issues kernels
only -- no memset, allocation or host synchronisation inside a call -- so a step captures
as it is.  Each test replays the graph several times, with the program's own eager work
(new inputs, an eager call of the same step) between replays, and checks every replay
bit for bit against the eager call on the same inputs."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import attention_accelerator_amd as gqa
from attention_accelerator_amd import stimulus
from _util import to_codes

pytestmark = pytest.mark.gpu


def _replays(q, graph_call, eager_call, n: int = 4):
    """Capture graph_call, then per replay: new Q (eager), replay, eager reference, compare."""
    torch.cuda.synchronize()
    graph_call()                      # warm-up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = graph_call()
    gen = torch.Generator("cuda").manual_seed(77)
    for r in range(n):
        q.copy_(torch.randn(q.shape, generator=gen, device=q.device).to(torch.bfloat16))
        g.replay()
        torch.cuda.synchronize()
        got = to_codes(out)
        want = to_codes(eager_call())
        torch.cuda.synchronize()
        assert np.array_equal(got, want), f"replay {r} differs from the eager call"


@pytest.mark.parametrize("path", ["single", "stream"])
def test_decode_graph_replays(dev, path):
    """The two decode launch shapes: one launch with its in-kernel merge counters, which
    each call leaves at zero for the next (small batch), and three launches (prepare,
    stream, merge)."""
    if path == "single":
        b = stimulus.decode_batch(2, 400, min_len=50, max_len=400, seed=21, device=dev)
    else:
        b = stimulus.decode_batch(8, 3000, min_len=100, max_len=3000, seed=22, device=dev)
    p = gqa.make_params(stream_k=path != "single")
    sl = b.seq_len.to(dev).to(torch.int32)
    qpos = (sl - 1).contiguous()
    q = torch.randn((b.k.shape[0], 32, 128), device=dev).to(torch.bfloat16)
    graph_call = gqa.PreparedDecode(q, b.k, b.v, qpos, sl, params=p)
    eager_call = gqa.PreparedDecode(q, b.k, b.v, qpos, sl, params=p)
    _replays(q, graph_call, eager_call)


@pytest.mark.parametrize("n_new", [4, 8, 40])
def test_prefill_graph_replays(dev, n_new):
    """Multi-token decode (stream-K path, T = 4 and 8) and chunked prefill (attention
    kernel, T = 40): every replay re-appends the same new rows and attends with new Q."""
    starts = [300, 77, 1024]
    cap = max(starts) + n_new + 8
    g = torch.Generator("cpu").manual_seed(23)
    batch = len(starts)
    kn = torch.randn((batch, n_new, 8, 128), generator=g).to(torch.bfloat16).to(dev)
    vn = torch.randn((batch, n_new, 8, 128), generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn((batch, 8, cap, 128), generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn((batch, 8, cap, 128), generator=g).to(torch.bfloat16).to(dev)
    q = torch.randn((batch, n_new, 32, 128), generator=g).to(torch.bfloat16).to(dev)
    st = torch.tensor(starts, dtype=torch.int32, device=dev)
    graph_call = gqa.PreparedPrefill(q, kn, vn, k, v, st)
    eager_call = gqa.PreparedPrefill(q, kn, vn, k, v, st)
    _replays(q, graph_call, eager_call)


class _NoAllocDecode:
    """gqa_decode_bf16_noalloc with its arguments bound (the library's own device array as the
    workspace): the warm-up call in _replays does the array's one-time set-up eagerly."""

    def __init__(self, q, k, v, qpos, sl, out):
        import ctypes
        from attention_accelerator_amd._lib import GqaKvLayout, lib
        self.p = gqa.make_params()
        self.lay = GqaKvLayout(k.stride(0), k.stride(1), k.stride(2), k.shape[2])
        self.out = out
        self._args = (ctypes.byref(self.p), q.data_ptr(), k.data_ptr(), v.data_ptr(), ctypes.byref(self.lay),
                      sl.data_ptr(), qpos.data_ptr(), q.shape[0], out.data_ptr())
        self._fn = lib().gqa_decode_bf16_noalloc

    def __call__(self):
        st = self._fn(*self._args, torch.cuda.current_stream().cuda_stream)
        assert st == 0, f"gqa_decode_bf16_noalloc status {st}"
        return self.out


@pytest.mark.parametrize("path", ["single", "stream"])
def test_noalloc_decode_graph_replays(dev, path):
    """The entry point that allocates nothing, captured: the one-launch plan (its piece
    counters live in the library's array and every call leaves them at zero) and the
    three-launch plan (B=64 ragged); each replay bit for bit against an eager call of the
    workspace entry point on the same inputs."""
    if path == "single":
        b = stimulus.decode_batch(2, 400, min_len=50, max_len=400, seed=24, device=dev)
    else:
        b = stimulus.decode_batch(64, 2048, min_len=512, max_len=2048, seed=25, gen_device="cuda", device=dev)
    sl = b.seq_len.to(dev).to(torch.int32)
    qpos = (sl - 1).contiguous()
    q = torch.randn((b.k.shape[0], 32, 128), device=dev).to(torch.bfloat16)
    out = torch.empty((b.k.shape[0], 32, 128), dtype=torch.bfloat16, device=dev)
    graph_call = _NoAllocDecode(q, b.k, b.v, qpos, sl, out)
    eager_call = gqa.PreparedDecode(q, b.k, b.v, qpos, sl)
    _replays(q, graph_call, eager_call)
