"""torch-facing operators over libgqa.so.

The call surface is the golden model's (pyfiles/gen_gqa_wrapper_vectors.py:121-139,
README.md:41-50): Q rows of one token, a K/V cache in position order,
`query_position` and `seq_len` in; 32 x 128 BF16 output rows out, in Q-head order.
Batches of independent sequences are the same call with a leading batch
dimension and per-sequence lengths.

Every op runs the HIP kernels of libgqa.so on the current torch stream and
raises if the library is not built; there is no CPU path.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Sequence, Union

import torch

from . import _lib
from ._lib import (GQA_PLAN_NO_MULTI_TOKEN, GQA_PLAN_STREAM_K, GQA_ROPE_K, GQA_ROPE_Q, GqaKvLayout, GqaPagedKv,
                   GqaParams, check, lib)

N_Q_HEADS = 32
N_KV_HEADS = 8
GROUP_SIZE = N_Q_HEADS // N_KV_HEADS
HEAD_DIM = 128
ROPE_THETA = 500000.0
DEFAULT_SCALE = 1.0 / math.sqrt(HEAD_DIM)

Lengths = Union[int, Sequence[int], torch.Tensor]


def make_params(*, rope_q: bool = True, rope_k: bool = False, theta: float = ROPE_THETA,
                scale: Optional[float] = None, n_q_heads: int = N_Q_HEADS,
                n_kv_heads: int = N_KV_HEADS, head_dim: int = HEAD_DIM, stream_wgs: int = 0,
                stream_k: bool = False, multi_token: bool = True) -> GqaParams:
    """The call parameters.  Plan choices (tests and tuning; the results stay within the same
    tolerance): stream_wgs > 0 sets the persistent workgroups of the stream-K kernels (0:
    four per CU), stream_k=True makes every contiguous decode call take the three-launch
    stream-K plan, multi_token=False sends chunks of at most 16 tokens through the prefill
    attention kernel.  Workspace sizes follow these fields, so size a workspace with the
    params of the call that will use it."""
    flags = ((GQA_ROPE_Q if rope_q else 0) | (GQA_ROPE_K if rope_k else 0)
             | (GQA_PLAN_STREAM_K if stream_k else 0) | (0 if multi_token else GQA_PLAN_NO_MULTI_TOKEN))
    return GqaParams(n_q_heads, n_kv_heads, head_dim,
                     DEFAULT_SCALE if scale is None else float(scale), float(theta), flags, int(stream_wgs))


def _plan_key(p: GqaParams, batch: int, capacity: int):
    return (int(batch), int(capacity), int(p.flags) & (GQA_PLAN_STREAM_K | GQA_PLAN_NO_MULTI_TOKEN),
            int(p.stream_wgs))


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _lengths_to_device(x: Lengths, batch: int, device: torch.device, name: str):
    """Returns (device int32 tensor, host int32 tensor or None)."""
    if isinstance(x, torch.Tensor) and x.is_cuda:
        if x.dtype != torch.int32 or x.numel() != batch:
            raise ValueError(f"{name} must be an int32 tensor of {batch} elements")
        return x.contiguous(), None
    host = torch.as_tensor(x, dtype=torch.int32).reshape(-1)
    if host.numel() == 1 and batch > 1:
        host = host.expand(batch)
    if host.numel() != batch:
        raise ValueError(f"{name} has {host.numel()} entries for a batch of {batch}")
    host = host.contiguous()
    return host.to(device, non_blocking=False), host


def decode_workspace_bytes(batch: int, capacity: int, params: Optional[GqaParams] = None) -> int:
    p = params or make_params()
    return int(lib().gqa_decode_workspace_bytes(ctypes.byref(p), int(batch), int(capacity)))


def new_workspace(batch: int, capacity: int, device, params: Optional[GqaParams] = None
                  ) -> torch.Tensor:
    """A decode workspace for `batch` sequences of up to `capacity` positions, prepared
    with gqa_decode_workspace_init.  Reuse it across calls with the same batch size on
    one stream; calls sharing it must not overlap."""
    p = params or make_params()
    nbytes = int(lib().gqa_decode_workspace_bytes(ctypes.byref(p), int(batch), int(capacity)))
    if nbytes == 0:
        check(_lib.GQA_ERR_INVALID_CONFIG, "gqa_decode_workspace_bytes")
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    check(lib().gqa_decode_workspace_init(ctypes.byref(p), int(batch), int(capacity), ws.data_ptr(),
                                          nbytes, _stream_handle(torch.device(device))),
          "gqa_decode_workspace_init")
    ws.gqa_decode_plan = _plan_key(p, batch, capacity)
    return ws


def _check_workspace_plan(workspace: torch.Tensor, p: GqaParams, batch: int, capacity: int) -> None:
    """A workspace from new_workspace carries the plan (batch, capacity, plan flags,
    stream_wgs) it was prepared for; the single-launch path's piece counters sit where that
    plan puts them, so another plan would find stale data there and leave rows unwritten.
    Reject the mismatch."""
    plan = getattr(workspace, "gqa_decode_plan", None)
    want = _plan_key(p, batch, capacity)
    if plan is not None and plan != want:
        raise ValueError(f"workspace was prepared for (batch, capacity, plan flags, stream_wgs) = {plan}, "
                         f"called with {want}; make one with new_workspace({batch}, {capacity}, ..., params)")


def gqa_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  query_position: Lengths, seq_len: Lengths, *, rope_q: bool = True,
                  rope_k: bool = False, theta: float = ROPE_THETA, scale: Optional[float] = None,
                  out: Optional[torch.Tensor] = None,
                  workspace: Optional[torch.Tensor] = None,
                  params: Optional[GqaParams] = None) -> torch.Tensor:
    """One GQA decode step (32 Q heads over 8 KV heads, head_dim 128, BF16).

    q        [32, 128] or [B, 32, 128] bfloat16 (CUDA/HIP)
    k_cache  [8, S, 128] or [B, 8, S, 128] bfloat16, positions in order; the last
             dim must be contiguous (any other strides, multiples of 8)
    v_cache  same shape and strides as k_cache
    query_position, seq_len: int, a sequence of B ints, or an int32 tensor.  Host
             values are validated first (1 <= seq_len <= S, 0 <= qpos < seq_len);
             device tensors are read by the kernel as they are.
    rope_q / rope_k: rotate Q at query_position / each K row at its position
             (the reference core does both; a cache stored post-RoPE sets rope_k=False)
    workspace: from new_workspace(B, S, device) to reuse across calls (else one is
             allocated and prepared per call)
    Returns out [.., 32, 128] bfloat16.  Key p contributes iff p < seq_len and
    p <= query_position.  Raises GqaConfigError for what the reference rejects."""
    single = q.dim() == 2
    if single:
        q, k_cache, v_cache = q.unsqueeze(0), k_cache.unsqueeze(0), v_cache.unsqueeze(0)
    if q.dim() != 3 or k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError("expected q [B,32,128] and k/v [B,8,S,128]")
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        if t.dtype != torch.bfloat16 or not t.is_cuda:
            raise ValueError(f"{name} must be a bfloat16 tensor on the GPU")
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share shape and strides")
    batch = q.shape[0]
    if k_cache.shape[0] != batch:
        raise ValueError("batch mismatch between q and the cache")
    if k_cache.stride(3) != 1:
        raise ValueError("cache rows must be contiguous in head_dim")
    q = q.contiguous()
    device = q.device
    capacity = k_cache.shape[2]
    p = params or make_params(rope_q=rope_q, rope_k=rope_k, theta=theta, scale=scale,
                              n_q_heads=q.shape[1], n_kv_heads=k_cache.shape[1],
                              head_dim=q.shape[2])
    sl_dev, sl_host = _lengths_to_device(seq_len, batch, device, "seq_len")
    qp_dev, qp_host = _lengths_to_device(query_position, batch, device, "query_position")
    if sl_host is not None and qp_host is not None:
        check(lib().gqa_validate_lengths(
            ctypes.cast(sl_host.data_ptr(), ctypes.POINTER(ctypes.c_int32)),
            ctypes.cast(qp_host.data_ptr(), ctypes.POINTER(ctypes.c_int32)), batch, capacity),
            "gqa_validate_lengths")
    ws_bytes = int(lib().gqa_decode_workspace_bytes(ctypes.byref(p), batch, capacity))
    if ws_bytes == 0:
        check(_lib.GQA_ERR_INVALID_CONFIG, "gqa_decode_workspace_bytes")
    if workspace is None:
        workspace = new_workspace(batch, capacity, device, p)
    elif workspace.numel() * workspace.element_size() < ws_bytes:
        raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} bytes; "
                         f"{ws_bytes} needed")
    _check_workspace_plan(workspace, p, batch, capacity)
    if out is None:
        out = torch.empty((batch, q.shape[1], q.shape[2]), dtype=torch.bfloat16, device=device)
    elif out.shape != (batch, q.shape[1], q.shape[2]) or out.dtype != torch.bfloat16 \
            or not out.is_contiguous():
        raise ValueError("out must be a contiguous bfloat16 [B,32,128] tensor")
    layout = GqaKvLayout(k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), capacity)
    status = lib().gqa_decode_bf16(
        ctypes.byref(p), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        ctypes.byref(layout), sl_dev.data_ptr(), qp_dev.data_ptr(), batch, out.data_ptr(),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        _stream_handle(device))
    check(status, "gqa_decode_bf16")
    return out[0] if single else out


gqa_decode = gqa_attention


def rope_half_split(rows: torch.Tensor, position: Union[int, torch.Tensor] = 0, *,
                    theta: float = ROPE_THETA, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """rotate_half RoPE of BF16 rows [N, 128] on the GPU (the rope_unit of rope_unit.v).

    position: an int p0 (row r at p0 + r, as tests/tb_rope_unit.sv drives it) or a
    device int32 tensor of N positions.  Output BF16 = round(f32(round(rope in double)))."""
    if rows.dtype != torch.bfloat16 or not rows.is_cuda or rows.dim() != 2 \
            or rows.shape[1] != HEAD_DIM or rows.stride(1) != 1:
        raise ValueError("rows must be a bfloat16 [N,128] GPU tensor with contiguous rows")
    if out is None:
        out = torch.empty_like(rows, memory_format=torch.contiguous_format)
    if out.shape != rows.shape or out.stride() != rows.stride():
        rows = rows.contiguous()
        if out.stride() != rows.stride():
            raise ValueError("out must match rows' layout")
    pos_ptr, pos0 = None, 0
    if isinstance(position, torch.Tensor):
        if not position.is_cuda or position.dtype != torch.int32 or position.numel() != rows.shape[0]:
            raise ValueError("position tensor must be int32 on the GPU with one entry per row")
        position = position.contiguous()
        pos_ptr = position.data_ptr()
    else:
        pos0 = int(position)
    status = lib().gqa_rope_rows_bf16(rows.data_ptr(), out.data_ptr(), rows.shape[0], rows.stride(0),
                                      pos_ptr, pos0, float(theta), _stream_handle(rows.device))
    check(status, "gqa_rope_rows_bf16")
    return out


class PreparedDecode:
    """A decode call with every argument bound once, for loops that repeat the same
    step (serving, benchmarking): calling it issues gqa_decode_bf16 on the current
    stream with no per-call tensor checks, allocation or host validation.

    Lengths must be device int32 tensors (validate them once with
    validate_lengths); the tensors passed in must stay alive while it is used."""

    def __init__(self, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 query_position: torch.Tensor, seq_len: torch.Tensor, *, rope_q: bool = True,
                 rope_k: bool = False, theta: float = ROPE_THETA, scale: Optional[float] = None,
                 out: Optional[torch.Tensor] = None, params: Optional[GqaParams] = None):
        if q.dim() != 3 or k_cache.dim() != 4:
            raise ValueError("expected q [B,32,128] and k/v [B,8,S,128]")
        if not (query_position.is_cuda and seq_len.is_cuda):
            raise ValueError("lengths must be device tensors")
        if k_cache.stride() != v_cache.stride() or k_cache.stride(3) != 1:
            raise ValueError("k_cache and v_cache must share strides with contiguous rows")
        self.batch = q.shape[0]
        self.capacity = k_cache.shape[2]
        self.params = params or make_params(rope_q=rope_q, rope_k=rope_k, theta=theta, scale=scale)
        self.layout = GqaKvLayout(k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
                                  self.capacity)
        self.workspace = new_workspace(self.batch, self.capacity, q.device, self.params)
        ws_bytes = self.workspace.numel()
        if out is not None and (out.shape != (self.batch, N_Q_HEADS, HEAD_DIM) or out.dtype != torch.bfloat16
                                or not out.is_contiguous() or out.device != q.device):
            raise ValueError("out must be a contiguous bfloat16 [B,32,128] tensor on q's device")
        self.out = out if out is not None else torch.empty(
            (self.batch, N_Q_HEADS, HEAD_DIM), dtype=torch.bfloat16, device=q.device)
        self._keep = (q.contiguous(), k_cache, v_cache, query_position.contiguous(),
                      seq_len.contiguous())
        qc, kc, vc, qp, sl = self._keep
        self._args = (ctypes.byref(self.params), qc.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                      ctypes.byref(self.layout), sl.data_ptr(), qp.data_ptr(), self.batch,
                      self.out.data_ptr(), self.workspace.data_ptr(), ws_bytes)
        self._fn = lib().gqa_decode_bf16
        self.device = q.device

    def __call__(self) -> torch.Tensor:
        status = self._fn(*self._args, _stream_handle(self.device))
        if status:
            check(status, "gqa_decode_bf16")
        return self.out


def _cache_layout(k_cache: torch.Tensor, v_cache: torch.Tensor) -> GqaKvLayout:
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must be [B,8,S,128] with the same shape and strides")
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
        if t.dtype != torch.bfloat16 or not t.is_cuda:
            raise ValueError(f"{name} must be a bfloat16 tensor on the GPU")
    if k_cache.stride(3) != 1:
        raise ValueError("cache rows must be contiguous in head_dim")
    return GqaKvLayout(k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), k_cache.shape[2])


def _start_tensor(start: Lengths, batch: int, capacity: int, n_new: int, device):
    """Device int32 start positions; host values are checked first
    (0 <= start <= capacity - n_new)."""
    if isinstance(start, torch.Tensor) and start.is_cuda:
        if start.dtype != torch.int32 or start.numel() != batch:
            raise ValueError(f"start must be an int32 tensor of {batch} elements")
        return start.contiguous()
    host = torch.as_tensor(start, dtype=torch.int32).reshape(-1)
    if host.numel() == 1 and batch > 1:
        host = host.expand(batch)
    if host.numel() != batch:
        raise ValueError(f"start has {host.numel()} entries for a batch of {batch}")
    if int(host.min()) < 0 or int(host.max()) > capacity - n_new:
        check(_lib.GQA_ERR_INVALID_CONFIG, "start positions")
    return host.contiguous().to(device)


def _capacity_arg(capacity) -> int:
    if isinstance(capacity, GqaParams):
        raise TypeError("prefill workspace size: the third argument is the cache capacity (positions "
                        "per sequence); pass params as a keyword, params=...")
    return int(capacity)


def prefill_workspace_bytes(batch: int, n_new: int, capacity: int, params: Optional[GqaParams] = None) -> int:
    """Workspace bytes of a gqa_prefill call: batch sequences, n_new new tokens each, a cache
    of `capacity` positions per sequence (chunks of more than 16 tokens stage 512 bytes per
    position of every (sequence, KV head) in it)."""
    p = params or make_params()
    return int(lib().gqa_prefill_workspace_bytes(ctypes.byref(p), int(batch), int(n_new), _capacity_arg(capacity)))


def prefill_rescored_rows(workspace: torch.Tensor, batch: int, n_new: int, capacity: int,
                          params: Optional[GqaParams] = None) -> int:
    """How many output rows the last gqa_prefill call on `workspace` recomputed in fp64 (the
    rows its MFMA kernels may have computed outside 64 BF16 ULP).  Synchronises the device."""
    p = params or make_params()
    off = int(lib().gqa_prefill_rescored_rows_offset(ctypes.byref(p), int(batch), int(n_new),
                                                     _capacity_arg(capacity)))
    if off == 0:
        check(_lib.GQA_ERR_INVALID_CONFIG, "gqa_prefill_rescored_rows_offset")
    word = workspace.view(torch.uint8)[off:off + 4].cpu().numpy().view("<u4")
    return int(word[0])


def gqa_prefill(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
                v_cache: torch.Tensor, start: Lengths, *, rope_q: bool = True, rope_k: bool = True,
                theta: float = ROPE_THETA, scale: Optional[float] = None,
                out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
                params: Optional[GqaParams] = None) -> torch.Tensor:
    """Chunked prefill: T new tokens per sequence after start[b] cached positions.

    q            [B, T, 32, 128] bfloat16 (rotated at positions start+t when rope_q)
    k_new, v_new [B, T, 8, 128] bfloat16 (K rotated at start+t when rope_k)
    k_cache, v_cache [B, 8, S, 128] bfloat16, rows < start post-RoPE; the chunk's rows are
             written at start+t (K rotated, rounded to BF16) before the attention
    start    int, B ints, or a device int32 tensor (host values checked:
             0 <= start <= S - T)
    Returns out [B, T, 32, 128]: token t attends to keys p <= start + t."""
    if q.dim() != 4 or k_new.dim() != 4 or v_new.shape != k_new.shape:
        raise ValueError("expected q [B,T,32,128] and k_new/v_new [B,T,8,128]")
    for name, t in (("q", q), ("k_new", k_new), ("v_new", v_new)):
        if t.dtype != torch.bfloat16 or not t.is_cuda:
            raise ValueError(f"{name} must be a bfloat16 tensor on the GPU")
    batch, n_new = q.shape[0], q.shape[1]
    if k_new.shape[:2] != (batch, n_new) or k_cache.shape[0] != batch:
        raise ValueError("batch / token count mismatch")
    layout = _cache_layout(k_cache, v_cache)
    p = params or make_params(rope_q=rope_q, rope_k=rope_k, theta=theta, scale=scale,
                              n_q_heads=q.shape[2], n_kv_heads=k_new.shape[2], head_dim=q.shape[3])
    device = q.device
    st = _start_tensor(start, batch, k_cache.shape[2], n_new, device)
    q, k_new, v_new = q.contiguous(), k_new.contiguous(), v_new.contiguous()
    ws_bytes = int(lib().gqa_prefill_workspace_bytes(ctypes.byref(p), batch, n_new, layout.capacity))
    if ws_bytes == 0:
        check(_lib.GQA_ERR_INVALID_CONFIG, "gqa_prefill_workspace_bytes")
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    elif workspace.numel() * workspace.element_size() < ws_bytes:
        raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} bytes; "
                         f"{ws_bytes} needed")
    if out is None:
        out = torch.empty(q.shape, dtype=torch.bfloat16, device=device)
    elif out.shape != q.shape or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("out must be a contiguous bfloat16 tensor shaped like q")
    status = lib().gqa_prefill_bf16(
        ctypes.byref(p), q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_cache.data_ptr(),
        v_cache.data_ptr(), ctypes.byref(layout), st.data_ptr(), batch, n_new, out.data_ptr(),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream_handle(device))
    check(status, "gqa_prefill_bf16")
    return out


class PreparedPrefill:
    """A chunked-prefill call with every argument bound once (the prefill counterpart of
    PreparedDecode): calling it issues gqa_prefill_bf16 on the current stream with no
    per-call checks or allocation.  start must be a device int32 tensor whose values
    satisfy 0 <= start <= S - T (checked on the device: a bad entry gives NaN rows); the
    tensors passed in must stay alive while it is used."""

    def __init__(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
                 v_cache: torch.Tensor, start: torch.Tensor, *, rope_q: bool = True, rope_k: bool = True,
                 theta: float = ROPE_THETA, scale: Optional[float] = None,
                 out: Optional[torch.Tensor] = None, params: Optional[GqaParams] = None):
        if q.dim() != 4 or k_new.dim() != 4 or v_new.shape != k_new.shape:
            raise ValueError("expected q [B,T,32,128] and k_new/v_new [B,T,8,128]")
        if not (isinstance(start, torch.Tensor) and start.is_cuda and start.dtype == torch.int32):
            raise ValueError("start must be a device int32 tensor")
        self.batch, self.n_new = q.shape[0], q.shape[1]
        if k_new.shape[:2] != (self.batch, self.n_new) or start.numel() != self.batch:
            raise ValueError("batch / token count mismatch")
        self.layout = _cache_layout(k_cache, v_cache)
        self.params = params or make_params(rope_q=rope_q, rope_k=rope_k, theta=theta, scale=scale)
        ws_bytes = int(lib().gqa_prefill_workspace_bytes(ctypes.byref(self.params), self.batch, self.n_new,
                                                          self.layout.capacity))
        if ws_bytes == 0:
            check(_lib.GQA_ERR_INVALID_CONFIG, "gqa_prefill_workspace_bytes")
        self.workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
        self.out = out if out is not None else torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
        self._keep = (q.contiguous(), k_new.contiguous(), v_new.contiguous(), k_cache, v_cache,
                      start.contiguous())
        qc, kn, vn, kc, vc, st = self._keep
        self._args = (ctypes.byref(self.params), qc.data_ptr(), kn.data_ptr(), vn.data_ptr(), kc.data_ptr(),
                      vc.data_ptr(), ctypes.byref(self.layout), st.data_ptr(), self.batch, self.n_new,
                      self.out.data_ptr(), self.workspace.data_ptr(), ws_bytes)
        self._fn = lib().gqa_prefill_bf16
        self.device = q.device

    def __call__(self) -> torch.Tensor:
        status = self._fn(*self._args, _stream_handle(self.device))
        if status:
            check(status, "gqa_prefill_bf16")
        return self.out

    def rescored_rows(self) -> int:
        """Output rows the last call recomputed in fp64 (synchronises the device)."""
        return prefill_rescored_rows(self.workspace, self.batch, self.n_new, self.layout.capacity, self.params)


def kv_append(k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
              v_cache: torch.Tensor, start: Lengths, *, rope_k: bool = True,
              theta: float = ROPE_THETA) -> None:
    """Write k_new / v_new [B, T, 8, 128] into the cache at positions start+t, K rotated
    at its position (rope_k) and rounded to BF16: the cache stays post-RoPE."""
    if k_new.dim() != 4 or v_new.shape != k_new.shape:
        raise ValueError("expected k_new/v_new [B,T,8,128]")
    for name, t in (("k_new", k_new), ("v_new", v_new)):
        if t.dtype != torch.bfloat16 or not t.is_cuda:
            raise ValueError(f"{name} must be a bfloat16 tensor on the GPU")
    batch, n_new = k_new.shape[0], k_new.shape[1]
    layout = _cache_layout(k_cache, v_cache)
    p = make_params(rope_q=False, rope_k=rope_k, theta=theta, n_kv_heads=k_new.shape[2],
                    head_dim=k_new.shape[3])
    st = _start_tensor(start, batch, k_cache.shape[2], n_new, k_new.device)
    k_new, v_new = k_new.contiguous(), v_new.contiguous()
    status = lib().gqa_kv_append_bf16(ctypes.byref(p), k_new.data_ptr(), v_new.data_ptr(),
                                      k_cache.data_ptr(), v_cache.data_ptr(), ctypes.byref(layout),
                                      st.data_ptr(), batch, n_new, _stream_handle(k_new.device))
    check(status, "gqa_kv_append_bf16")


BLOCK_SIZE = 16   # positions per block of a paged cache (the core's KV_BLOCK_LEN)


def _paged_layout(k_pool: torch.Tensor, v_pool: torch.Tensor, block_table: torch.Tensor
                  ) -> GqaPagedKv:
    """Pools [n_blocks, 8, 16, 128] bfloat16 (any strides with contiguous rows), block
    table [B, max_blocks] int32 on the device."""
    if k_pool.dim() != 4 or k_pool.shape != v_pool.shape or k_pool.stride() != v_pool.stride():
        raise ValueError("k_pool and v_pool must be [n_blocks,8,16,128] with the same strides")
    if k_pool.shape[2] != BLOCK_SIZE:
        raise ValueError(f"blocks hold {BLOCK_SIZE} positions")
    for name, t in (("k_pool", k_pool), ("v_pool", v_pool)):
        if t.dtype != torch.bfloat16 or not t.is_cuda:
            raise ValueError(f"{name} must be a bfloat16 tensor on the GPU")
    if k_pool.stride(3) != 1:
        raise ValueError("pool rows must be contiguous in head_dim")
    if block_table.dim() != 2 or block_table.dtype != torch.int32 or not block_table.is_cuda:
        raise ValueError("block_table must be an int32 [B, max_blocks] tensor on the GPU")
    if k_pool.shape[1] != N_KV_HEADS or k_pool.shape[3] != HEAD_DIM:
        raise ValueError(f"pools hold {N_KV_HEADS} KV heads of {HEAD_DIM} dimensions per block")
    return GqaPagedKv(k_pool.stride(0), k_pool.stride(1), k_pool.stride(2), BLOCK_SIZE,
                      block_table.shape[1], k_pool.shape[0])


def gqa_decode_paged(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                     block_table: torch.Tensor, query_position: Lengths, seq_len: Lengths, *,
                     rope_q: bool = True, rope_k: bool = False, theta: float = ROPE_THETA,
                     scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                     workspace: Optional[torch.Tensor] = None,
                     params: Optional[GqaParams] = None) -> torch.Tensor:
    """gqa_attention over a paged cache: q [B, 32, 128]; k_pool, v_pool [n_blocks, 8, 16,
    128]; block_table [B, max_blocks] int32 (block j of sequence b holds positions
    16j .. 16j+15).  Host lengths are checked against capacity = 16 * max_blocks."""
    if q.dim() != 3 or q.dtype != torch.bfloat16 or not q.is_cuda or q.shape[1:] != (N_Q_HEADS, HEAD_DIM):
        raise ValueError("q must be a bfloat16 [B,32,128] tensor on the GPU")
    layout = _paged_layout(k_pool, v_pool, block_table)
    batch = q.shape[0]
    if block_table.shape[0] != batch:
        raise ValueError("block_table has one row per sequence")
    capacity = BLOCK_SIZE * block_table.shape[1]
    device = q.device
    p = params or make_params(rope_q=rope_q, rope_k=rope_k, theta=theta, scale=scale)
    sl_dev, sl_host = _lengths_to_device(seq_len, batch, device, "seq_len")
    qp_dev, qp_host = _lengths_to_device(query_position, batch, device, "query_position")
    if sl_host is not None and qp_host is not None:
        check(lib().gqa_validate_lengths(
            ctypes.cast(sl_host.data_ptr(), ctypes.POINTER(ctypes.c_int32)),
            ctypes.cast(qp_host.data_ptr(), ctypes.POINTER(ctypes.c_int32)), batch, capacity),
            "gqa_validate_lengths")
    ws_bytes = int(lib().gqa_decode_paged_workspace_bytes(ctypes.byref(p), batch,
                                                          block_table.shape[1]))
    if ws_bytes == 0:
        check(_lib.GQA_ERR_INVALID_CONFIG, "gqa_decode_paged_workspace_bytes")
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    elif workspace.numel() * workspace.element_size() < ws_bytes:
        raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} bytes; "
                         f"{ws_bytes} needed")
    if out is None:
        out = torch.empty((batch, N_Q_HEADS, HEAD_DIM), dtype=torch.bfloat16, device=device)
    elif out.shape != (batch, N_Q_HEADS, HEAD_DIM) or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("out must be a contiguous bfloat16 [B,32,128] tensor")
    q = q.contiguous()
    bt = block_table.contiguous()
    status = lib().gqa_decode_paged_bf16(
        ctypes.byref(p), q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), ctypes.byref(layout),
        bt.data_ptr(), sl_dev.data_ptr(), qp_dev.data_ptr(), batch, out.data_ptr(),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream_handle(device))
    check(status, "gqa_decode_paged_bf16")
    return out


def kv_append_paged(k_new: torch.Tensor, v_new: torch.Tensor, k_pool: torch.Tensor,
                    v_pool: torch.Tensor, block_table: torch.Tensor, start: Lengths, *,
                    rope_k: bool = True, theta: float = ROPE_THETA) -> None:
    """kv_append into a paged cache (rows to block block_table[b][(start+t)//16])."""
    if k_new.dim() != 4 or v_new.shape != k_new.shape:
        raise ValueError("expected k_new/v_new [B,T,8,128]")
    for name, t in (("k_new", k_new), ("v_new", v_new)):
        if t.dtype != torch.bfloat16 or not t.is_cuda:
            raise ValueError(f"{name} must be a bfloat16 tensor on the GPU")
    layout = _paged_layout(k_pool, v_pool, block_table)
    batch, n_new = k_new.shape[0], k_new.shape[1]
    p = make_params(rope_q=False, rope_k=rope_k, theta=theta)
    st = _start_tensor(start, batch, BLOCK_SIZE * block_table.shape[1], n_new, k_new.device)
    k_new, v_new = k_new.contiguous(), v_new.contiguous()
    bt = block_table.contiguous()
    status = lib().gqa_kv_append_paged_bf16(ctypes.byref(p), k_new.data_ptr(), v_new.data_ptr(),
                                            k_pool.data_ptr(), v_pool.data_ptr(), ctypes.byref(layout),
                                            bt.data_ptr(), st.data_ptr(), batch, n_new,
                                            _stream_handle(k_new.device))
    check(status, "gqa_kv_append_paged_bf16")


def validate_lengths(seq_len, query_position, capacity: int) -> None:
    """Host check of lengths (raises GqaConfigError), gen_gqa_wrapper_vectors.py:73-78."""
    sl = torch.as_tensor(seq_len, dtype=torch.int32).reshape(-1).contiguous()
    qp = torch.as_tensor(query_position, dtype=torch.int32).reshape(-1).contiguous()
    if sl.numel() != qp.numel():
        raise ValueError("seq_len and query_position differ in length")
    check(lib().gqa_validate_lengths(ctypes.cast(sl.data_ptr(), ctypes.POINTER(ctypes.c_int32)),
                                     ctypes.cast(qp.data_ptr(), ctypes.POINTER(ctypes.c_int32)),
                                     sl.numel(), int(capacity)), "gqa_validate_lengths")


def profile_enable(max_calls: int) -> None:
    """Start recording kernel times of up to max_calls decode or prefill calls (0 stops)."""
    check(lib().gqa_profile_enable(int(max_calls)), "gqa_profile_enable")


def profile_read():
    """-> (first_kernel_ms_total, second_kernel_ms_total, calls) recorded since the last
    read: decode calls {stream, merge}, prefill calls {KV append, attention}."""
    p = _lib.GqaProfile()
    check(lib().gqa_profile_read(ctypes.byref(p)), "gqa_profile_read")
    return p.kernel_ms[0], p.kernel_ms[1], p.calls


def profile_read_stages():
    """-> ([stage_ms_total] * 4, calls) recorded since the last read: decode {stream, merge,
    0, 0}, prefill {append + staging + reduce, attention, rescore, 0}, prefill of at most 16
    new tokens {preparation, stream, merge, rescore}."""
    ms = (ctypes.c_double * 4)()
    n = ctypes.c_int32(0)
    check(lib().gqa_profile_read_stages(ms, 4, ctypes.byref(n)), "gqa_profile_read_stages")
    return list(ms), n.value
