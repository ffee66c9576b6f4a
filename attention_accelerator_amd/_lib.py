"""ctypes binding of libgqa.so (the C ABI declared in include/gqa.h).

torch is imported first so that libgqa.so's libamdhip64.so.7 dependency
resolves to the HIP runtime torch already loaded: device pointers and streams
from torch are then valid in the library.  There is no fallback: if the library
is missing the import of this module's `lib()` raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("GQA_LIBRARY", PKG_DIR / "libgqa.so"))

GQA_OK = 0
GQA_ERR_INVALID_CONFIG = 1
GQA_ERR_BAD_POINTER = 2
GQA_ERR_WORKSPACE = 3
GQA_ERR_HIP = 4

GQA_ROPE_Q = 1
GQA_ROPE_K = 2
GQA_PLAN_STREAM_K = 4
GQA_PLAN_NO_MULTI_TOKEN = 8

# Every function include/gqa.h declares (checked by the CPU test suite).
EXPORTS = (
    "gqa_validate_registers",
    "gqa_validate_lengths",
    "gqa_decode_workspace_bytes",
    "gqa_decode_workspace_init",
    "gqa_decode_bf16",
    "gqa_decode_bf16_noalloc",
    "gqa_decode_paged_workspace_bytes",
    "gqa_decode_paged_bf16",
    "gqa_kv_append_paged_bf16",
    "gqa_prefill_workspace_bytes",
    "gqa_prefill_bf16",
    "gqa_prefill_rescored_rows_offset",
    "gqa_kv_append_bf16",
    "gqa_rope_rows_bf16",
    "gqa_profile_enable",
    "gqa_profile_read",
    "gqa_profile_read_stages",
    "gqa_status_string",
    "gqa_abi_version",
)


class GqaParams(ctypes.Structure):
    _fields_ = [
        ("n_q_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("scale", ctypes.c_double),
        ("rope_theta", ctypes.c_double),
        ("flags", ctypes.c_uint32),
        ("stream_wgs", ctypes.c_int32),
    ]


class GqaKvLayout(ctypes.Structure):
    _fields_ = [
        ("batch_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64),
        ("pos_stride", ctypes.c_int64),
        ("capacity", ctypes.c_int32),
    ]


class GqaPagedKv(ctypes.Structure):
    _fields_ = [
        ("block_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64),
        ("pos_stride", ctypes.c_int64),
        ("block_size", ctypes.c_int32),
        ("max_blocks", ctypes.c_int32),
        ("n_blocks", ctypes.c_int32),
    ]


class GqaProfile(ctypes.Structure):
    _fields_ = [
        ("kernel_ms", ctypes.c_double * 2),
        ("calls", ctypes.c_int32),
    ]


class GqaError(RuntimeError):
    """A non-zero status from libgqa.so."""

    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {status_string(status)} (status {status})")


class GqaConfigError(GqaError, ValueError):
    """GQA_ERR_INVALID_CONFIG: the configuration the reference core rejects at start."""


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() first")
    L = ctypes.CDLL(str(LIB_PATH))
    vp = ctypes.c_void_p
    i32p = ctypes.POINTER(ctypes.c_int32)
    L.gqa_validate_registers.argtypes = [ctypes.c_int32] * 7 + [ctypes.c_uint16]
    L.gqa_validate_registers.restype = ctypes.c_int
    L.gqa_validate_lengths.argtypes = [i32p, i32p, ctypes.c_int32, ctypes.c_int32]
    L.gqa_validate_lengths.restype = ctypes.c_int
    L.gqa_decode_workspace_bytes.argtypes = [ctypes.POINTER(GqaParams), ctypes.c_int32,
                                             ctypes.c_int32]
    L.gqa_decode_workspace_bytes.restype = ctypes.c_size_t
    L.gqa_decode_workspace_init.argtypes = [ctypes.POINTER(GqaParams), ctypes.c_int32,
                                            ctypes.c_int32, vp, ctypes.c_size_t, vp]
    L.gqa_decode_workspace_init.restype = ctypes.c_int
    L.gqa_decode_bf16.argtypes = [ctypes.POINTER(GqaParams), vp, vp, vp,
                                  ctypes.POINTER(GqaKvLayout), vp, vp, ctypes.c_int32, vp, vp,
                                  ctypes.c_size_t, vp]
    L.gqa_decode_bf16.restype = ctypes.c_int
    L.gqa_decode_bf16_noalloc.argtypes = [ctypes.POINTER(GqaParams), vp, vp, vp,
                                          ctypes.POINTER(GqaKvLayout), vp, vp, ctypes.c_int32, vp, vp]
    L.gqa_decode_bf16_noalloc.restype = ctypes.c_int
    L.gqa_decode_paged_workspace_bytes.argtypes = [ctypes.POINTER(GqaParams), ctypes.c_int32,
                                                   ctypes.c_int32]
    L.gqa_decode_paged_workspace_bytes.restype = ctypes.c_size_t
    L.gqa_decode_paged_bf16.argtypes = [ctypes.POINTER(GqaParams), vp, vp, vp,
                                        ctypes.POINTER(GqaPagedKv), vp, vp, vp, ctypes.c_int32, vp,
                                        vp, ctypes.c_size_t, vp]
    L.gqa_decode_paged_bf16.restype = ctypes.c_int
    L.gqa_kv_append_paged_bf16.argtypes = [ctypes.POINTER(GqaParams), vp, vp, vp, vp,
                                           ctypes.POINTER(GqaPagedKv), vp, vp, ctypes.c_int32,
                                           ctypes.c_int32, vp]
    L.gqa_kv_append_paged_bf16.restype = ctypes.c_int
    L.gqa_prefill_workspace_bytes.argtypes = [ctypes.POINTER(GqaParams), ctypes.c_int32,
                                              ctypes.c_int32, ctypes.c_int32]
    L.gqa_prefill_workspace_bytes.restype = ctypes.c_size_t
    L.gqa_prefill_bf16.argtypes = [ctypes.POINTER(GqaParams), vp, vp, vp, vp, vp,
                                   ctypes.POINTER(GqaKvLayout), vp, ctypes.c_int32, ctypes.c_int32,
                                   vp, vp, ctypes.c_size_t, vp]
    L.gqa_prefill_bf16.restype = ctypes.c_int
    L.gqa_prefill_rescored_rows_offset.argtypes = [ctypes.POINTER(GqaParams), ctypes.c_int32,
                                                   ctypes.c_int32, ctypes.c_int32]
    L.gqa_prefill_rescored_rows_offset.restype = ctypes.c_size_t
    L.gqa_kv_append_bf16.argtypes = [ctypes.POINTER(GqaParams), vp, vp, vp, vp,
                                     ctypes.POINTER(GqaKvLayout), vp, ctypes.c_int32, ctypes.c_int32,
                                     vp]
    L.gqa_kv_append_bf16.restype = ctypes.c_int
    L.gqa_rope_rows_bf16.argtypes = [vp, vp, ctypes.c_int64, ctypes.c_int64, vp, ctypes.c_int32,
                                     ctypes.c_double, vp]
    L.gqa_rope_rows_bf16.restype = ctypes.c_int
    L.gqa_profile_enable.argtypes = [ctypes.c_int32]
    L.gqa_profile_enable.restype = ctypes.c_int
    L.gqa_profile_read.argtypes = [ctypes.POINTER(GqaProfile)]
    L.gqa_profile_read.restype = ctypes.c_int
    L.gqa_profile_read_stages.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.c_int32,
                                          ctypes.POINTER(ctypes.c_int32)]
    L.gqa_profile_read_stages.restype = ctypes.c_int
    L.gqa_status_string.argtypes = [ctypes.c_int]
    L.gqa_status_string.restype = ctypes.c_char_p
    L.gqa_abi_version.argtypes = []
    L.gqa_abi_version.restype = ctypes.c_uint32
    _lib = L
    return L


def status_string(status: int) -> str:
    return lib().gqa_status_string(int(status)).decode()


def check(status: int, what: str) -> None:
    if status == GQA_OK:
        return
    if status == GQA_ERR_INVALID_CONFIG:
        raise GqaConfigError(status, what)
    raise GqaError(status, what)
