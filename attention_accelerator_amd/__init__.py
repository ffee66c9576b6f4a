"""MI355X-native GQA attention step (Llama-3-8B geometry) behind a C ABI.

Public surface:
  gqa_attention / gqa_decode   one decode step, batch of sequences (HIP kernels)
  gqa_decode_paged             the same over a paged cache (block tables, blocks of 16)
  gqa_prefill                  chunked prefill, T new tokens per sequence (HIP/MFMA kernels)
  kv_append, kv_append_paged   KV append with RoPE on insert (HIP kernel)
  rope_half_split              rotate_half RoPE of BF16 rows (HIP kernel)
  decode_workspace_bytes       workspace size of a decode call
  prefill_rescored_rows        output rows a prefill call recomputed in fp64 (measurement)
Tools: check (output checker), mem_runner (.mem stimulus -> GPU -> .mem output),
memfmt (.mem codec), stimulus (synthetic inputs), build (hipcc in-tree build).
"""
from .attention import (DEFAULT_SCALE, GROUP_SIZE, HEAD_DIM, N_KV_HEADS, N_Q_HEADS,  # noqa: F401
                        ROPE_THETA, PreparedDecode, PreparedPrefill, decode_workspace_bytes, gqa_attention,
                        gqa_decode, gqa_decode_paged, gqa_prefill, kv_append, kv_append_paged,
                        make_params, new_workspace, prefill_rescored_rows, prefill_workspace_bytes,
                        profile_enable, profile_read, profile_read_stages, rope_half_split,
                        validate_lengths)
from ._lib import GqaConfigError, GqaError  # noqa: F401

__version__ = "0.1.0"
