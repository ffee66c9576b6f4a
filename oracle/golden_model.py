"""Pure-Python restatement of the reference golden model (test infrastructure only).

Only tests/, the smoke check and the benchmark's CPU-baseline leg import this
module; the product path never does.  Each function cites the reference code it
restates; the arithmetic is IEEE double exactly as the reference's stdlib Python
performs it, so on the reference's own cases the results are bit-identical to the
.mem files its generator writes (pinned against tests/golden/).

Pure-Python loops: use for small cases only.  oracle/oracle.py holds the
compiled (C) restatement of the same attention loop for large ones.
"""
from __future__ import annotations

import math
import random
import struct
import sys
from pathlib import Path
from typing import Iterable, List, Optional, Sequence

# ----------------------------------------------------------------------------
# BF16 and .mem codecs -- pyfiles/gqa_reference.py:15-57
# ----------------------------------------------------------------------------


def f32_to_bf16(value: float) -> int:
    """pyfiles/gqa_reference.py:15-19: double -> f32 via struct (RNE, raises
    OverflowError past the f32 range) -> BF16 with (bits + 0x7FFF + lsb) >> 16."""
    bits = struct.unpack(">I", struct.pack(">f", float(value)))[0]
    lsb = (bits >> 16) & 1
    return ((bits + 0x7FFF + lsb) >> 16) & 0xFFFF


def bf16_to_f32(bits: int) -> float:
    """pyfiles/gqa_reference.py:22-23: exact widening."""
    return struct.unpack(">f", struct.pack(">I", (bits & 0xFFFF) << 16))[0]


def pack_bf16(values: Iterable[int]) -> str:
    """pyfiles/gqa_reference.py:26-28: element 0 is the rightmost 4 hex digits."""
    return "".join(f"{v & 0xFFFF:04x}" for v in reversed(list(values)))


def unpack_bf16(line: str, elements: int) -> List[int]:
    """pyfiles/gqa_reference.py:31-36 ('_' separators allowed, length checked)."""
    text = line.strip().replace("_", "")
    if len(text) != elements * 4:
        raise ValueError(f"expected {elements * 4} hex digits, got {len(text)}")
    return [int(text[len(text) - 4 * (i + 1):len(text) - 4 * i], 16) for i in range(elements)]


def write_mem(path: Path, rows: Iterable[Iterable[int]]) -> None:
    """pyfiles/gqa_reference.py:39-41: one packed row per line, trailing newline."""
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text("\n".join(pack_bf16(r) for r in rows) + "\n")


def read_mem(path: Path, elements: int) -> List[List[int]]:
    """pyfiles/gqa_reference.py:44-46: blank lines and // comments skipped."""
    return [unpack_bf16(ln, elements) for ln in Path(path).read_text().splitlines()
            if ln.strip() and not ln.lstrip().startswith("//")]


def ulp_distance(a: int, b: int) -> int:
    """pyfiles/gqa_reference.py:49-53: distance of sign-magnitude codes mapped
    onto a monotonic line (+0 and -0 both map to 0x8000)."""
    def ordered(x: int) -> int:
        return 0x8000 - (x & 0x7FFF) if x & 0x8000 else 0x8000 + x
    return abs(ordered(a) - ordered(b))


def scale_for_head_dim(head_dim: int) -> int:
    """pyfiles/gqa_reference.py:56-57: BF16 code of 1/sqrt(d) (0x3db5 at d=128)."""
    return f32_to_bf16(1.0 / math.sqrt(head_dim))


def element_fails(want: int, got: int, max_ulp: int) -> bool:
    """The checker's per-element policy, pyfiles/check_gqa_output.py:57-64: fail when
    the distance exceeds max_ulp unless both BF16 exponent fields are <= 0x3d."""
    if ulp_distance(want, got) <= max_ulp:
        return False
    return not (((want >> 7) & 0xFF) <= 0x3D and ((got >> 7) & 0xFF) <= 0x3D)


# ----------------------------------------------------------------------------
# RoPE and the golden attention -- pyfiles/gen_gqa_wrapper_vectors.py
# ----------------------------------------------------------------------------


def chunks(row: Sequence[int], tile_dim: int):
    """pyfiles/gen_gqa_wrapper_vectors.py:20-22."""
    for start in range(0, len(row), tile_dim):
        yield list(row[start:start + tile_dim])


def rope_half_split(row: Sequence[float], position: int, theta: float = 500000.0) -> List[float]:
    """pyfiles/gen_gqa_wrapper_vectors.py:25-35: rotate_half pairing (i, i+n/2)."""
    half = len(row) // 2
    out = list(row)
    for i in range(half):
        angle = position * theta ** (-2.0 * i / len(row))
        c, s = math.cos(angle), math.sin(angle)
        x, y = row[i], row[i + half]
        out[i] = x * c - y * s
        out[i + half] = x * s + y * c
    return out


def golden_attention(q_bits, k_bits, v_bits, seq_len: int, query_position: int,
                     *, rope_q: bool = True, rope_k: bool = True, theta: float = 500000.0,
                     scale: Optional[float] = None) -> List[List[int]]:
    """pyfiles/gen_gqa_wrapper_vectors.py:124-139 for one query token.

    q_bits[qh][d], k_bits/v_bits[kh][p][d] are BF16 codes (rows past seq_len ignored).
    rope_q / rope_k select which operands are rotated (the reference rotates both;
    a cache stored post-RoPE sets rope_k=False).  Returns out[qh][d] BF16 codes."""
    q_heads, kv_heads = len(q_bits), len(k_bits)
    head_dim = len(q_bits[0])
    group = q_heads // kv_heads
    qpos = query_position

    def prep(row, pos, rot):
        vals = [bf16_to_f32(x) for x in row]
        return rope_half_split(vals, pos, theta) if rot else vals

    q_ref = [prep(row, qpos, rope_q) for row in q_bits]
    k_ref = [[prep(row, p, rope_k) for p, row in enumerate(head[:seq_len])] for head in k_bits]
    v_ref = [[[bf16_to_f32(x) for x in row] for row in head[:seq_len]] for head in v_bits]
    sc = 1.0 / math.sqrt(head_dim) if scale is None else scale
    golden = []
    for qh in range(q_heads):
        kh = qh // group
        scores = [sum(q_ref[qh][d] * k_ref[kh][p][d] for d in range(head_dim)) * sc
                  for p in range(qpos + 1)]
        max_score = max(scores)
        weights = [math.exp(s - max_score) for s in scores]
        normalizer = sum(weights)
        golden.append([f32_to_bf16(sum(weights[p] * v_ref[kh][p][d]
                                       for p in range(qpos + 1)) / normalizer)
                       for d in range(head_dim)])
    return golden


# ----------------------------------------------------------------------------
# Stimulus -- pyfiles/gen_gqa_wrapper_vectors.py:79-119
# ----------------------------------------------------------------------------


def kv_input_len(seq_len: int, kv_block_len: int) -> int:
    """pyfiles/gen_gqa_wrapper_vectors.py:83: seq_len rounded up to whole blocks."""
    return ((seq_len + kv_block_len - 1) // kv_block_len) * kv_block_len


def stimulus(mode: str, seq_len: int, seed: int, *, q_heads: int = 32, kv_heads: int = 8,
             head_dim: int = 128, kv_block_len: int = 16):
    """Inputs as BF16 codes, restating pyfiles/gen_gqa_wrapper_vectors.py:79-107.

    mode "smoke":  Q = K = 0, V[h][p][d] = 0.03125(1+h) + 0.0078125p + 0.001953125(d%17)
    mode "random": uniform(-0.25, 0.25) drawn q -> k -> v, head -> position -> dim;
                   pad rows are zero and consume no draws.
    mode "normal": this build's N(0,1) variant (random.gauss) in the same draw order.
    Returns (q[qh][d], k[kh][p][d], v[kh][p][d]) with kv_input_len(...) positions."""
    rng = random.Random(seed)
    n_pos = kv_input_len(seq_len, kv_block_len)
    if mode == "smoke":
        q = [[0.0] * head_dim for _ in range(q_heads)]
        k = [[[0.0] * head_dim for _ in range(n_pos)] for _ in range(kv_heads)]
        v = [[[(0.03125 * (1 + h) + 0.0078125 * p + 0.001953125 * (d % 17)) if p < seq_len else 0.0
               for d in range(head_dim)] for p in range(n_pos)] for h in range(kv_heads)]
    elif mode in ("random", "normal"):
        draw = (lambda: rng.uniform(-0.25, 0.25)) if mode == "random" else (lambda: rng.gauss(0.0, 1.0))
        q = [[draw() for _ in range(head_dim)] for _ in range(q_heads)]
        k = [[[(draw() if p < seq_len else 0.0) for _ in range(head_dim)] for p in range(n_pos)]
             for _ in range(kv_heads)]
        v = [[[(draw() if p < seq_len else 0.0) for _ in range(head_dim)] for p in range(n_pos)]
             for _ in range(kv_heads)]
    else:
        raise ValueError(f"unknown mode {mode!r}")
    q_bits = [[f32_to_bf16(x) for x in row] for row in q]
    k_bits = [[[f32_to_bf16(x) for x in row] for row in head] for head in k]
    v_bits = [[[f32_to_bf16(x) for x in row] for row in head] for head in v]
    return q_bits, k_bits, v_bits


def beats(q_bits, k_bits, v_bits, tile_dim: int = 16):
    """AXIS beat order, pyfiles/gen_gqa_wrapper_vectors.py:111-119: Q rows head by head,
    then K (and V) head -> position -> 16-element beat, pad rows included."""
    qb = [b for row in q_bits for b in chunks(row, tile_dim)]
    kb = [b for head in k_bits for row in head for b in chunks(row, tile_dim)]
    vb = [b for head in v_bits for row in head for b in chunks(row, tile_dim)]
    return qb, kb, vb


def config_text(*, seq_len: int, head_dim: int, tile_dim: int, q_heads: int, kv_heads: int,
                kv_block_len: int, query_position: int, mode: str, seed: int) -> str:
    """gqa_config.txt, pyfiles/gen_gqa_wrapper_vectors.py:145-152 (same keys and order)."""
    n_pos = kv_input_len(seq_len, kv_block_len)
    return (f"SEQ_LEN={seq_len}\nHEAD_DIM={head_dim}\nTILE_DIM={tile_dim}\n"
            f"N_Q_HEADS={q_heads}\nN_KV_HEADS={kv_heads}\nGROUP_SIZE={q_heads // kv_heads}\n"
            f"KV_BLOCK_LEN={kv_block_len}\n"
            f"QUERY_POSITION={query_position}\nKV_INPUT_SEQ_LEN={n_pos}\n"
            f"SCALE_BF16=0x{scale_for_head_dim(head_dim):04x}\n"
            f"MODE={mode}\nSEED={seed}\n"
            f"VALID_INPUT_BF16_VECTORS={q_heads * head_dim + 2 * kv_heads * seq_len * head_dim}\n"
            f"TRANSPORT_BF16_VECTORS={q_heads * head_dim + 2 * kv_heads * n_pos * head_dim}\n")


def python_sum_mode() -> int:
    """0 when this interpreter's sum() adds floats left to right (CPython <= 3.11),
    1 when it is Neumaier-compensated (CPython >= 3.12)."""
    return 1 if sys.version_info >= (3, 12) else 0
