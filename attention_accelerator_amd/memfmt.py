"""The reference's .mem text format and gqa_config.txt, vectorised with numpy.

Format (pyfiles/gqa_reference.py:26-46): one packed row per line as hex, element
0 in the rightmost four digits; blank lines and lines starting with // are
skipped; '_' separators are ignored.  Stimulus files carry 16-element beats in
the order Q: head -> beat, K/V: head -> position -> beat
(pyfiles/gen_gqa_wrapper_vectors.py:111-119); output files carry one 128-element
row per Q head (pyfiles/check_gqa_output.py:4-7).
"""
from __future__ import annotations

from pathlib import Path
from typing import Dict

import numpy as np


def read_mem(path: Path, elements: int) -> np.ndarray:
    """-> uint16 [rows, elements]."""
    rows = []
    for line in Path(path).read_text().splitlines():
        if not line.strip() or line.lstrip().startswith("//"):
            continue
        text = line.strip().replace("_", "")
        if len(text) != elements * 4:
            raise ValueError(f"{path}: expected {elements * 4} hex digits, got {len(text)}")
        rows.append(text)
    if not rows:
        return np.zeros((0, elements), dtype=np.uint16)
    vals = np.frombuffer(bytes.fromhex("".join(rows)), dtype=">u2").astype(np.uint16)
    return vals.reshape(len(rows), elements)[:, ::-1].copy()


def format_mem(rows: np.ndarray) -> str:
    rows = np.asarray(rows, dtype=np.uint16)
    if rows.ndim != 2:
        raise ValueError("rows must be 2-D")
    width = rows.shape[1] * 4
    text = np.ascontiguousarray(rows[:, ::-1]).astype(">u2").tobytes().hex()
    return "\n".join(text[i:i + width] for i in range(0, len(text), width)) + "\n"


def write_mem(path: Path, rows: np.ndarray) -> None:
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(format_mem(rows))


def read_config(path: Path) -> Dict[str, str]:
    """KEY=VALUE lines of gqa_config.txt (pyfiles/gen_gqa_wrapper_vectors.py:145-152)."""
    cfg: Dict[str, str] = {}
    for line in Path(path).read_text().splitlines():
        if "=" in line:
            k, v = line.split("=", 1)
            cfg[k.strip()] = v.strip()
    return cfg


def config_int(cfg: Dict[str, str], key: str, default=None) -> int:
    if key not in cfg:
        if default is None:
            raise KeyError(key)
        return default
    return int(cfg[key], 0)


def beats_to_rows(beats: np.ndarray, head_dim: int) -> np.ndarray:
    """[n_beats, tile_dim] -> [n_rows, head_dim] (beats of a row are consecutive)."""
    beats = np.asarray(beats, dtype=np.uint16)
    return beats.reshape(-1, head_dim)
