"""Compile libgqa.so for gfx950 in-tree with hipcc (no JIT cache, no torch extension ABI)."""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
SOURCES = ("gqa_abi.hip", "gqa_decode.hip", "gqa_prefill.hip", "gqa_multitoken.hip", "gqa_rope.hip")
OUT = PKG / "libgqa.so"

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Wall", "-Wno-unused-command-line-argument",
    # packed fp32 VALU ops stay off (the compiler would otherwise form v_pk_* from scalar code)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def build(verbose: bool = False) -> Path:
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{ROOT / 'include'}", f"-I{CSRC}", "-o", str(OUT) + ".tmp",
           *[str(CSRC / s) for s in SOURCES]]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    text = "\n".join(ln for ln in res.stdout.splitlines() if "packed-fp32-ops" not in ln)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{text}")
    if verbose and text.strip():
        print(text)
    os.replace(str(OUT) + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
