#!/usr/bin/env python3
"""Write the golden fixtures under tests/golden/ by running the reference's own
stdlib-only vector generators once, in this container, into a temp directory.

Why run them: the exact stimulus (the ``random.Random(seed)`` draw order and the
``.mem`` beat packing of pyfiles/gen_gqa_wrapper_vectors.py:79-119) and the
bit-exact golden rows it writes (:121-144) are pinned by nothing the reference
commits (its .gitignore drops every ``*.mem``).  Only their outputs are kept:

* per attention case: ``<case>/gqa_golden.mem`` and ``<case>/gqa_config.txt``
  verbatim, plus ``<case>/stimulus.sha256`` (digests of gqa_q/k/v.mem);
* RoPE (pyfiles/gen_rope_test_vectors.py): digests of in.mem / golden.mem plus
  the first 32 golden rows;
* BF16 add/mul (pyfiles/gen_bf16_primitive_vectors.py): digests of its four
  word files (they pin f32_to_bf16's double->f32->BF16 rounding).

Nothing here is imported by the product or by any GPU run; the fixtures are
data.  Re-run with ``python3 tests/golden/make_fixtures.py`` (needs the
reference checkout at /root/reference).
"""
from __future__ import annotations

import hashlib
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

REF = Path("/root/reference/pyfiles")
HERE = Path(__file__).resolve().parent

# name, mode, seq_len, seed (None = generator default), query_position (None = seq_len-1),
# kv_block_len.  The first six are pyfiles/run_gqa_regression.py:13-20 verbatim; the
# rest fill the gaps the reference never exercises (causal != padding, longer rows,
# the 4-entry PYNQ-Z2 block padding).
CASES = (
    ("smoke_len1", "smoke", 1, None, None, 16),
    ("random_len15", "random", 15, 20260815, None, 16),
    ("random_len16", "random", 16, 20260816, None, 16),
    ("random_len17_bp", "random", 17, 20260817, None, 16),
    ("random_len30", "random", 30, 20260805, None, 16),
    ("random_len32_bp", "random", 32, 20260832, None, 16),
    ("smoke_len16_default", "smoke", 16, None, None, 16),
    ("smoke_len30_qpos11", "smoke", 30, None, 11, 16),
    ("random_len30_qpos17", "random", 30, 20260901, 17, 16),
    ("random_len1", "random", 1, 20260902, None, 16),
    ("random_len77_qpos40", "random", 77, 20260903, 40, 16),
    ("random_len130", "random", 130, 20260904, None, 16),
    ("random_len13_blk4", "random", 13, 20260905, None, 4),
)


def sha(path: Path) -> str:
    return hashlib.sha256(path.read_bytes()).hexdigest()


def run(args: list[str]) -> None:
    subprocess.run([sys.executable, *args], cwd=REF, check=True,
                   stdout=subprocess.DEVNULL)


def main() -> None:
    with tempfile.TemporaryDirectory() as tmp_s:
        tmp = Path(tmp_s)
        for name, mode, seq_len, seed, qpos, blk in CASES:
            out = tmp / name
            cmd = [str(REF / "gen_gqa_wrapper_vectors.py"), "--out-dir", str(out),
                   "--mode", mode, "--seq-len", str(seq_len), "--kv-block-len", str(blk)]
            if seed is not None:
                cmd += ["--seed", str(seed)]
            if qpos is not None:
                cmd += ["--query-position", str(qpos)]
            run(cmd)
            dst = HERE / name
            dst.mkdir(parents=True, exist_ok=True)
            shutil.copyfile(out / "gqa_golden.mem", dst / "gqa_golden.mem")
            shutil.copyfile(out / "gqa_config.txt", dst / "gqa_config.txt")
            (dst / "stimulus.sha256").write_text(
                "".join(f"{sha(out / f)}  {f}\n" for f in ("gqa_q.mem", "gqa_k.mem", "gqa_v.mem")))
            print(f"[{name}] fixtures written")

        rope = tmp / "rope"
        run([str(REF / "gen_rope_test_vectors.py"), "--out-dir", str(rope)])
        dst = HERE / "rope"
        dst.mkdir(parents=True, exist_ok=True)
        (dst / "rope.sha256").write_text(
            "".join(f"{sha(rope / f)}  {f}\n" for f in ("in.mem", "golden.mem")))
        lines = (rope / "golden.mem").read_text().splitlines()
        (dst / "golden_rows0_31.mem").write_text("\n".join(lines[:32 * 8]) + "\n")
        print("[rope] fixtures written")

        prim = tmp / "bf16"
        run([str(REF / "gen_bf16_primitive_vectors.py"), "--out-dir", str(prim)])
        dst = HERE / "bf16_primitives"
        dst.mkdir(parents=True, exist_ok=True)
        (dst / "bf16_primitives.sha256").write_text(
            "".join(f"{sha(prim / f)}  {f}\n"
                    for f in ("a.mem", "b.mem", "add_golden.mem", "mul_golden.mem")))
        shutil.copyfile(prim / "config.txt", dst / "config.txt")
        print("[bf16_primitives] fixtures written")


if __name__ == "__main__":
    main()
