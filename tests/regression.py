#!/usr/bin/env python3
"""Reproducible end-to-end GQA regressions on the GPU: the flow of
pyfiles/run_gqa_regression.py with the Vivado/XSim step replaced by
attention_accelerator_amd.mem_runner.

Per case (pyfiles/run_gqa_regression.py:13-20): generate vectors with
oracle/gen_vectors.py (same files as the reference generator) -> run the GPU
kernel on them (VECTORS_DIR, OUTPUT_BACKPRESSURE has no meaning here) -> the
runner prints PASS:/FAIL: against gqa_golden.mem, and the output file is checked
again with the checker's CLI (pyfiles/check_gqa_output.py) -> then the
invalid-configuration case (N_Q_HEADS=31) must print
"PASS: invalid configuration rejected" (:66-77).
"""
from __future__ import annotations

import argparse
import contextlib
import io
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

CASES = (
    ("smoke_len1", "smoke", 1, None, False),
    ("random_len15", "random", 15, 20260815, False),
    ("random_len16", "random", 16, 20260816, False),
    ("random_len17_bp", "random", 17, 20260817, True),
    ("random_len30", "random", 30, 20260805, False),
    ("random_len32_bp", "random", 32, 20260832, True),
)


def _run_runner(vectors: Path, env_extra: dict, in_process: bool) -> tuple[int, str]:
    if not in_process:
        env = os.environ.copy()
        env.update(env_extra)
        env["VECTORS_DIR"] = str(vectors)
        res = subprocess.run([sys.executable, "-m", "attention_accelerator_amd.mem_runner"],
                             cwd=ROOT, env=env, text=True, stdout=subprocess.PIPE,
                             stderr=subprocess.STDOUT)
        return res.returncode, res.stdout
    from attention_accelerator_amd import mem_runner
    buf = io.StringIO()
    argv = ["--vectors", str(vectors)]
    if env_extra.get("INVALID_CONFIG") == "1":
        argv.append("--invalid-config")
    with contextlib.redirect_stdout(buf):
        rc = mem_runner.main(argv)
    return rc, buf.getvalue()


def run(out_dir: Path, keep_going: bool = False, generate_only: bool = False,
        in_process: bool = False) -> int:
    failures = []
    for name, mode, seq_len, seed, backpressure in CASES:
        vectors = out_dir / name / "vectors"
        vectors.mkdir(parents=True, exist_ok=True)
        cmd = [sys.executable, str(ROOT / "oracle" / "gen_vectors.py"), "--out-dir", str(vectors),
               "--mode", mode, "--seq-len", str(seq_len)]
        if seed is not None:
            cmd += ["--seed", str(seed)]
        res = subprocess.run(cmd, text=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
        print(f"[{name}] vector generation\n{res.stdout}", end="")
        if res.returncode:
            failures.append(name)
        elif not generate_only:
            rc, text = _run_runner(vectors, {}, in_process)
            (out_dir / name / "runner.log").write_text(text)
            passed = rc == 0 and "PASS:" in text
            if passed:
                from attention_accelerator_amd import check
                buf = io.StringIO()
                try:
                    with contextlib.redirect_stdout(buf):
                        check.main(["--golden", str(vectors / "gqa_golden.mem"),
                                    "--actual", str(vectors / "gqa_rtl_out.mem"), "--show-rows", "0"])
                except SystemExit as e:
                    passed = False
                    buf.write(str(e))
                passed = passed and "PASS:" in buf.getvalue()
                text += buf.getvalue()
            print(f"[{name}] {'PASS' if passed else 'FAIL'}\n{text}", end="")
            if not passed:
                failures.append(name)
        if failures and not keep_going:
            break
    if not generate_only and not failures:
        name = "invalid_config"
        rc, text = _run_runner(out_dir / "smoke_len1" / "vectors", {"INVALID_CONFIG": "1"},
                               in_process)
        passed = rc == 0 and "PASS: invalid configuration rejected" in text
        print(f"[{name}] {'PASS' if passed else 'FAIL'}\n{text}", end="")
        if not passed:
            failures.append(name)
    if failures:
        print("GQA REGRESSION FAILED: " + ", ".join(failures))
        return 1
    if generate_only:
        print(f"GQA REGRESSION VECTORS GENERATED: {len(CASES)} datapath cases")
    else:
        print(f"GQA REGRESSION PASSED: {len(CASES)} datapath cases plus invalid-config rejection")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--out-dir", type=Path, default=Path("build/gqa_regression"))
    ap.add_argument("--keep-going", action="store_true")
    ap.add_argument("--generate-only", action="store_true")
    ap.add_argument("--in-process", action="store_true",
                    help="run the GPU step in this process instead of a subprocess per case")
    args = ap.parse_args()
    return run(args.out_dir.resolve(), args.keep_going, args.generate_only, args.in_process)


if __name__ == "__main__":
    raise SystemExit(main())
