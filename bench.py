#!/usr/bin/env python3
"""Benchmark: batched ragged GQA decode on one MI355X.

Workload (default): B=64 sequences, KV lengths drawn uniformly from [512, 8192]
(seed 20260805), cache capacity 8192, 32 Q / 8 KV heads, head_dim 128, BF16
N(0,1) inputs, K cache stored post-RoPE (RoPE on Q in the kernel), query_position
= length - 1, unused cache rows NaN.  One step = one gqa_decode_bf16 call (prepare,
stream and merge kernels) on inputs already resident in HBM.

Prints one JSON line: value = algorithmic HBM bytes of the step / time per step
(GB/s) over K uninstrumented steps, ms_per_step, the roofline of the dominant kernel
(the stream kernel), timed with HIP events around each of its launches in a second
region of K steps, and the CPU baseline (the compiled oracle on a bounded sample of
the same batch, 1 core).

--workload prefill_b4_512_over_8192 times the chunked prefill instead: B=4, 512 new
tokens per sequence after an 8192-token post-RoPE cache, RoPE on Q and the new K
(one step = one gqa_prefill_bf16 call: KV append + attention), with a 512 MiB write
between steps so that no step finds the 142 MB of K/V in the Infinity Cache.  value =
algorithmic flops / time per step (TFLOP/s) and the roofline is MFMA (BF16 dense peak).

--workload multitoken_b64_ragged_512_8192_t4 times multi-token decode (e.g. verifying 4
drafted tokens): the default batch's lengths, the last 4 positions of each sequence being
new tokens that one gqa_prefill_bf16 call appends (K rotated) and attends causally.  value =
the attention's algorithmic HBM bytes (every K/V row the last token sees, Q in, O out) /
time per step (GB/s); the roofline is HBM.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "GQA decode µs/step + achieved HBM GB/s, B=64 ragged ctx 512–8192"
HBM_PEAK_GBS = 8000.0
WORKLOADS = {
    # name: (batch, capacity, min_len, max_len)
    "decode_b64_ragged_512_8192": (64, 8192, 512, 8192),
    "decode_b1_4096": (1, 4096, None, None),
    "decode_b8_131072": (8, 131072, None, None),
    # the north-star batch through a paged cache (blocks of 16 positions, shuffled pool)
    "decode_paged_b64_ragged_512_8192": (64, 8192, 512, 8192),
}
PREFILL_WORKLOADS = {
    # name: (batch, new tokens, cached positions)
    "prefill_b4_512_over_8192": (4, 512, 8192),
}
MULTI_WORKLOADS = {
    # name: (batch, capacity, min_len, max_len, new tokens): the decode batch's lengths, whose
    # last `new` positions are the new tokens (appended with RoPE, then attended causally)
    "multitoken_b64_ragged_512_8192_t4": (64, 8192, 512, 8192, 4),
    "multitoken_b64_ragged_512_8192_t8": (64, 8192, 512, 8192, 8),
    "multitoken_b64_ragged_512_8192_t16": (64, 8192, 512, 8192, 16),
}
MFMA_BF16_PEAK_TFLOPS = 2500.0
TRAFFIC_FILES = {
    "decode_b64_ragged_512_8192": ROOT / "profiles" / "decode_stream_b64_ragged_traffic.txt",
    "multitoken_b64_ragged_512_8192_t4": ROOT / "profiles" / "mt_stream_b64_ragged_t4_traffic.txt",
    "multitoken_b64_ragged_512_8192_t8": ROOT / "profiles" / "mt_stream_b64_ragged_t8_traffic.txt",
    "multitoken_b64_ragged_512_8192_t16": ROOT / "profiles" / "mt_stream_b64_ragged_t16_traffic.txt",
}


def read_traffic(workload: str):
    """HBM bytes per launch of the workload's dominant kernel measured with rocprofv3 --pmc
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration), if committed."""
    f = TRAFFIC_FILES.get(workload)
    if f is None or not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch="):
            return float(line.split("=", 1)[1])
    return None


def calibrate_copy(torch, dev):
    """Five plain 1 GiB device copies: the known-size kernel the PMC byte counters are
    scaled by."""
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def codes_of(t):
    """bfloat16 tensor -> uint16 BF16 codes on the host."""
    import numpy as np
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def parity_summary(want, want64, got) -> dict:
    """The GPU rows against the oracle's rows for the same inputs: worst BF16 ULP, elements
    over 64 ULP under the reference checker's policy (pyfiles/check_gqa_output.py:57-64),
    and the largest |GPU - golden| against the golden's float64 value (before rounding)."""
    import numpy as np

    from attention_accelerator_amd.check import failures, ulp_distance
    want = np.asarray(want, dtype=np.uint16).reshape(-1, 128)
    got = np.asarray(got, dtype=np.uint16).reshape(-1, 128)
    gv = (got.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    wv = (want.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    w64 = np.asarray(want64).reshape(-1, 128)
    return {"max_ulp": int(ulp_distance(want, got).max()),
            "max_abs_err_vs_f64": float(np.abs(gv - w64).max()),
            # the golden's own BF16 rows are this far from its float64 values (output rounding)
            "golden_bf16_max_abs_err_vs_f64": float(np.abs(wv - w64).max()),
            "fails_64ulp": int(failures(want, got, 64).sum()), "elements": int(want.size)}


def fp32_attention(q_ref, k_ref, v_ref, n_keys: int):
    """The attention step in float32 (torch on the CPU): q_ref [32, 128] rotated and k_ref,
    v_ref [8, >= n_keys, 128] as the golden prepares them (double), rounded to float32 first;
    scores * 1/sqrt(128), softmax and weighted V in float32.  Returns [32, 128] float64."""
    import math

    import numpy as np
    import torch
    q = torch.from_numpy(np.ascontiguousarray(q_ref, dtype=np.float32)).view(8, 4, 128)
    k = torch.from_numpy(np.ascontiguousarray(k_ref[:, :n_keys], dtype=np.float32))
    v = torch.from_numpy(np.ascontiguousarray(v_ref[:, :n_keys], dtype=np.float32))
    s = torch.matmul(q, k.transpose(1, 2).contiguous()) * np.float32(1.0 / math.sqrt(128))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v).reshape(32, 128).numpy().astype(np.float64)


def fp32_summary(parity: dict, got_rows, want64_rows, ref32_rows) -> dict:
    """Adds the largest |GPU - fp32 reference| and |golden - fp32 reference| to parity."""
    import numpy as np
    got = (np.asarray(got_rows, dtype=np.uint16).reshape(-1, 128).astype(np.uint32) << 16).view(np.float32)
    r32 = np.asarray(ref32_rows).reshape(-1, 128)
    parity["max_abs_err_vs_fp32_ref"] = float(np.abs(got.astype(np.float64) - r32).max())
    parity["golden_f64_max_abs_diff_vs_fp32_ref"] = float(np.abs(np.asarray(want64_rows).reshape(-1, 128) - r32).max())
    return parity


def fp32_chunk_rows(qc, kc, vc, knc, vnc, s0: int, rows):
    """fp32_attention for tokens `rows` of one chunk: qc [T, 32, 128], knc / vnc [T, 8, 128]
    BF16 codes of the new rows, kc / vc [8, s0, 128] the cache before the chunk (post-RoPE);
    token t at position s0 + t sees the cache and new rows 0..t (K rotated at s0 + u in
    double, unrounded, as the golden). Returns [len(rows), 32, 128]."""
    import numpy as np

    from oracle import oracle as orc
    k_all = np.stack([np.concatenate([orc.prepare_rows(kc[h], False), orc.prepare_rows(knc[:, h], True, s0)])
                      for h in range(8)])
    v_all = np.stack([np.concatenate([orc.prepare_rows(vc[h], False), orc.prepare_rows(vnc[:, h], False)])
                      for h in range(8)])
    def q_at(t):
        return np.stack([orc.prepare_rows(qc[t, h][None], True, s0 + t)[0] for h in range(32)])
    return np.stack([fp32_attention(q_at(t), k_all, v_all, s0 + t + 1) for t in rows])


def python_golden(q, k, v, seq_len: int, qpos: int, nbytes: int, what: str) -> dict:
    """The reference's own arithmetic, pure Python (oracle/golden_model.golden_attention,
    a restatement of pyfiles/gen_gqa_wrapper_vectors.py:124-139), timed on one query token
    (all 32 heads), 1 thread; q [32, 128], k / v [8, >= seq_len, 128] BF16 codes, K taken
    as post-RoPE (Q rotated)."""
    from oracle import golden_model as gm
    qb, kb, vb = q.tolist(), k[:, :seq_len].tolist(), v[:, :seq_len].tolist()
    t0 = time.perf_counter()
    gm.golden_attention(qb, kb, vb, seq_len, qpos, rope_q=True, rope_k=False)
    t = time.perf_counter() - t0
    return {"value": round(nbytes / t / 1e9, 6), "unit": "GB/s", "cores": 1, "seconds": round(t, 2),
            "sample": f"{what}: {seq_len} keys, all 32 heads, pure-Python golden loop"}


def cpu_baseline(batch, gpu_out, budget_s: float = 12.0):
    """The compiled oracle (C restatement of the golden loop, double, 1 thread) on the
    first sequences of the same batch until ~budget_s of CPU work; the GPU's rows for
    those sequences against its rows (parity), and the pure-Python golden loop on the
    batch's shortest sequence beside it."""
    import numpy as np

    from attention_accelerator_amd.stimulus import algorithmic_bytes_decode
    from oracle import oracle as orc

    done, t_total, lens, wants, wants64 = 0, 0.0, [], [], []
    bsz = batch.q.shape[0]
    while done < bsz and t_total < budget_s:
        n = int(batch.seq_len[done])
        q = codes_of(batch.q[done:done + 1])
        k = codes_of(batch.k[done:done + 1, :, :n])
        v = codes_of(batch.v[done:done + 1, :, :n])
        t0 = time.perf_counter()
        w, w64 = orc.decode(q, k, v, batch.seq_len[done:done + 1].numpy(),
                            batch.query_pos[done:done + 1].numpy(), want_f64=True)
        t_total += time.perf_counter() - t0
        wants.append(w)
        wants64.append(w64)
        lens.append(n)
        done += 1
    gbs = algorithmic_bytes_decode(lens) / t_total / 1e9
    ref32 = []
    for b in range(done):
        n, qp = lens[b], int(batch.query_pos[b])
        qc, kc, vc = codes_of(batch.q[b]), codes_of(batch.k[b, :, :n]), codes_of(batch.v[b, :, :n])
        q_ref = np.stack([orc.prepare_rows(qc[h][None], True, qp)[0] for h in range(32)])
        k_ref = np.stack([orc.prepare_rows(kc[h], False) for h in range(8)])
        v_ref = np.stack([orc.prepare_rows(vc[h], False) for h in range(8)])
        ref32.append(fp32_attention(q_ref, k_ref, v_ref, qp + 1))
    s = int(np.argmin(batch.seq_len.numpy()))
    n = int(batch.seq_len[s])
    py = python_golden(codes_of(batch.q[s]), codes_of(batch.k[s, :, :n]), codes_of(batch.v[s, :, :n]), n,
                       int(batch.query_pos[s]), algorithmic_bytes_decode([n]), f"sequence {s} (the shortest)")
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": (f"sequences 0..{done - 1} of the same batch ({done} of {bsz}, "
                       f"{sum(lens)} keys, all 32 heads), compiled oracle in double, "
                       f"{t_total:.2f} s; os.cpu_count()={os.cpu_count()}, "
                       f"affinity={len(os.sched_getaffinity(0))}"),
            "parity": fp32_summary(parity_summary(np.concatenate(wants), np.concatenate(wants64), gpu_out[:done]),
                                   gpu_out[:done], np.concatenate(wants64), np.stack(ref32)),
            "python_golden": py}

def prefill_flops(batch: int, n_new: int, start: int) -> int:
    """QK^T and PV multiply-adds of a chunk, 2 flops each: token t sees start+t+1 keys."""
    keys = n_new * start + n_new * (n_new + 1) // 2
    return batch * 32 * keys * 128 * 4


def prefill_cpu_baseline(q, kn, vn, k, v, starts, gpu_out, budget_s: float = 12.0):
    """The compiled oracle (double, 1 thread) on the first rows of sequence 0, the GPU's
    rows against its rows (parity), and the pure-Python golden loop on token 0 beside it."""
    import numpy as np

    from oracle import oracle as orc

    s0 = int(starts[0])
    qc, knc, vnc = codes_of(q[:1]), codes_of(kn[:1]), codes_of(vn[:1])
    kc, vc = codes_of(k[:1, :, :s0]), codes_of(v[:1, :, :s0])
    rows, t_total, step, wants, wants64 = [], 0.0, 8, [], []
    while t_total < budget_s and len(rows) < q.shape[1]:
        batch_rows = list(range(len(rows), min(len(rows) + step, q.shape[1])))
        t0 = time.perf_counter()
        w, w64 = orc.prefill(qc, kc, vc, knc, vnc, np.asarray([s0]), rows=batch_rows, want_f64=True)
        t_total += time.perf_counter() - t0
        wants.append(w)
        wants64.append(w64)
        rows += batch_rows
    flops = sum(32 * (s0 + t + 1) * 128 * 4 for t in rows)
    # token 0 of sequence 0 sees the cache and its own new row (timing only: the new K row
    # enters unrotated and this output is not compared)
    k0 = np.concatenate([kc[0], knc[0, :1].reshape(8, 1, 128)], axis=1)
    v0 = np.concatenate([vc[0], vnc[0, :1].reshape(8, 1, 128)], axis=1)
    py = python_golden(qc[0, 0], k0, v0, s0 + 1, s0, 32 * (s0 + 1) * 128 * 4, "token 0 of sequence 0")
    py["unit"] = "FLOP/s"
    py["value"] = round(32 * (s0 + 1) * 128 * 4 / py["seconds"], 1)
    return {"value": round(flops / t_total / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": (f"tokens 0..{rows[-1]} of sequence 0 ({len(rows)} of {q.shape[1]} tokens, all "
                       f"32 heads, {s0} cached keys), compiled oracle in double, {t_total:.2f} s; "
                       f"os.cpu_count()={os.cpu_count()}, affinity={len(os.sched_getaffinity(0))}"),
            "parity": fp32_summary(parity_summary(np.concatenate(wants, axis=1), np.concatenate(wants64, axis=1),
                                                  gpu_out[:1, :len(rows)]),
                                   gpu_out[:1, :len(rows)], np.concatenate(wants64, axis=1),
                                   fp32_chunk_rows(qc[0], kc[0], vc[0], knc[0], vnc[0], s0, rows)),
            "python_golden": py}


def spin_up(call, torch, seconds: float) -> None:
    """Repeat the step, untimed, until the GPU has run it for `seconds`: the engine clock
    ramps over the first tens of milliseconds of load (B=64 decode: 201.6 us per step over
    the first 100 steps after 10 warm-up steps, 193.5 us from then on), and the timed steps
    should see the clock a sustained workload runs at."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            call()
        torch.cuda.synchronize()


def bench_prefill(args, torch, gqa, dev) -> int:
    bsz, n_new, start = PREFILL_WORKLOADS[args.workload]
    cap = start + n_new
    g = torch.Generator("cuda").manual_seed(args.seed)
    q = (torch.randn((bsz, n_new, 32, 128), generator=g, device=dev) * args.q_scale).to(torch.bfloat16)
    kn = torch.randn((bsz, n_new, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    vn = torch.randn((bsz, n_new, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    k = torch.full((bsz, 8, cap, 128), float("nan"), dtype=torch.bfloat16, device=dev)
    v = torch.full_like(k, float("nan"))
    k[:, :, :start] = torch.randn((bsz, 8, start, 128), generator=g, device=dev).to(torch.bfloat16)
    v[:, :, :start] = torch.randn((bsz, 8, start, 128), generator=g, device=dev).to(torch.bfloat16)
    k_host, v_host = (k.cpu(), v.cpu()) if not args.no_cpu_baseline else (None, None)
    starts = torch.full((bsz,), start, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    flops = prefill_flops(bsz, n_new, start)
    print(f"[bench] {args.workload}: B={bsz} new={n_new} start={start} flops/step={flops}",
          file=sys.stderr, flush=True)

    call = gqa.PreparedPrefill(q, kn, vn, k, v, starts, out=out)

    spin_up(call, torch, args.spinup_s)
    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    for i in range(args.steps):
        flush.fill_(i & 0xFF)                      # outside the timed pair of events
        evs[i][0].record()
        call()
        evs[i][1].record()
    torch.cuda.synchronize()
    ms_per_step = sum(a.elapsed_time(b) for a, b in evs) / args.steps

    attn_ms = append_ms = None
    if not args.no_profile:
        gqa.profile_enable(args.steps)
        for i in range(args.steps):
            flush.fill_(i & 0xFF)
            call()
        torch.cuda.synchronize()
        st_ms, n = gqa.profile_read_stages()
        gqa.profile_enable(0)
        append_ms, attn_ms, rescore_ms = st_ms[0] / n, st_ms[1] / n, st_ms[2] / n
    print(f"[bench] {args.steps} steps: {ms_per_step * 1e3:.2f} us/step", file=sys.stderr, flush=True)

    torch.cuda.synchronize()
    gpu_out = None if args.no_cpu_baseline else codes_of(out)     # the last step's rows
    rescored = call.rescored_rows()                               # the last step's fp64 rows
    tflops = flops / (ms_per_step * 1e-3) / 1e12
    roofline = None
    if attn_ms:
        achieved = flops / (attn_ms * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                    "traffic": None, "kernel": "prefill_attn_kernel",
                    "kernel_us": round(attn_ms * 1e3, 2), "append_stage_us": round(append_ms * 1e3, 2),
                    "rescore_us": round(rescore_ms * 1e3, 2), "flops_per_launch": flops}
    result = {
        "metric": "GQA chunked prefill µs/step + MFMA TFLOP/s, B=4 512 new over 8192 cached",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_step": round(ms_per_step * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": f"synthetic N(0,1) BF16, seed {args.seed}",
        "config": {"workload": args.workload, "batch": bsz, "new_tokens": n_new,
                   "cached": start, "q_heads": 32, "kv_heads": 8, "head_dim": 128,
                   "rope": "q and new k", "precision": "BF16 K/V staged exactly as fp16 (power-of-two "
                   "scale per 64-position block); Q, the chunk's K and P in two fp16 parts; fp32 MFMA "
                   "accumulation per 64-key block, fp64 across blocks; fp64 rescore of flagged rows",
                   "flops_per_step": flops, "spinup_s": args.spinup_s, "q_scale": args.q_scale,
                   "rescored_rows": rescored, "output_rows": bsz * n_new * 32},
        "roofline": roofline,
        "cpu_baseline": None if args.no_cpu_baseline else prefill_cpu_baseline(
            q, kn, vn, k_host, v_host, [start] * bsz, gpu_out),
    }
    print(json.dumps(result), flush=True)
    return 0


def multitoken_bytes(lengths, n_new: int) -> int:
    """HBM bytes of the attention: every K and V row each sequence's last token sees, once,
    the Q rows in and the output rows out (the append's own traffic is not counted)."""
    kv = sum(2 * 8 * 128 * 2 * int(x) for x in lengths)
    return kv + 2 * len(lengths) * n_new * 32 * 128 * 2


def multitoken_cpu_baseline(q, kn, vn, k, v, starts, n_new: int, gpu_out, budget_s: float = 12.0):
    """The compiled oracle (double, 1 thread) on whole sequences (all new tokens) from 0 on,
    the GPU's rows against its rows (parity), and the pure-Python golden loop on the first
    new token of the shortest sequence beside it."""
    import numpy as np

    from oracle import oracle as orc

    done, t_total, byts, wants, wants64 = 0, 0.0, 0, [], []
    while t_total < budget_s and done < q.shape[0]:
        b, s0 = done, int(starts[done])
        qc, knc, vnc = codes_of(q[b:b + 1]), codes_of(kn[b:b + 1]), codes_of(vn[b:b + 1])
        kc, vc = codes_of(k[b:b + 1, :, :s0]), codes_of(v[b:b + 1, :, :s0])
        t0 = time.perf_counter()
        w, w64 = orc.prefill(qc, kc, vc, knc, vnc, np.asarray([s0]), rows=list(range(n_new)), want_f64=True)
        t_total += time.perf_counter() - t0
        wants.append(w)
        wants64.append(w64)
        byts += multitoken_bytes([s0 + n_new], n_new)
        done += 1
    ref32 = [fp32_chunk_rows(codes_of(q[b]), codes_of(k[b, :, :int(starts[b])]), codes_of(v[b, :, :int(starts[b])]),
                             codes_of(kn[b]), codes_of(vn[b]), int(starts[b]), range(n_new)) for b in range(done)]
    b = int(np.argmin(np.asarray(starts)))
    s0 = int(starts[b])
    qc, knc, vnc = codes_of(q[b]), codes_of(kn[b]), codes_of(vn[b])
    k0 = np.concatenate([codes_of(k[b, :, :s0]), knc[0].reshape(8, 1, 128)], axis=1)   # timing only
    v0 = np.concatenate([codes_of(v[b, :, :s0]), vnc[0].reshape(8, 1, 128)], axis=1)
    py = python_golden(qc[0], k0, v0, s0 + 1, s0, multitoken_bytes([s0 + 1], 1),
                       f"new token 0 of sequence {b} (the shortest)")
    return {"value": round(byts / t_total / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": (f"sequences 0..{done - 1} ({done} of {q.shape[0]}, all {n_new} new tokens, all 32 "
                       f"heads), compiled oracle in double, {t_total:.2f} s; "
                       f"os.cpu_count()={os.cpu_count()}, affinity={len(os.sched_getaffinity(0))}"),
            "parity": fp32_summary(parity_summary(np.concatenate(wants), np.concatenate(wants64), gpu_out[:done]),
                                   gpu_out[:done], np.concatenate(wants64), np.stack(ref32)),
            "python_golden": py}


def bench_multitoken(args, torch, gqa, dev, stimulus) -> int:
    bsz, cap, lo, hi, n_new = MULTI_WORKLOADS[args.workload]
    batch = stimulus.decode_batch(bsz, cap, min_len=lo, max_len=hi, seed=args.seed, device=dev,
                                  gen_device="cuda")
    lens = [int(x) for x in batch.seq_len]
    g = torch.Generator("cuda").manual_seed(args.seed + 1)
    q = (torch.randn((bsz, n_new, 32, 128), generator=g, device=dev) * args.q_scale).to(torch.bfloat16)
    kn = torch.randn((bsz, n_new, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    vn = torch.randn((bsz, n_new, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    starts_l = [x - n_new for x in lens]
    starts = torch.tensor(starts_l, dtype=torch.int32, device=dev)
    k_host, v_host = (batch.k.cpu(), batch.v.cpu()) if not args.no_cpu_baseline else (None, None)
    out = torch.empty_like(q)
    step_bytes = multitoken_bytes(lens, n_new)
    print(f"[bench] {args.workload}: B={bsz} new={n_new} keys={sum(lens)} bytes/step={step_bytes}",
          file=sys.stderr, flush=True)
    call = gqa.PreparedPrefill(q, kn, vn, batch.k, batch.v, starts, out=out)

    spin_up(call, torch, args.spinup_s)
    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        call()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps

    attn_ms = append_ms = None
    if not args.no_profile:
        gqa.profile_enable(args.steps)
        for _ in range(args.steps):
            call()
        torch.cuda.synchronize()
        st_ms, n = gqa.profile_read_stages()
        gqa.profile_enable(0)
        append_ms, attn_ms = st_ms[0] / n, st_ms[1] / n
        merge_ms, rescore_ms = st_ms[2] / n, st_ms[3] / n
    print(f"[bench] {args.steps} steps: {ms_per_step * 1e3:.2f} us/step", file=sys.stderr, flush=True)
    gpu_out = None if args.no_cpu_baseline else codes_of(out)     # the last step's rows
    rescored = call.rescored_rows()                               # the last step's fp64 rows
    if args.calibrate_copy:
        calibrate_copy(torch, dev)
    roofline = None
    if attn_ms:
        # Chunks of at most 16 new tokens run the stream-K path (stages: preparation with
        # the append, the stream kernel, the merge, the rescore); longer ones the prefill
        # attention kernel (stages: append + staging + reduce, attention, rescore).
        stream_k = n_new <= 16
        achieved = step_bytes / (attn_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": read_traffic(args.workload) if stream_k else None,
                    "kernel": "mt_stream_kernel" if stream_k else "prefill_attn_kernel",
                    "kernel_us": round(attn_ms * 1e3, 2),
                    ("prepare_us" if stream_k else "append_us"): round(append_ms * 1e3, 2),
                    **({"merge_us": round(merge_ms * 1e3, 2), "rescore_us": round(rescore_ms * 1e3, 2)}
                       if stream_k else {"rescore_us": round(merge_ms * 1e3, 2)}),
                    "bytes_per_launch": step_bytes}
    result = {
        "metric": f"GQA multi-token decode µs/step + achieved HBM GB/s, B=64 ragged ctx 512–8192, {n_new} new tokens",
        "value": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_step": round(ms_per_step * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic N(0,1) BF16, seed {args.seed}",
        "config": {"workload": args.workload, "batch": bsz, "new_tokens": n_new, "keys": sum(lens),
                   "q_heads": 32, "kv_heads": 8, "head_dim": 128, "rope": "q and new k",
                   "bytes_per_step": step_bytes, "spinup_s": args.spinup_s, "q_scale": args.q_scale,
                   "rescored_rows": rescored, "output_rows": bsz * n_new * 32},
        "roofline": roofline,
        "cpu_baseline": None if args.no_cpu_baseline else multitoken_cpu_baseline(
            q, kn, vn, k_host, v_host, starts_l, n_new, gpu_out),
    }
    print(json.dumps(result), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--spinup-s", type=float, default=0.3,
                    help="seconds of untimed steps before the warm-up (engine clock ramp)")
    ap.add_argument("--workload", choices=sorted(WORKLOADS) + sorted(PREFILL_WORKLOADS) + sorted(MULTI_WORKLOADS),
                    default="decode_b64_ragged_512_8192")
    ap.add_argument("--seed", type=int, default=20260805)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-profile", action="store_true",
                    help="skip the per-kernel HIP events inside the timed region")
    ap.add_argument("--graph", action="store_true",
                    help="decode workloads: time replays of one captured step (HIP graph)")
    ap.add_argument("--q-scale", type=float, default=1.0,
                    help="prefill and multi-token workloads: Q drawn as N(0, q_scale^2) (a peaked "
                         "softmax for q_scale > 1; the headline workloads use 1)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run plain 1 GiB device copies (PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the decode shards by sequence or KV head with no exchange between GPUs)",
              file=sys.stderr)
        return 2

    import torch

    import attention_accelerator_amd as gqa
    from attention_accelerator_amd import stimulus
    from attention_accelerator_amd.attention import PreparedDecode, validate_lengths

    dev = torch.device("cuda", 0)
    if args.workload in PREFILL_WORKLOADS:
        return bench_prefill(args, torch, gqa, dev)
    if args.workload in MULTI_WORKLOADS:
        return bench_multitoken(args, torch, gqa, dev, stimulus)
    bsz, cap, lo, hi = WORKLOADS[args.workload]
    batch = stimulus.decode_batch(bsz, cap, min_len=lo, max_len=hi, seed=args.seed,
                                  device=dev, gen_device="cuda")
    validate_lengths(batch.seq_len, batch.query_pos, cap)
    lens = [int(x) for x in batch.seq_len]
    step_bytes = stimulus.algorithmic_bytes_decode(lens)
    # The split kernel reads K/V rows, Q rows and the lengths; the combine writes O.
    split_bytes = step_bytes - bsz * stimulus.N_Q_HEADS * stimulus.HEAD_DIM * 2
    if args.workload.startswith("decode_paged"):
        # Scatter every (sequence, 16-position block) to a random pool block.
        nb = cap // 16
        kp = batch.k.view(bsz, 8, nb, 16, 128).permute(0, 2, 1, 3, 4).reshape(bsz * nb, 8, 16, 128)
        vp = batch.v.view(bsz, 8, nb, 16, 128).permute(0, 2, 1, 3, 4).reshape(bsz * nb, 8, 16, 128)
        perm = torch.randperm(bsz * nb, generator=torch.Generator().manual_seed(args.seed)).to(dev)
        k_pool = torch.empty_like(kp)
        v_pool = torch.empty_like(vp)
        k_pool[perm] = kp
        v_pool[perm] = vp
        table = perm.view(bsz, nb).to(torch.int32).contiguous()
        del kp, vp
        qp_dev, sl_dev = batch.query_pos.to(dev), batch.seq_len.to(dev)
        ws = torch.empty(gqa.attention.decode_workspace_bytes(bsz, cap), dtype=torch.uint8,
                         device=dev)
        out = torch.empty((bsz, 32, 128), dtype=torch.bfloat16, device=dev)

        def call():
            gqa.gqa_decode_paged(batch.q, k_pool, v_pool, table, qp_dev, sl_dev, out=out,
                                 workspace=ws)
    else:
        call = PreparedDecode(batch.q, batch.k, batch.v, batch.query_pos.to(dev),
                              batch.seq_len.to(dev))
    print(f"[bench] {args.workload}: B={bsz} keys={sum(lens)} bytes/step={step_bytes}",
          file=sys.stderr, flush=True)

    spin_up(call, torch, args.spinup_s)
    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()

    # --graph: the timed steps replay one captured step (the library issues kernels only,
    # so a step captures as it is) instead of issuing its launches from the host.
    step = call
    if args.graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            call()
        step = graph.replay
        step()
        torch.cuda.synchronize()

    # A step whose K/V fit in the 256 MB Infinity Cache would find them there on every
    # repeat; such workloads write 512 MiB between steps (outside the timed events) and
    # time each step on its own.
    flushed = step_bytes < (1 << 30)
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev) if flushed else None

    # Timed region 1 (the headline): K plain steps.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    if flushed:
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(args.steps)]
        for i in range(args.steps):
            flush.fill_(i & 0xFF)
            evs[i][0].record()
            step()
            evs[i][1].record()
        torch.cuda.synchronize()
        ms_per_step = sum(a.elapsed_time(b) for a, b in evs) / args.steps
    else:
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(args.steps):
            step()
        ev1.record()
        torch.cuda.synchronize()
        ms_per_step = ev0.elapsed_time(ev1) / args.steps
    wall = time.perf_counter() - t0

    # Timed region 2: the same K steps with the library's HIP events recorded around
    # each kernel on the launch stream (gqa_profile_*), for the per-kernel roofline.
    # The event records add a few microseconds per step, so this region is not the
    # headline.
    split_ms = combine_ms = None
    if not args.no_profile:
        gqa.profile_enable(args.steps)
        torch.cuda.synchronize()
        for i in range(args.steps):
            if flushed:
                flush.fill_(i & 0xFF)
            call()
        torch.cuda.synchronize()
        s_ms, c_ms, n = gqa.profile_read()
        gqa.profile_enable(0)
        split_ms, combine_ms = s_ms / n, c_ms / n
    print(f"[bench] {args.steps} steps: {ms_per_step * 1e3:.2f} us/step (events), "
          f"wall {wall / args.steps * 1e6:.2f} us/step{' (cache flushed between steps)' if flushed else ''}",
          file=sys.stderr, flush=True)

    if args.calibrate_copy:
        calibrate_copy(torch, dev)
    res = call()
    torch.cuda.synchronize()
    gpu_out = None if args.no_cpu_baseline else codes_of(out if res is None else res)

    gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    roofline = None
    if split_ms:
        achieved = split_bytes / (split_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": read_traffic(args.workload),
                    "kernel": "decode_stream_kernel", "kernel_us": round(split_ms * 1e3, 2),
                    "merge_us": round(combine_ms * 1e3, 2), "bytes_per_launch": split_bytes}
    result = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_step": round(ms_per_step * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic N(0,1) BF16, seed {args.seed}, lengths U[{lo},{hi}]" if lo else
                f"synthetic N(0,1) BF16, seed {args.seed}",
        "config": {"workload": args.workload, "batch": bsz, "capacity": cap,
                   "min_len": lo, "max_len": hi, "total_keys": sum(lens), "q_heads": 32,
                   "kv_heads": 8, "head_dim": 128, "rope": "q", "accumulate": "fp64 scores, softmax and weighted V (fp64 MFMA)",
                   "bytes_per_step": step_bytes,
                   "infinity_cache": "flushed between steps" if flushed else "working set > 1 GiB",
                   "spinup_s": args.spinup_s, "graph": bool(args.graph)},
        "roofline": roofline,
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline(
            stimulus.DecodeBatch(batch.q.cpu(), batch.k, batch.v, batch.seq_len,
                                 batch.query_pos), gpu_out),
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
