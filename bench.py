#!/usr/bin/env python3
"""Benchmark of the quantized decode hot path on one MI355X.

Workload (the LM-head configuration, 262144 x 640): one step is
  * Q8_0 GEMV 262144 x 640 (36-byte blocks) -> fp32 logits -> fused softmax + argmax
  * Q4_0 GEMV 262144 x 640 (20-byte blocks) -> fp32 logits -> fused softmax + argmax
on seeded synthetic weights (scale |N(0,0.01)|, uniform quants) and an N(0,1) hidden
vector, all resident in HBM before timing. Copies of the weights are rotated (four of the
Q8_0 matrix, 760 MB; six of the Q4_0 one, 636 MB) so that the steps read their weights from
HBM, not the 256 MB last-level cache.

value = algorithmic bytes of a step (M*ceil(K/32)*B_blk + 4K + 4M per GEMV, plus 1 MiB
read + 1 MiB written per softmax) / step time.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--decode-steps N]
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
M_LM, K_LM = 262144, 640
METRIC = "Q4_0/Q8_0 GEMV HBM GB/s (% of peak) + decode tok/s, Gemma-3-270M shape"


def gemv_bytes(dtype: int, m: int, k: int) -> int:
    from sapphire_amd import synth
    return m * ((k + 31) // 32) * synth.BLOCK_BYTES[dtype] + 4 * k + 4 * m


def traffic_from_profiles():
    """HBM bytes per launch of the Q8_0 LM-head GEMV, from the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, calibrated against a copy kernel)."""
    path = os.path.join(ROOT, "profiles", "gemv_lm_head_traffic.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_q8_0_lm_head\s*[:=]\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


def host_cpu() -> dict:
    """The host's CPU model, its logical CPU count and the CPUs this process may use."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"cpu_model": model, "nproc": os.cpu_count(), "usable_cpus": usable}


def cpu_threads() -> int:
    """Threads for the CPU legs: the CPUs this process may use, capped by OMP_NUM_THREADS
    (the box's CPU share) and 16."""
    usable = host_cpu()["usable_cpus"]
    return max(1, min(usable, int(os.environ.get("OMP_NUM_THREADS", usable)), 16))


def cpu_baseline(x, w8, w4, min_reps: int = 20, min_reps_1t: int = 5, budget_s: float = 20.0):
    """The reference's own pooled kernel_gemv (compiled from its sources into oracle/_ref) on
    this host, or the oracle's restatement when that was not built: the median over reps of one
    Q8_0 + one Q4_0 GEMV 262144x640, with the box's threads and with one thread."""
    from oracle.oracle import Oracle, Reference
    from sapphire_amd import synth
    threads = cpu_threads()
    if Reference.available():
        ref, kind = Reference(), "reference"
        run = lambda dt, w, n: ref.gemv(dt, w, x, nthreads=n)   # noqa: E731
    else:
        orc, kind = Oracle(), "port"
        run = lambda dt, w, n: orc.gemv(dt, w, x, nthreads=n)   # noqa: E731
    pair = gemv_bytes(synth.Q8_0, M_LM, K_LM) + gemv_bytes(synth.Q4_0, M_LM, K_LM)

    def median_rate(nth, reps_min):
        rates, t_start = [], time.perf_counter()
        run(synth.Q8_0, w8, nth)                      # warm-up (pool start, page faults)
        while len(rates) < reps_min or time.perf_counter() - t_start < budget_s / 2:
            t0 = time.perf_counter()
            run(synth.Q8_0, w8, nth)
            run(synth.Q4_0, w4, nth)
            rates.append(pair / (time.perf_counter() - t0) / 1e9)
        return float(np.median(rates)), len(rates), time.perf_counter() - t_start

    med, reps, secs = median_rate(threads, min_reps)
    med1, reps1, secs1 = median_rate(1, min_reps_1t)
    return {
        "value": round(med, 2), "unit": "GB/s", "cores": threads, "kind": kind,
        "value_1_thread": round(med1, 2), **host_cpu(),
        "sample": f"median of {reps} reps of (Q8_0 + Q4_0 GEMV 262144x640) with the pooled kernel_gemv on "
                  f"{threads} threads ({secs:.1f} s), and of {reps1} reps on 1 thread ({secs1:.1f} s)",
    }


def ref_decode_rate(m, k, v, tok, prefill, n):
    """Tokens/s of the reference engine (oracle/_ref, or the oracle's restatement when it was not
    built) over n greedy steps from the given KV cache, session set-up excluded: the time of n + 1
    steps minus that of one step. Returns (tok/s, kind, tokens of the n + 1 steps)."""
    from oracle.oracle import oracle_decode, Oracle, ref_decode, ref_decode_available
    if ref_decode_available():
        go, kind = (lambda steps: ref_decode(m, k.copy(), v.copy(), tok, prefill, steps)[0]), "reference"
    else:
        orc = Oracle()
        go, kind = (lambda steps: oracle_decode(orc, m, k.copy(), v.copy(), tok, prefill, steps,
                                                nthreads=cpu_threads())[0]), "port"
    t0 = time.perf_counter()
    go(1)
    t1 = time.perf_counter()
    toks = go(n + 1)
    t2 = time.perf_counter()
    return n / ((t2 - t1) - (t1 - t0)), kind, [int(t) for t in toks]


def decode_leg(steps: int, cpu: bool, seed: int = 20260101, prefill: int = 1024):
    """Greedy decode of the Gemma-3-270M-shaped Q4_0 model on the GPU (device-resident engine,
    one HIP graph per step), and the reference engine compiled from its sources (oracle/_ref)
    on this host's cores for a few steps of the same model as the CPU baseline."""
    from sapphire_amd import model as smodel
    from sapphire_amd import synth
    from sapphire_amd.engine import bench_decode
    m = smodel.synthetic_model(smodel.GEMMA3_270M, seed)
    k, v = m.kv_prefill(prefill)
    out = bench_decode(steps, seed=seed, prefill=prefill, m=m, kv=(k, v))
    # prefill of a 1024-token prompt into an empty cache (chunks of 16 through the batched GEMMs)
    from sapphire_amd.engine import Decoder
    dec = Decoder(m)
    prompt = synth.rng(seed, 77).integers(0, m.cfg.vocab, prefill).astype(np.int32)
    dec.prefill(prompt[:64], 0)                      # warm-up
    pf_ms = min(dec.prefill(prompt, 0) for _ in range(3))
    dec.close()
    out["prefill"] = {"tokens": prefill, "ms": round(pf_ms, 3), "tok_per_s": round(prefill / (pf_ms * 1e-3), 1),
                      "form": "chunks of 16 tokens, projections as matrix-core GEMMs",
                      "reference": "quantized prompt batches are rejected by the reference's pool (pool.c:318-321); "
                                   "its prompt rate is its one-token decode rate (cpu_baseline.tok_per_s)"}
    # the same model with the reference's own LM head: the BF16 embedding table (tied)
    tied_cfg = dataclasses.replace(m.cfg, lm_dtype=synth.BF16)
    tied = dataclasses.replace(m, cfg=tied_cfg, lm_head=m.embed_bf16)
    out["tied_bf16_lm_head"] = {kk: vv for kk, vv in bench_decode(steps, seed=seed, prefill=prefill, m=tied,
                                                                    kv=(k, v)).items()
                                if kk in ("ms_per_token", "tok_per_s", "weight_bytes_per_token", "first_tokens")}
    if cpu:
        tok = smodel.start_token(m.cfg, seed)
        rate, kind, toks = ref_decode_rate(m, k, v, tok, prefill, steps)
        out["cpu_baseline"] = {
            "tok_per_s": round(rate, 2), "kind": kind, "cores": os.cpu_count(), **host_cpu(),
            "sample": f"{steps} greedy steps of the same model and KV cache through the reference's session and "
                      f"layer functions (session set-up excluded); its pool starts one thread per online CPU "
                      f"(pool.c:159)",
            "tokens_match_gpu": toks[:len(out["first_tokens"])] == out["first_tokens"],
        }
    return out


def lm_head_gemm(blocks, batch: int, seed: int, iters: int = 20):
    """The batched decode's dominant kernel alone: Q4_0 262144 x 1152 times 16 vectors on the
    matrix cores (four weight copies rotated, 4 x 189 MB > the 256 MB last-level cache)."""
    from sapphire_amd import load, synth
    from sapphire_amd.device import DeviceArray, QMatrix, Timer, check
    L = load()
    m, k = blocks.shape[0], blocks.shape[1] * 32
    qs = [QMatrix(synth.Q4_0, blocks, layout=2) for _ in range(4)]
    X = DeviceArray.from_numpy(synth.normal_f32((batch, k), seed, 77))
    Y = DeviceArray.empty(batch * m)
    ws = DeviceArray(L.sapphire_gemm_workspace_bytes(synth.Q4_0, m, k))
    run = lambda i: check(L.sapphire_gemm_q_dev(synth.Q4_0, 2, qs[i % 4].ptr(), m, k, X.ptr, batch, Y.ptr,  # noqa: E731
                                                ws.ptr, None))
    for i in range(4):
        run(i)
    check(L.sapphire_synchronize())
    t = Timer(None)
    t.start()
    for i in range(iters):
        run(i)
    us = t.stop() / iters * 1e3
    algo = m * (k // 32) * synth.BLOCK_BYTES[synth.Q4_0] + 4 * batch * (k + m)
    out = {
        "shape": f"{m}x{k} Q4_0, {batch} sequences", "us": round(us, 2),
        "GB/s": round(algo / (us * 1e-6) / 1e9, 1), "frac_hbm_peak": round(algo / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "TFLOP/s": round(2.0 * batch * m * k / (us * 1e-6) / 1e12, 1), "algorithmic_bytes": algo,
    }
    # the form a greedy decode step runs: the same rows reduced to one token per sequence
    # inside the GEMM (no logits stored), then one short kernel over the workgroups' partials
    T = DeviceArray.empty(batch, np.int32)
    run_g = lambda i: check(L.sapphire_gemm_q_greedy_dev(synth.Q4_0, qs[i % 4].ptr(), m, k, X.ptr, batch,  # noqa: E731
                                                         T.ptr, ws.ptr, None))
    for i in range(4):
        run_g(i)
    check(L.sapphire_synchronize())
    t.start()
    for i in range(iters):
        run_g(i)
    ug = t.stop() / iters * 1e3
    algo_g = m * (k // 32) * synth.BLOCK_BYTES[synth.Q4_0] + 4 * batch * k + 4 * batch
    out["greedy_with_finish_kernel"] = {
        "us": round(ug, 2), "GB/s": round(algo_g / (ug * 1e-6) / 1e9, 1),
        "frac_hbm_peak": round(algo_g / (ug * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "algorithmic_bytes": algo_g,
    }
    return out


def decode_batch_leg(steps: int, cpu: bool, seed: int = 20260101, prefill: int = 1024, batch: int = 16):
    """Batched greedy decode of the Gemma-3-1B-shaped Q4_0 model, 16 sequences in lock step
    (projections as matrix-core GEMMs). CPU baseline: the reference engine (oracle/_ref) decodes
    one sequence at a time (it has no quantized batch path, pool.c:318-321), so its tokens/s
    for 16 sequences is its one-sequence rate, timed for a few steps of the same model."""
    from sapphire_amd import model as smodel
    from sapphire_amd.engine import bench_decode_batch
    m = smodel.synthetic_model(smodel.GEMMA3_1B, seed)
    k, v = m.kv_prefill(prefill)
    out = bench_decode_batch(steps, batch=batch, seed=seed, prefill=prefill, m=m, kv=(k, v))
    out["lm_head_gemm"] = lm_head_gemm(m.lm_head, batch, seed)
    # the same model with the reference's own LM head: the BF16 embedding table (tied)
    from sapphire_amd import synth
    tied = dataclasses.replace(m, cfg=dataclasses.replace(m.cfg, lm_dtype=synth.BF16), lm_head=m.embed_bf16)
    out["tied_bf16_lm_head"] = {kk: vv for kk, vv in bench_decode_batch(steps, batch=batch, seed=seed,
                                                                          prefill=prefill, m=tied, kv=(k, v)).items()
                                if kk in ("ms_per_step", "tok_per_s", "weight_bytes_per_step")}
    if cpu:
        rate, kind, _ = ref_decode_rate(m, k, v, out["first_tokens"][0], prefill, steps)
        out["cpu_baseline"] = {
            "tok_per_s": round(rate, 2), "kind": kind, "cores": os.cpu_count(), **host_cpu(),
            "sample": f"{steps} greedy steps of one sequence of the same model through the reference's session "
                      f"and layer functions (session set-up excluded); its pool starts one thread per online "
                      f"CPU (pool.c:159)",
        }
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--decode-steps", type=int, default=64, help="greedy decode steps (0 skips decode)")
    ap.add_argument("--batch-steps", type=int, default=32,
                    help="steps of the 16-sequence Gemma-3-1B-shaped batched decode (0 skips it)")
    ap.add_argument("--profile-kernels", action="store_true",
                    help="only launch each LM-head kernel 10 times plus a 256 MiB device copy (the "
                         "calibration kernel of the FETCH_SIZE/WRITE_SIZE counters), for rocprofv3")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the path has no multi-GPU mode; run it with --gpus 1.",
              file=sys.stderr)
        return 2

    from sapphire_amd import load, synth
    from sapphire_amd.device import DeviceArray, QMatrix, Timer, check
    L = load()
    if L.sapphire_device_count() < 1:
        print("no GPU visible", file=sys.stderr)
        return 1

    seed = 20260101
    w8 = synth.quant_matrix(synth.Q8_0, M_LM, K_LM, seed, 1)
    w4 = synth.quant_matrix(synth.Q4_0, M_LM, K_LM, seed, 2)
    x = synth.normal_f32(K_LM, seed, 3)
    # Weight copies rotated so that the launches read HBM, not the 256 MB last-level cache. Of
    # copies read back to back the first of each cycle keeps part of itself in that cache (about
    # 10 % faster in a read-only probe), so the rotation is long: at most one launch in four (six)
    # finds its copy partly cached.
    n_sets = 4        # Q8_0 copies: 4 x 190 MB (also the BF16 / F32 copies)
    n_sets4 = 6       # Q4_0 copies: 6 x 106 MB
    LAY = 2   # TILED: the matrix-core layout kernel_gemv uses for matrices this long
    q8 = [QMatrix(synth.Q8_0, w8, layout=LAY) for _ in range(n_sets)]
    q4 = [QMatrix(synth.Q4_0, w4, layout=LAY) for _ in range(n_sets4)]
    dx = DeviceArray.from_numpy(x)
    logits = DeviceArray.empty(M_LM)
    probs = DeviceArray.empty(M_LM)
    arg = DeviceArray.empty(1, np.int32)
    stream = L.sapphire_stream_create()

    def step(i):
        """One pass over the LM head of each dtype: GEMV with the softmax/argmax epilogue."""
        check(L.sapphire_gemv_softmax_dev(synth.Q8_0, LAY, q8[i % n_sets].ptr(), M_LM, K_LM, dx.ptr, logits.ptr,
                                          probs.ptr, arg.ptr, stream))
        check(L.sapphire_gemv_softmax_dev(synth.Q4_0, LAY, q4[i % n_sets4].ptr(), M_LM, K_LM, dx.ptr, logits.ptr,
                                          probs.ptr, arg.ptr, stream))

    if args.profile_kernels:
        copy_bytes = 256 << 20
        src, dst = DeviceArray(copy_bytes), DeviceArray(copy_bytes)
        check(L.sapphire_memset(src.ptr, 1, copy_bytes), "memset")
        for i in range(10):
            step(i)
        for i in range(10):
            check(L.sapphire_gemv_q_dev(synth.Q8_0, LAY, q8[i % n_sets].ptr(), M_LM, K_LM, dx.ptr, logits.ptr, stream))
            check(L.sapphire_gemv_q_dev(synth.Q4_0, LAY, q4[i % n_sets4].ptr(), M_LM, K_LM, dx.ptr, logits.ptr, stream))
        for i in range(10):
            check(L.sapphire_memcpy_d2d(dst.ptr, src.ptr, copy_bytes, stream), "copy")
        check(L.sapphire_stream_synchronize(stream))
        print(json.dumps({"profile_kernels": "done", "copy_bytes": copy_bytes}), flush=True)
        return 0

    for i in range(args.warmup):
        step(i)
    check(L.sapphire_stream_synchronize(stream))

    # whole steps, back to back
    t = Timer(stream)
    t.start()
    for i in range(args.steps):
        step(i)
    ms_total = t.stop()
    ms_step = ms_total / args.steps

    # each kernel alone, back to back on the bench stream (HIP events on that stream); the
    # Q8_0 GEMV is the dominant kernel of the step and gives roofline.achieved
    def time_alone(fn, iters=20, warm=3):
        for i in range(warm):
            fn(i)
        tt = Timer(stream)
        tt.start()
        for i in range(iters):
            fn(i)
        return tt.stop() / iters
    q8_ms = time_alone(lambda i: check(L.sapphire_gemv_q_dev(
        synth.Q8_0, LAY, q8[i % n_sets].ptr(), M_LM, K_LM, dx.ptr, logits.ptr, stream)))
    q4_ms = time_alone(lambda i: check(L.sapphire_gemv_q_dev(
        synth.Q4_0, LAY, q4[i % n_sets4].ptr(), M_LM, K_LM, dx.ptr, logits.ptr, stream)))
    q8sm_ms = time_alone(lambda i: check(L.sapphire_gemv_softmax_dev(
        synth.Q8_0, LAY, q8[i % n_sets].ptr(), M_LM, K_LM, dx.ptr, logits.ptr, probs.ptr, arg.ptr, stream)))
    sm_ms = time_alone(lambda i: check(L.sapphire_softmax_argmax_dev(logits.ptr, M_LM, probs.ptr, arg.ptr, stream)))

    # The same LM head held as BF16 / F32 rows (a weight-tied embedding), on the element
    # types' own GEMV kernel; four copies of each rotate so the weights come from HBM.
    # the small GEMVs of one decode layer (Gemma-3-270M MLP shapes), PACKED layout: per call
    # time of 200 back-to-back launches on the bench stream (weights stay in the 256 MB MALL,
    # so these are launch- and latency-bound, not HBM-bound)
    small = {}
    for name, dt, shapes in (("gemv_q8_0_2048x640", synth.Q8_0, [(2048, 640)]),
                             ("gemv_q4_0_pair_2048x640_640x2048", synth.Q4_0, [(2048, 640), (640, 2048)])):
        mats = [(QMatrix(dt, synth.quant_matrix(dt, m_, k_, seed, 50 + m_), layout=1), m_, k_) for m_, k_ in shapes]
        xs = [DeviceArray.from_numpy(synth.normal_f32(k_, seed, 60 + k_)) for _, _, k_ in mats]
        ys = [DeviceArray.empty(m_) for _, m_, _ in mats]

        def call(i, mats=mats, xs=xs, ys=ys, dt=dt):
            for (qm, m_, k_), xx, yy in zip(mats, xs, ys):
                check(L.sapphire_gemv_q_dev(dt, 1, qm.ptr(), m_, k_, xx.ptr, yy.ptr, stream))
        s_ms = time_alone(call, iters=200, warm=10)
        sb = sum(gemv_bytes(dt, m_, k_) for _, m_, k_ in mats)
        small[name] = {"us_per_call": round(s_ms * 1e3, 2), "GB/s": round(sb / (s_ms * 1e-3) / 1e9, 1),
                       "bytes": sb}
    f_lines = {}
    qout = DeviceArray(gemv_bytes(synth.Q8_0, M_LM, K_LM))
    for name, dt, es in (("gemv_bf16_lm_head", synth.BF16, 2), ("gemv_f32_lm_head", synth.F32, 4)):
        tile = synth.normal_f32((M_LM // 64, K_LM), seed, 40 + dt, 0.0, 0.05)
        if dt == synth.BF16:
            tile = (tile.view(np.uint32) >> 16).astype(np.uint16)
        tile = np.ascontiguousarray(np.tile(tile, (64, 1)))
        mats = [DeviceArray.from_numpy(tile) for _ in range(n_sets)]
        del tile
        f_ms = time_alone(lambda i: check(L.sapphire_gemv_f_dev(dt, mats[i % n_sets].ptr, M_LM, K_LM, dx.ptr,
                                                                 logits.ptr, stream)))
        fb = M_LM * K_LM * es + 4 * K_LM + 4 * M_LM
        f_lines[name] = {"us": round(f_ms * 1e3, 2), "GB/s": round(fb / (f_ms * 1e-3) / 1e9, 1),
                         "frac_peak": round(fb / (f_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if dt == synth.BF16:
            # the batched form (16 vectors) on the matrix cores: weights read once
            xb = DeviceArray.from_numpy(synth.normal_f32((16, K_LM), seed, 45))
            yb = DeviceArray.empty(16 * M_LM)
            g_ms = time_alone(lambda i: check(L.sapphire_gemm_bf16_dev(mats[i % n_sets].ptr, M_LM, K_LM, xb.ptr, K_LM,
                                                                       16, yb.ptr, M_LM, stream)))
            gb = M_LM * K_LM * 2 + 16 * 4 * (K_LM + M_LM)
            f_lines["gemm_bf16_lm_head_16_vectors"] = {
                "us": round(g_ms * 1e3, 2), "GB/s": round(gb / (g_ms * 1e-3) / 1e9, 1),
                "frac_peak": round(gb / (g_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "TFLOP/s": round(2 * 16 * M_LM * K_LM / (g_ms * 1e-3) / 1e12, 1)}
            xb.free()
            yb.free()
        # the Q4_0 / Q8_0 producer over the same rows: bytes = source + blocks
        for qdt in (synth.Q4_0, synth.Q8_0):
            q_ms = time_alone(lambda i: check(L.sapphire_quantize_dev(qdt, dt, mats[i % n_sets].ptr, M_LM, K_LM,
                                                                      qout.ptr, stream)))
            qb = M_LM * K_LM * es + gemv_bytes(qdt, M_LM, K_LM) - 4 * K_LM - 4 * M_LM
            f_lines[f"quantize_{'bf16' if dt == synth.BF16 else 'f32'}_to_{synth.DTYPE_NAME[qdt].lower()}"
                    f"_lm_head"] = {"us": round(q_ms * 1e3, 2), "GB/s": round(qb / (q_ms * 1e-3) / 1e9, 1),
                                    "frac_peak": round(qb / (q_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        for m_ in mats:
            m_.free()

    b8, b4 = gemv_bytes(synth.Q8_0, M_LM, K_LM), gemv_bytes(synth.Q4_0, M_LM, K_LM)
    b_sm = 2 * 4 * M_LM
    step_bytes = b8 + b4 + 2 * b_sm
    value = step_bytes / (ms_step * 1e-3) / 1e9
    achieved = b8 / (q8_ms * 1e-3) / 1e9

    decode = None
    if args.decode_steps > 0:
        decode = decode_leg(args.decode_steps, cpu=not args.no_cpu)
    decode_batch = None
    if args.batch_steps > 0:
        decode_batch = decode_batch_leg(args.batch_steps, cpu=not args.no_cpu)

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Q8_0/Q4_0 blocks, N(0,1) activations)",
        "config": {
            "workload": "lm_head 262144x640: Q8_0 GEMV + softmax/argmax, Q4_0 GEMV + softmax/argmax "
                        "(softmax partials fused into the GEMV epilogue)",
            "weights_rotated": {"q8_0": n_sets, "q4_0": n_sets4}, "step_bytes": step_bytes,
        },
        "roofline": {
            "bound": "hbm", "kernel": "gemv_q8_0 262144x640",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(),
        },
        "kernels": {
            "gemv_q8_0_lm_head": {"us": round(q8_ms * 1e3, 2), "GB/s": round(achieved, 1),
                                  "frac_peak": round(achieved / HBM_PEAK_GBS, 4)},
            "gemv_q4_0_lm_head": {"us": round(q4_ms * 1e3, 2), "GB/s": round(b4 / (q4_ms * 1e-3) / 1e9, 1),
                                  "frac_peak": round(b4 / (q4_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
            "gemv_q8_0_lm_head_with_softmax_epilogue": {"us": round(q8sm_ms * 1e3, 2)},
            "softmax_argmax_262144_standalone": {"us": round(sm_ms * 1e3, 2)},
            **f_lines,
            **small,
        },
        "decode": decode,
        "decode_batch16_gemma3_1b": decode_batch,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(x, w8, w4)
    print(json.dumps(out), flush=True)
    L.sapphire_stream_destroy(stream)
    return 0


if __name__ == "__main__":
    sys.exit(main())
