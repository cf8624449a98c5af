#!/usr/bin/env python3
"""Throughput of the denoising path on one MI355X: LLaDA-8B architecture, Q4_K_M,
32-token prompt + B=256 masks, 16 steps, entropy_exit remasking with the inter-step
KV cache (diffuse_generate; tools/main-bench.cpp measures the same call).

One bench step = one diffuse_generate of 256 tokens (16 denoising steps).  Weights
are random-init N(0, 0.02) from seed 0 with norms 1.0, written as GGUF and
quantised with the Q4_K_M mixture by the library's generator; the prompt is 32
ids drawn uniformly from [0, 126000) with seed 1.  Prints one JSON line.

Beside the headline: the other single-GPU workloads of the benchmark set (LLaDA-8B
32 + 64 low_confidence without cache; Dream-7B 64 + 64 entropy_exit with cache; the
sampler over a [256 x 126464] logits block; 8 x (512 + 256) sequences on LLaDA-8B Q8_0
generating concurrently; Dream-7B ar_generate decode), and the CPU baseline (the oracle,
a restatement of the reference's CPU path, timed on this host).
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "diffuse-cpp_amd"))

import dfx  # noqa: E402

B, PROMPT, STEPS = 256, 32, 16
MFMA_F16_PEAK_TFLOPS = 2500.0      # MI355X dense f16 MFMA
HBM_PEAK_GBS = 8000.0
# The reference's published CPU rate: 1586 ms per Q4_K_M denoising step at 96 rows on a
# 12-core EPYC 4465P (research/benchmark/RESULTS.md:50-54), 2 * 96 * 7.497e9 FLOP per step.
GGML_GFLOPS_PER_CORE = 2.0 * 96 * 7.497e9 / 1.586 / 12 / 1e9


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def model_path(tag, scheme, seed):
    d = os.environ.get("DFX_BENCH_DIR", "/tmp")
    return os.path.join(d, f"dfx-{tag}-{scheme}-s{seed}.gguf")


def ensure_model(tag="llada8b", arch=None, scheme="q4_k_m", seed=0):
    """Generated once per machine (the parity tests share the file naming)."""
    p = model_path(tag, scheme, seed)
    stamp = p + ".ok"
    if not (os.path.exists(p) and os.path.exists(stamp)):
        t = time.time()
        dfx.synth_model(p, arch or dfx.LLADA_8B, scheme=scheme, seed=seed, sigma=0.02, n_threads=16)
        open(stamp, "w").write("ok\n")
        log(f"generated {p} in {time.time() - t:.1f}s")
    return p


def time_generations(ctx, prompt, n_gen, params, reps, warmup):
    for _ in range(warmup):
        ctx.generate(prompt, n_gen, params)
    stats = dfx.GenStats()
    dfx.sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        ctx.generate(prompt, n_gen, params, stats)
    dfx.sync()
    return (time.perf_counter() - t0) / reps, stats


def cpu_baseline(path, row_plan, n_threads):
    """The CPU oracle (a restatement of the reference's GGML CPU path, run here as the
    reference cannot be built) timed on this host's cores, on a bounded sample:
      * a whole 16-step generation (entropy_exit + cache, 32 + 256) of a two-layer model of
        the LLaDA-8B width (vocab head, embedding and sampler at full size), timed end to end;
      * the 32-layer and the 1-layer forward over the 288-row step-0 sequence, whose
        difference gives the cost of one layer per row;
    the full-depth generation = the two-layer one + 30 layers' cost at the rows of every
    step.  Its GEMM rate per core is reported beside the reference's published rate."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import oracle_py as O
    spent = 0.0
    # two-layer generate, timed
    arch2 = dict(dfx.LLADA_8B, n_layer=2)
    p2 = ensure_model("llada8b-2l", arch2, "q4_k_m", 0)
    om2 = O.OracleModel(p2)
    prompt = np.random.default_rng(1).integers(0, 126000, PROMPT).astype(np.int32)
    t = time.perf_counter()
    _, st = om2.generate(prompt, B, n_steps=STEPS, remasking=dfx.ENTROPY_EXIT, use_cache=True, seed=42,
                         n_threads=n_threads)
    t_gen2 = time.perf_counter() - t
    spent += t_gen2
    rows2 = [st.rows_per_step[i] for i in range(st.actual_steps)]
    # per-layer-row cost from a 1-layer and the full-depth forward (better of two runs)
    om = O.OracleModel(path)
    L = om.m.n_layer
    M = PROMPT + B
    toks = np.random.default_rng(1).integers(0, 126000, M).astype(np.int32)
    times = {}
    for nl in (1, L):
        om.m.n_layer = nl
        best = float("inf")
        for _ in range(2):
            t = time.perf_counter()
            om.forward_full(toks, n_threads=n_threads)
            dt = time.perf_counter() - t
            spent += dt
            best = min(best, dt)
        times[nl] = best
    om.m.n_layer = L
    t_layer_row = max(times[L] - times[1], 1e-9) / ((L - 1) * M)
    total = t_gen2 + (L - 2) * t_layer_row * sum(rows2)
    gflop_layer = 2.0 * (4 * 4096 * 4096 + 3 * 4096 * 12288) * M / 1e9
    gflops_core = gflop_layer / max(t_layer_row * M, 1e-9) / n_threads
    value = B / total
    return {
        "value": round(value, 4), "unit": "tok/s", "cores": n_threads, "kind": "port",
        "sample": (f"oracle (GGML-semantics C++ restatement, {n_threads} threads, AVX2 integer block dots): "
                   f"a whole 16-step generate (entropy_exit + cache, 32 + 256) of a 2-layer LLaDA-8B-width "
                   f"model timed end to end ({t_gen2:.1f}s, rows {rows2}), plus 30 layers at those rows from "
                   f"the 32- and 1-layer 288-row forwards (better of 2 each); {spent:.1f}s of CPU time in all"),
        "two_layer_generate_s": round(t_gen2, 2),
        "step0_forward_s": round(times[L], 3),
        "ms_per_denoise_step": round(1000 * total / STEPS, 1),
        "layer_gflops_per_core": round(gflops_core, 2),
        "reference_published_gflops_per_core": round(GGML_GFLOPS_PER_CORE, 2),
        # the same generation at the reference's published per-core GEMM rate on these cores
        "value_at_reference_rate": round(value * GGML_GFLOPS_PER_CORE / gflops_core, 4),
    }


def config_llada_b64(model):
    """LLaDA-8B Q4_K_M, 32 + 64 masks, low_confidence, no cache, 16 steps (96 rows a step)."""
    prompt = np.random.default_rng(1).integers(0, 126000, 32).astype(np.int32)
    ctx = dfx.Context(model, 96)
    params = dfx.SamplerParams.make(n_steps=16, remasking=dfx.LOW_CONFIDENCE, use_cache=False, seed=42)
    sec, st = time_generations(ctx, prompt, 64, params, 3, 1)
    ctx.close()
    return {"workload": "LLaDA-8B Q4_K_M, prompt 32 + B=64, 16 steps, low_confidence, no cache",
            "tok_s": round(64 / sec, 2), "ms_per_generation": round(1000 * sec, 3),
            "ms_per_denoise_step": round(st.forward_ms / max(st.actual_steps, 1), 3),
            "rows_per_step": [st.rows_per_step[i] for i in range(st.actual_steps)]}


def config_dream():
    """Dream-7B Q4_K_M, 64 + 64 masks, entropy_exit + cache, 16 steps."""
    path = ensure_model("dream7b", dfx.DREAM_7B, "q4_k_m", 2)
    model = dfx.Model(path)
    prompt = np.random.default_rng(3).integers(0, 151643, 64).astype(np.int32)
    ctx = dfx.Context(model, 128)
    params = dfx.SamplerParams.make(n_steps=16, remasking=dfx.ENTROPY_EXIT, use_cache=True, seed=42,
                                    entropy_threshold=1.5)
    sec, st = time_generations(ctx, prompt, 64, params, 3, 1)
    ctx.close()
    model.close()
    steps = [round(st.step_ms[i], 3) for i in range(st.actual_steps)]
    return {"workload": "Dream-7B Q4_K_M, prompt 64 + B=64, 16 steps, entropy_exit + inter-step KV cache",
            "tok_s": round(64 / sec, 2), "ms_per_generation": round(1000 * sec, 3),
            "ms_per_denoise_step_full": steps[0] if steps else None,
            "ms_per_denoise_step_cached_mean": round(float(np.mean(steps[1:])), 3) if len(steps) > 1 else None,
            "rows_per_step": [st.rows_per_step[i] for i in range(st.actual_steps)]}


DREAM_Q4KM_WEIGHT_BYTES = 4.223e9   # Dream-7B Q4_K_M matrices (embedding excluded), read once per decode pass


def config_ar(reps=3):
    """ar_generate on Dream-7B Q4_K_M (the Qwen2 architecture the reference's AR path targets):
    prompt 64, 128 greedy tokens (temperature 0, repeat penalty 1.1 over 64), 1 warm-up + reps.
    Decode is one pass over every weight per token: its HBM rate is the matrices' bytes
    over the mean time per decoded token."""
    path = ensure_model("dream7b", dfx.DREAM_7B, "q4_k_m", 2)
    model = dfx.Model(path)
    prompt = np.random.default_rng(3).integers(0, 151643, 64).astype(np.int32)
    ctx = dfx.Context(model, 64 + 128)
    params = dfx.ArParams.make(temperature=0.0)
    runs = []
    for i in range(1 + reps):
        st = dfx.ArStats()
        toks = ctx.ar_generate(prompt, 128, params, stats=st)
        if i:
            runs.append((st.prefill_ms, st.decode_ms, st.n_decoded, st.total_ms, len(toks)))
    ctx.close()
    model.close()
    pre = float(np.mean([r[0] for r in runs]))
    dec_ms = float(np.mean([r[1] / max(r[2], 1) for r in runs]))
    tot = float(np.mean([r[3] for r in runs]))
    gbs = DREAM_Q4KM_WEIGHT_BYTES / (dec_ms * 1e-3) / 1e9
    return {"workload": "ar_generate, Dream-7B Q4_K_M, prompt 64, 128 tokens greedy (repeat penalty 1.1 / 64)",
            "prefill_ms": round(pre, 3), "prefill_tok_s": round(64 / (pre * 1e-3), 1),
            "decode_ms_per_token": round(dec_ms, 4), "decode_tok_s": round(1000.0 / dec_ms, 1),
            "gen_tok_s": round(runs[0][4] / (tot * 1e-3), 1), "generated": runs[0][4],
            "decode_weight_gbs": round(gbs, 1), "decode_frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4)}


def config_batched():
    """The batched long-context workload: 8 independent sequences of a 512-token prompt + B=256
    masks on LLaDA-8B Q8_0 (seed 5), 16 steps, low_confidence with the inter-step cache (the
    header's default policy).  The sequences run at the same time, one context each (own
    stream) on one shared model, from 8 host threads; tok/s = 8 x 256 / the wall time of the
    whole batch.  One warm-up batch, then one timed batch; a single sequence alone is timed
    beside it."""
    import threading
    path = ensure_model("llada8b", dfx.LLADA_8B, "q8_0", 5)
    model = dfx.Model(path)
    S, P, Bm = 8, 512, 256
    prompts = [np.random.default_rng(50 + i).integers(0, 126000, P).astype(np.int32) for i in range(S)]
    ctxs = [dfx.Context(model, P + Bm) for _ in range(S)]
    params = dfx.SamplerParams.make(n_steps=16, remasking=dfx.LOW_CONFIDENCE, use_cache=True, seed=42)
    stats = [dfx.GenStats() for _ in range(S)]

    def batch():
        errors = []

        def run(i):
            try:
                ctxs[i].generate(prompts[i], Bm, params, stats[i])
            except Exception as e:   # noqa: BLE001 - re-raised below
                errors.append(e)
        th = [threading.Thread(target=run, args=(i,)) for i in range(S)]
        dfx.sync()
        t0 = time.perf_counter()
        for t in th:
            t.start()
        for t in th:
            t.join()
        dfx.sync()
        if errors:
            raise errors[0]
        return time.perf_counter() - t0
    batch()
    sec = batch()
    one, st1 = time_generations(ctxs[0], prompts[0], Bm, params, 1, 0)
    for c in ctxs:
        c.close()
    model.close()
    return {"workload": "8 x (512 + 256) LLaDA-8B Q8_0, 16 steps, low_confidence + inter-step KV cache, "
                        "8 contexts generating concurrently",
            "tok_s": round(S * Bm / sec, 2), "ms_per_batch": round(1000 * sec, 1),
            "single_sequence_ms": round(1000 * one, 1),
            "single_ms_per_denoise_step_full": round(st1.step_ms[0], 3),
            "rows_per_step": [st1.rows_per_step[i] for i in range(st1.actual_steps)]}


def config_sampler():
    """The sampler over [256 x 126464] f32 logits N(0, sigma), sigma in {0.5, 2, 8} (seed 4):
    row statistics (softmax max / sum, entropy, top-2), candidate records and the selection
    of the 16 to unmask (256 / 16), on device.  HBM rate of the statistics pass: the logits
    block read once (129.5 MB) over its time."""
    R, V, L = 256, 126464, dfx.lib
    rows = dfx.Buf.of(np.arange(R, dtype=np.int32))
    pos = dfx.Buf.of(np.arange(R, dtype=np.int32) + 32)
    st, cand, order, nun = dfx.Buf(R * 16), dfx.Buf(R * 16), dfx.Buf(R * 4), dfx.Buf(4)
    out = {}
    for sigma in (0.5, 2.0, 8.0):
        x = dfx.Buf.of(np.random.default_rng(4).standard_normal((R, V), dtype=np.float32) * np.float32(sigma))

        def run():
            dfx.check(L().dfx_row_stats(x.ptr, V, rows.ptr, R, V, st.ptr, None), "row_stats")
            dfx.check(L().dfx_make_candidates(st.ptr, pos.ptr, R, 0, cand.ptr, None), "candidates")
            dfx.check(L().dfx_select(cand.ptr, R, dfx.ENTROPY_EXIT, 1.5, R // 16, order.ptr, nun.ptr, None), "select")

        def timed(fn, reps=20):
            for _ in range(3):
                fn()
            tm, ms = C.c_void_p(), C.c_float()
            dfx.check(L().dfx_timer_start(C.byref(tm), None), "timer")
            for _ in range(reps):
                fn()
            dfx.check(L().dfx_timer_stop(tm, None, C.byref(ms)), "timer")
            return 1000.0 * ms.value / reps
        total_us = timed(run)
        stats_us = timed(lambda: dfx.check(L().dfx_row_stats(x.ptr, V, rows.ptr, R, V, st.ptr, None), "row_stats"))
        gbs = R * V * 4 / (stats_us * 1e-6) / 1e9
        out[f"sigma_{sigma:g}"] = {"us_per_step": round(total_us, 2), "row_stats_us": round(stats_us, 2),
                                   "row_stats_gbs": round(gbs, 1), "frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        del x
    return {"workload": "sampler: [256 x 126464] f32 logits N(0, sigma), stats + candidates + select 16",
            "results": out}


def committed_traffic():
    """HBM bytes per Q4_K GEMM launch of this workload, from the committed rocprofv3
    counter summary (FETCH_SIZE / WRITE_SIZE scaled by a plain copy's readings), or
    None if the summary is absent."""
    f = os.path.join(REPO, "profiles", "q4k_gemm_hbm_traffic_llada8b_q4km_b256.md")
    try:
        for line in open(f):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":")[1]))
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3, help="timed diffuse_generate calls")
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-configs", action="store_true", help="skip the other workloads")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--launch", choices=("graphs", "direct"), default="graphs",
                    help="per-step layer stacks replayed from captured HIP graphs (default) or launched "
                         "kernel by kernel (the same kernels; for tools that trace launches one by one)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 3 device-to-device copies of 512 MiB (reference kernel for the "
                         "FETCH_SIZE / WRITE_SIZE counter scale) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        n = 512 << 20
        a, b = dfx.Buf(n), dfx.Buf(n)
        a.zero()
        for _ in range(3):
            dfx.check(dfx.lib().dfx_memcpy_d2d(b.ptr, a.ptr, n, None), "copy")
        dfx.sync()
        print(json.dumps({"copy_calibration_bytes": n, "copies": 3}))
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: --gpus {args.gpus} is not supported (the denoising path is "
              f"single-GPU; see the sharding design notes)", file=sys.stderr)
        sys.exit(2)
    if dfx.device_count() < 1:
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)

    path = ensure_model()
    t = time.time()
    model = dfx.Model(path)
    ctx = dfx.Context(model, PROMPT + B)
    ctx.set_device_loop(True, graphs=args.launch == "graphs")
    log(f"model loaded in {time.time() - t:.1f}s")
    prompt = np.random.default_rng(1).integers(0, 126000, PROMPT).astype(np.int32)
    params = dfx.SamplerParams.make(n_steps=STEPS, remasking=dfx.ENTROPY_EXIT, use_cache=True, seed=42,
                                    entropy_threshold=1.5)
    for _ in range(args.warmup):
        ctx.generate(prompt, B, params)

    # Timed region for `value`: K generations with no per-GEMM events on the stream.
    stats = dfx.GenStats()
    dfx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ctx.generate(prompt, B, params, stats)
    dfx.sync()
    elapsed = time.perf_counter() - t0
    log(f"timed {args.steps} generations: {1000 * elapsed / args.steps:.2f} ms each")
    # The same K generations again with a HIP event pair around every GEMM launch on the
    # engine stream: the roofline's average launch time comes from these events.  The
    # event packets slow the stream a little, so this pass does not give `value`.
    ctx.profile(True)
    dfx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ctx.generate(prompt, B, params)
    dfx.sync()
    elapsed_prof = time.perf_counter() - t0
    prof = {t: ctx.profile_read(t) for t in (dfx.TYPE_Q4_K, dfx.TYPE_Q6_K)}
    q4_big = ctx.profile_read(dfx.TYPE_Q4_K, 1)     # M > 96: MFMA-bound shapes (mostly k_q4k_w<2, 1, 2>)
    q4_small = ctx.profile_read(dfx.TYPE_Q4_K, 2)   # M <= 96: weight-bandwidth-bound shapes
    ctx.profile(False)
    ctx.close()

    steps_done = stats.actual_steps
    rows = [stats.rows_per_step[i] for i in range(steps_done)]
    step_ms = [round(stats.step_ms[i], 3) for i in range(steps_done)]
    ms_per_gen = 1000 * elapsed / args.steps
    q4 = prof[dfx.TYPE_Q4_K]
    achieved = q4_big["flops"] / (q4_big["ms"] * 1e-3) / 1e12 if q4_big["ms"] > 0 else 0.0
    achieved_all = q4["flops"] / (q4["ms"] * 1e-3) / 1e12 if q4["ms"] > 0 else 0.0
    small_gbs = q4_small["bytes"] / (q4_small["ms"] * 1e-3) / 1e9 if q4_small["ms"] > 0 else 0.0

    configs = None
    if not args.no_configs:
        configs = {}
        t = time.time()
        configs["llada8b_q4km_b64_low_confidence_no_cache"] = config_llada_b64(model)
        log(f"B=64 workload took {time.time() - t:.1f}s")
    model.close()
    if configs is not None:
        t = time.time()
        configs["dream7b_q4km_b64_entropy_exit_cache"] = config_dream()
        log(f"Dream workload took {time.time() - t:.1f}s")
        t = time.time()
        configs["sampler_256x126464"] = config_sampler()
        log(f"sampler workload took {time.time() - t:.1f}s")
        t = time.time()
        configs["ar_dream7b_q4km_decode"] = config_ar()
        log(f"AR workload took {time.time() - t:.1f}s")
        t = time.time()
        configs["batched_8x768_llada8b_q8_0"] = config_batched()
        log(f"batched long-context workload took {time.time() - t:.1f}s")

    cpu = None
    if not args.no_cpu:
        n_thr = args.cpu_threads or min(os.cpu_count() or 1, 16)
        t = time.time()
        cpu = cpu_baseline(path, rows, n_thr)
        log(f"cpu baseline leg took {time.time() - t:.1f}s")

    out = {
        "metric": "gen tok/s + ms/denoise step, LLaDA-8B Q4_K_M B=256 s=16, 1 MI355X",
        "value": round(B * args.steps / elapsed, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_gen, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k_m weights, int8-quantised activations (exact integer MFMA sums), f32 accumulation",
        "data": "synthetic: random-init N(0,0.02) LLaDA-8B weights (seed 0), 32 random prompt ids (seed 1)",
        "config": {"workload": "LLaDA-8B arch Q4_K_M, prompt 32 + B=256 masks, 16 steps, entropy_exit + "
                               "inter-step KV cache (diffuse_generate)",
                   "prompt": PROMPT, "B": B, "denoise_steps": STEPS, "actual_steps": steps_done,
                   "rows_per_step": rows, "layer_launch": args.launch},
        "ms_per_denoise_step": round(stats.forward_ms / max(steps_done, 1), 3),
        "ms_per_denoise_step_full": step_ms[0] if step_ms else None,
        "ms_per_denoise_step_cached_mean": round(float(np.mean(step_ms[1:])), 3) if len(step_ms) > 1 else None,
        "step_forward_ms": step_ms,
        "roofline": {
            "kernel": "Q4_K GEMM calls over more than 96 rows: k_q4k_w<2, 1, 2> (exact dequant-fused MFMA GEMM, "
                      "LDS-DMA fed, 64-row tiles; the gate|up call with SwiGLU in its epilogue), k_q4k_w<3, 1, 2> "
                      "(96-row tiles) where that saves a round of workgroups, k_q4k<1, 1, 4> / <1, 1, 2> where the "
                      "row count favours 32-row tiles; a split-K reduction is included when one is launched",
            "bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4), "traffic": committed_traffic(),
            "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
            "algorithmic_bytes_per_launch": round(q4_big["bytes"] / max(q4_big["launches"], 1)),
            "launches": q4_big["launches"],
            "avg_launch_us": round(1000 * q4_big["ms"] / max(q4_big["launches"], 1), 3),
            "flops_per_launch": round(q4_big["flops"] / max(q4_big["launches"], 1), 1),
            "gemm_share_of_time": round((q4["ms"] + prof[dfx.TYPE_Q6_K]["ms"]) / (1000 * elapsed_prof), 4),
            "events_pass_tok_s": round(B * args.steps / elapsed_prof, 2),
            "all_q4k_calls_tflops": round(achieved_all, 2),
            "small_rows": {"kernel": "Q4_K GEMM calls over at most 96 rows", "bound": "hbm",
                           "achieved": round(small_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(small_gbs / HBM_PEAK_GBS, 4), "launches": q4_small["launches"],
                           "avg_launch_us": round(1000 * q4_small["ms"] / max(q4_small["launches"], 1), 3)},
        },
        "cpu_baseline": cpu,
        "other_workloads": configs,
    }
    if cpu:
        out["vs_cpu"] = round(out["value"] / cpu["value"], 1)
        out["vs_cpu_at_reference_rate"] = round(out["value"] / cpu["value_at_reference_rate"], 1)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
