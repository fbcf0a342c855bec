#!/usr/bin/env python3
"""Benchmark of the dequant-GEMV hot path on one MI355X.

Workload (benchmark config 1, the record's `value`): batch-1 dequant-GEMV over
the seven Qwen3-4B layer shapes (q 4096x2560, k/v 1024x2560, o 2560x4096,
gate/up 9728x2560, down 2560x9728) in the v3 scheme (6-bit codes, two-plane
device layout), synthetic blocks and x ~ N(0,1) fp32 drawn with the configs'
PRNG (xoshiro256++ seeded 0x12345678, Box-Muller in f32, as the reference's
evaluator draws x; wpcg.synth.wpc_blocks / wpc_x). One step = one pass
of the seven GEMVs in four launches (q/k/v share their input and a launch, as
do gate/up; o and down run alone, as in a decode layer where their inputs come
from other operations). Weights are HBM-cold: the steps rotate over enough
device copies of the layer to exceed the 256 MB Infinity Cache (>= 1 GB), and
the launches are replayed from HIP graphs so host launch cost is not timed.
Exactly --warmup untimed steps, then exactly --steps timed steps.

value = algorithmic bytes per step x steps / time, with
bytes(GEMV) = rows*(cols/128)*BPB + 4*cols + 4*rows, BPB = 100 (v3) / 68 (v4).

Also measured in the same run (under `config`):
  per_shape   each config-1 GEMV alone, HBM-cold, GB/s and % of peak;
  cfg0        the config-0 v4 GEMV 4864x896, HBM-cold (rotated over >= 1 GB)
              and cache-hot (one copy), launch after launch;
  decode      greedy decode of the Qwen3-30B-A3B-shaped v4 model (config 3);
  decode_dense greedy decode of the dense Qwen3-4B-shaped v4 model (config 2);
  gemm        the batched v4 GEMM at Gemma-12B shapes (config 4);
  large_gemv  the FAST kernel on the config-3 lm_head shape (165 MB).
CPU baselines run the oracle's AVX2 restatement of the reference kernels on
the host, with the box's CPU share (at most 16 threads) and with 1 thread,
recording nproc and the CPU model.

`--gpus N` with N > 1 is refused: this build measures one GPU.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "wpc-engine_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "dequant-GEMV HBM GB/s (% of peak); decode tok/s Qwen3-30B-A3B-shape v4"
PEAK_GBPS = 8000.0
QWEN3_4B = [("q_proj", 4096, 2560), ("k_proj", 1024, 2560), ("v_proj", 1024, 2560),
            ("o_proj", 2560, 4096), ("gate_proj", 9728, 2560), ("up_proj", 9728, 2560),
            ("down_proj", 2560, 9728)]
BPB = {3: 100, 4: 68}
# HBM bytes per launch of the FAST kernel in this workload, measured with
# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (bench.py --pmc-pass) and scaled by
# the same counters' reading for a copy kernel of known size; see
# profiles/k_gemv_fast_cfg1_v3_traffic.txt. None where not measured.
TRAFFIC = {(3, "fast"): 20051404}
TRAFFIC_SOURCE = ("profiles/k_gemv_fast_cfg1_v3_traffic.txt: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE "
                  "passes over bench.py --pmc-pass (the workload rotated over >= 1 GB, HBM-cold), scaled by "
                  "a 256 MiB device copy's readings")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemv_bytes(rows, cols, scheme):
    return rows * (cols // 128) * BPB[scheme] + 4 * cols + 4 * rows


def host_info():
    """nproc, the threads this process may use, the CPU model, and the
    thread count of the all-cores baseline: the CPUs this process may run on,
    capped at OMP_NUM_THREADS and at 16 (the host-CPU share of one GPU on
    the benchmark machines)."""
    nproc = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = nproc
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    omp = os.environ.get("OMP_NUM_THREADS", "")
    cap = int(omp) if omp.isdigit() and int(omp) > 0 else affinity
    return {"nproc": nproc, "affinity": affinity, "cpu_model": model,
            "threads_all": max(1, min(affinity, cap, 16))}


def timed_median(fn, budget_s, min_reps=20):
    """Median wall time of fn() after one warm-up call: at least min_reps
    calls, more while budget_s lasts."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_reps or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_gemv_baseline(scheme, shapes, blocks, xs, budget_s, what):
    """The oracle's AVX2 restatement of the reference row kernel
    (matvec_v{3,4}_fused) on the host cores, rows split over threads as
    WpcLinear*::matvec does with rayon (wpc_weights_v4.rs:165-193), on the
    given matrices: all cores and 1 core, median of >= 20 passes each."""
    import oracle as O
    hi = host_info()
    kern = O.KERNEL_AVX2 if O.have_avx2() else O.KERNEL_FUSED
    step_bytes = sum(gemv_bytes(r, c, scheme) for _, r, c in shapes)
    res = {}
    for key, threads, budget in (("all", hi["threads_all"], budget_s), ("one", 1, budget_s / 2)):
        def one_pass(threads=threads):
            for (name, r, c), b in zip(shapes, blocks):
                O.linear_matvec(scheme, b, r, c, xs[c], None, kern, threads)
        med, n = timed_median(one_pass, budget)
        res[key] = (step_bytes / med / 1e9, med, n, threads)
    kname = "AVX2 intrinsics" if kern == O.KERNEL_AVX2 else "scalar fmaf"
    return {
        "value": round(res["all"][0], 3),
        "unit": "GB/s",
        "cores": res["all"][3],
        "kind": "port",
        "one_core_value": round(res["one"][0], 3),
        "nproc": hi["nproc"],
        "cpu_model": hi["cpu_model"],
        "sample": (f"{what} ({step_bytes / 1e6:.2f} MB per pass): median of {res['all'][2]} passes on "
                   f"{res['all'][3]} threads (all of this process's CPUs, at most 16) and of "
                   f"{res['one'][2]} on 1 thread; {kname} restatement of matvec_v{scheme}_fused, rows "
                   f"split over threads as rayon does; nproc {hi['nproc']}, {hi['cpu_model']}"),
    }


QWEN3_30B_A3B = dict(n_layers=48, hidden=2048, n_heads=32, n_kv_heads=4, head_dim=128, inter=0,
                     vocab=151936, n_experts=128, top_k=8, moe_inter=768, norm_topk=1, tied=0,
                     max_pos=512, eps=1e-6, rope_theta=1e6)
QWEN3_4B_DENSE = dict(n_layers=36, hidden=2560, n_heads=32, n_kv_heads=8, head_dim=128, inter=9728,
                      vocab=151936, n_experts=0, top_k=0, moe_inter=0, norm_topk=1, tied=1,
                      max_pos=512, eps=1e-6, rope_theta=1e6)
DECODE_MODELS = {
    "decode": (QWEN3_30B_A3B, "Qwen3-30B-A3B-shaped, v4 (48 layers, hidden 2048, 32q/4kv x 128, 128 experts "
                              "top-8, moe_inter 768, vocab 151936 untied, fp32 router)"),
    "decode_dense": (QWEN3_4B_DENSE, "Qwen3-4B-shaped dense, v4 (36 layers, hidden 2560, 32q/8kv x 128, "
                               "intermediate 9728 SwiGLU, vocab 151936 tied)"),
}


def decode_token_bytes(c, bpb=68):
    """Weight bytes one decode token reads: attention, the MLP (or the router,
    fp32, and the top-k experts), the output head (KV cache excluded)."""
    H, hd = c["hidden"], c["head_dim"]
    qd, kvd = c["n_heads"] * hd, c["n_kv_heads"] * hd
    blocks = lambda r, k: r * (k // 128) * bpb  # noqa: E731
    attn = blocks(qd, H) + 2 * blocks(kvd, H) + blocks(H, qd)
    if c["n_experts"]:
        mlp = c["top_k"] * (2 * blocks(c["moe_inter"], H) + blocks(H, c["moe_inter"])) + c["n_experts"] * H * 4
    else:
        mlp = 2 * blocks(c["inter"], H) + blocks(H, c["inter"])
    return c["n_layers"] * (attn + mlp) + blocks(c["vocab"], H)


def kv_bytes_per_token(c, n_prompt, n_new):
    """fp32 K and V bytes read per decode step, averaged over the timed steps
    (positions n_prompt .. n_prompt + n_new - 2): every layer reads
    2 * n_kv_heads * head_dim * 4 bytes per cached position."""
    per_pos = c["n_layers"] * 2 * c["n_kv_heads"] * c["head_dim"] * 4
    mean_len = n_prompt + 1 + (n_new - 2) / 2.0
    return per_pos * mean_len


def decode_bench(ctx, wpcg, synth, key, n_prompt, n_new, cpu_tokens, eager=False, n_exact=64,
                 prefill_timing=True):
    """Greedy decode of a config-2/3 model: seeded weights ~N(0, 0.02)
    encoded as the artifact compiler does (layer 0 from fresh draws, later
    layers seeded row permutations of it: distinct weights, every token
    reads all its bytes from HBM), FAST generation of n_new tokens after an
    n_prompt-token prompt timed with HIP events around the replayed steps,
    EXACT generation of n_exact tokens and the number of leading ids the two
    share, the batched prefill of the prompt, and (cpu_tokens > 0) the
    oracle's decode of the same model at the same positions: bit identity of
    EXACT's logits and the CPU baseline (oracle_check). Returns the
    record's object."""
    import numpy as np
    cfg, desc = DECODE_MODELS[key]
    t0 = time.perf_counter()
    model = wpcg.Model(ctx, wpcg.SCHEME_V4, wpcg.ModelConfig(**cfg))
    keep = {} if cpu_tokens else None
    resident = 0
    for name, arr in synth.model_tensors(cfg, 4, 30, wpcg.encode, derive_layers=True):
        model.set_tensor(name, arr)
        resident += arr.nbytes
        if keep is not None:
            keep[name] = arr
    log(f"{key} model built in {time.perf_counter() - t0:.1f} s ({resident / 1e9:.2f} GB resident)")
    prompt = np.random.default_rng(31).integers(0, cfg["vocab"], n_prompt).astype(np.uint32)
    if eager:  # launch by launch, for kernel traces (a trace cannot see inside graph replays)
        model.set_graphs(False)
    out = {}
    for mode, mk, n in ((wpcg.MODE_FAST, "fast", n_new), (wpcg.MODE_EXACT, "exact", n_exact)):
        if n < 2:
            continue
        model.set_mode(mode)
        model.generate(prompt, n)            # warm-up (graph capture)
        ids, ms = model.generate(prompt, n)
        out[mk] = ((n - 1) / (ms / 1e3), ms / (n - 1), ids)
        log(f"{key} {mk}: {out[mk][0]:.1f} tok/s ({out[mk][1]:.3f} ms/token, {n - 1} steps)")
    m = min(n_new, n_exact)
    same = None
    if "exact" in out:
        same = int(np.argmax(np.concatenate([out["fast"][2][:m] != out["exact"][2][:m], [True]])))
        log(f"{key}: FAST greedy ids equal EXACT's for {same} of {m}")
    # the prompt alone: batched prefill (FAST) against the same tokens step
    # by step, each timed from an empty cache to the last token's logits
    model.set_mode(wpcg.MODE_FAST)
    pre = {}
    for pk, batched in (("batched", True), ("steps", False)) if prefill_timing else ():
        model.set_prefill(batched)
        model.reset()
        model.prefill(prompt, want_logits=False)  # warm-up
        model.reset()
        t1 = time.perf_counter()
        _, first = model.prefill(prompt, want_logits=False)
        pre[pk] = (time.perf_counter() - t1, first)
    model.set_prefill(True)
    if pre:
        log(f"{key} prefill of {n_prompt} tokens: batched {pre['batched'][0] * 1e3:.1f} ms, "
            f"step by step {pre['steps'][0] * 1e3:.1f} ms")
    tok_bytes = decode_token_bytes(cfg)
    kv = kv_bytes_per_token(cfg, n_prompt, n_new)
    rec = {
        "model": desc,
        "mode": "fast",
        "prompt_tokens": int(n_prompt),
        "new_tokens": int(n_new),
        "tok_s": round(out["fast"][0], 2),
        "ms_per_token": round(out["fast"][1], 4),
        "exact_tok_s": round(out["exact"][0], 2) if "exact" in out else None,
        "fast_ids_equal_exact": f"{same} of {m}" if same is not None else None,
        "prefill": {"tokens": int(n_prompt), "ms": round(pre["batched"][0] * 1e3, 2),
                    "tok_s": round(n_prompt / pre["batched"][0], 1),
                    "stepwise_ms": round(pre["steps"][0] * 1e3, 2),
                    "first_token_equal_stepwise": bool(pre["batched"][1] == pre["steps"][1])} if pre else None,
        "weight_bytes_per_token": tok_bytes,
        "kv_bytes_per_token_mean": round(kv),
        "achieved_gbps": round((tok_bytes + kv) * out["fast"][0] / 1e9, 1),
        "roofline_tok_s": round(PEAK_GBPS * 1e9 / (tok_bytes + kv), 1),
        "frac_of_roofline": round(out["fast"][0] * (tok_bytes + kv) / (PEAK_GBPS * 1e9), 4),
        "resident_gb": round(resident / 1e9, 2),
        "data": "synthetic: weights N(0,0.02) then v4-encoded (layer 0 drawn, later layers seeded row "
                "permutations of it), norms 1.0, prompt of random ids",
    }
    if cpu_tokens:
        rec.update(oracle_check(model, wpcg, cfg, keep, prompt, key, cpu_tokens))
    model.close()
    return rec


def oracle_check(model, wpcg, cfg, keep, prompt, key, n_steps):
    """The full-depth model against the oracle (the CPU restatement of the
    reference's forward_token, model.rs:419-547 / qwen3_moe_model.rs:406-542)
    at the positions the GPU decode runs: the oracle runs the prompt on all
    host threads, then n_steps greedy steps, timed (the CPU baseline, at
    positions n_prompt .. n_prompt + n_steps - 1), then two more steps on
    one thread. The GPU model in EXACT mode runs the same prompt and steps,
    each step's logits compared with the oracle's bit for bit; in FAST mode
    the same, each step's logits within 1e-5 of the oracle's range and the
    greedy ids compared. Returns the record's fields."""
    import numpy as np
    import oracle as O
    kern = O.KERNEL_AVX2 if O.have_avx2() else O.KERNEL_FUSED
    hi = host_info()
    n_prompt = len(prompt)
    ref = O.Model(cfg, keep, cfg["max_pos"], kern, hi["threads_all"])
    t0 = time.perf_counter()
    for t in prompt[:-1]:
        ref.forward_token(int(t))
    t_prompt = time.perf_counter() - t0
    r_last = ref.forward_token(int(prompt[-1]))
    ref_logits, ids = [], []
    tok = O.argmax(r_last)
    t1 = time.perf_counter()
    for _ in range(n_steps):
        ids.append(tok)
        r = ref.forward_token(tok)
        ref_logits.append(r)
        tok = O.argmax(r)
    t_all = time.perf_counter() - t1
    n_one = 2
    t2 = time.perf_counter()
    for _ in range(n_one):
        r = ref.forward_token(tok, threads=1)
        tok = O.argmax(r)
    t_one = time.perf_counter() - t2
    ref.close()
    log(f"{key} oracle: prompt of {n_prompt} in {t_prompt:.1f} s, {n_steps} steps "
        f"{n_steps / t_all:.3f} tok/s on {hi['threads_all']} threads, {n_one / t_one:.3f} on 1")
    u32 = lambda a: np.ascontiguousarray(a, np.float32).view(np.uint32)  # noqa: E731
    out = {}
    for mode, mk in ((wpcg.MODE_EXACT, "exact"), (wpcg.MODE_FAST, "fast")):
        model.set_mode(mode)
        model.reset()
        g_last, _ = model.prefill(prompt, want_logits=True)
        same, worst, ids_same = [], 0.0, 0
        for i in range(n_steps):
            g, a = model.forward_token(ids[i])
            r = ref_logits[i]
            same.append(bool(np.array_equal(u32(g), u32(r))))
            span = float(r.max() - r.min())
            worst = max(worst, float(np.max(np.abs(g.astype(np.float64) - r))) / span)
            ids_same += int(a == (ids[i + 1] if i + 1 < n_steps else O.argmax(r)))
        prompt_same = bool(np.array_equal(u32(g_last), u32(r_last)))
        out[mk] = (sum(same), worst, ids_same, prompt_same)
        log(f"{key} {mk} vs oracle at positions {n_prompt}..{n_prompt + n_steps - 1}: "
            f"{sum(same)} of {n_steps} steps bit-identical, worst {worst:.2e} of the logit range, "
            f"{ids_same} of {n_steps} greedy ids equal; last prompt logits "
            f"{'bit-identical' if prompt_same else 'differ'}")
    model.set_mode(wpcg.MODE_FAST)
    return {
        "exact_equal_oracle": f"{out['exact'][0]} of {n_steps}",
        "exact_prompt_logits_equal_oracle": out["exact"][3],
        "fast_vs_oracle": {"max_err_of_logit_range": float(f"{out['fast'][1]:.3e}"),
                           "greedy_ids_equal": f"{out['fast'][2]} of {n_steps}"},
        "oracle_check": (f"full depth ({cfg['n_layers']} layers): the oracle ran the {n_prompt}-token "
                         f"prompt and {n_steps} greedy steps (positions {n_prompt}..{n_prompt + n_steps - 1}); "
                         f"the GPU model ran the same prompt and the oracle's ids, logits compared per step"),
        "cpu_baseline": {
            "tok_s": round(n_steps / t_all, 3), "cores": hi["threads_all"], "kind": "port",
            "one_core_tok_s": round(n_one / t_one, 3), "nproc": hi["nproc"], "cpu_model": hi["cpu_model"],
            "sample": (f"{n_steps} forward_token steps at positions {n_prompt}..{n_prompt + n_steps - 1} on "
                       f"{hi['threads_all']} threads, then {n_one} at the next positions on 1 thread, after the "
                       f"{n_prompt}-token prompt: the same model on the host (oracle restatement, "
                       f"{'AVX2' if kern == O.KERNEL_AVX2 else 'scalar'} GEMV, rows split over threads as "
                       f"rayon does)")},
    }


GEMMA_12B = [("gate/up_proj", 15360, 3840), ("down_proj", 3840, 15360)]
MFMA_BF16_TFLOPS = 2500.0  # MI355X dense bf16


def bf16_bits(x):
    """fp32 -> bf16 bit patterns (round to nearest even, finite inputs)."""
    import numpy as np
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def gemm_bench(ctx, wpcg, synth, cpu):
    """Benchmark config 4: batched v4 dequant-GEMM on the Gemma-12B-shaped
    gate/up (15360x3840) and down (3840x15360) matrices, M in {1, 4, 16, 64}
    activations (bf16 for M >= 4; M = 1 is the fp32 GEMV), HBM-cold over 34
    rotated copies (1.07 GB), replayed from a HIP graph. The time of a call
    includes every launch it makes (for M > 16 the X packing kernel too).
    Bytes = W + M*K*2 (bf16 X; 4 for the fp32 GEMV) + M*N*4."""
    import numpy as np
    e0, e1 = ctx.event(), ctx.event()
    out = {}
    for name, rows, cols in GEMMA_12B:
        base = wpcg.WpcLinear.from_blocks(ctx, 4, synth.random_v4_blocks(rows, cols, 41), rows, cols)
        base.set_mode(wpcg.MODE_FAST)
        wbytes = rows * (cols // 128) * 68
        lins = [base] + [base.clone() for _ in range(-(-int(1.0e9) // wbytes) - 1)]
        for M in (1, 4, 16, 64):
            X = np.random.default_rng(M).standard_normal((M, cols)).astype(np.float32)
            dt = wpcg.DTYPE_F32 if M == 1 else wpcg.DTYPE_BF16
            xd = ctx.upload(X if M == 1 else bf16_bits(X))
            yd = ctx.alloc(M * rows * 4)
            body = lambda: [l.gemm_dev(xd, M, yd, dt) for l in lins]
            body()
            ctx.sync()
            g = ctx.capture(body)
            g.launch()
            ctx.sync()
            reps = 10
            e0.record()
            for _ in range(reps):
                g.launch()
            e1.record()
            ctx.sync()
            us = e0.elapsed_ms(e1) * 1e3 / (reps * len(lins))
            alg = wbytes + M * cols * (4 if M == 1 else 2) + M * rows * 4
            tflops = 2.0 * M * rows * cols / us / 1e6
            out[f"{name} M={M}"] = {"us": round(us, 3), "gbps": round(alg / us / 1e3, 1),
                                    "frac_hbm": round(alg / us / 1e3 / PEAK_GBPS, 4),
                                    "tflops": round(tflops, 1),
                                    "frac_mfma_bf16": round(tflops / MFMA_BF16_TFLOPS, 4)}
            log(f"gemm {name} M={M}: {us:.2f} us, {alg / us / 1e3:.0f} GB/s, {tflops:.1f} TFLOP/s")
            del g
            xd.free()
            yd.free()
        for l in lins:
            l.close()
    rec = {"workload": "cfg4: batched v4 dequant-GEMM, Gemma-12B gate/up 15360x3840 and down 3840x15360, "
                       "HBM-cold, bf16 X for M >= 4 (matrix cores), fp32 x GEMV for M = 1",
           "results": out}
    if cpu:
        import oracle as O
        rows, cols = GEMMA_12B[0][1], GEMMA_12B[0][2]
        blocks = synth.random_v4_blocks(rows, cols, 41)
        X = np.random.default_rng(4).standard_normal((4, cols)).astype(np.float32)
        kern = O.KERNEL_AVX2 if O.have_avx2() else O.KERNEL_FUSED
        threads = host_info()["threads_all"]
        O.linear_matmul_v4(blocks, rows, cols, X[:1], kern, threads)  # warm-up
        t1 = time.perf_counter()
        n = 0
        while time.perf_counter() - t1 < 2.0 or n < 2:
            O.linear_matmul_v4(blocks, rows, cols, X, kern, threads)
            n += 1
        us = (time.perf_counter() - t1) / n * 1e6
        rec["cpu_baseline"] = {"us_gate_up_M4": round(us, 1), "cores": threads, "kind": "port",
                               "sample": f"{n} calls of 4 per-token matvecs (the reference's path for a "
                                         f"batch) on the gate/up matrix, oracle AVX2 restatement"}
        log(f"gemm CPU baseline: gate/up M=4 {us:.0f} us on {threads} threads")
    return rec


def large_gemv_bench(ctx, wpcg, synth):
    """The largest GEMV of the config-3 decode, its lm_head shape (151936 x
    2048, v4, 165 MB) as a plain FAST GEMV with an fp32 x, HBM-cold over 7
    rotated copies (1.16 GB), replayed from a HIP graph: the kernel's
    bandwidth once a launch is large enough to stream (the config-1 launches
    are 8-39 MB each and bound by their memory round trip)."""
    import numpy as np
    rows, cols = 151936, 2048
    base = wpcg.WpcLinear.from_blocks(ctx, 4, synth.random_v4_blocks(rows, cols, 77), rows, cols)
    base.set_mode(wpcg.MODE_FAST)
    lins = [base] + [base.clone() for _ in range(6)]
    xd = ctx.upload(synth.random_x(cols, seed=5))
    yd = ctx.alloc(4 * rows)
    body = lambda: [l.matvec_dev(xd, yd) for l in lins]
    body()
    ctx.sync()
    g = ctx.capture(body)
    g.launch()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    reps = 10
    e0.record()
    for _ in range(reps):
        g.launch()
    e1.record()
    ctx.sync()
    us = e0.elapsed_ms(e1) * 1e3 / (reps * len(lins))
    alg = gemv_bytes(rows, cols, 4)
    del g
    for l in lins:
        l.close()
    xd.free()
    yd.free()
    gbps = alg / us / 1e3
    log(f"large GEMV v4 {rows}x{cols}: {us:.2f} us, {gbps:.0f} GB/s ({100 * gbps / PEAK_GBPS:.1f}% of peak)")
    return {"shape": f"v4 {rows}x{cols} (config-3 lm_head), FAST, fp32 x, HBM-cold over 7 copies",
            "us": round(us, 3), "gbps": round(gbps, 1), "frac_hbm": round(gbps / PEAK_GBPS, 4),
            "algorithmic_bytes": alg}


def prefill_trace(wpcg, synth, layers, n_prompt):
    """Four FAST prefills of the config-3 model cut to `layers` layers, each
    timed; for rocprofv3 kernel traces of the batched prefill."""
    import numpy as np
    cfg = dict(QWEN3_30B_A3B, n_layers=layers)
    ctx = wpcg.Context(0)
    model = wpcg.Model(ctx, wpcg.SCHEME_V4, wpcg.ModelConfig(**cfg))
    for name, arr in synth.model_tensors(cfg, 4, 30, wpcg.encode, derive_layers=True):
        model.set_tensor(name, arr)
    model.set_mode(wpcg.MODE_FAST)
    prompt = np.random.default_rng(31).integers(0, cfg["vocab"], n_prompt).astype(np.uint32)
    for _ in range(4):
        model.reset()
        t0 = time.perf_counter()
        model.prefill(prompt, want_logits=False)
        log(f"prefill of {n_prompt} tokens, {layers} layers: {(time.perf_counter() - t0) * 1e3:.2f} ms")
    model.close()
    ctx.close()
    return 0


def rotation_runner(ctx, copies, step_for_copy):
    """run(n): exactly n steps, step i on copy i % copies, replayed from HIP
    graphs: one graph per full rotation and one per remainder length."""
    graphs = {}

    def graph(k):
        if k not in graphs:
            graphs[k] = ctx.capture(lambda: [step_for_copy(i) for i in range(k)])
        return graphs[k]

    def run(n):
        q, r = divmod(n, copies)
        for _ in range(q):
            graph(copies).launch()
        if r:
            graph(r).launch()

    def warm():
        graph(copies)  # capture before any timed region
        return graphs
    return run, warm, graphs


# --series-eager: the per-shape and config-0 series launch one by one instead
# of replaying a graph (for kernel traces: rocprofv3 ended the process on a
# graph of several hundred launches); their times then include host launch
# cost, so such a run's JSON is not a measurement of record.
SERIES_EAGER = False


def gemv_series_us(ctx, wpcg, lins, xd, yd, reps=8):
    """Device time of one launch of lins[i].matvec(x), launched one after the
    other (each waits for the previous on the stream) over every member of
    lins, from a replayed graph: the mean over reps replays."""
    body = lambda: [l.matvec_dev(xd, yd) for l in lins]  # noqa: E731
    if SERIES_EAGER:
        body()
        ctx.sync()
        e0, e1 = ctx.event(), ctx.event()
        e0.record()
        for _ in range(reps):
            body()
        e1.record()
        ctx.sync()
        return e0.elapsed_ms(e1) * 1e3 / (reps * len(lins))
    g = ctx.capture(body)
    g.launch()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    e0.record()
    for _ in range(reps):
        g.launch()
    e1.record()
    ctx.sync()
    us = e0.elapsed_ms(e1) * 1e3 / (reps * len(lins))
    del g
    return us


def per_shape_bench(ctx, wpcg, scheme, shapes, blocks, xs, min_bytes, fast_kernel=0):
    """Each config-1 GEMV alone (the step's own matrices and x): FAST,
    HBM-cold (rotated over >= min_bytes of device copies of that matrix),
    launch after launch."""
    out = {}
    for i, (name, r, c) in enumerate(shapes):
        base = wpcg.WpcLinear.from_blocks(ctx, scheme, blocks[i], r, c)
        base.set_mode(wpcg.MODE_FAST).set_fast_kernel(fast_kernel)
        n = max(1, -(-int(min_bytes) // base.device_bytes()))
        lins = [base] + [base.clone() for _ in range(n - 1)]
        xd = ctx.upload(xs[c])
        yd = ctx.alloc(4 * r)
        us = gemv_series_us(ctx, wpcg, lins, xd, yd)
        alg = gemv_bytes(r, c, scheme)
        out[name] = {"shape": f"{r}x{c}", "us": round(us, 3), "gbps": round(alg / us / 1e3, 1),
                     "frac_hbm": round(alg / us / 1e3 / PEAK_GBPS, 4), "bytes": alg, "copies": n}
        log(f"per-shape {name} {r}x{c}: {us:.2f} us, {alg / us / 1e3:.0f} GB/s over {n} copies")
        for l in lins:
            l.close()
        xd.free()
        yd.free()
    return out


def cfg0_bench(ctx, wpcg, synth, min_bytes, cpu_budget, fast_kernel=0):
    """Benchmark config 0: the v4 GEMV 4864x896 (Qwen2.5-0.5B MLP up-proj),
    FAST, fp32 x. HBM-cold: launch after launch over >= min_bytes of device
    copies (each launch's weights come from HBM); cache-hot: the same launches
    on one copy (resident in the Infinity Cache after the first)."""
    rows, cols = 4864, 896
    blocks = synth.wpc_blocks(4, rows, cols, matrix_id=0)  # the configs' PRNG (synth.WPC_SEED)
    x = synth.wpc_x(cols)
    base = wpcg.WpcLinear.from_blocks(ctx, 4, blocks, rows, cols).set_mode(wpcg.MODE_FAST)
    base.set_fast_kernel(fast_kernel)
    n = max(1, -(-int(min_bytes) // base.device_bytes()))
    lins = [base] + [base.clone() for _ in range(n - 1)]
    xd = ctx.upload(x)
    yd = ctx.alloc(4 * rows)
    cold = gemv_series_us(ctx, wpcg, lins, xd, yd)
    hot = gemv_series_us(ctx, wpcg, [base] * n, xd, yd)
    alg = gemv_bytes(rows, cols, 4)
    for l in lins:
        l.close()
    xd.free()
    yd.free()
    log(f"cfg0 v4 {rows}x{cols}: HBM-cold {cold:.3f} us ({alg / cold / 1e3:.0f} GB/s), "
        f"cache-hot {hot:.3f} us ({alg / hot / 1e3:.0f} GB/s)")
    rec = {"shape": f"v4 {rows}x{cols}", "bytes": alg, "copies": n,
           "hbm_cold": {"us": round(cold, 3), "gbps": round(alg / cold / 1e3, 1),
                        "frac_hbm": round(alg / cold / 1e3 / PEAK_GBPS, 4)},
           "cache_hot": {"us": round(hot, 3), "gbps": round(alg / hot / 1e3, 1),
                         "frac_hbm": round(alg / hot / 1e3 / PEAK_GBPS, 4)},
           "north_star_us_at_70pct": round(alg / (0.7 * PEAK_GBPS) / 1e3, 3)}
    if cpu_budget:
        rec["cpu_baseline"] = cpu_gemv_baseline(4, [("up_proj", rows, cols)], [blocks], {cols: x},
                                                cpu_budget, "the config-0 v4 GEMV 4864x896")
        log(f"cfg0 CPU baseline {rec['cpu_baseline']['value']} GB/s on {rec['cpu_baseline']['cores']} "
            f"threads, {rec['cpu_baseline']['one_core_value']} on 1")
    return rec


def summarize_profile(out_dir, match=""):
    """Print rocprofv3 CSV output (run on the CPU, after a traced run) grouped by
    kernel and launch shape: kernel traces as launches, mean and median
    duration (end - start), counter collections as the mean value of each
    counter per dispatch. `match` keeps the kernels whose name contains it."""
    import csv
    import glob
    import collections

    def grid_of(row, axis):
        g = int(row.get(f"Grid_Size_{axis}") or 1)
        w = int(row.get(f"Workgroup_Size_{axis}") or 1)
        return g // max(w, 1)

    def short(name):
        return name.replace("wpcg::(anonymous namespace)::", "").split("(")[0].replace("void ", "")

    found = False
    for path in sorted(glob.glob(os.path.join(out_dir, "**", "*kernel_trace.csv"), recursive=True)):
        found = True
        groups = collections.defaultdict(list)
        with open(path) as f:
            for row in csv.DictReader(f):
                if match and match not in row["Kernel_Name"]:
                    continue
                key = (short(row["Kernel_Name"]), grid_of(row, "X"), grid_of(row, "Y"))
                groups[key].append((int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3)
        print(f"# {os.path.relpath(path, out_dir)}: kernel, workgroups x by y, launches, mean us, median us")
        for (name, gx, gy), v in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
            print(f"{name:44s} {gx:6d} x {gy:<3d} {len(v):7d} {statistics.mean(v):9.2f} "
                  f"{statistics.median(v):9.2f}")
    for path in sorted(glob.glob(os.path.join(out_dir, "**", "*counter_collection.csv"), recursive=True)):
        found = True
        groups = collections.defaultdict(lambda: collections.defaultdict(float))
        with open(path) as f:
            for row in csv.DictReader(f):
                if match and match not in row["Kernel_Name"]:
                    continue
                wg = int(row.get("Workgroup_Size") or 1)
                key = (short(row["Kernel_Name"]), int(row.get("Grid_Size") or 0) // max(wg, 1))
                # one row per dispatch and counter (dimensions already summed)
                did = int(row.get("Dispatch_Id") or row.get("Correlation_Id") or 0)
                groups[key][(row["Counter_Name"], did)] += float(row["Counter_Value"])
        print(f"# {os.path.relpath(path, out_dir)}: kernel, workgroups, counter, dispatches, "
              "mean per dispatch, last dispatch")
        for (name, wgs), vals in sorted(groups.items()):
            per = collections.defaultdict(list)
            for (cn, did), v in sorted(vals.items(), key=lambda kv: kv[0][1]):
                per[cn].append(v)
            for cn, v in sorted(per.items()):
                print(f"{name:44s} {wgs:7d} {cn:28s} {len(v):6d} {statistics.mean(v):16.1f} {v[-1]:16.1f}")
    if not found:
        print(f"no rocprofv3 CSV output under {out_dir}", file=sys.stderr)
        return 1
    return 0


def main():
    if "--summarize" in sys.argv:
        ap = argparse.ArgumentParser()
        ap.add_argument("--summarize", required=True, metavar="DIR",
                        help="print a rocprofv3 --output-format csv directory grouped by kernel and shape")
        ap.add_argument("--match", default="", help="only kernels whose name contains this")
        a = ap.parse_args()
        return summarize_profile(a.summarize, a.match)
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--scheme", type=int, default=3, choices=(3, 4))
    ap.add_argument("--mode", default="fast", choices=("exact", "fast"))
    ap.add_argument("--fast-kernel", default="mfma", choices=("mfma", "valu"),
                    help="FAST GEMV kernel of the config-1 step, per-shape and config-0 lines: matrix cores "
                         "with int8 x digits (mfma) or fp32 on the vector ALU (valu)")
    ap.add_argument("--min-bytes", type=float, default=1.0e9,
                    help="rotated working set, bytes (>= 1 GB defeats the 256 MB MALL)")
    ap.add_argument("--cpu-seconds", type=float, default=6.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--normal-exit", action="store_true",
                    help="leave through the runtime's exit path even with WPCG_HARD_EXIT=1 "
                         "(profilers finalize there)")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="short run for rocprofv3 --pmc passes (no timing, no JSON)")
    ap.add_argument("--only", default="",
                    help="comma list of extra sections to run (per_shape,cfg0,large_gemv,gemm,decode,"
                         "decode_dense, or none for the config-1 line alone); default: all")
    ap.add_argument("--no-decode", action="store_true", help="skip both decode measurements")
    ap.add_argument("--decode-prompt", type=int, default=256)
    ap.add_argument("--decode-new", type=int, default=256)
    ap.add_argument("--dense-prompt", type=int, default=128)
    ap.add_argument("--decode-cpu-tokens", type=int, default=8,
                    help="oracle steps after the prompt: the full-depth bit-identity check and the "
                         "CPU baseline (0: neither)")
    ap.add_argument("--decode-exact", type=int, default=64,
                    help="EXACT-mode decode steps timed and compared with FAST's ids (< 2: none)")
    ap.add_argument("--no-prefill-timing", action="store_true",
                    help="skip the batched-vs-stepwise prefill timing of the decode sections")
    ap.add_argument("--decode-eager", action="store_true",
                    help="decode steps launch by launch instead of graph replays (for kernel traces)")
    ap.add_argument("--no-gemm", action="store_true", help="skip the batched GEMM (config 4) lines")
    ap.add_argument("--series-eager", action="store_true",
                    help="per-shape and config-0 series launched one by one (kernel traces only)")
    ap.add_argument("--no-large-gemv", action="store_true",
                    help="skip the lm_head-shaped v4 GEMV line (165 MB per launch)")
    ap.add_argument("--prefill-trace", type=int, default=0, metavar="LAYERS",
                    help="only: build the config-3 model with LAYERS layers and run four FAST prefills "
                         "of --decode-prompt tokens (for kernel traces), then exit")
    args = ap.parse_args()

    global SERIES_EAGER
    SERIES_EAGER = args.series_eager
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build "
              "(the single-GPU kernel is the unit of work; see the sharding design notes).",
              file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2
    sections = {"per_shape", "cfg0", "large_gemv", "gemm", "decode", "decode_dense"}
    if args.only:
        want = {w.strip() for w in args.only.split(",") if w.strip()} - {"none"}
        bad = want - sections
        if bad:
            print(f"--only: unknown sections {sorted(bad)}", file=sys.stderr)
            return 2
        sections = want
    if args.no_decode:
        sections -= {"decode", "decode_dense"}
    if args.no_gemm:
        sections.discard("gemm")
    if args.no_large_gemv:
        sections.discard("large_gemv")

    import numpy as np

    import wpcg
    from wpcg import synth

    if args.prefill_trace:
        return prefill_trace(wpcg, synth, args.prefill_trace, args.decode_prompt)

    scheme = args.scheme
    mode = wpcg.MODE_EXACT if args.mode == "exact" else wpcg.MODE_FAST
    log(f"generating v{scheme} blocks for the seven Qwen3-4B shapes (xoshiro256++, seed "
        f"{synth.WPC_SEED:#x}, the configs' PRNG)")
    blocks = [synth.wpc_blocks(scheme, r, c, matrix_id=1 + i) for i, (_, r, c) in enumerate(QWEN3_4B)]
    xs = {c: synth.wpc_x(c) for c in sorted({c for _, _, c in QWEN3_4B})}

    ctx = wpcg.Context(0)
    fast_kernel = wpcg.FAST_KERNEL_VALU if args.fast_kernel == "valu" else wpcg.FAST_KERNEL_MFMA
    base = [wpcg.WpcLinear.from_blocks(ctx, scheme, b, r, c).set_fast_kernel(fast_kernel)
            for b, (_, r, c) in zip(blocks, QWEN3_4B)]
    step_bytes = sum(gemv_bytes(r, c, scheme) for _, r, c in QWEN3_4B)
    weight_bytes = sum(l.device_bytes() for l in base)
    copies = max(1, int(np.ceil(args.min_bytes / weight_bytes)))
    log(f"layer weights {weight_bytes / 1e6:.1f} MB; {copies} device copies "
        f"({copies * weight_bytes / 1e9:.2f} GB rotated)")
    sets = [base] + [[l.clone() for l in base] for _ in range(copies - 1)]
    xb = {c: ctx.upload(x) for c, x in xs.items()}
    yb = {name: ctx.alloc(4 * r) for name, r, _ in QWEN3_4B}
    names = [n for n, _, _ in QWEN3_4B]

    def step_launches(s):
        """One step's launches: q/k/v share their input and one launch, as do
        gate/up; o and down run alone (their inputs come from other ops)."""
        L = dict(zip(names, s))
        return [
            lambda: wpcg.matvec_multi([L["q_proj"], L["k_proj"], L["v_proj"]], [xb[2560]] * 3,
                                      [yb["q_proj"], yb["k_proj"], yb["v_proj"]]),
            lambda: L["o_proj"].matvec_dev(xb[4096], yb["o_proj"]),
            lambda: wpcg.matvec_multi([L["gate_proj"], L["up_proj"]], [xb[2560]] * 2,
                                      [yb["gate_proj"], yb["up_proj"]]),
            lambda: L["down_proj"].matvec_dev(xb[9728], yb["down_proj"]),
        ]

    def one_step(i):
        for fn in step_launches(sets[i % copies]):
            fn()

    def launch_durations(rounds):
        """Average device duration of one launch, from an event pair recorded
        on the launch's own stream right before and after it."""
        evs = [(ctx.event(), ctx.event()) for _ in range(4 * len(sets))]
        total, n = 0.0, 0
        for _ in range(rounds):
            k = 0
            for s in sets:
                for fn in step_launches(s):
                    a, b = evs[k]
                    k += 1
                    a.record()
                    fn()
                    b.record()
            ctx.sync()
            for a, b in evs:
                total += a.elapsed_ms(b)
                n += 1
        return total / n * 1e3, n

    def measure(mode, steps, warmup):
        """Exactly `warmup` untimed steps, then exactly `steps` timed ones."""
        for s in sets:
            for l in s:
                l.set_mode(mode)
        run, warm, graphs = rotation_runner(ctx, copies, one_step)
        warm()
        run(warmup)
        if steps % copies:
            run(steps % copies)  # capture the remainder graph outside the timed region
        ctx.sync()
        e0, e1 = ctx.event(), ctx.event()
        e0.record()
        run(steps)
        e1.record()
        ctx.sync()
        ms = e0.elapsed_ms(e1)
        graphs.clear()
        n_launch = steps * (4 if mode == wpcg.MODE_FAST else len(QWEN3_4B))
        return step_bytes * steps / (ms / 1e3) / 1e9, ms, ms * 1e3 / n_launch, n_launch

    if args.pmc_pass:
        # short run for hardware-counter passes: a few rotations of the FAST
        # steps, then one plain copy kernel of known size (the calibration of
        # the FETCH_SIZE / WRITE_SIZE counters against a known byte count)
        for s in sets:
            for l in s:
                l.set_mode(mode)
        for _ in range(4):
            for i in range(copies):
                one_step(i)
        ctx.sync()
        n = 256 << 20  # bytes read and bytes written by the copy kernel
        src, dst = ctx.alloc(n), ctx.alloc(n)
        wpcg.check(wpcg.lib.wpcg_memcpy_d2d(ctx.h, dst.ptr, src.ptr, n))
        ctx.sync()
        log(f"pmc pass: {4 * copies} steps, then one device copy of {n} bytes "
            "(the runtime's copy kernel)")
        return 0

    other = "exact" if args.mode == "fast" else "fast"
    log(f"timing {other} mode ({copies} steps)")
    o_val = measure(wpcg.MODE_EXACT if other == "exact" else wpcg.MODE_FAST, copies, copies)[0]
    log(f"{other}: {o_val:.1f} GB/s ({100 * o_val / PEAK_GBPS:.1f}% of peak)")
    log(f"timing {args.mode} mode: {args.warmup} warm-up steps, {args.steps} timed steps")
    value, ms, avg_launch_us, n_launch = measure(mode, args.steps, args.warmup)
    steps = args.steps
    log(f"{args.mode}: {value:.1f} GB/s ({100 * value / PEAK_GBPS:.1f}% of peak), "
        f"{ms / steps * 1e3:.2f} us/step, {n_launch} launches, avg {avg_launch_us:.2f} us")
    # The graphs replay the launches back to back on one stream, so the
    # event-timed region divided by the launches is the kernel's average
    # launch duration (inter-kernel gaps included; rocprofv3's kernel trace
    # of the same command gives the same average within a few percent).
    dur_us = avg_launch_us
    launch_bytes = step_bytes / (n_launch // steps)
    achieved = launch_bytes / dur_us / 1e3
    eager_us, n_eager = launch_durations(max(1, -(-100 // copies)))
    log(f"avg launch {dur_us:.2f} us -> {achieved:.1f} GB/s per launch; eager launches between "
        f"event pairs: {eager_us:.2f} us ({n_eager} launches, dispatch latency included)")

    cpu = None
    if not args.no_cpu_baseline:
        log(f"CPU baseline (~{1.5 * args.cpu_seconds:.0f} s)")
        cpu = cpu_gemv_baseline(scheme, QWEN3_4B, blocks, xs, args.cpu_seconds,
                                f"passes over the seven Qwen3-4B v{scheme} matrices")
        log(f"CPU baseline {cpu['value']} GB/s on {cpu['cores']} threads, {cpu['one_core_value']} on 1")

    for lst in sets:  # free the rotated GEMV copies first
        for l in lst:
            l.close()
    cpu_budget = 0 if args.no_cpu_baseline else args.cpu_seconds / 2
    per_shape = per_shape_bench(ctx, wpcg, scheme, QWEN3_4B, blocks, xs, args.min_bytes, fast_kernel) \
        if "per_shape" in sections else None
    cfg0 = cfg0_bench(ctx, wpcg, synth, args.min_bytes, cpu_budget, fast_kernel) if "cfg0" in sections else None
    large = large_gemv_bench(ctx, wpcg, synth) if "large_gemv" in sections else None
    gemm = gemm_bench(ctx, wpcg, synth, not args.no_cpu_baseline) if "gemm" in sections else None
    cpu_tokens = 0 if args.no_cpu_baseline else args.decode_cpu_tokens
    decode = decode_bench(ctx, wpcg, synth, "decode", args.decode_prompt, args.decode_new, cpu_tokens,
                          args.decode_eager, args.decode_exact, not args.no_prefill_timing) \
        if "decode" in sections else None
    decode_dense = decode_bench(ctx, wpcg, synth, "decode_dense", args.dense_prompt, args.decode_new,
                                cpu_tokens, args.decode_eager, args.decode_exact, not args.no_prefill_timing) \
        if "decode_dense" in sections else None

    kname = f"k_gemv_exact<{scheme}>" if mode == wpcg.MODE_EXACT else \
        f"k_gemv_valu<{scheme}>" if fast_kernel == wpcg.FAST_KERNEL_VALU else f"k_gemv_fast<{scheme}, 0, 0, 4>"
    rec = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": ("synthetic, the configs' PRNG (xoshiro256++ seeded 0x12345678 as wpc-eval/src/main.rs:77-82, "
                 "Box-Muller in f32; one stream per matrix row): codes uniform, zp f16(N(-0.03,0.005)), "
                 "scale f16(U(0.002,0.006)), x N(0,1)"),
        "config": {
            "workload": (f"cfg1: v{scheme} dequant-GEMV batch 1 over the seven Qwen3-4B layer shapes "
                         f"(q/k/v/o/gate/up/down) in 4 launches per step, HBM-cold over {copies} rotated "
                         f"copies"),
            "scheme": f"v{scheme}",
            "mode": args.mode,
            "fast_kernel": args.fast_kernel,
            "bytes_per_step": step_bytes,
            "pct_of_peak": round(100 * value / PEAK_GBPS, 2),
            "launches_per_step": n_launch // steps,
            f"{other}_mode_gbps": round(o_val, 2),
            "per_shape": per_shape,
            "cfg0": cfg0,
            "decode": decode,
            "decode_dense": decode_dense,
            "gemm": gemm,
            "large_gemv": large,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": kname,
            "achieved": round(achieved, 2),
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBPS, 4),
            "avg_launch_us": round(dur_us, 3),
            "eager_launch_us": round(eager_us, 3),
            "algorithmic_bytes_per_launch": round(launch_bytes),
            "traffic": TRAFFIC.get((scheme, args.mode)),
            "traffic_source": TRAFFIC_SOURCE if (scheme, args.mode) in TRAFFIC else None,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    try:
        rc = main()
    except BaseException:  # noqa: B902  (report, then leave through the same exit)
        import traceback
        traceback.print_exc()
        rc = 1
    _w = sys.modules.get("wpcg")
    if _w is not None and _w.gpu_used():
        if "--normal-exit" in sys.argv:
            _w.NORMAL_EXIT = True
        rc = _w.finish(rc)  # see wpcg.NORMAL_EXIT
    sys.exit(rc)
