#!/usr/bin/env python3
"""Benchmark: BASELINE configs[3] on one MI355X.

Workload (one "step"): the 2B hybrid (24 layers, 3:1 gated-delta-net : attention, int4 group-32
weights, random init, vocab 151936) encodes a 512-token state of uniform-random ids once
(Engine::forward with keep), then answers 3 questions of 40 random tokens each from the state's
snapshot (2, 3 and 5 option rows + the last row), the pointer head scoring each.  That is the
reference's Decider::ask_all (src/lib.rs:183-199) on token ids.

Reported: `value` = prefill tokens/s (512-token state forwards), `ms_per_step` = ask_all latency
(state prefill + 3 questions + head), plus the per-phase times, the roofline of the dominant kernel
class (the prefill int4 GEMM, timed live with HIP events on the stream it runs on) and the CPU
baseline (the C oracle on the host cores, a bounded prefill sample of the same model).
"""
import argparse
import json
import os
import statistics
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

STATE_LEN, N_QUESTIONS, Q_LEN = 512, 3, 40
OPTIONS = [[3, 17], [5, 12, 30], [2, 9, 18, 27, 36]]
PEAK_MFMA_F16 = 2500.0   # TFLOP/s, MI355X dense fp16
PEAK_HBM = 8000.0        # GB/s


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemm_roofline(pkg, cfg, reps=20):
    """Average launch duration of the prefill GEMM kernel over the 2B's per-layer GEMM mix at
    M = 512, timed with HIP events on the stream the kernels are launched on."""
    import torch
    d, inter = cfg["hidden_size"], cfg["intermediate_size"]
    import sdamd.synth as synth
    n_gdn = sum(k == "linear_attention" for k in cfg["layer_types"])
    n_att = sum(k == "full_attention" for k in cfg["layer_types"])
    H, dv = cfg["linear_num_key_heads"], cfg["linear_value_head_dim"]
    hq, hd = cfg["num_attention_heads"], cfg["head_dim"]
    shapes = ([(synth.in_proj_rows(cfg), d), (d, H * dv)] * n_gdn + [(synth.qkv_rows(cfg), d), (d, hq * hd)] * n_att
              + [(2 * inter, d), (d, inter)] * (n_gdn + n_att))
    M = STATE_LEN
    uniq = sorted(set(shapes))
    bufs = {}
    for (N, K) in uniq:
        W = torch.randint(0, 2 ** 31, (N * K // 8,), dtype=torch.int32, device="cuda")
        S = (torch.rand(N * K // 32, device="cuda") * 0.01 + 0.005).half()
        bufs[(N, K)] = (W, S, torch.empty(M * N, dtype=torch.float16, device="cuda"))
    A = torch.randn(M * max(K for _, K in uniq), device="cuda").half()
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    def run():
        for (N, K) in shapes:
            W, S, Y = bufs[(N, K)]
            pkg.op_matmul(A.data_ptr(), W.data_ptr(), S.data_ptr(), Y.data_ptr(), M, N, K, False, -1, sp)

    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    launches = reps * len(shapes)
    avg_s = e0.elapsed_time(e1) / 1e3 / launches
    flops = sum(2.0 * M * N * K for N, K in shapes) / len(shapes)
    achieved = flops / avg_s / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_MFMA_F16, "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_MFMA_F16, 4), "traffic": None,
            "kernel": "k_gemm_w4<8,2,false> (prefill int4 GEMM, M=512)",
            "avg_launch_us": round(avg_s * 1e6, 2), "flops_per_launch": flops, "launches_timed": launches}


def cpu_baseline(model_dir, vocab, n_tokens=64):
    """The C oracle (a CPU port of the reference kernels) on the host cores: prefill of n_tokens."""
    import numpy as np
    from oracle import torso
    om = torso.OracleModel(model_dir)
    ids = np.random.default_rng(7).integers(0, vocab, n_tokens)
    t = time.perf_counter()
    om.forward(ids, [n_tokens - 1])
    dt = time.perf_counter() - t
    return {"value": round(n_tokens / dt, 3), "unit": "tokens/s", "cores": torso.lib().or_num_threads(),
            "kind": "port",
            "sample": f"prefill of {n_tokens} random tokens on the same 2B model ({dt:.1f} s of CPU time; "
                      f"the reference's wgpu/lavapipe path cannot be built here: no cargo, no Vulkan ICD)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--model-dir", default=os.path.join(tempfile.gettempdir(), "sd_bench_2b"))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-roofline", action="store_true")
    ap.add_argument("--profile", action="store_true", help="also print the per-kernel-label breakdown")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}): every state and question is independent, "
              "so more GPUs would each run their own requests; there is no multi-GPU path to measure.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import __graft_entry__ as entry
    pkg = entry._import_pkg()
    pkg.lib()
    import sdamd.synth as synth

    t = time.perf_counter()
    model_dir = synth.write_model(args.model_dir, synth.CONFIG_2B, vocab=synth.VOCAB_2B, seed=0)
    log(f"model ready in {time.perf_counter() - t:.1f} s: {model_dir}")
    t = time.perf_counter()
    eng, head, dcfg = pkg.load_decider(model_dir)
    log(f"{eng.adapter}: weights loaded in {time.perf_counter() - t:.1f} s")
    d = eng.hidden_size()
    rng = np.random.default_rng(2026)
    state = rng.integers(0, synth.VOCAB_2B, STATE_LEN).astype(np.uint32)
    questions = [rng.integers(0, synth.VOCAB_2B, Q_LEN).astype(np.uint32) for _ in range(N_QUESTIONS)]
    temp = float(dcfg["temperature"])

    def step():
        t0 = time.perf_counter()
        out = eng.forward(state, [], keep=True, timed=True)
        t1 = time.perf_counter()
        snap = out.snapshot
        qgpu, probs = [], []
        for q, opts in zip(questions, OPTIONS):
            o = eng.forward(q, opts + [Q_LEN - 1], cache=snap, timed=True)
            probs.append(head.probs(o.hidden, d, temp))
            qgpu.append(o.gpu_ms)
        t2 = time.perf_counter()
        snap.free()
        return t1 - t0, t2 - t1, out.gpu_ms, qgpu, probs

    for i in range(args.warmup):
        step()
        log(f"warmup {i + 1}/{args.warmup} done")
    torch.cuda.synchronize()
    pre, qs, pre_gpu, q_gpu = [], [], [], []
    t_start = time.perf_counter()
    for i in range(args.steps):
        a, b, g, qg, probs = step()
        pre.append(a)
        qs.append(b)
        pre_gpu.append(g)
        q_gpu.extend(qg)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    log(f"timed {args.steps} steps in {wall:.3f} s")
    ask = [a + b for a, b in zip(pre, qs)]
    value = STATE_LEN * len(pre) / sum(pre)
    res = {
        "metric": "prefill tokens/s + ask_all latency (ms), 2B hybrid, 512-tok state, 1 GPU",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * wall / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 x int4 (f32 accumulate; f32 recurrent state)",
        "data": "synthetic: random-init 2B weights (seed 0), uniform-random token ids",
        "config": {"workload": "configs[3]: 2B hybrid, 512-token state prefill + ask_all of 3 x 40-token questions",
                   "layers": 24, "hidden": d, "vocab": synth.VOCAB_2B, "state_tokens": STATE_LEN,
                   "questions": N_QUESTIONS, "question_tokens": Q_LEN, "options": [len(o) for o in OPTIONS]},
        "ask_all_ms": round(1e3 * statistics.mean(ask), 3),
        "ask_all_p50_ms": round(1e3 * statistics.median(ask), 3),
        "prefill_ms": round(1e3 * statistics.mean(pre), 3),
        "prefill_gpu_ms": round(statistics.mean(pre_gpu), 3),
        "question_ms": round(1e3 * statistics.mean(qs) / N_QUESTIONS, 3),
        "question_gpu_ms": round(statistics.mean(q_gpu), 3),
        "probs_last_step": [[round(float(x), 5) for x in p] for p in probs],
    }
    if args.profile:
        prof = eng.profile(state)
        res["profile_prefill_ms"] = {k: round(v, 4) for k, v in prof}
        prof_q = eng.profile(questions[0])
        res["profile_question_ms"] = {k: round(v, 4) for k, v in prof_q}
    if not args.no_roofline:
        res["roofline"] = gemm_roofline(pkg, synth.CONFIG_2B)
    if not args.no_cpu_baseline:
        eng.free()
        res["cpu_baseline"] = cpu_baseline(model_dir, synth.VOCAB_2B)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
