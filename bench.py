#!/usr/bin/env python3
"""Benchmark: BASELINE configs[3] on one MI355X.

Workload (one "step"): the 2B hybrid (24 layers, 3:1 gated-delta-net : attention, int4 group-32
weights, random init, vocab 151936) encodes a 512-token state of uniform-random ids once
(Engine::forward with keep), then answers 3 questions of 40 random tokens each from the state's
snapshot (2, 3 and 5 option rows + the last row), the pointer head scoring each.  That is the
reference's Decider::ask_all (src/lib.rs:183-199) on token ids; the three question forwards run as
independent sequences of one batched forward (the same results as three forwards), and the head
(src/head.rs:55-77, f64) runs on the device after it.

Reported: `value` = prefill tokens/s (512-token state forwards), `ms_per_step` = ask_all latency
(state prefill + 3 questions + head), plus the per-phase times (questions_ms: the batched question
forward with the pointer head on the device), the roofline of the dominant kernel
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


GEMM_LABELS = ("in_proj", "out_proj", "qkv", "o_proj", "gate_up", "down")
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "gemm_w4_prefill_512_traffic.txt")


def gemm_shapes(cfg):
    """(label, N, K) of every int4 GEMM launch of one forward, in plan order (src/engine.rs:475-518)."""
    import sdamd.synth as synth
    d, inter = cfg["hidden_size"], cfg["intermediate_size"]
    H, dv = cfg["linear_num_key_heads"], cfg["linear_value_head_dim"]
    hq, hd = cfg["num_attention_heads"], cfg["head_dim"]
    out = []
    for kind in cfg["layer_types"]:
        if kind == "linear_attention":
            out += [("in_proj", synth.in_proj_rows(cfg), d), ("out_proj", d, H * dv)]
        else:
            out += [("qkv", synth.qkv_rows(cfg), d), ("o_proj", d, hq * hd)]
        out += [("gate_up", 2 * inter, d), ("down", d, inter)]
    return out


def read_traffic():
    """HBM bytes per GEMM launch from the committed rocprofv3 counter summary, or None."""
    try:
        with open(TRAFFIC_SUMMARY) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def gemm_roofline(eng, state, cfg, reps=5):
    """The prefill int4 GEMM (k_gemm_w4, M = 512) inside the engine's own 512-token forward: each
    GEMM is one launch whose own start and end HIP records into a pair of events on the engine's
    stream (hipExtLaunchKernel, Engine.profile).  achieved = algorithmic flops per launch / average
    launch duration."""
    shapes = gemm_shapes(cfg)
    M = len(state)
    total_ms = []
    for _ in range(reps):
        prof = dict(eng.profile(state))
        total_ms.append(sum(prof[k] for k in GEMM_LABELS))
    ms = statistics.median(total_ms)
    launches = len(shapes)
    avg_s = ms / 1e3 / launches
    flops = sum(2.0 * M * N * K for _, N, K in shapes) / launches
    achieved = flops / avg_s / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_MFMA_F16, "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_MFMA_F16, 4), "traffic": read_traffic(),
            "kernel": "k_gemm_w4 (int4 g32 fused-dequant MFMA GEMM, prefill M=512, the 2B's 96 GEMMs)",
            "avg_launch_us": round(avg_s * 1e6, 2), "flops_per_launch": flops,
            "algorithmic_bytes_per_launch": sum(N * K // 2 + N * K // 16 + 2 * M * K + 2 * M * N
                                                for _, N, K in shapes) / launches,
            "launches_timed": launches * reps}


def pmc_workload(eng, state):
    """What the rocprofv3 counter runs profile: a plain copy kernel of known size (torch.neg over
    256 MiB of f32: 256 MiB read + 256 MiB written), then one eager 512-token forward."""
    import torch
    n = 64 << 20
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    eng.profile(state)
    torch.cuda.synchronize()
    log(f"pmc workload done: copy kernel of {4 * n} bytes each way, one {len(state)}-token forward")


def traffic_summary(fetch_dir, write_dir, cfg, state_len):
    """Reads the per-dispatch FETCH_SIZE and WRITE_SIZE (KiB) of the two counter runs, scales each
    by the ratio of the copy kernel's known bytes to its counter reading, and prints the summary
    that read_traffic() parses."""
    import csv
    import glob

    def per_kernel(d, counter):
        rows = []
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as f:
                for r in csv.DictReader(f):
                    if r["Counter_Name"] == counter:
                        rows.append((r["Kernel_Name"], float(r["Counter_Value"])))
        if not rows:
            raise SystemExit(f"no {counter} rows under {d}")
        copy = [v for k, v in rows if "neg_kernel" in k]
        gemm = [v for k, v in rows if "k_gemm_w4" in k]
        if not copy or not gemm:
            raise SystemExit(f"{counter}: copy kernel or GEMM dispatches missing under {d}")
        return statistics.median(copy), sum(gemm) / len(gemm), len(gemm)

    copy_bytes = 4 * (64 << 20)
    fc, fg, nf = per_kernel(fetch_dir, "FETCH_SIZE")
    wc, wg, nw = per_kernel(write_dir, "WRITE_SIZE")
    kf, kw = copy_bytes / (fc * 1024), copy_bytes / (wc * 1024)
    traffic = fg * 1024 * kf + wg * 1024 * kw
    shapes = gemm_shapes(cfg)
    alg = sum(N * K // 2 + N * K // 16 + 2 * state_len * K + 2 * state_len * N for _, N, K in shapes) / len(shapes)
    print(f"# HBM traffic of k_gemm_w4 in one eager {state_len}-token prefill of the 2B (rocprofv3 --pmc)")
    print("# commands (R = repository root, run from /tmp):")
    print("#   rocprofv3 --pmc FETCH_SIZE --output-format csv -d FETCH_DIR -o run -- python3 $R/bench.py --pmc-workload")
    print("#   rocprofv3 --pmc WRITE_SIZE --output-format csv -d WRITE_DIR -o run -- python3 $R/bench.py --pmc-workload")
    print("#   python3 $R/bench.py --traffic-summary FETCH_DIR WRITE_DIR")
    print(f"# copy kernel (torch.neg, {copy_bytes} B each way): FETCH_SIZE {fc:.1f} KiB -> factor {kf:.4f}; "
          f"WRITE_SIZE {wc:.1f} KiB -> factor {kw:.4f}")
    print(f"# k_gemm_w4: {nf} dispatches, mean FETCH_SIZE {fg:.1f} KiB, mean WRITE_SIZE {wg:.1f} KiB")
    print(f"# algorithmic bytes per launch (weights + scales + A + Y as f16): {alg:.0f}")
    print(f"fetch_bytes_per_launch: {fg * 1024 * kf:.0f}")
    print(f"write_bytes_per_launch: {wg * 1024 * kw:.0f}")
    print(f"traffic_bytes_per_launch: {traffic:.0f}")


def trace_summary(trace_dir):
    """Per-kernel totals of a `rocprofv3 --kernel-trace` run of this script, then the kernels of the
    last state prefill and of the last batched question forward, then the GEMM launches of the
    roofline's eager forwards.  Each forward starts with one k_embed launch; the forwards of a step
    alternate prefill, questions; the roofline's forwards follow a marker kernel of torch's."""
    import csv
    import glob
    rows = []
    for path in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        with open(path) as f:
            for r in csv.DictReader(f):
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    if not rows:
        raise SystemExit(f"no kernel_trace.csv under {trace_dir}")
    rows.sort()

    import re

    def short(name):
        """k_gemm_w4<4,3,false,false> from the (demangled or mangled) kernel name."""
        m = re.match(r"_ZN2sd12_GLOBAL__N_1(\d+)", name)
        if m:  # mangled: length-prefixed name, then I<template args>E of integer/bool literals
            n = int(m.group(1))
            base = name[m.end():m.end() + n]
            rest = name[m.end() + n:]
            if rest.startswith("I"):
                args = re.findall(r"L([ib])(\d+)E", rest[:rest.find("EE") + 2])
                base += "<" + ",".join(v if t == "i" else ("true" if v == "1" else "false") for t, v in args) + ">"
            return base
        name = name.replace("void ", "").replace("sd::(anonymous namespace)::", "")
        return name.split("(")[0]

    def table(rs, title):
        agg = {}
        for s, e, k in rs:
            a = agg.setdefault(short(k), [0, 0.0])
            a[0] += 1
            a[1] += (e - s) / 1e3
        busy = sum(v[1] for v in agg.values())
        print(title)
        print(f"  {'kernel':44s} {'calls':>6s} {'total us':>10s} {'avg us':>8s} {'%':>6s}")
        for k, (n, us) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
            print(f"  {k:44s} {n:6d} {us:10.1f} {us / n:8.2f} {100 * us / busy:6.2f}")
        return busy

    table(rows, "# per-kernel totals over the whole run")

    def is_marker(name):
        return "at::native" in name or name.startswith("_ZN2at6native")

    mark = next((i for i, r in enumerate(rows) if is_marker(r[2])), len(rows))
    steps_rows, roof_rows = rows[:mark], [r for r in rows[mark:] if not is_marker(r[2])]
    starts = [i for i, r in enumerate(steps_rows) if "k_embed" in r[2]]
    fwd = [steps_rows[a:b] for a, b in zip(starts, starts[1:] + [len(steps_rows)])]
    for kind, idx in (("state prefill", range(0, len(fwd), 2)), ("batched question forward", range(1, len(fwd), 2))):
        idx = list(idx)
        if not idx:
            continue
        f = fwd[idx[-1]]
        print()
        span = (f[-1][1] - f[0][0]) / 1e3
        busy = table(f, f"# one {kind} (last of {len(idx)}): {len(f)} kernels, first start to last end "
                        f"{span:.1f} us")
        print(f"  kernel busy {busy:.1f} us, gaps {span - busy:.1f} us")
        g = [(e - s) / 1e3 for s, e, k in f if "k_gemm_w4" in k]
        if g:
            print(f"  k_gemm_w4 launches in this forward: {len(g)}, average duration {sum(g) / len(g):.2f} us")
    g = [(e - s) / 1e3 for s, e, k in roof_rows if "k_gemm_w4" in k]
    if g:
        n_fwd = sum(1 for r in roof_rows if "k_embed" in r[2])
        print()
        print(f"# roofline: the GEMM launches of its {n_fwd} eager {STATE_LEN}-token forwards (Engine.profile)")
        print(f"  k_gemm_w4 launches: {len(g)}, average duration {sum(g) / len(g):.2f} us")


def _dev(a):
    """numpy array -> device bytes (torch is only the allocator)."""
    import numpy as np
    import torch
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.uint8).reshape(-1).copy()).cuda()


def _timed(fn, reps):
    """Average device ms of fn() over reps calls on torch's current stream (after one warm-up)."""
    import torch
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / reps


def kernel_bench(pkg, reps=50):
    """BASELINE configs[0..2] as kernel-level measurements (parity for them is in tests/): the int4
    GEMM on one linear layer, the GEMM set of one decoder layer at M = 512 and M = 8, and one gated
    delta net layer.  Weights are repacked once (sd_op_repack_w4), as the engine does at load."""
    import numpy as np
    import torch
    import sdamd.synth as synth
    stream = torch.cuda.current_stream().cuda_stream
    rng = np.random.default_rng(0)
    out = {"metric": "kernel-level configs[0..2] (int4 GEMM, layer GEMM set, gated delta net layer), 1 GPU",
           "unit": "us", "data": "synthetic (BASELINE configs distributions, seed 0)"}

    def gemm(M, N, K):
        A = rng.standard_normal((M, K)).astype(np.float16)
        W = synth.pack_nibbles(rng.integers(0, 16, size=(N, K), dtype=np.uint32))
        S = rng.uniform(0.005, 0.02, size=(N, K // 32)).astype(np.float16)
        dA, dW, dS = _dev(A), _dev(W), _dev(S)
        dY = torch.empty(M * N * 2, dtype=torch.uint8, device="cuda")
        pkg.op_repack_w4(dW.data_ptr(), dS.data_ptr(), N, K, stream)
        exact = M <= 20
        ms = _timed(lambda: pkg.op_matmul(dA.data_ptr(), dW.data_ptr(), dS.data_ptr(), dY.data_ptr(), M, N, K, exact,
                                          -1, True, stream), reps)
        wbytes = N * K // 2 + N * K // 16
        io = 2 * M * K + 2 * M * N
        return {"M": M, "N": N, "K": K, "us": round(ms * 1e3, 2),
                "tflops": round(2.0 * M * N * K / ms / 1e9, 1),
                "mfma_frac": round(2.0 * M * N * K / ms / 1e9 / PEAK_MFMA_F16, 4),
                "gbps": round((wbytes + io) / ms / 1e6, 1),
                "hbm_frac": round((wbytes + io) / ms / 1e6 / PEAK_HBM, 4)}

    out["cfg0_linear"] = gemm(128, 6144, 2048)
    layer = [("q", 2048, 2048), ("k", 512, 2048), ("v", 512, 2048), ("o", 2048, 2048), ("gate", 6144, 2048),
             ("up", 6144, 2048), ("down", 2048, 6144)]
    fused = [("qkv", 5120, 2048), ("in_proj", 8256, 2048), ("gate_up", 12288, 2048), ("o", 2048, 2048),
             ("down", 2048, 6144)]
    for M in (512, 8):
        rs = {name: gemm(M, N, K) for name, N, K in layer}
        tot_us = sum(r["us"] for r in rs.values())
        flops = sum(2.0 * M * N * K for _, N, K in layer)
        wbytes = sum(N * K // 2 + N * K // 16 for _, N, K in layer)
        out[f"cfg1_layer_M{M}"] = {"shapes": rs, "total_us": round(tot_us, 2),
                                   "tflops": round(flops / tot_us / 1e6, 1),
                                   "mfma_frac": round(flops / tot_us / 1e6 / PEAK_MFMA_F16, 4),
                                   "weight_gbps": round(wbytes / tot_us / 1e3, 1),
                                   "hbm_frac": round(wbytes / tot_us / 1e3 / PEAK_HBM, 4)}
        if M == 512:
            out["cfg1_fused_M512"] = {name: gemm(M, N, K) for name, N, K in fused}
            # the vendor library's f16 GEMM (torch.matmul -> hipBLASLt) on the same shapes, with f16
            # weights (4x the weight bytes, no dequant): what the hardware gives a plain GEMM here
            for name, N, K in fused:
                a16 = torch.randn(M, K, dtype=torch.float16, device="cuda")
                b16 = torch.randn(N, K, dtype=torch.float16, device="cuda")
                ms = _timed(lambda: torch.matmul(a16, b16.t()), reps)
                out["cfg1_fused_M512"][name]["hipblaslt_f16_us"] = round(ms * 1e3, 2)
    # one gated delta net layer (prep + scan), T = 512, 16 heads, dk = dv = 128
    T, H, dk, dv = 512, 16, 128, 128
    C = 2 * H * dk + H * dv
    qkv = rng.standard_normal((T, C)).astype(np.float32)
    for j in range(2 * H):  # q and k rows L2-normalized per head (the kernel normalizes again)
        blk = qkv[:, j * dk:(j + 1) * dk]
        blk /= np.linalg.norm(blk, axis=1, keepdims=True)
    big = np.zeros((T, 2 * H), np.float16)
    big[:, :H] = rng.standard_normal((T, H)).astype(np.float16)   # a: g = -softplus(a)
    big[:, H:] = rng.standard_normal((T, H)).astype(np.float16)   # b: beta = sigmoid(b)
    d_qkv, d_big = _dev(qkv), _dev(big)
    d_nA, d_dtb = _dev(np.full(H, -1.0, np.float32)), _dev(np.zeros(H, np.float32))
    d_state = torch.zeros(H * dk * dv, dtype=torch.float32, device="cuda")
    d_o = torch.empty(T * H * dv, dtype=torch.float32, device="cuda")
    ms = _timed(lambda: pkg.op_gdn(d_qkv.data_ptr(), d_big.data_ptr(), 2 * H, 0, H, d_nA.data_ptr(), d_dtb.data_ptr(),
                                   T, H, dk, dv, d_state.data_ptr(), 0, d_o.data_ptr(), stream), reps)
    alg = 4 * T * H * (2 * dk + dv) + 8 * T * H + 4 * T * H * dv + 4 * H * dk * dv
    out["cfg2_gdn_layer"] = {"T": T, "H": H, "us": round(ms * 1e3, 2), "algorithmic_bytes": alg,
                             "gbps": round(alg / ms / 1e6, 1), "hbm_frac": round(alg / ms / 1e6 / PEAK_HBM, 4),
                             "recurrent_equiv_tflops": round(7.0 * T * H * dk * dv / ms / 1e9, 2)}
    return out


def sweep_bench(eng, head, temp, n_states=64, n_q=8, seed=4):
    """64 independent states of U[128, 2048] random tokens, each encoded once
    (forward with keep), then 8 questions of U[24, 64] tokens answered from its snapshot as one
    batched forward with the device head.  Aggregate prefill tokens/s; per-question latency = the
    wall time of the batch that answers it.  A first pass over the same inputs builds the per-length
    plans (captured graphs) and is reported separately as the cold pass."""
    import numpy as np
    import sdamd.synth as synth
    rng = np.random.default_rng(seed)
    work = []
    for _ in range(n_states):
        L = int(rng.integers(128, 2049))
        state = rng.integers(0, synth.VOCAB_2B, L).astype(np.uint32)
        qs = [rng.integers(0, synth.VOCAB_2B, int(rng.integers(24, 65))).astype(np.uint32) for _ in range(n_q)]
        opts = [sorted(rng.choice(len(q) - 1, int(rng.integers(2, 6)), replace=False).tolist()) for q in qs]
        work.append((state, qs, opts))

    def run_pass():
        pre_tok, pre_s, q_lat = 0, 0.0, []
        for state, qs, opts in work:
            t0 = time.perf_counter()
            snap = eng.forward(state, [], keep=True).snapshot
            t1 = time.perf_counter()
            eng.ask_batch(head, qs, opts, [temp] * n_q, cache=snap)
            t2 = time.perf_counter()
            snap.free()
            pre_tok += len(state)
            pre_s += t1 - t0
            q_lat.extend([t2 - t1] * n_q)
        q_lat.sort()
        return pre_tok / pre_s, q_lat

    t = time.perf_counter()
    cold_rate, _ = run_pass()
    log(f"sweep cold pass (plans built) in {time.perf_counter() - t:.1f} s")
    rate, q_lat = run_pass()
    return {"metric": "configs[4] sweep: aggregate prefill tokens/s, per-question latency p50/p99 (ms)",
            "prefill_tokens_per_s": round(rate, 1), "cold_pass_prefill_tokens_per_s": round(cold_rate, 1),
            "states": n_states, "questions_per_state": n_q,
            "question_p50_ms": round(1e3 * q_lat[len(q_lat) // 2], 3),
            "question_p99_ms": round(1e3 * q_lat[min(len(q_lat) - 1, int(0.99 * len(q_lat)))], 3),
            "data": "synthetic: random-init 2B, uniform-random ids; lengths U[128, 2048], questions U[24, 64], "
                    "2-5 options each"}


def cpu_baseline(model_dir, vocab, n_tokens=STATE_LEN):
    """The C oracle (a CPU port of the reference kernels) on the host cores: one prefill of
    n_tokens random ids (the 512-token state of the workload; about 15-20 s on 16 cores)."""
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
    ap.add_argument("--pmc-workload", action="store_true",
                    help="run only the workload of the rocprofv3 counter runs (copy kernel + one prefill)")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="print the HBM traffic summary from two rocprofv3 --pmc output folders (no GPU)")
    ap.add_argument("--trace-summary", metavar="TRACE_DIR",
                    help="print the kernel summary of a rocprofv3 --kernel-trace output folder (no GPU)")
    ap.add_argument("--kernels", action="store_true",
                    help="kernel-level BASELINE configs[0..2] instead of the ask_all workload (one JSON line)")
    ap.add_argument("--sweep", action="store_true",
                    help="BASELINE configs[4] (64 states, 8 questions each) instead of the ask_all workload")
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return
    if args.traffic_summary:
        import __graft_entry__ as entry
        entry._import_pkg()
        import sdamd.synth as synth
        traffic_summary(*args.traffic_summary, synth.CONFIG_2B, STATE_LEN)
        return
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
    if args.kernels:
        print(json.dumps(kernel_bench(pkg)), flush=True)
        return

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
    if args.pmc_workload:
        pmc_workload(eng, state)
        return
    if args.sweep:
        print(json.dumps(sweep_bench(eng, head, temp)), flush=True)
        return

    def step():
        t0 = time.perf_counter()
        out = eng.forward(state, [], keep=True, timed=True)
        t1 = time.perf_counter()
        snap = out.snapshot
        # the questions continue from the snapshot as independent sequences of one batched forward,
        # the pointer head runs on the device behind it
        probs, qgpu = eng.ask_batch(head, questions, OPTIONS, [temp] * N_QUESTIONS, cache=snap, timed=True)
        t2 = time.perf_counter()
        snap.free()
        return t1 - t0, t2 - t1, out.gpu_ms, [qgpu], probs

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
        "questions_ms": round(1e3 * statistics.mean(qs), 3),
        "questions_gpu_ms": round(statistics.mean(q_gpu), 3),
        "probs_last_step": [[round(float(x), 5) for x in p] for p in probs],
    }
    if args.profile:
        prof = eng.profile(state)
        res["profile_prefill_ms"] = {k: round(v, 4) for k, v in prof}
        prof_q = eng.profile(questions[0])
        res["profile_question_ms"] = {k: round(v, 4) for k, v in prof_q}
    if not args.no_roofline:
        # a marker kernel of torch's separates the timed steps from the roofline's forwards in a
        # kernel trace of this script (see trace_summary)
        torch.ones(1, device="cuda")
        torch.cuda.synchronize()
        res["roofline"] = gemm_roofline(eng, state, synth.CONFIG_2B)
    if not args.no_cpu_baseline:
        eng.free()
        res["cpu_baseline"] = cpu_baseline(model_dir, synth.VOCAB_2B)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
