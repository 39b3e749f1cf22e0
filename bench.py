"""Benchmark of the MI355X attention + quantized-matmul hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

Prints ONE JSON line.  Workloads (synthetic seeded inputs of the named shapes,
random-init weights; all inputs resident in HBM before timing):

  lm_decode   (default) the full Qwen3-8B-shape batched CFG decode step on the
              ggml backend: 36 layers, hidden 4096, 32 q / 8 KV heads d128,
              FFN 12288, vocab 151936, Q8_0 weights (--wtype q6_k), f16 KV
              cache at 4096 x 2 sets.  value = 2 tokens / the GPU time of one
              step's HIP-graph replay (HIP events on the backend stream; inputs
              resident), wall_tok_s = the same with each step's host input
              uploads, launch and logits / hidden readback included; roofline = the
              step's largest kernel (the MLP gate_up GEMV with its RMS-norm
              prologue and SwiGLU epilogue) alone; step_roofline = the step's algorithmic bytes /
              its GPU time from HIP events on the backend stream.
  gemv_q8_0   Q8_0 decode GEMV: W 12288 x 4096 Q8_0, x [2 x 4096] f32 -> [2 x 12288]
              (one step = activation quantisation + GEMV).  8 weight copies
              (428 MB) rotate so the 256 MB Infinity Cache cannot hold them.
  fa_decode   GQA decode attention: B=2 (CFG), 32 q / 8 KV heads, D=128, KV 2048,
              Q f32, K/V f16, no mask.  16 K/V copies rotate (269 MB).

The roofline object times the dominant kernel (or the one call it belongs
to) alone: its launches are captured into a HIP graph and replayed between
HIP events on the stream they are launched on; the cpu_baseline object times
the in-repo C restatement of ggml-CPU arithmetic (oracle/, "port") on a
bounded sample.
"""
import argparse
import ctypes
import json
import os
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "LM decode tok/s (CFG B=2, Q8_0, KV 4096); DiT attn TFLOP/s; % roofline"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="lm_decode",
                    choices=["lm_decode", "gemv_q8_0", "fa_decode", "fa_prefill", "fa_dit", "gemm_q4_k",
                             "dit_block", "depth"])
    ap.add_argument("--wtype", default="q8_0", choices=["q8_0", "q6_k", "q5_k_m", "bf16"],
                    help="lm_decode weight type (q5_k_m: Q5_K with the bumped layers' V / down in Q6_K)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    return ap.parse_args()


def graph_time(torch, fn, n, reps=10):
    """Per-launch time of n launches of fn(i) captured into one HIP graph on a
    side stream, replayed reps times between HIP events on that stream (the
    launch gaps of a graph replay, as in the decode step)."""
    hip = ctypes.CDLL("libamdhip64.so")
    s = torch.cuda.Stream()
    st = ctypes.c_void_p(s.cuda_stream)
    with torch.cuda.stream(s):
        fn(0, st)
    torch.cuda.synchronize()
    assert hip.hipStreamBeginCapture(st, 2) == 0
    for i in range(n):
        fn(i, st)
    g = ctypes.c_void_p()
    assert hip.hipStreamEndCapture(st, ctypes.byref(g)) == 0
    ex = ctypes.c_void_p()
    assert hip.hipGraphInstantiate(ctypes.byref(ex), g, None, None, ctypes.c_size_t(0)) == 0
    assert hip.hipGraphLaunch(ex, st) == 0
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        assert hip.hipGraphLaunch(ex, st) == 0
        e1.record(s)
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e-3 / n)
    hip.hipGraphExecDestroy(ex)
    hip.hipGraphDestroy(g)
    return float(np.mean(ts)), float(np.min(ts))


def profile_value(name, key, conv=float):
    """A `key: value` line of the committed rocprofv3 summary profiles/<name>.md,
    or None."""
    p = ROOT / "profiles" / (name + ".md")
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith(key + ":"):
            return conv(line.split(":", 1)[1].strip())
    return None


def mfma_counters(name):
    """MFMA busy fraction and MFMA f16 FLOPs per launch of the profiled
    kernel(s), from the rocprofv3 PMC passes in profiles/<name>.md
    (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x 1024 SIMDs) and
    SQ_INSTS_VALU_MFMA_MOPS_F16 x 512)."""
    util = profile_value(name, "mfma_busy_frac")
    flops = profile_value(name, "mfma_f16_flops_per_launch")
    if util is None and flops is None:
        return None
    return {"mfma_busy_frac": util, "mfma_f16_flops_per_launch": flops, "source": "profiles/%s.md" % name}


def profile_traffic(name):
    """HBM bytes per launch of a kernel, from the committed rocprofv3 PMC
    summary profiles/<name>.md (its `traffic_bytes_per_launch:` line), or None."""
    p = ROOT / "profiles" / (name + ".md")
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1].strip())
    return None


def cpu_rate(fn, seconds):
    """Seconds per call of fn() over about `seconds` of repeated calls."""
    t0 = time.perf_counter()
    it = 0
    while time.perf_counter() - t0 < seconds or it == 0:
        fn()
        it += 1
    return (time.perf_counter() - t0) / it, it


def cpu_threads():
    """Threads the CPU baseline runs with: the CPUs this process may use
    (affinity mask, capped by OMP_NUM_THREADS), as the oracle's default."""
    import oracle

    return oracle.default_threads()


def half_threads():
    """The reference's default CPU thread count, hardware_concurrency() / 2
    (src/backend.h:25-31), within the CPUs this process may use."""
    return max(1, min((os.cpu_count() or 2) // 2, cpu_threads()))


def host_cpu():
    """The host CPU as lscpu reports it: model, sockets x physical cores per
    socket, threads per core, plus the logical CPUs online and this process's
    share."""
    import subprocess

    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass

    def num(k):
        v = info.get(k, "")
        return int(v) if v.isdigit() else None

    sockets, cps, tpc = num("Socket(s)"), num("Core(s) per socket"), num("Thread(s) per core")
    return {"model": info.get("Model name"), "sockets": sockets, "physical_cores": sockets * cps if sockets and cps
            else None, "threads_per_core": tpc, "logical_cpus": os.cpu_count(), "process_cpus": cpu_threads()}


def via_backend(pkg, make, reps=20):
    """The same op through the ggml-backend boundary: a graph of n_ops
    independent nodes of it (one per rotated input copy) built with the ggml
    API and run by ggml_backend_graph_compute on the MI355X backend.  make(og)
    creates the tensors and ops on the OpGraph og and returns (outputs, n_ops,
    upload) where upload() sets the inputs after allocation.  Reported: GPU
    time per op of the replayed graph (HIP events on the backend stream) and
    the host wall clock per op of graph_compute + synchronize."""
    import importlib

    og_mod = importlib.import_module(pkg.__name__ + ".opgraph")
    og = og_mod.OpGraph(n_tensors=256)
    try:
        outs, n_ops, upload = make(og)
        og.build(outs)
        upload()
        for _ in range(3):  # eager, captured, first replay
            og.compute()
        og.synchronize()
        og.gpu_time(reset=True)
        t0 = time.perf_counter()
        for _ in range(reps):
            og.compute()
        og.synchronize()
        wall = (time.perf_counter() - t0) / reps
        ms, n = og.gpu_time()
        replays, eager = og.graph_stats()
    finally:
        og.close()
    return {"path": "ggml_backend_graph_compute, MI355X backend, HIP-graph replay", "ops_per_graph": n_ops,
            "gpu_us_per_op": round(ms / max(n, 1) * 1e3 / n_ops, 3), "wall_us_per_op": round(wall * 1e6 / n_ops, 3),
            "replays": replays, "eager": eager}


def bench_gemv(args, torch, pkg):
    import oracle

    mm, synth = pkg.mmhip, pkg.synth
    N, K, M = 12288, 4096, 2
    copies = 8
    Ws = [mm.QuantWeight.from_gguf(mm.Q8_0, synth.gguf_blocks_torch(mm.Q8_0, N, K, 1002 + c), N, K)
          for c in range(copies)]
    x = torch.from_numpy(synth.normal_np((M, K), 1003)).cuda()
    y = torch.empty((M, N), device="cuda")
    L = mm.load()
    ws = torch.empty(L.mmhip_mul_mat_workspace(mm.Q8_0, N, K, M), dtype=torch.uint8, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def step(i):
        W = Ws[i % copies]
        rc = L.mmhip_mul_mat(mm.Q8_0, ctypes.c_void_p(W.data.data_ptr()), N, K, W.row_bytes,
                             ctypes.c_void_p(x.data_ptr()), K, M, ctypes.c_void_p(y.data_ptr()), N,
                             ctypes.c_void_p(ws.data_ptr()), ws.numel(), st)
        assert rc == 0, L.mmhip_last_error()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt / args.steps * 1e3

    # dominant kernel alone: the GEMV on pre-quantised activations, launches
    # replayed as a HIP graph (the kernel's own duration, as in a decode step)
    xq = mm.quantize_act(mm.Q8_0, x)

    def gemv(i, s):
        W = Ws[i % copies]
        rc = L.mmhip_mul_mat_q(mm.Q8_0, ctypes.c_void_p(W.data.data_ptr()), N, K, W.row_bytes,
                               ctypes.c_void_p(xq.data_ptr()), M, ctypes.c_void_p(y.data_ptr()), N, s)
        assert rc == 0

    avg_s, med_s = graph_time(torch, gemv, 4 * copies)
    alg_bytes = N * K // 32 * 34 + M * K * 4 + M * N * 4  # weights + f32 x + f32 y
    achieved = alg_bytes / avg_s / 1e9

    del xq
    raw = synth.gguf_blocks_np(mm.Q8_0, N, K, 1002)
    xh = synth.normal_np((M, K), 1003)

    def make(og):
        x_t = og.tensor(mm.F32, [K, M])
        ws_t = [og.tensor(mm.Q8_0, [K, N]) for _ in range(copies)]
        outs = [og.mul_mat(w, x_t) for w in ws_t]

        def upload():
            og.set(x_t, xh)
            for w in ws_t:
                og.set(w, raw)
        return outs, copies, upload

    backend = via_backend(pkg, make)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_gemv(oracle, synth, N, K, M, args.cpu_seconds)
    step_bytes = alg_bytes
    return {
        "metric": "Q8_0 decode GEMV effective HBM GB/s (W 12288x4096, CFG B=2)",
        "value": round(step_bytes / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "ms_per_step": round(ms, 5),
        "dtype": "q8_0xq8_0->f32 (int8 dot)",
        "config": {"workload": "Q8_0 decode GEMV W[12288x4096] x[2x4096] f32", "weight_copies_rotated": copies,
                   "step": "quantize_act + gemv"},
        "via_backend": backend,
        "roofline": {"bound": "hbm", "kernel": "k_gemv_q8_0<2,2,4,true>", "achieved": round(achieved, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "avg_launch_us": round(avg_s * 1e6, 3), "min_launch_us": round(med_s * 1e6, 3),
                     "alg_bytes_per_launch": alg_bytes, "traffic": profile_traffic("gemv_q8_0_12288x4096_m2")},
        "cpu_baseline": cpu,
    }


def cpu_gemv(oracle, synth, N, K, M, seconds):
    n_thr = cpu_threads()
    rows = 2048  # bounded sample: 2048 of the 12288 rows
    raw = synth.gguf_blocks_np(8, rows, K, 7)
    x = synth.normal_np((M, K), 8)
    oracle.mul_mat_ggml(8, raw, rows, K, x, nthreads=n_thr)
    nbytes = rows * K // 32 * 34 + M * K * 4 + M * rows * 4
    dt, it = cpu_rate(lambda: oracle.mul_mat_ggml(8, raw, rows, K, x, nthreads=n_thr), seconds)
    nh = half_threads()
    dt_h, _ = cpu_rate(lambda: oracle.mul_mat_ggml(8, raw, rows, K, x, nthreads=nh), seconds / 2)
    gbs = nbytes / dt / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": n_thr, "kind": "port",
            "half_threads": {"value": round(nbytes / dt_h / 1e9, 3), "cores": nh},
            "sample": f"ggml-CPU-semantics Q8_0 mul_mat (oracle/oracle.c) on {rows} of {N} rows, K={K}, M={M}, "
                      f"{it} reps in {seconds:.0f}s"}


def bench_fa(args, torch, pkg):
    import oracle

    mm, synth = pkg.mmhip, pkg.synth
    B, Hq, Hkv, D, nkv = 2, 32, 8, 128, 2048
    copies = 16
    q = torch.from_numpy(synth.normal_np((B, Hq, 1, D), 1001)).cuda()
    g = torch.Generator(device="cuda")
    g.manual_seed(1001)
    ks = [torch.randn((B, Hkv, nkv, D), device="cuda", generator=g).half() for _ in range(copies)]
    vs = [torch.randn((B, Hkv, nkv, D), device="cuda", generator=g).half() for _ in range(copies)]
    out = torch.empty((B, 1, Hq, D), device="cuda")
    L = mm.load()
    qv = mm.view_of(q)
    kvs = [(mm.view_of(k), mm.view_of(v)) for k, v in zip(ks, vs)]
    need = L.mmhip_flash_attn_workspace(ctypes.byref(qv), ctypes.byref(kvs[0][0]), ctypes.byref(kvs[0][1]))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    scale = float(np.float32(1 / np.sqrt(D)))

    def step(i, s=None):
        kv, vv = kvs[i % copies]
        rc = L.mmhip_flash_attn_ext(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), None, scale,
                                    ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()), need,
                                    st if s is None else s)
        assert rc == 0, L.mmhip_last_error()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    # one attention call = the split-KV kernel + the split combine, replayed
    # as a HIP graph
    avg_s, med_s = graph_time(torch, step, 4 * copies)
    alg_bytes = B * Hq * D * 4 * 2 + 2 * B * Hkv * nkv * D * 2
    achieved = alg_bytes / avg_s / 1e9
    qh = q.cpu().numpy()
    kh = ks[0].cpu().numpy()

    def make(og):
        q_t = og.tensor(mm.F32, [D, 1, Hq, B])
        kv_t = [(og.tensor(mm.F16, [D, nkv, Hkv, B]), og.tensor(mm.F16, [D, nkv, Hkv, B])) for _ in range(copies)]
        outs = [og.flash_attn(q_t, k_t, v_t, None, scale) for k_t, v_t in kv_t]

        def upload():
            og.set(q_t, qh)
            for k_t, v_t in kv_t:
                og.set(k_t, kh)
                og.set(v_t, kh)
        return outs, copies, upload

    backend = via_backend(pkg, make)
    cpu = None
    if not args.no_cpu:
        qn = q.cpu().numpy()
        kn = ks[0].cpu().numpy()
        vn = vs[0].cpu().numpy()
        n_thr = cpu_threads()
        dt, it = cpu_rate(lambda: oracle.flash_attn_ext(qn, kn, vn, None, scale, "ggml", nthreads=n_thr),
                          args.cpu_seconds)
        nh = half_threads()
        dt_h, _ = cpu_rate(lambda: oracle.flash_attn_ext(qn, kn, vn, None, scale, "ggml", nthreads=nh),
                           args.cpu_seconds / 2)
        cpu = {"value": round(alg_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": n_thr, "kind": "port",
               "half_threads": {"value": round(alg_bytes / dt_h / 1e9, 3), "cores": nh},
               "sample": f"ggml-CPU-semantics flash_attn_ext (oracle/oracle.c), full shape, {it} reps"}
    return {
        "metric": "GQA decode attention effective HBM GB/s (B=2, 32q/8kv, D128, KV 2048)",
        "value": round(alg_bytes / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "ms_per_step": round(ms, 5),
        "dtype": "f16 K/V, f32 accumulate",
        "config": {"workload": "GQA decode FA B=2 Hq=32 Hkv=8 D=128 KV=2048 no mask", "kv_copies_rotated": copies},
        "via_backend": backend,
        "roofline": {"bound": "hbm", "kernel": "k_fa_dec_mfma<128,8,1,false> + k_fa_combine (one attention call)",
                     "achieved": round(achieved, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "avg_launch_us": round(avg_s * 1e6, 3), "min_launch_us": round(med_s * 1e6, 3),
                     "alg_bytes_per_launch": alg_bytes, "traffic": profile_traffic("fa_decode_gqa_b2_kv2048")},
        "cpu_baseline": cpu,
    }


def _fa_common(args, torch, pkg, B, Hq, Hkv, S, D, causal, seed, copies):
    mm, synth = pkg.mmhip, pkg.synth
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    qs = [torch.randn((B, Hq, S, D), device="cuda", generator=g).half().float() for _ in range(copies)]
    ks = [torch.randn((B, Hkv, S, D), device="cuda", generator=g).half() for _ in range(copies)]
    vs = [torch.randn((B, Hkv, S, D), device="cuda", generator=g).half() for _ in range(copies)]
    mask = None
    if causal:
        mask = torch.full((S, S), float("-inf"), device="cuda").triu(1).half().view(1, 1, S, S)
    out = torch.empty((B, S, Hq, D), device="cuda")
    L = mm.load()
    views = [(mm.view_of(q), mm.view_of(k), mm.view_of(v)) for q, k, v in zip(qs, ks, vs)]
    mv = mm.view_of(mask) if mask is not None else None
    need = L.mmhip_flash_attn_workspace(ctypes.byref(views[0][0]), ctypes.byref(views[0][1]),
                                        ctypes.byref(views[0][2]))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    scale = float(np.float32(1 / np.sqrt(D)))

    def step(i, s=None):
        qv, kv, vv = views[i % copies]
        rc = L.mmhip_flash_attn_ext(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                                    ctypes.byref(mv) if mv is not None else None, scale,
                                    ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()), need,
                                    st if s is None else s)
        assert rc == 0, L.mmhip_last_error()

    return step


def _timed(args, torch, step, copies):
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    # the roofline's launches replayed as a HIP graph (kernel durations
    # without per-call host dispatch)
    avg_s, min_s = graph_time(torch, step, 4 * copies)
    return ms, avg_s, min_s


MFMA_PEAK_TFLOPS = 2500.0


def bench_fa_mfma(args, torch, pkg, causal):
    import oracle

    if causal:
        B, Hq, Hkv, S, D, seed = 2, 32, 8, 1024, 128, 1003
        flops = 4.0 * B * Hq * D * S * (S + 1) / 2
        name = "causal prefill attention B=2 S=1024 Hq=32 Hkv=8 D=128"
    else:
        B, Hq, Hkv, S, D, seed = 2, 16, 16, 4096, 128, 1004
        flops = 4.0 * B * Hq * S * S * D
        name = "DiT bidirectional attention B=2 S=4096 H=16 D=128"
    prof = "fa_prefill_causal_b2_s1024_gqa" if causal else "fa_dit_b2_s4096_h16_d128"
    copies = 2
    step = _fa_common(args, torch, pkg, B, Hq, Hkv, S, D, causal, seed, copies)
    ms, avg_s, med_s = _timed(args, torch, step, copies)
    tf = flops / avg_s / 1e12
    mm = pkg.mmhip
    rng = np.random.default_rng(seed + 100)
    qh = rng.standard_normal((B, Hq, S, D)).astype(np.float16).astype(np.float32)
    kh = rng.standard_normal((B, Hkv, S, D)).astype(np.float16)
    mh = np.triu(np.full((S, S), -np.inf, np.float32), 1).astype(np.float16) if causal else None
    scale = float(np.float32(1 / np.sqrt(D)))

    def make(og):
        m_t = og.tensor(mm.F16, [S, S]) if causal else None
        ops = [(og.tensor(mm.F32, [D, S, Hq, B]), og.tensor(mm.F16, [D, S, Hkv, B]), og.tensor(mm.F16, [D, S, Hkv, B]))
               for _ in range(copies)]
        outs = [og.flash_attn(q_t, k_t, v_t, m_t, scale) for q_t, k_t, v_t in ops]

        def upload():
            if causal:
                og.set(m_t, mh)
            for q_t, k_t, v_t in ops:
                og.set(q_t, qh)
                og.set(k_t, kh)
                og.set(v_t, kh)
        return outs, copies, upload

    backend = via_backend(pkg, make, reps=5)
    backend["tflops_per_op"] = round(flops / (backend["gpu_us_per_op"] * 1e-6) / 1e12, 2)
    backend["note"] = ("measured after the C-ABI timings: the same kernel runs slower once the MFMA load has been "
                       "sustained for a while (clock drop visible in the kernel trace)")
    cpu = None
    if not args.no_cpu:
        rng = np.random.default_rng(seed)
        rows = 16 if causal else 4  # bounded sample of query rows per head
        q = rng.standard_normal((B, Hq, rows, D)).astype(np.float32)
        k = rng.standard_normal((B, Hkv, S, D)).astype(np.float16)
        v = rng.standard_normal((B, Hkv, S, D)).astype(np.float16)
        n_thr = cpu_threads()
        dt, it = cpu_rate(lambda: oracle.flash_attn_ext(q, k, v, None, 1 / np.sqrt(D), "ggml", nthreads=n_thr),
                          args.cpu_seconds)
        nh = half_threads()
        dt_h, _ = cpu_rate(lambda: oracle.flash_attn_ext(q, k, v, None, 1 / np.sqrt(D), "ggml", nthreads=nh),
                           args.cpu_seconds / 2)
        cpu_flops = 4.0 * B * Hq * rows * S * D
        cpu = {"value": round(cpu_flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": n_thr, "kind": "port",
               "half_threads": {"value": round(cpu_flops / dt_h / 1e12, 5), "cores": nh},
               "sample": f"ggml-CPU-semantics flash_attn_ext (oracle/oracle.c): {rows} query rows per head against "
                         f"all {S} keys, {it} reps"}
    return {
        "metric": ("causal prefill" if causal else "DiT") + " attention TFLOP/s",
        "value": round(flops / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "ms_per_step": round(ms, 4),
        "dtype": "f16 MFMA, f32 accumulate",
        "config": {"workload": name, "mask": "causal f16" if causal else "none"},
        "via_backend": backend,
        "roofline": {"bound": "mfma",
                     "kernel": ("k_fa_dma<true> + k_fa_row_end mask prepass (one attention call)" if causal
                                else "k_fa_dma<false>"),
                     "achieved": round(tf, 2),
                     "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tf / MFMA_PEAK_TFLOPS, 4),
                     "avg_launch_us": round(avg_s * 1e6, 2), "min_launch_us": round(med_s * 1e6, 2),
                     "alg_flops_per_launch": flops, "traffic": profile_traffic(prof),
                     "mfma_counters": mfma_counters(prof)},
        "cpu_baseline": cpu,
    }


def bench_gemm(args, torch, pkg):
    import oracle

    mm, synth = pkg.mmhip, pkg.synth
    N, K, M = 6144, 2048, 8192
    copies = 2
    Ws = [mm.QuantWeight.from_gguf(mm.Q4_K, synth.gguf_blocks_torch(mm.Q4_K, N, K, 1005 + c), N, K)
          for c in range(copies)]
    g = torch.Generator(device="cuda")
    g.manual_seed(1006)
    xs = [torch.randn((M, K), device="cuda", generator=g) for _ in range(copies)]
    y = torch.empty((M, N), device="cuda")
    L = mm.load()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws_n = L.mmhip_mul_mat_workspace(mm.Q4_K, N, K, M)
    ws = torch.empty(max(ws_n, 1), dtype=torch.uint8, device="cuda")

    def step(i, s=None):
        W, x = Ws[i % copies], xs[i % copies]
        rc = L.mmhip_mul_mat(mm.Q4_K, ctypes.c_void_p(W.data.data_ptr()), N, K, W.row_bytes,
                             ctypes.c_void_p(x.data_ptr()), K, M, ctypes.c_void_p(y.data_ptr()), N,
                             ctypes.c_void_p(ws.data_ptr()), ws_n, st if s is None else s)
        assert rc == 0, L.mmhip_last_error()

    ms, avg_s, med_s = _timed(args, torch, step, copies)
    flops = 2.0 * M * N * K
    tf = flops / avg_s / 1e12
    raw = synth.gguf_blocks_np(mm.Q4_K, N, K, 1005)
    xh = np.random.default_rng(1006).standard_normal((M, K)).astype(np.float32)

    def make(og):
        ops = [(og.tensor(mm.Q4_K, [K, N]), og.tensor(mm.F32, [K, M])) for _ in range(copies)]
        outs = [og.mul_mat(w_t, x_t) for w_t, x_t in ops]

        def upload():
            for w_t, x_t in ops:
                og.set(w_t, raw)
                og.set(x_t, xh)
        return outs, copies, upload

    backend = via_backend(pkg, make, reps=5)
    backend["tflops_per_op"] = round(flops / (backend["gpu_us_per_op"] * 1e-6) / 1e12, 2)
    backend["note"] = ("measured after the C-ABI timings: the same kernel runs slower once the MFMA load has been "
                       "sustained for a while (clock drop visible in the kernel trace)")
    cpu = None
    if not args.no_cpu:
        rows = 64
        raw = synth.gguf_blocks_np(mm.Q4_K, rows, K, 9)
        x = synth.normal_np((64, K), 10)
        n_thr = cpu_threads()
        dt, it = cpu_rate(lambda: oracle.mul_mat_ggml(mm.Q4_K, raw, rows, K, x, nthreads=n_thr), args.cpu_seconds)
        nh = half_threads()
        dt_h, _ = cpu_rate(lambda: oracle.mul_mat_ggml(mm.Q4_K, raw, rows, K, x, nthreads=nh), args.cpu_seconds / 2)
        cpu = {"value": round(2.0 * 64 * rows * K / dt / 1e12, 5), "unit": "TFLOP/s", "cores": n_thr,
               "half_threads": {"value": round(2.0 * 64 * rows * K / dt_h / 1e12, 5), "cores": nh},
               "kind": "port", "sample": f"ggml-CPU-semantics Q4_K x Q8_K mul_mat (oracle/oracle.c): {rows} weight "
                                         f"rows x 64 tokens, K={K}, {it} reps"}
    return {
        "metric": "Q4_K GEMM TFLOP/s (DiT QKV projection 2048->6144, 8192 tokens)",
        "value": round(flops / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "ms_per_step": round(ms, 4),
        "dtype": "f16 MFMA (Q4_K dequantised to f16 rows once per call), f32 accumulate",
        "config": {"workload": "Q4_K GEMM W[6144x2048] x[8192x2048] f32 -> f32"},
        "via_backend": backend,
        "roofline": {"bound": "mfma", "kernel": "k_xw_to_f16<Q4_K> (activations and weights to f16, one launch) + k_gemm_q<f16 weights, 4-stage DMA ring, four waves> "
                                               "(one mul_mat call)", "achieved": round(tf, 2),
                     "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tf / MFMA_PEAK_TFLOPS, 4),
                     "avg_launch_us": round(avg_s * 1e6, 2), "min_launch_us": round(med_s * 1e6, 2),
                     "alg_flops_per_launch": flops, "traffic": profile_traffic("gemm_q4_k_6144x2048_m8192"),
                     "mfma_counters": mfma_counters("gemm_q4_k_6144x2048_m8192")},
        "cpu_baseline": cpu,
    }


def dit_block_flops(S, B, dim=2048, ff=8192, heads=32, hd=64):
    """FLOPs of one DiT block: the six projections (q, k, v, o, ff_in emitting
    2 ff, ff_out) and bidirectional attention (QK^T and PV)."""
    M = S * B
    return 2.0 * M * (4 * dim * dim + dim * 2 * ff + ff * dim) + 4.0 * B * heads * S * S * hd


def cpu_dit_block(oracle, dg, w, x, pos):
    """One DiT block (src/dit.h:183-247) composed from the oracle's
    ggml-CPU-semantics restatements; x [B, S, dim] f32."""
    B, S, dim = x.shape
    H, D, ff = dg.N_HEADS, dg.HEAD_DIM, dg.FF_INNER
    Q8 = 8

    def mm(name, a, n_out):
        return oracle.mul_mat_ggml(Q8, w[name], n_out, a.shape[-1], a.reshape(-1, a.shape[-1])).reshape(B, S, n_out)

    def ln(a, g_, b_):
        return oracle.layer_norm(a, dg.LN_EPS) * g_ + b_

    h = ln(x, w["norm1_w"], w["norm1_b"])
    q, k, v = (mm(n, h, dim).reshape(B * S, H, D) for n in ("wq", "wk", "wv"))
    pos_b = np.tile(pos, B)
    q = oracle.rope_neox(q, pos_b, dg.ROTARY_DIM, dg.ROPE_BASE).reshape(B, S, H, D).transpose(0, 2, 1, 3)
    k = oracle.rope_neox(k, pos_b, dg.ROTARY_DIM, dg.ROPE_BASE).reshape(B, S, H, D).transpose(0, 2, 1, 3)
    v = v.reshape(B, S, H, D).transpose(0, 2, 1, 3)
    a = oracle.flash_attn_ext(np.ascontiguousarray(q), np.ascontiguousarray(k).astype(np.float16),
                              np.ascontiguousarray(v).astype(np.float16), None, float(np.float32(1 / np.sqrt(D))))
    x = x + mm("wo", a.reshape(B, S, H * D), dim)
    h = ln(x, w["norm2_w"], w["norm2_b"])
    f = mm("ff_in_w", h, 2 * ff) + w["ff_in_b"]
    act = oracle.swiglu(np.concatenate([f[..., ff:], f[..., :ff]], axis=-1))
    return x + (mm("ff_out_w", act, dim) + w["ff_out_b"])


def bench_dit_block(args, torch, pkg):
    """The DiT block (src/dit.h:183-247) at the model's shape, S = 690 tokens
    (T = 689 latent frames + the timestep token), CFG B = 2, Q8_0 weights:
    a graph of NB chained blocks (distinct weights) through
    ggml_backend_graph_compute on the MI355X backend, HIP-graph replay."""
    import importlib

    import oracle

    og_mod = importlib.import_module(pkg.__name__ + ".opgraph")
    dg = importlib.import_module(pkg.__name__ + ".ditgraph")
    mm = pkg.mmhip
    S, B, NB = 690, 2, 4
    ws = [dg.synth_block(3000 + i) for i in range(NB)]
    x0 = np.random.default_rng(3100).standard_normal((B, S, dg.DIM)).astype(np.float32)
    pos = np.arange(S, dtype=np.int32)
    g = og_mod.OpGraph(n_tensors=64 * NB)
    try:
        blks = [dg.Block(g) for _ in range(NB)]
        tx = g.tensor(og_mod.F32, [dg.DIM, S, B])
        tp = g.tensor(26, [S])  # GGML_TYPE_I32
        out = tx
        for b in blks:
            out = dg.build_block(g, b, out, tp, S, B)
        g.build([out])
        for b, w in zip(blks, ws):
            b.upload(g, w)
        g.set(tx, x0)
        g.set(tp, pos)
        for _ in range(args.warmup + 2):
            g.compute()
        g.synchronize()
        g.gpu_time(reset=True)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            g.compute()
        g.synchronize()
        wall = (time.perf_counter() - t0) / args.steps
        gms, n = g.gpu_time()
        replays, eager = g.graph_stats()
        f16_bytes = g.f16_weight_bytes()
    finally:
        g.close()
    us_block = gms / max(n, 1) * 1e3 / NB
    flops = dit_block_flops(S, B)
    # dominant kernel: the ff_in projection (2048 -> 16384, 1380 tokens) as the block runs it: f16 activations
    # from the LayerNorm, bias, SwiGLU of the two halves and the f16 rounding for ff_out in the epilogue, on
    # the f16 copy of the weights that the backend makes for a repeating graph (one k_gemm_q launch on the
    # DMA ring), C-ABI, graph replay
    M, N, K = S * B, 2 * dg.FF_INNER, dg.DIM
    W = mm.QuantWeight.from_gguf(mm.Q8_0, ws[0]["ff_in_w"], N, K)
    xs = torch.randn((M, K), device="cuda").half()
    bias = torch.from_numpy(ws[0]["ff_in_b"]).cuda()
    hh = torch.empty((M, N // 2), dtype=torch.float16, device="cuda")
    L = mm.load()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    wh = torch.empty(L.mmhip_weights_f16_bytes(N, K), dtype=torch.uint8, device="cuda")
    assert L.mmhip_weights_to_f16(mm.Q8_0, P(W.data), N, K, W.row_bytes, P(wh), None) == 0, L.mmhip_last_error()
    assert L.mmhip_register_weights_f16(P(W.data), N, K, P(wh)) == 0, L.mmhip_last_error()

    def step(i, s):
        rc = L.mmhip_mul_mat_bias_swiglu_h(mm.Q8_0, P(W.data), N, K, W.row_bytes, P(xs), M, P(bias), 0, None, P(hh),
                                           s)
        assert rc == 0, L.mmhip_last_error()

    try:
        avg_s, min_s = graph_time(torch, step, 10)
    finally:
        torch.cuda.synchronize()
        L.mmhip_unregister_weights_f16(P(W.data))
    gf = 2.0 * M * N * K
    tf = gf / avg_s / 1e12
    cpu = None
    if not args.no_cpu:
        Sc = 32
        xc = x0[:, :Sc].copy()
        dt, it = cpu_rate(lambda: cpu_dit_block(oracle, dg, ws[0], xc, np.arange(Sc, dtype=np.int32)), args.cpu_seconds)
        cpu = {"value": round(dit_block_flops(Sc, B) / dt / 1e12, 5), "unit": "TFLOP/s",
               "cores": cpu_threads(), "kind": "port",
               "sample": f"one DiT block from the oracle's ggml-CPU-semantics restatements (Q8_0 mul_mat, LayerNorm, "
                         f"NeoX RoPE, flash_attn_ext, SwiGLU): S={Sc} tokens x B={B}, {it} reps"}
    return {
        "metric": "DiT block TFLOP/s (S=690 tokens, CFG B=2, Q8_0, dim 2048, 32x64 heads, FF 8192)",
        "value": round(flops / (us_block * 1e-6) / 1e12, 2),
        "unit": "TFLOP/s",
        "ms_per_step": round(us_block * 1e-3, 4),
        "dtype": "f16 MFMA (Q8_0 dequantised to f16 copies once per weight), f32 glue",
        "config": {"workload": f"DiT block x{NB} chained through ggml_backend_graph_compute, S={S}, B={B}, Q8_0"},
        "via_backend": {"path": "ggml_backend_graph_compute, MI355X backend, HIP-graph replay", "blocks_per_graph": NB,
                        "gpu_us_per_block": round(us_block, 2), "wall_us_per_block": round(wall * 1e6 / NB, 2),
                        "replays": replays, "eager": eager, "f16_weight_copy_bytes": f16_bytes},
        "roofline": {"bound": "mfma",
                     "kernel": "k_gemm_q<f16 weight copy, 4-stage DMA ring> with bias + SwiGLU + f16 epilogue "
                               "(ff_in 2048->16384, 1380 tokens)",
                     "achieved": round(tf, 2), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / MFMA_PEAK_TFLOPS, 4), "avg_launch_us": round(avg_s * 1e6, 2),
                     "min_launch_us": round(min_s * 1e6, 2), "alg_flops_per_launch": gf,
                     "traffic": profile_traffic("dit_block_s690_b2_q8_0"),
                     "mfma_counters": mfma_counters("dit_block_s690_b2_q8_0")},
        "cpu_baseline": cpu,
    }


def bench_depth(args, torch, pkg):
    """The RVQ depth decoder's 4-layer transformer stack (src/depth-decoder.h:
    196-236) at its last step, S = 8 positions x the CFG pair (B = 2, 16
    tokens), Q8_0 weights, through ggml_backend_graph_compute on the MI355X
    backend (HIP-graph replay).  The roofline call is the gate projection
    (6144 x 4096) at 16 tokens through the C-ABI (two 8-column GEMV groups)."""
    import importlib

    import oracle

    og_mod = importlib.import_module(pkg.__name__ + ".opgraph")
    dg = importlib.import_module(pkg.__name__ + ".depthgraph")
    mm = pkg.mmhip
    S, B, NL = 8, 2, 4
    ws = [dg.synth_layer(3200 + i) for i in range(NL)]
    x0 = np.random.default_rng(3300).standard_normal((B, S, dg.DIM)).astype(np.float32)
    g = og_mod.OpGraph(n_tensors=100 * NL)
    try:
        ls = [dg.Layer(g) for _ in range(NL)]
        tx = g.tensor(og_mod.F32, [dg.DIM, S, B])
        out = tx
        for lw in ls:
            out = dg.build_layer(g, lw, out, S, B)
        g.build([out])
        for lw, w in zip(ls, ws):
            lw.upload(g, w)
        g.set(tx, x0)
        for _ in range(args.warmup + 2):
            g.compute()
        g.synchronize()
        g.gpu_time(reset=True)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            g.compute()
        g.synchronize()
        wall = (time.perf_counter() - t0) / args.steps
        gms, n = g.gpu_time()
        replays, eager = g.graph_stats()
    finally:
        g.close()
    us = gms / max(n, 1) * 1e3
    wbytes = NL * (4 * dg.DIM * dg.DIM + 3 * dg.DIM * dg.FF_INNER) * 34 // 32
    M, N, K = S * B, dg.FF_INNER, dg.DIM
    W = mm.QuantWeight.from_gguf(mm.Q8_0, ws[0]["w_gate"], N, K)
    xs = torch.randn((M, K), device="cuda")
    y = torch.empty((M, N), device="cuda")
    L = mm.load()
    ws_n = L.mmhip_mul_mat_workspace(mm.Q8_0, N, K, M)
    wsb = torch.empty(ws_n, dtype=torch.uint8, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())

    def step(i, s):
        rc = L.mmhip_mul_mat(mm.Q8_0, P(W.data), N, K, W.row_bytes, P(xs), K, M, P(y), N, P(wsb), ws_n, s)
        assert rc == 0, L.mmhip_last_error()

    avg_s, min_s = graph_time(torch, step, 10)
    alg = N * K * 34 // 32 + M * K * 4 + M * N * 4
    cpu = None
    if not args.no_cpu:
        raw = ws[0]["w_gate"][:512]
        xc = x0.reshape(-1, dg.DIM)
        n_thr = cpu_threads()
        dt, it = cpu_rate(lambda: oracle.mul_mat_ggml(mm.Q8_0, raw, 512, K, xc, nthreads=n_thr), args.cpu_seconds)
        cpu = {"value": round(512 * K * 34 / 32 / dt / 1e9, 3), "unit": "GB/s (weight bytes streamed)", "cores": n_thr,
               "kind": "port", "sample": f"ggml-CPU-semantics Q8_0 mul_mat (oracle/oracle.c): 512 gate rows x {M} "
                                         f"tokens, K={K}, {it} reps"}
    return {
        "metric": "Depth decoder 4-layer stack weight GB/s (S=8 steps, CFG B=2, Q8_0, 16 x 256 heads, FF 6144)",
        "value": round(wbytes / (us * 1e-6) / 1e9, 2),
        "unit": "GB/s",
        "ms_per_step": round(us * 1e-3, 4),
        "dtype": "int8 dots on Q8_0-quantised activations (GEMV), f32 attention",
        "config": {"workload": f"depth decoder layers x{NL} through ggml_backend_graph_compute, S={S}, B={B}, Q8_0"},
        "via_backend": {"path": "ggml_backend_graph_compute, MI355X backend, HIP-graph replay", "layers_per_graph": NL,
                        "gpu_us_per_stack": round(us, 2), "wall_us_per_stack": round(wall * 1e6, 2),
                        "replays": replays, "eager": eager},
        "roofline": {"bound": "hbm", "kernel": "k_quant_q8_0 + k_gemv_q8_0_mfma<2> (gate 6144x4096, 16 tokens, int8 MFMA)",
                     "achieved": round(alg / avg_s / 1e9, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(alg / avg_s / 1e9 / HBM_PEAK_GBS, 4), "avg_launch_us": round(avg_s * 1e6, 2),
                     "min_launch_us": round(min_s * 1e6, 2), "alg_bytes_per_launch": alg,
                     "traffic": profile_traffic("depth_stack_s8_b2_q8_0")},
        "cpu_baseline": cpu,
    }


# Algorithmic HBM bytes of one Qwen3-8B-shape CFG decode step at KV 4096:
# weights + KV read + norm weights + logits + KV write (per step, both rows).
def lm_bumped_layers(cfg):
    """Layers whose V / down projections take bump_type (the "_M" rule of
    tools/quantize.cpp:127-150)."""
    L = cfg["n_layers"]
    if not cfg.get("bump_type"):
        return []
    return [l for l in range(L) if l < L // 9 or l >= L - L // 7 or l % 3 == 0]


def lm_step_bytes(cfg, wtype):
    size = {8: (32, 34), 14: (256, 210), 13: (256, 176), 12: (256, 144), 30: (1, 2)}

    def nbytes(n, t):
        be, bb = size[t]
        return n * bb // be

    H, D, Nh, Nkv, F, V, L = (cfg["hidden"], cfg["head_dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["ffn"],
                              cfg["vocab"], cfg["n_layers"])
    bumped = set(lm_bumped_layers(cfg))
    weights = nbytes(H * V, wtype)
    for l in range(L):
        bt = cfg["bump_type"] if l in bumped else wtype
        weights += (nbytes(H * (Nh * D + Nkv * D) + Nh * D * H + H * 2 * F, wtype) +
                    nbytes(H * Nkv * D + F * H, bt))
    kv_len, sets = 4096, 2
    kv_read = L * 2 * sets * Nkv * kv_len * D * 2
    norms = (L * (2 * H + 2 * D) + H) * 4
    logits = sets * V * 4
    kv_write = L * 2 * sets * Nkv * D * 2
    return weights + kv_read + norms + logits + kv_write


def bench_lm(args, torch, pkg):
    import importlib

    lm_mod = importlib.import_module(pkg.__name__ + ".lm")
    cfg = dict(lm_mod.QWEN3_8B)
    cfg["wtype"] = {"q8_0": 8, "q6_k": 14, "q5_k_m": 13, "bf16": 30}[args.wtype]
    cfg["bump_type"] = 14 if args.wtype == "q5_k_m" else 0
    lm = lm_mod.Lm(seed=1005, **cfg)
    lm.fill_kv(0, 4095, seed=1)
    lm.fill_kv(1, 4095, seed=2)
    emb = np.random.default_rng(1005).standard_normal((2, cfg["hidden"])).astype(np.float32)

    def step():
        # every step attends over KV 4096 (positions reset to 4095); the
        # step reads its logits and final hidden states back to the host, as
        # the reference does after every batched decode (src/qwen3-lm.h:923-927)
        lm.set_pos(0, 4095)
        lm.set_pos(1, 4095)
        lm.decode(emb, [0, 1])

    for _ in range(max(args.warmup, 3)):
        step()
    lm.gpu_ms(reset=True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    dt = (time.perf_counter() - t0) / args.steps
    gpu_s = lm.gpu_ms() / 1e3  # HIP events on the backend stream around each graph replay
    step_bytes = lm_step_bytes(cfg, cfg["wtype"])
    achieved = step_bytes / gpu_s / 1e9
    replays, eager = lm.graph_stats()
    nodes = lm.graph_nodes()
    lm.close()
    if cfg["wtype"] == 30:
        dom = lm_dominant_kernel_bf16(torch, pkg, cfg)
    elif cfg["wtype"] == 13:
        dom = lm_dominant_kernel_gemv(torch, pkg, cfg)
    else:
        dom = lm_dominant_kernel(torch, pkg, cfg)
    cpu = None
    if not args.no_cpu and cfg["wtype"] != 30:
        cpu = cpu_lm(args, lm_mod, cfg)
    return {
        "metric": "LM decode tok/s (CFG B=2, %s, KV 4096)" % args.wtype.upper(),
        # inputs resident: the GPU time of the step's graph replay; the host
        # input uploads of each step are in the wall-clock figures beside it
        "value": round(2.0 / gpu_s, 2),
        "unit": "tok/s",
        "ms_per_step": round(gpu_s * 1e3, 4),
        "wall_tok_s": round(2.0 / dt, 2),
        "wall_ms_per_step": round(dt * 1e3, 4),
        "dtype": (args.wtype + " weights (int8-dot GEMV), f16 KV, f32 activations") if args.wtype != "bf16" else
                 "bf16 weights x bf16-rounded activations (f32 sums), f16 KV, f32 activations",
        "config": {"workload": "Qwen3-8B-shape batched CFG decode step: 36 layers, hidden 4096, 32q/8kv d128, "
                               "FFN 12288 SwiGLU, vocab 151936, KV 4096 x 2 sets",
                   "weights": args.wtype, "graph_nodes": nodes, "graph_replays": replays, "eager_runs": eager,
                   "tokens_per_step": 2},
        "roofline": dom,
        "step_roofline": {"bound": "hbm", "kernel": "whole decode step (one HIP-graph replay of %d ggml nodes)" % nodes,
                          "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(achieved / HBM_PEAK_GBS, 4), "alg_bytes_per_step": step_bytes,
                          "gpu_us_per_step": round(gpu_s * 1e6, 2), "wall_us_per_step": round(dt * 1e6, 2)},
        "cpu_baseline": cpu,
    }


def lm_dominant_kernel(torch, pkg, cfg):
    """The step's largest kernel alone: the MLP gate_up GEMV with the RMS norm
    in its prologue and the SwiGLU + the down GEMV's Q8_0 quantisation in its
    epilogue (W [2 ffn x hidden] Q8_0, 2 columns), six weight copies (642 MB)
    rotating past the 256 MB Infinity Cache, launches replayed as a HIP graph
    like the step's."""
    mm, synth = pkg.mmhip, pkg.synth
    N, K, M = 2 * cfg["ffn"], cfg["hidden"], 2
    F = N // 2
    wt = cfg["wtype"]
    copies = 6
    L = mm.load()
    if not L.mmhip_rms_norm_mul_mat_glu_supported(wt, N, K, M):
        return None
    Ws = [mm.QuantWeight.from_gguf(wt, synth.gguf_blocks_torch(wt, N, K, 2001 + c), N, K) for c in range(copies)]
    x = torch.from_numpy(synth.normal_np((M, K), 2011)).cuda()
    nw = torch.ones(K, device="cuda")
    xq = torch.empty(L.mmhip_act_bytes(mm.Q8_0, F, M), dtype=torch.uint8, device="cuda")

    def launch(i, st):
        W = Ws[i % copies]
        rc = L.mmhip_rms_norm_mul_mat_glu(wt, ctypes.c_void_p(W.data.data_ptr()), N, K, W.row_bytes,
                                          ctypes.c_void_p(x.data_ptr()), K, M, ctypes.c_void_p(nw.data_ptr()), 1e-6, 0,
                                          ctypes.c_void_p(xq.data_ptr()), None, st)
        assert rc == 0, L.mmhip_last_error()

    avg_s, min_s = graph_time(torch, launch, 36)
    # weights + x + norm weight + the Q8_0 SwiGLU rows written (int8 + f32 block scales)
    alg_bytes = Ws[0].data.numel() + M * K * 4 + K * 4 + M * F + M * (F // 32) * 4
    achieved = alg_bytes / avg_s / 1e9
    del Ws
    torch.cuda.empty_cache()
    return {"bound": "hbm", "kernel": "k_gemv_q8_0_norm_glu<2>: RMS norm + gate_up GEMV %d x %d Q8_0 + SwiGLU, "
                                      "2 columns (the decode step's largest kernel)" % (N, K),
            "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": profile_traffic("gemv_norm_glu_gate_up_24576x4096_m2"),
            "avg_launch_us": round(avg_s * 1e6, 3), "min_launch_us": round(min_s * 1e6, 3),
            "alg_bytes_per_launch": alg_bytes}


def lm_dominant_kernel_gemv(torch, pkg, cfg):
    """The Q5_K_M step's largest kernel alone: the gate_up GEMV with the RMS
    norm and the Q8_K quantisation in its prologue (W [2 ffn x hidden] Q5_K,
    2 columns; the step's SwiGLU is a separate quantising pass), six weight
    copies (415 MB) rotating past the 256 MB Infinity Cache, replayed as a
    HIP graph."""
    mm, synth = pkg.mmhip, pkg.synth
    N, K, M = 2 * cfg["ffn"], cfg["hidden"], 2
    wt = cfg["wtype"]
    copies = 6
    L = mm.load()
    if not L.mmhip_rms_norm_mul_mat_supported(wt, N, K, M):
        return None
    Ws = [mm.QuantWeight.from_gguf(wt, synth.gguf_blocks_torch(wt, N, K, 2201 + c), N, K) for c in range(copies)]
    x = torch.from_numpy(synth.normal_np((M, K), 2211)).cuda()
    nw = torch.ones(K, device="cuda")
    y = torch.empty((M, N), device="cuda")

    def launch(i, st):
        W = Ws[i % copies]
        rc = L.mmhip_rms_norm_mul_mat(wt, ctypes.c_void_p(W.data.data_ptr()), N, K, W.row_bytes,
                                      ctypes.c_void_p(x.data_ptr()), K, M, ctypes.c_void_p(nw.data_ptr()), 1e-6, None,
                                      None, 0, ctypes.c_void_p(y.data_ptr()), N, st)
        assert rc == 0, L.mmhip_last_error()

    avg_s, min_s = graph_time(torch, launch, 36)
    # weights + x + norm weight + y
    alg_bytes = Ws[0].data.numel() + M * K * 4 + K * 4 + M * N * 4
    achieved = alg_bytes / avg_s / 1e9
    del Ws
    torch.cuda.empty_cache()
    return {"bound": "hbm", "kernel": "k_gemv_q45_K_pro<2,1,PRO_NORM,Q5>: RMS norm + gate_up GEMV %d x %d Q5_K, "
                                      "2 columns (the Q5_K_M step's largest kernel)" % (N, K),
            "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profile_traffic("lm_decode_q5_k_m_kv4096"),
            "avg_launch_us": round(avg_s * 1e6, 3), "min_launch_us": round(min_s * 1e6, 3),
            "alg_bytes_per_launch": alg_bytes}


def lm_dominant_kernel_bf16(torch, pkg, cfg):
    """The BF16 step's largest kernel alone: the gate_up decode GEMV with the
    RMS norm in its prologue and the SwiGLU in its epilogue (W [2 ffn x
    hidden] bf16, 2 columns), three weight copies (1.2 GB) rotating past the
    256 MB Infinity Cache, replayed as a HIP graph."""
    L = pkg.mmhip.load()
    N, K, M = 2 * cfg["ffn"], cfg["hidden"], 2
    copies = 3
    if not L.mmhip_mul_mat_bf16_dec_supported(N, K, M, 1):
        return None
    g = torch.Generator(device="cuda")
    g.manual_seed(2101)
    Ws = [(torch.randn((N, K), device="cuda", generator=g) * 0.02).to(torch.bfloat16) for _ in range(copies)]
    x = torch.randn((M, K), device="cuda", generator=g)
    nw = torch.ones(K, device="cuda")
    y = torch.empty((M, N // 2), device="cuda")

    def launch(i, st):
        W = Ws[i % copies]
        rc = L.mmhip_mul_mat_bf16_dec(ctypes.c_void_p(W.data_ptr()), N, K, K, ctypes.c_void_p(x.data_ptr()), K, M,
                                      ctypes.c_void_p(nw.data_ptr()), 1e-6, None, 0, 1, ctypes.c_void_p(y.data_ptr()),
                                      N // 2, st)
        assert rc == 0, L.mmhip_last_error()

    avg_s, min_s = graph_time(torch, launch, 36)
    alg_bytes = N * K * 2 + M * K * 4 + K * 4 + M * (N // 2) * 4
    achieved = alg_bytes / avg_s / 1e9
    del Ws
    torch.cuda.empty_cache()
    return {"bound": "hbm", "kernel": "k_gemv_bf16_dec<2,NORM,GLU>: RMS norm + gate_up GEMV %d x %d BF16 + SwiGLU, "
                                      "2 columns (the BF16 step's largest kernel)" % (N, K),
            "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "avg_launch_us": round(avg_s * 1e6, 3), "min_launch_us": round(min_s * 1e6, 3),
            "alg_bytes_per_launch": alg_bytes}


def cpu_lm(args, lm_mod, cfg):
    """One decoder layer and the lm_head at the full shape through the
    ggml-CPU-semantics restatement, extrapolated to 36 layers."""
    import oracle

    sys.path.insert(0, str(ROOT / "tests"))
    n_thr = cpu_threads()
    H, D, Nh, Nkv, F, V = cfg["hidden"], cfg["head_dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["ffn"], cfg["vocab"]
    t = cfg["wtype"]
    rng = np.random.default_rng(7)
    import importlib

    synth = importlib.import_module(lm_mod.__name__.rsplit(".", 1)[0] + ".synth")
    W = {n: synth.gguf_blocks_np(t, r, k, 50 + i) for i, (n, r, k) in enumerate(
        [("qkv", Nh * D + 2 * Nkv * D, H), ("o", H, Nh * D), ("gu", 2 * F, H), ("down", H, F)])}
    bt = cfg.get("bump_type") or t
    n_bumped = len(lm_bumped_layers(cfg))
    if n_bumped:
        W.update({n: synth.gguf_blocks_np(tt, r, k, 60 + i) for i, (n, tt, r, k) in enumerate(
            [("qk", t, Nh * D + Nkv * D, H), ("v", bt, Nkv * D, H), ("down_b", bt, H, F)])})
    kc = rng.standard_normal((2, Nkv, 4096, D)).astype(np.float16)
    vc = rng.standard_normal((2, Nkv, 4096, D)).astype(np.float16)
    x = rng.standard_normal((2, H)).astype(np.float32)
    wn = np.ones(H, np.float32)

    def layer(nt, bumped=False):
        h = oracle.rms_norm_mul(x, wn, 1e-6)
        if bumped:
            qkv = np.concatenate([oracle.mul_mat_ggml(t, W["qk"], Nh * D + Nkv * D, H, h, nthreads=nt),
                                  oracle.mul_mat_ggml(bt, W["v"], Nkv * D, H, h, nthreads=nt)], axis=1)
        else:
            qkv = oracle.mul_mat_ggml(t, W["qkv"], Nh * D + 2 * Nkv * D, H, h, nthreads=nt)
        q = oracle.rope_neox(qkv[:, :Nh * D].reshape(2, Nh, D), np.array([4095, 4095], np.int32), D, 1e6)
        o = oracle.flash_attn_ext(np.ascontiguousarray(q[:, :, None]), kc, vc, None, 1 / np.sqrt(D), "ggml",
                                  nthreads=nt).reshape(2, Nh * D)
        h2 = x + oracle.mul_mat_ggml(t, W["o"], H, Nh * D, np.asarray(o, np.float32), nthreads=nt)
        gu = oracle.mul_mat_ggml(t, W["gu"], 2 * F, H, oracle.rms_norm_mul(h2, wn, 1e-6), nthreads=nt)
        if bumped:
            return h2 + oracle.mul_mat_ggml(bt, W["down_b"], H, F, oracle.swiglu(gu), nthreads=nt)
        return h2 + oracle.mul_mat_ggml(t, W["down"], H, F, oracle.swiglu(gu), nthreads=nt)

    rows = 8192  # lm_head sample: 8192 of the 151936 vocab rows
    Wl = synth.gguf_blocks_np(t, rows, H, 99)

    def step_s(nt, seconds):
        if n_bumped:
            # one layer of each kind, weighted by how many of the 36 there are
            t_plain, it = cpu_rate(lambda: layer(nt), seconds / 2)
            t_bump, it_b = cpu_rate(lambda: layer(nt, True), seconds / 2)
            t_layer = ((36 - n_bumped) * t_plain + n_bumped * t_bump) / 36
            it += it_b
        else:
            t_layer, it = cpu_rate(lambda: layer(nt), seconds)
        t_head, _ = cpu_rate(lambda: oracle.mul_mat_ggml(t, Wl, rows, H, x, nthreads=nt), 0.0)
        return 36 * t_layer + t_head * V / rows, t_layer, it

    step, t_layer, it = step_s(n_thr, args.cpu_seconds)
    nh = half_threads()
    step_h, _, _ = step_s(nh, args.cpu_seconds / 2)
    return {"value": round(2.0 / step, 4), "unit": "tok/s", "cores": n_thr, "kind": "port",
            "half_threads": {"value": round(2.0 / step_h, 4), "cores": nh},
            "sample": f"ggml-CPU-semantics restatement (oracle/): {it} full-shape decoder layer(s) at KV 4096 "
                      f"({t_layer * 1e3:.0f} ms each) and an 8192-row lm_head slice, extrapolated to 36 layers + "
                      f"the 151936-row lm_head ({step:.2f} s per 2-token step)"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU sharding is design-only",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    pkg.mmhip.load()
    res = {
        "lm_decode": lambda: bench_lm(args, torch, pkg),
        "gemv_q8_0": lambda: bench_gemv(args, torch, pkg),
        "fa_decode": lambda: bench_fa(args, torch, pkg),
        "fa_prefill": lambda: bench_fa_mfma(args, torch, pkg, True),
        "fa_dit": lambda: bench_fa_mfma(args, torch, pkg, False),
        "gemm_q4_k": lambda: bench_gemm(args, torch, pkg),
        "dit_block": lambda: bench_dit_block(args, torch, pkg),
        "depth": lambda: bench_depth(args, torch, pkg),
    }[args.workload]()
    line = {
        "metric": res["metric"],
        "value": res["value"],
        "unit": res["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": res["dtype"],
        "data": "synthetic (seeded), random-init weights",
        "config": res["config"],
        "roofline": res["roofline"],
        "cpu_baseline": res["cpu_baseline"],
        "baseline_metric": METRIC,
    }
    for k in ("step_roofline", "wall_tok_s", "wall_ms_per_step", "via_backend"):
        if k in res:
            line[k] = res[k]
    if isinstance(line["cpu_baseline"], dict):
        line["cpu_baseline"]["host"] = host_cpu()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
