"""Benchmark of the quantised-matmul + MoE-FFN hot path on one MI355X.

Workload: the TinyLlama-1.1B Q4_K_M matmul set —
22 layers x {q, k, v, o, gate, up (Q4_K), down (Q6_K)} plus the Q6_K lm_head,
22 distinct weight copies (664 MB, beyond the 256 MB Infinity Cache) —
applied to fp32 activations at decode batch 1 with the *_batch_matmul
semantics (CE:255-378).  One step = one pass over the whole set.  Inputs are
resident in HBM before the timed region.  `value` is the algorithmic HBM
bandwidth of that pass (weight bytes + activations + fp32 outputs) / time.

Also reported (same JSON line): batch 4 and 8 passes, configs[0] (Q8_0 GEMV
5632x2048 rotated over 24 copies), the roofline of the dominant kernel (the
Q4_K gate/up GEMV, timed with HIP events on its own stream) and the
reference's own C path (oracle/_ref, AVX2 + OpenMP) timed on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from mojollama_amd import kernels as K  # noqa: E402
from mojollama_amd import workloads as W  # noqa: E402

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the roofline kernel (fused Q4_K gate+up GEMV, B=1) from
# FETCH_SIZE / WRITE_SIZE counter runs calibrated on a copy of known size:
# profiles/gemv_gate_up_q4k_traffic.md (commands and raw counter values).
GATE_UP_TRAFFIC_BYTES = 13273463


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the host-CPU reference timing")
    ap.add_argument("--no-extra", action="store_true", help="only the configs[1] decode set")
    ap.add_argument("--kernel", choices=("gate_up", "copy"),
                    help="run only 50 launches of one kernel and exit, for counter runs (rocprofv3 --pmc): the "
                         "fused Q4_K gate+up GEMV of the roofline, or a 256 MiB device copy to calibrate bytes")
    return ap.parse_args()


def kernel_only(torch, dev, which):
    """50 launches of one kernel, nothing else on the GPU besides set-up."""
    if which == "copy":
        a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        a.fill_(1)
        torch.cuda.synchronize()
        for _ in range(50):
            b.copy_(a)
    else:
        rng = np.random.default_rng(2)
        raw = np.concatenate([W.gen_weights(rng, W.QT_Q4_K, 5632, 2048) for _ in range(2)])
        m = Matrix(dev, K.Q4_K_GGML, raw, 11264, 2048)
        x = torch.randn(1, 2048, device="cuda")
        o = torch.empty(1, 11264, device="cuda")
        torch.cuda.synchronize()
        for _ in range(50):
            dev.gemv(m.sem, m.packed, x, m.rows, m.cols, out=o)
    torch.cuda.synchronize()
    print(f"[bench] {which}: 50 launches done", file=sys.stderr, flush=True)


class Matrix:
    def __init__(self, dev, sem, raw, rows, cols):
        import torch
        self.sem, self.rows, self.cols = sem, rows, cols
        self.raw_bytes = raw.size
        self.packed = dev.pack(sem, torch.from_numpy(raw).cuda(), rows, cols)


def build_tinyllama(dev, rng, n_layers):
    """Per layer the device copies are laid out as a decode engine runs them:
    q/k/v rows concatenated into one 2560x2048 matrix (one launch, like the
    reference's fused QKV tensors and batch_qkv_omp), o, gate/up rows
    concatenated into one 11264x2048 matrix (batch_gate_up_omp), and down."""
    import torch
    layers = []
    for _ in range(n_layers):
        raw = {name: W.gen_weights(rng, qt, rows, cols) for name, rows, cols, qt in W.TINYLLAMA_MATS}
        qkv = np.concatenate([raw["q"], raw["k"], raw["v"]])
        gu = np.concatenate([raw["gate"], raw["up"]])
        layers.append([("qkv", Matrix(dev, K.Q4_K_GGML, qkv, 2560, 2048)),
                       ("o", Matrix(dev, K.Q4_K_GGML, raw["o"], 2048, 2048)),
                       ("gate_up", Matrix(dev, K.Q4_K_GGML, gu, 11264, 2048)),
                       ("down", Matrix(dev, K.Q6_K_SEQ, raw["down"], 2048, 5632))])
    name, rows, cols, qt = W.TINYLLAMA_LM_HEAD
    lm = Matrix(dev, K.Q6_K_SEQ, W.gen_weights(rng, qt, rows, cols), rows, cols)
    return layers, lm


def algo_bytes(m, B):
    return m.raw_bytes + B * (m.cols + m.rows) * 4


def time_region(torch, fn, steps, warmup):
    """ms per call of fn (a sequence of kernel launches), captured once into a
    HIP graph and replayed: host launch overhead stays out of the figure.
    Timed with events on the stream the kernels run on."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(st)
    for _ in range(steps):
        g.replay()
    t1.record(st)
    t1.synchronize()
    return t0.elapsed_time(t1) / steps  # ms per step


def gpu_info(torch):
    p = torch.cuda.get_device_properties(0)
    return f"{p.name} ({getattr(p, 'gcnArchName', '?')}, {p.multi_processor_count} CUs)"


def cpu_reference(layers_np, lm_np, B, passes=5):
    """The reference's q4_k/q6_k_batch_matmul (oracle/_ref/libref.so, built from
    /root/reference with its Dockerfile recipe) on a bounded sample: the first
    layers' 7 matrices + lm_head at batch B."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    if not O.ref_available():
        return None
    cores = min(len(os.sched_getaffinity(0)), 16)
    os.environ.setdefault("OMP_PROC_BIND", "close")
    os.environ.setdefault("OMP_PLACES", "cores")
    ref = O.RefLib()
    ref.so.set_num_threads(cores)
    work = [(m, r, c, qt) for mats in layers_np for (m, r, c, qt) in mats] + [lm_np]
    x = {c: W.gen_x(np.random.default_rng(5), B, c) for c in (2048, 5632)}
    outs = {r: np.zeros(B * r, np.float32) for (_, r, _, _) in work}
    fns = {12: ref.so.q4_k_batch_matmul, 14: ref.so.q6_k_batch_matmul}
    nbytes = sum(w.size + B * (r + c) * 4 for (w, r, c, _) in work)

    def one():
        for (w, r, c, qt) in work:
            fns[qt](w.ctypes.data_as(K.cu), x[c].ctypes.data_as(K.cf), outs[r].ctypes.data_as(K.cf), r, c, B)
    for _ in range(3):
        one()
    ts = []
    for _ in range(passes):
        t = time.perf_counter()
        one()
        ts.append(time.perf_counter() - t)
    med = float(np.median(ts))
    return {"value": round(nbytes / med / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "reference",
            "sample": f"q4_k/q6_k_batch_matmul (oracle/_ref, AVX2+OpenMP, {cores} threads) over "
                      f"{len(layers_np)} TinyLlama layers (7 matrices each) + lm_head, B={B}, "
                      f"{nbytes / 1e6:.1f} MB per pass, median of {passes} passes after 3 warmups",
            "ms_per_pass": round(med * 1e3, 3)}


MFMA_BF16_PEAK_TFLOPS = 2500.0


def cpu_batch_matmul_reference(name, raw_np, R, C, M, reps=3):
    """The reference's *_batch_matmul (oracle/_ref, AVX2 + OpenMP) on one matrix at batch M:
    median seconds per call after one warm-up, or None when the reference build is absent."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    if not O.ref_available():
        return None, 0
    cores = min(len(os.sched_getaffinity(0)), 16)
    ref = O.RefLib()
    ref.so.set_num_threads(cores)
    fn = getattr(ref.so, name)
    x = W.gen_x(np.random.default_rng(6), M, C)
    out = np.zeros(M * R, np.float32)
    call = lambda: fn(raw_np.ctypes.data_as(K.cu), x.ctypes.data_as(K.cf), out.ctypes.data_as(K.cf), R, C, M)  # noqa: E731
    call()
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        call()
        ts.append(time.perf_counter() - t)
    return float(np.median(ts)), cores


def bench_prefill(torch, dev, args, with_cpu=False):
    """Q4_K gate/up 5632x2048 and Q6_K down 2048x5632 at M in {128, 512, 1280}
    bf16-valued activations, *_batch_matmul semantics, through the MFMA GEMM; with_cpu adds
    the reference's q4_k/q6_k_batch_matmul at M = 128 on the host cores."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    out = {}
    mats = {"gate_q4k": (K.Q4_K_GGML, W.QT_Q4_K, 5632, 2048), "down_q6k": (K.Q6_K_SEQ, W.QT_Q6_K, 2048, 5632)}
    cpu_names = {"gate_q4k": "q4_k_batch_matmul", "down_q6k": "q6_k_batch_matmul"}
    for name, (sem, qt, R, C) in mats.items():
        raw = W.gen_weights_torch(gen, qt, R, C)
        if with_cpu:
            sec, cores = cpu_batch_matmul_reference(cpu_names[name], raw.cpu().numpy(), R, C, 128)
            if sec:
                tf = 2.0 * R * C * 128 / sec / 1e12
                out.setdefault("cpu_baseline", {})[f"{name}_M128"] = {
                    "value": round(tf, 4), "unit": "TFLOP/s", "cores": cores, "kind": "reference",
                    "ms": round(sec * 1e3, 2),
                    "sample": f"{cpu_names[name]} (oracle/_ref, AVX2+OpenMP, {cores} threads), B=128, median of 3"}
                print(f"[bench] CPU reference {cpu_names[name]} M=128: {sec * 1e3:.1f} ms, {tf * 1e3:.1f} GFLOP/s",
                      file=sys.stderr, flush=True)
        packed = dev.pack(sem, raw, R, C)
        for M in (128, 512, 1280):
            x = torch.randn(M, C, device="cuda", generator=gen).bfloat16().float()
            o = torch.empty(M, R, device="cuda")
            ws = dev.workspace(sem, C, M, x.device, R)
            ms = time_region(torch, lambda: dev.gemv(sem, packed, x, R, C, out=o, ws=ws), max(5, args.steps), args.warmup)
            flops = 2.0 * R * C * M
            out[f"{name}_M{M}"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
                                   "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)}
            print(f"[bench] prefill {name} M={M}: {ms * 1e3:.1f} us, {out[f'{name}_M{M}']['TFLOP/s']} TFLOP/s",
                  file=sys.stderr, flush=True)
    return out


def bench_moe(torch, dev, args, tag, with_cpu, sizes=(1, 1280)):
    """one MoE FFN layer (all experts resident) at decode
    batch 1 and at 10 x 128 = 1280 tokens; tokens/s = tokens / layer time."""
    wl = W.moe_workload(tag, max(sizes))
    c = wl["cfg"]
    N, E, Kk, M = c["N"], c["E"], c["K"], c["M"]
    qts = wl["qts"]
    renorm = 1
    gates, ups, downs = wl["gates"], wl["ups"], wl["downs"]
    router_np, x_np = wl["router"], wl["x"]
    router = torch.from_numpy(router_np).cuda()
    layer = dev.moe_prepare(qts, N, M, E, Kk, gates, ups, downs, router, renorm)
    x = torch.from_numpy(x_np).cuda()
    res = {}
    wbytes_expert = sum(W.row_bytes(q, cols) * rows for q, rows, cols in ((qts[0], M, N), (qts[1], M, N), (qts[2], N, M)))
    for Tn in sizes:
        xs = x[:Tn].contiguous()
        o = torch.empty(Tn, N, device="cuda")
        layer.workspace(Tn)
        ms = time_region(torch, lambda: layer.forward(xs, out=o), max(5, args.steps), args.warmup)
        idx = torch.empty(Tn, Kk, dtype=torch.int32, device="cuda")
        layer.forward(xs, idx=idx)
        n_exp = int(torch.unique(idx).numel())
        flops = 2.0 * Tn * Kk * (3 * M * N) + 2.0 * Tn * N * E
        nbytes = n_exp * wbytes_expert + E * N * 4 + 2 * Tn * N * 4
        r = {"us": round(ms * 1e3, 1), "tokens/s": round(Tn / (ms * 1e-3), 1), "experts_touched": n_exp,
             "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2)}
        if Tn == 1:
            r["hbm_frac"] = round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        else:
            r["mfma_frac"] = round(flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)
        res[f"T{Tn}"] = r
        print(f"[bench] MoE {tag} T={Tn}: {ms * 1e3:.1f} us, {r['tokens/s']} tokens/s", file=sys.stderr, flush=True)
    if with_cpu:
        res["cpu_baseline"] = cpu_moe_reference(tag, qts, N, M, E, Kk, gates, ups, downs, router_np, x_np)
    del layer
    torch.cuda.empty_cache()
    return res


def cpu_moe_reference(tag, qts, N, M, E, Kk, gates, ups, downs, router_np, x_np, n_tok=16):
    """The reference's moe_forward_omp (oracle/_ref, AVX2 + OpenMP) per token with
    the renormalised C routing, on the first n_tok tokens of the same workload."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    if not O.ref_available():
        return None
    cores = min(len(os.sched_getaffinity(0)), 16)
    ref = O.RefLib()
    ref.so.set_num_threads(cores)
    orc = O.Oracle()
    idx, w = orc.route(router_np, x_np[:n_tok], Kk, renorm=True)
    need = sorted(set(int(e) for e in idx.ravel()))
    host = {e: (gates[e].cpu().numpy(), ups[e].cpu().numpy(), downs[e].cpu().numpy()) for e in need}
    dummy = host[need[0]]
    g = [host.get(e, dummy)[0] for e in range(E)]
    u = [host.get(e, dummy)[1] for e in range(E)]
    d = [host.get(e, dummy)[2] for e in range(E)]
    ref.moe_forward(g, u, d, x_np[0], M, N, qts, idx[0], w[0])   # warm-up
    t0 = time.perf_counter()
    for t in range(n_tok):
        ref.moe_forward(g, u, d, x_np[t], M, N, qts, idx[t], w[t])
    dt = time.perf_counter() - t0
    return {"value": round(n_tok / dt, 2), "unit": "tokens/s", "cores": cores, "kind": "reference",
            "sample": f"moe_forward_omp (oracle/_ref) on {n_tok} tokens of the {tag} workload, C routing "
                      f"(renormalised top-{Kk}) precomputed, {cores} OpenMP threads"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported: the multi-GPU sharding "
              "(row-sharded GEMV, expert-parallel MoE) is a design in DESIGN.md, not a run.", file=sys.stderr)
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = K.DeviceOps()
    torch.cuda.set_device(0)
    if args.kernel:
        kernel_only(torch, dev, args.kernel)
        return
    rng = np.random.default_rng(2)
    n_layers = W.TINYLLAMA_LAYERS
    print(f"[bench] building {n_layers} TinyLlama layers + lm_head on {gpu_info(torch)}", file=sys.stderr, flush=True)
    layers, lm = build_tinyllama(dev, rng, n_layers)
    allm = [m for mats in layers for (_, m) in mats] + [lm]

    def make_pass(B):
        xs = {c: torch.randn(B, c, device="cuda") for c in (2048, 5632)}
        outs = {m.rows: torch.empty(B, m.rows, device="cuda") for m in allm}
        ws = {}

        def run():
            for m in allm:
                dev.gemv(m.sem, m.packed, xs[m.cols], m.rows, m.cols, out=outs[m.rows], ws=ws.get(m.cols))
        return run

    results = {}
    for B in (1, 4, 8):
        ms = time_region(torch, make_pass(B), args.steps if B == 1 else max(3, args.steps // 2), args.warmup)
        nbytes = sum(algo_bytes(m, B) for m in allm)
        results[B] = (ms, nbytes / (ms * 1e-3) / 1e9)
        print(f"[bench] TinyLlama set B={B}: {ms:.3f} ms/pass, {results[B][1]:.1f} GB/s", file=sys.stderr, flush=True)

    # dominant kernel: the fused Q4_K gate/up GEMV (11264x2048) at B=1, rotating over the 22 layer copies
    gu = [m for mats in layers for (n, m) in mats if n == "gate_up"]
    x1 = torch.randn(1, 2048, device="cuda")
    o1 = torch.empty(1, 11264, device="cuda")

    def gu_pass():
        for m in gu:
            dev.gemv(m.sem, m.packed, x1, m.rows, m.cols, out=o1)
    ms_gu = time_region(torch, gu_pass, max(5, args.steps), args.warmup)
    per_launch_s = ms_gu * 1e-3 / len(gu)
    gu_bytes = algo_bytes(gu[0], 1)
    achieved = gu_bytes / per_launch_s / 1e9
    print(f"[bench] Q4_K gate_up 11264x2048 GEMV: {per_launch_s * 1e6:.2f} us/launch, {achieved:.1f} GB/s",
          file=sys.stderr, flush=True)

    # Q8_0 GEMV 5632x2048 B=1, 24 rotated copies (295 MB)
    q8 = [Matrix(dev, K.Q8_0, W.gen_weights(np.random.default_rng(100 + i), W.QT_Q8_0, 5632, 2048), 5632, 2048)
          for i in range(24)]
    xq = torch.from_numpy(W.gen_x(np.random.default_rng(0), 1, 2048)).cuda()
    oq = torch.empty(1, 5632, device="cuda")

    def q8_pass():
        for m in q8:
            dev.gemv(m.sem, m.packed, xq, 5632, 2048, out=oq)
    ms_q8 = time_region(torch, q8_pass, max(5, args.steps), args.warmup)
    q8_gbs = algo_bytes(q8[0], 1) / (ms_q8 * 1e-3 / len(q8)) / 1e9
    print(f"[bench] Q8_0 5632x2048 GEMV: {ms_q8 * 1e3 / len(q8):.2f} us/launch, {q8_gbs:.1f} GB/s", file=sys.stderr,
          flush=True)
    q8_cpu = None
    if not args.no_cpu:
        # the reference's q8_0_batch_matmul at B = 1 on the host cores, 24 rotating matrices (over 280 MB)
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        if O.ref_available():
            w8 = [W.gen_weights(np.random.default_rng(100 + i), W.QT_Q8_0, 5632, 2048) for i in range(24)]
            cores = min(len(os.sched_getaffinity(0)), 16)
            ref = O.RefLib()
            ref.so.set_num_threads(cores)
            xh = W.gen_x(np.random.default_rng(0), 1, 2048)
            oh = np.zeros(5632, np.float32)
            ref.so.q8_0_batch_matmul(w8[0].ctypes.data_as(K.cu), xh.ctypes.data_as(K.cf), oh.ctypes.data_as(K.cf),
                                     5632, 2048, 1)   # warm-up
            t0 = time.perf_counter()
            for w in w8 * 2:
                ref.so.q8_0_batch_matmul(w.ctypes.data_as(K.cu), xh.ctypes.data_as(K.cf), oh.ctypes.data_as(K.cf),
                                         5632, 2048, 1)
            sec = (time.perf_counter() - t0) / (2 * len(w8))
            q8_cpu = {"value": round(algo_bytes(q8[0], 1) / sec / 1e9, 2), "unit": "GB/s", "cores": cores,
                      "kind": "reference", "us": round(sec * 1e6, 1),
                      "sample": f"q8_0_batch_matmul (oracle/_ref, AVX2+OpenMP, {cores} threads), B=1, "
                                f"48 calls over 24 rotating 12 MB matrices"}
            print(f"[bench] CPU reference q8_0_batch_matmul: {sec * 1e6:.1f} us, {q8_cpu['value']} GB/s",
                  file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu:
        r2 = np.random.default_rng(2)
        sample_layers = []
        for _ in range(2):
            sample_layers.append([(W.gen_weights(r2, qt, rows, cols), rows, cols, qt)
                                  for (_, rows, cols, qt) in W.TINYLLAMA_MATS])
        name, rows, cols, qt = W.TINYLLAMA_LM_HEAD
        cpu = cpu_reference(sample_layers, (W.gen_weights(r2, qt, rows, cols), rows, cols, qt), 1)
        if cpu:
            print(f"[bench] CPU reference: {cpu['value']} GB/s on {cpu['cores']} threads", file=sys.stderr, flush=True)

    extra = {}
    if not args.no_extra:
        extra["configs2_prefill_gemm"] = bench_prefill(torch, dev, args, with_cpu=not args.no_cpu)
        extra["configs3_gptoss_moe"] = bench_moe(torch, dev, args, "gptoss", with_cpu=not args.no_cpu)
        extra["configs4_qwen3_moe"] = bench_moe(torch, dev, args, "qwen3", with_cpu=not args.no_cpu)

    ms1, gbs1 = results[1]
    line = {
        "metric": "quant GEMV HBM GB/s (% of peak) + MoE-FFN layer tokens/s, batch 1 and 10",
        "value": round(gbs1, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms1, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (fp32 activations as three int8 digit planes, int32 dot4 per 16-weight run, fp32 scales and accumulation)",
        "data": "synthetic (BASELINE.json distributions, seeded)",
        "config": {"workload": "configs[1] TinyLlama-1.1B Q4_K_M matmul set (22 layers + lm_head), decode B=1, "
                               "*_batch_matmul semantics, qkv and gate/up fused per layer (89 launches per pass)",
                   "hbm_frac": round(gbs1 / HBM_PEAK_GBS, 4),
                   "B4": {"ms_per_pass": round(results[4][0], 4), "GB/s": round(results[4][1], 1)},
                   "B8": {"ms_per_pass": round(results[8][0], 4), "GB/s": round(results[8][1], 1)},
                   "configs0_q8_0_gemv": {"us": round(ms_q8 * 1e3 / len(q8), 3), "GB/s": round(q8_gbs, 1),
                                          "hbm_frac": round(q8_gbs / HBM_PEAK_GBS, 4), "cpu_baseline": q8_cpu}},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": GATE_UP_TRAFFIC_BYTES,
                     "kernel": f"k_gemv_p<Q4_K_GGML,B=1> fused gate+up 11264x2048 ({gu_bytes:,} algorithmic B/launch)"},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
