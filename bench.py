"""Benchmark of the quantised-matmul + MoE-FFN hot path on one MI355X.

Headline: the TinyLlama-1.1B Q4_K_M matmul set
(22 layers x {qkv, o, gate/up (Q4_K), down (Q6_K)} + the Q6_K lm_head, 22
distinct weight copies = 664 MB, beyond the 256 MB Infinity Cache) run as a
decode step at batch 1 with the *_batch_matmul semantics (CE:255-378): each
layer's RMSNorm is fused into the qkv and gate/up GEMVs, the residual adds
into the o and down GEMVs and the SiLU product into the down GEMV's staging,
and every matrix consumes the previous one's output (the attention between
qkv and o is outside this path: o takes the q rows).  One step = one decode
pass (89 dependent launches).  Inputs are resident in HBM before the timed
region.  `value` = algorithmic HBM bytes of the pass (weights + activations in
+ fp32 outputs) / time.

Also in the JSON line: the same pass at batch 4 and 8; the 89 GEMVs with
independent inputs (the earlier form of this metric); each matrix kind's
per-launch time next to a plain read of the same bytes in one launch; the
Q8_0 GEMV of configs[0]; the prefill GEMMs of configs[2]; the MoE layers of
configs[3] / configs[4] at T = 1 (hot and cold experts) and T = 1280; the
drop-in host-ABI latency per call; the roofline of the dominant kernel (HIP
events on the stream it runs on); and the reference's own C (oracle/_ref,
AVX2 + OpenMP) timed on this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import os


def host_cpu():
    """(threads to use, CPU description): the physical cores this process may
    run on, at most 16 (one GPU's share of the box's cores), and the host's
    model name with its family / model / stepping numbers and physical core
    count (sockets x cores) from /proc/cpuinfo."""
    aff = os.sched_getaffinity(0)
    model, cores, all_cores, cur, ids = "unknown", set(), set(), {}, {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f.read().split("\n") + [""]:
                if not line.strip():
                    if cur.get("processor") is not None:
                        key = (cur.get("physical id", "0"), cur.get("core id", cur["processor"]))
                        all_cores.add(key)
                        if int(cur["processor"]) in aff:
                            cores.add(key)
                    cur = {}
                    continue
                k, _, v = line.partition(":")
                k = k.strip()
                cur[k] = v.strip()
                if k == "model name":
                    model = v.strip()
                if k in ("cpu family", "model", "stepping") and k not in ids:
                    ids[k] = v.strip()
    except OSError:
        pass
    n = len(cores)
    if n < max(1, len(aff) // 4):   # a virtualised cpuinfo that does not list the cores this process may use
        n = len(aff)
    desc = {"model_name": model, "family": ids.get("cpu family"), "model": ids.get("model"),
            "stepping": ids.get("stepping"), "physical_cores": len(all_cores), "logical_cpus_visible": len(aff)}
    return max(1, min(n, 16)), desc


# The host reference runs in a child process (bench.py --cpu-leg NAME) that
# imports no torch and has its OpenMP binding (OMP_PROC_BIND=close,
# OMP_PLACES=cores, BENCHMARK_CHANGELOG.md:66-69) in the environment from its
# start; this process keeps its OpenMP runtime unbound, because a bound
# runtime pins the initial thread to one core, which the child would inherit.
CPU_THREADS, CPU_MODEL = host_cpu()

import argparse  # noqa: E402
import ctypes  # noqa: E402
import json  # noqa: E402
import sys  # noqa: E402
import time  # noqa: E402

import numpy as np  # noqa: E402

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from mojollama_amd import kernels as K  # noqa: E402
from mojollama_amd import workloads as W  # noqa: E402
from mojollama_amd.decode_chain import EPS, DecodeChain, Matrix, algo_bytes, build_tinyllama  # noqa: E402,F401

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
# HBM bytes per launch of a decode-chain GEMV kind, from FETCH_SIZE /
# WRITE_SIZE counter runs (bench.py --kernel gate_up) calibrated on a copy of
# known size (bench.py --kernel copy): FETCH 6526.2 KiB x 1.99982 + WRITE
# 22.0 KiB for the fused gate+up launch.  profiles/gemv_gate_up_q4k_traffic.md
# gives the commands and raw values; re-measure after any change to that kernel.
ROOFLINE_TRAFFIC_BYTES = {"gate_up": 13350224}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the host-CPU reference timing")
    ap.add_argument("--no-extra", action="store_true", help="only the configs[1] decode set")
    ap.add_argument("--cpu-leg", choices=CPU_LEGS, help="(internal) run one host-CPU reference leg and print it")
    ap.add_argument("--kernel", choices=("gate_up", "down", "gate_up_b8", "down_b8", "copy", "gemm_gate",
                                         "gemm_down", "moe_gptoss", "moe_qwen3", "long_q4k", "long_mxfp4"),
                    help="run only a few launches of one kernel and exit, for counter runs (rocprofv3 --pmc): the "
                         "decode chain's fused gate+up or down GEMV (50), a 256 MiB device copy to calibrate bytes "
                         "(50), the configs[2] GEMMs (10), the MoE layers at T = 1280 (5 forwards), or the "
                         "16384 x 16384 batch-1 GEMV (20)")
    return ap.parse_args()


def ref_lib():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    if not O.ref_available():
        return None, None
    return O, O.RefLib()


def median_time(fn, reps, warm=3):
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return float(np.median(ts))


def cpu_tag(cores, model):
    """cores: the threads the reference ran on; model: host_cpu()'s description."""
    if isinstance(model, dict):
        model = (f"{model['model_name']} (family {model['family']} model {model['model']} stepping "
                 f"{model['stepping']}; {model['physical_cores']} physical cores, {model['logical_cpus_visible']} "
                 "logical CPUs visible to this process)")
    return {"cores": cores, "cpu_model": model, "kind": "reference", "omp_proc_bind": os.environ.get("OMP_PROC_BIND"),
            "omp_places": os.environ.get("OMP_PLACES")}


# ------------------------------------------------------------------ GPU helpers
def time_region(torch, fn, steps, warmup):
    """ms per call of fn (a sequence of kernel launches), captured once into a
    HIP graph and replayed: host launch overhead stays out of the figure.
    Timed with events on the stream the graph replays on."""
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


def kernel_only(torch, dev, which):
    """A few launches of one kernel, nothing else on the GPU besides set-up."""
    if which == "copy":
        a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        a.fill_(1)
        torch.cuda.synchronize()
        for _ in range(50):
            b.copy_(a)
    elif which in ("gemm_gate", "gemm_down"):
        # configs[2] prefill at M = 1280: the Q4_K gate (5632x2048) or the Q6_K down (2048x5632), 10 launches
        gen = torch.Generator(device="cuda").manual_seed(3)
        sem, qt, R, C = (K.Q4_K_GGML, W.QT_Q4_K, 5632, 2048) if which.endswith("gate") else \
            (K.Q6_K_SEQ, W.QT_Q6_K, 2048, 5632)
        packed = dev.pack(sem, W.gen_weights_torch(gen, qt, R, C), R, C)
        x = torch.randn(1280, C, device="cuda", generator=gen).bfloat16().float()
        o = torch.empty(1280, R, device="cuda")
        ws = dev.workspace(sem, C, 1280, x.device, R)
        for _ in range(10):
            dev.gemv(sem, packed, x, R, C, out=o, ws=ws)
    elif which in ("long_q4k", "long_mxfp4"):
        # the batch-1 decode GEMV on a 16384 x 16384 matrix (bench_long_gemv), 20 launches
        # rotating over copies that together exceed the Infinity Cache
        gen = torch.Generator(device="cuda").manual_seed(5)
        sem, qt = (K.Q4_K_GGML, W.QT_Q4_K) if which.endswith("q4k") else (K.MXFP4, W.QT_MXFP4)
        copies, _ = long_gemv_copies(torch, dev, gen, sem, qt)
        x = torch.randn(1, LONG_GEMV, device="cuda", generator=gen)
        o = torch.empty(1, LONG_GEMV, device="cuda")
        for i in range(20):
            dev.gemv(sem, copies[i % len(copies)], x, LONG_GEMV, LONG_GEMV, out=o)
    elif which in ("moe_gptoss", "moe_qwen3"):
        # the MoE layer at T = 1280, 5 forwards
        wl = W.moe_workload(which.split("_")[1], 1280)
        c = wl["cfg"]
        layer = dev.moe_prepare(wl["qts"], c["N"], c["M"], c["E"], c["K"], wl["gates"], wl["ups"], wl["downs"],
                                torch.from_numpy(wl["router"]).cuda(), 1)
        x = torch.from_numpy(wl["x"]).cuda()
        o = torch.empty(1280, c["N"], device="cuda")
        for _ in range(5):
            layer.forward(x, out=o)
    else:
        # the decode chain's fused gate+up or down GEMV; *_b8: at batch 8 (the integer-MFMA kernel)
        B = 8 if which.endswith("_b8") else 1
        layers, lm, on = build_tinyllama(dev, np.random.default_rng(2), 1)
        ch = DecodeChain(torch, dev, layers, lm, on, B)
        ch.run()
        torch.cuda.synchronize()
        L = layers[0]
        for _ in range(50):
            if which.startswith("gate_up"):
                dev.gemv_fused(L["gate_up"].sem, L["gate_up"].packed, ch.xb, 5632, 2048, ch.f_gu[0], out=ch.h,
                               ws=ch.ws)
            else:
                dev.gemv_fused(L["down"].sem, L["down"].packed, ch.h, 2048, 5632, ch.f_down, out=ch.xa, ws=ch.ws)
    torch.cuda.synchronize()
    print(f"[bench] {which}: launches done", file=sys.stderr, flush=True)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------------ legs
def bench_kinds(torch, dev, layers, lm, out_norm, args):
    """Each matrix kind at B=1, rotating over the 22 layer copies: the chain's
    fused GEMV per launch, and a plain read of the same packed bytes in one
    launch (mllm_read_probe): the ceiling a single launch over those bytes has."""
    sink = torch.empty(64, dtype=torch.uint8, device="cuda")
    ch = DecodeChain(torch, dev, layers, lm, out_norm, 1)
    ch.run()
    res = {}
    kinds = {
        "qkv": (lambda L: dev.gemv_fused(L["qkv"].sem, L["qkv"].packed, ch.xa, 2560, 2048, ch.f_qkv[0], out=ch.qkv,
                                         ws=ch.ws)),
        "o": (lambda L: dev.gemv_fused(L["o"].sem, L["o"].packed, ch.qkv.data_ptr(), 2048, 2048, ch.f_o, out=ch.xb,
                                       ws=ch.ws, B=1)),
        "gate_up": (lambda L: dev.gemv_fused(L["gate_up"].sem, L["gate_up"].packed, ch.xb, 5632, 2048, ch.f_gu[0],
                                             out=ch.h, ws=ch.ws)),
        "down": (lambda L: dev.gemv_fused(L["down"].sem, L["down"].packed, ch.h, 2048, 5632, ch.f_down, out=ch.xa,
                                          ws=ch.ws)),
    }
    for name, fn in kinds.items():
        ms = time_region(torch, lambda: [fn(L) for L in layers], max(5, args.steps), args.warmup)
        mats = [L[name] for L in layers]
        rd = time_region(torch, lambda: [dev.so.mllm_read_probe(m.packed.data_ptr(), m.packed.numel() // 16 * 16,
                                                                sink.data_ptr(), dev._stream()) for m in mats],
                         max(5, args.steps), args.warmup)
        us, rus = ms * 1e3 / len(layers), rd * 1e3 / len(layers)
        gbs = algo_bytes(mats[0], 1) / (us * 1e-6) / 1e9
        res[name] = {"us": round(us, 2), "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                     "plain_read_us": round(rus, 2), "frac_of_plain_read": round(rus / us, 3),
                     "bytes": algo_bytes(mats[0], 1)}
        log(f"{name}: {us:.2f} us/launch ({gbs:.0f} GB/s), plain read of the same bytes {rus:.2f} us")
    # lm_head: one copy; each launch follows a 300+ MB read of the layer weights so it starts cold
    flush = [L["gate_up"] for L in layers]
    fl = lambda: [dev.so.mllm_read_probe(m.packed.data_ptr(), m.packed.numel() // 16 * 16, sink.data_ptr(),  # noqa
                                         dev._stream()) for m in flush]
    t_fl = time_region(torch, fl, max(5, args.steps), args.warmup)
    t_lm = time_region(torch, lambda: (fl(), dev.gemv_fused(lm.sem, lm.packed, ch.xa, 32000, 2048, ch.f_lm,
                                                             out=ch.logits, ws=ch.ws)), max(5, args.steps), args.warmup)
    t_rd = time_region(torch, lambda: (fl(), dev.so.mllm_read_probe(lm.packed.data_ptr(), lm.packed.numel() // 16 * 16,
                                                                     sink.data_ptr(), dev._stream())),
                       max(5, args.steps), args.warmup)
    us, rus = (t_lm - t_fl) * 1e3, (t_rd - t_fl) * 1e3
    gbs = algo_bytes(lm, 1) / (us * 1e-6) / 1e9
    res["lm_head"] = {"us": round(us, 2), "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                      "plain_read_us": round(rus, 2), "frac_of_plain_read": round(rus / us, 3),
                      "bytes": algo_bytes(lm, 1)}
    log(f"lm_head: {us:.2f} us ({gbs:.0f} GB/s), plain read {rus:.2f} us")
    return res


LONG_GEMV = 16384   # rows = columns of the long-matrix GEMV


def long_gemv_copies(torch, dev, gen, sem, qt):
    """Packed copies of one 16384 x 16384 matrix, two or more so that together
    they exceed the 256 MB Infinity Cache (launches rotate over them)."""
    R = C = LONG_GEMV
    raw = W.gen_weights_torch(gen, qt, R, C)
    nbytes = raw.numel()
    copies = [dev.pack(sem, raw, R, C) for _ in range(max(2, -(-320_000_000 // nbytes)))]
    del raw
    return copies, nbytes


def bench_long_gemv(torch, dev, args):
    """The batch-1 decode GEMV on one long matrix per format (16384 x 16384,
    143-285 MB: a launch long enough for its steady rate to show), against a
    plain read of the same bytes; each timed replay runs 8 launches rotating
    over copies that together exceed the Infinity Cache."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    sink = torch.empty(64, dtype=torch.uint8, device="cuda")
    res = {}
    R = C = LONG_GEMV
    reps = 8
    for name, sem, qt in (("Q4_K", K.Q4_K_GGML, W.QT_Q4_K), ("Q6_K", K.Q6_K_SEQ, W.QT_Q6_K),
                          ("Q8_0", K.Q8_0, W.QT_Q8_0), ("MXFP4", K.MXFP4, W.QT_MXFP4)):
        copies, nbytes = long_gemv_copies(torch, dev, gen, sem, qt)
        x = torch.randn(1, C, device="cuda")
        o = torch.empty(1, R, device="cuda")

        def run():
            for i in range(reps):
                dev.gemv(sem, copies[i % len(copies)], x, R, C, out=o)

        def read():
            for i in range(reps):
                p = copies[i % len(copies)]
                dev.so.mllm_read_probe(p.data_ptr(), p.numel() // 16 * 16, sink.data_ptr(), dev._stream())
        ms = time_region(torch, run, max(5, args.steps), args.warmup) / reps
        rd = time_region(torch, read, max(5, args.steps), args.warmup) / reps
        gbs = (nbytes + 4 * (R + C)) / (ms * 1e-3) / 1e9
        res[name] = {"us": round(ms * 1e3, 1), "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                     "plain_read_us": round(rd * 1e3, 1), "frac_of_plain_read": round(rd / ms, 3),
                     "MB": round(nbytes / 1e6, 1), "copies": len(copies)}
        log(f"long GEMV {name} {R}x{C} B=1: {ms * 1e3:.1f} us, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%}); "
            f"plain read {rd * 1e3:.1f} us ({len(copies)} copies)")
        del copies
        torch.cuda.empty_cache()
    return res


def bench_q8(torch, dev, args):
    """Q8_0 GEMV 5632x2048 B=1 rotated over 24 copies (295 MB)."""
    sink = torch.empty(64, dtype=torch.uint8, device="cuda")
    raws = [W.gen_weights(np.random.default_rng(100 + i), W.QT_Q8_0, 5632, 2048) for i in range(24)]
    q8 = [Matrix(dev, K.Q8_0, r, 5632, 2048) for r in raws]
    xq = torch.from_numpy(W.gen_x(np.random.default_rng(0), 1, 2048)).cuda()
    oq = torch.empty(1, 5632, device="cuda")
    ms = time_region(torch, lambda: [dev.gemv(m.sem, m.packed, xq, 5632, 2048, out=oq) for m in q8],
                     max(5, args.steps), args.warmup)
    rd = time_region(torch, lambda: [dev.so.mllm_read_probe(m.packed.data_ptr(), m.packed.numel() // 16 * 16,
                                                            sink.data_ptr(), dev._stream()) for m in q8],
                     max(5, args.steps), args.warmup)
    us, rus = ms * 1e3 / len(q8), rd * 1e3 / len(q8)
    gbs = algo_bytes(q8[0], 1) / (us * 1e-6) / 1e9
    res = {"us": round(us, 3), "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
           "plain_read_us": round(rus, 2), "frac_of_plain_read": round(rus / us, 3)}
    log(f"Q8_0 5632x2048 GEMV: {us:.2f} us/launch, {gbs:.1f} GB/s; plain read {rus:.2f} us")
    # the drop-in host ABI per call: quant_matmul_omp(Q8_0) with x in / y out over PCIe and a sync
    lib = dev.so
    xh = W.gen_x(np.random.default_rng(0), 1, 2048)
    oh = np.zeros(5632, np.float32)
    call = lambda i: lib.quant_matmul_omp(raws[i % 24].ctypes.data_as(K.cu), xh.ctypes.data_as(K.cf),  # noqa: E731
                                          oh.ctypes.data_as(K.cf), 5632, 2048, 8)
    for i in range(24):
        call(i)   # uploads each matrix once
    ts = []
    for i in range(48):
        t = time.perf_counter()
        call(i)
        ts.append(time.perf_counter() - t)
    res["host_abi_quant_matmul_omp_us"] = round(float(np.median(ts)) * 1e6, 1)
    log(f"host-ABI quant_matmul_omp(Q8_0 5632x2048): {res['host_abi_quant_matmul_omp_us']} us per call")
    return res


def bench_prefill(torch, dev, args):
    """Q4_K gate/up 5632x2048 and Q6_K down 2048x5632 at M in {128, 512, 1280},
    *_batch_matmul semantics, through mllm_gemv (the fp16-plane GEMM: weights decoded
    from the packed bytes in registers, activations staged inside the timed region).
    Activations bf16-valued (one fp16 plane after scaling) and, at M=1280, general
    fp32 (two planes, twice the MFMA work)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    out = {}
    mats = {"gate_q4k": (K.Q4_K_GGML, W.QT_Q4_K, 5632, 2048), "down_q6k": (K.Q6_K_SEQ, W.QT_Q6_K, 2048, 5632)}
    for name, (sem, qt, R, C) in mats.items():
        raw = W.gen_weights_torch(gen, qt, R, C)
        packed = dev.pack(sem, raw, R, C)
        for M, act in ((128, "bf16"), (512, "bf16"), (1280, "bf16"), (1280, "fp32")):
            x = torch.randn(M, C, device="cuda", generator=gen)
            if act == "bf16":
                x = x.bfloat16().float()
            o = torch.empty(M, R, device="cuda")
            ws = dev.workspace(sem, C, M, x.device, R)
            ms = time_region(torch, lambda: dev.gemv(sem, packed, x, R, C, out=o, ws=ws), max(5, args.steps),
                             args.warmup)
            flops = 2.0 * R * C * M
            tf = round(flops / (ms * 1e-3) / 1e12, 1)
            key = f"{name}_M{M}" + ("" if act == "bf16" else "_fp32_act")
            out[key] = {"us": round(ms * 1e3, 2), "TFLOP/s": tf,
                        "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4), "activations": act}
            log(f"prefill {name} M={M} ({act} activations): {ms * 1e3:.1f} us, {tf} TFLOP/s")
    return out


def bench_moe(torch, dev, args, tag, sizes=(1, 1280)):
    """one MoE FFN layer (all experts resident) at decode
    batch 1 and at 10 x 128 = 1280 tokens; tokens/s = tokens / layer time.  T=1
    is timed twice: replaying one token (its experts stay in the caches) and
    cycling over 32 tokens whose expert sets together exceed the 256 MB
    Infinity Cache (each call streams its experts from HBM)."""
    wl = W.moe_workload(tag, max(sizes))
    c = wl["cfg"]
    N, E, Kk, M = c["N"], c["E"], c["K"], c["M"]
    qts = wl["qts"]
    gates, ups, downs = wl["gates"], wl["ups"], wl["downs"]
    router_np, x_np = wl["router"], wl["x"]
    router = torch.from_numpy(router_np).cuda()
    layer = dev.moe_prepare(qts, N, M, E, Kk, gates, ups, downs, router, 1)
    x = torch.from_numpy(x_np).cuda()
    res = {}
    wbytes_expert = sum(W.row_bytes(q, cols) * rows for q, rows, cols in ((qts[0], M, N), (qts[1], M, N), (qts[2], N, M)))

    def layer_bytes(n_exp, Tn):
        return n_exp * wbytes_expert + E * N * 4 + 2 * Tn * N * 4

    for Tn in sizes:
        xs = x[:Tn].contiguous()
        o = torch.empty(Tn, N, device="cuda")
        layer.workspace(Tn)
        ms = time_region(torch, lambda: layer.forward(xs, out=o), max(5, args.steps), args.warmup)
        idx = torch.empty(Tn, Kk, dtype=torch.int32, device="cuda")
        layer.forward(xs, idx=idx)
        n_exp = int(torch.unique(idx).numel())
        flops = 2.0 * Tn * Kk * (3 * M * N) + 2.0 * Tn * N * E
        nbytes = layer_bytes(n_exp, Tn)
        r = {"us": round(ms * 1e3, 1), "tokens/s": round(Tn / (ms * 1e-3), 1), "experts_touched": n_exp,
             "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2)}
        if Tn == 1:
            r["hbm_frac"] = round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
            r["note"] = "one token replayed: its experts stay in L2 / Infinity Cache"
        else:
            r["mfma_frac"] = round(flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)
        res[f"T{Tn}"] = r
        log(f"MoE {tag} T={Tn}: {ms * 1e3:.1f} us, {r['tokens/s']} tokens/s")
    # the batched path over load-time bf16 expert copies (mllm_moe_dense_experts:
    # MXFP4 matrices left on the bf16-tile GEMM, bit-identical results), where the
    # layer has any (none at configs[3] / configs[4]: the fp16-plane GEMM takes them)
    big = max(sizes)
    if big > 24:
        dl = dev.moe_prepare(qts, N, M, E, Kk, gates, ups, downs, router, 1)
        nbytes_dense = dl.dense_experts()
        if nbytes_dense > 0:
            xs = x[:big].contiguous()
            o = torch.empty(big, N, device="cuda")
            dl.workspace(big)
            ms = time_region(torch, lambda: dl.forward(xs, out=o), max(5, args.steps), args.warmup)
            flops = 2.0 * big * Kk * (3 * M * N) + 2.0 * big * N * E
            res[f"T{big}_dense_experts"] = {
                "us": round(ms * 1e3, 1), "tokens/s": round(big / (ms * 1e-3), 1),
                "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2),
                "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                "dense_copy_GB": round(nbytes_dense / 1e9, 2),
                "note": "expert matrices as load-time bf16 copies (exact for MXFP4), outputs bit-identical"}
            log(f"MoE {tag} T={big} over bf16 expert copies ({nbytes_dense / 1e9:.2f} GB): {ms * 1e3:.1f} us, "
                f"{big / (ms * 1e-3):.1f} tokens/s")
        del dl
    # cold decode: 32 single-token calls over distinct tokens per replay
    R = 32
    outs = [torch.empty(1, N, device="cuda") for _ in range(R)]
    xs1 = [x[t:t + 1].contiguous() for t in range(R)]
    layer.workspace(1)
    ms = time_region(torch, lambda: [layer.forward(xs1[t], out=outs[t]) for t in range(R)], max(5, args.steps // 2),
                     args.warmup)
    idx = torch.empty(R, Kk, dtype=torch.int32, device="cuda")
    layer.forward(x[:R].contiguous(), idx=idx)
    touched = int(torch.unique(idx).numel())
    per = ms / R
    nb = layer_bytes(Kk, 1)
    res["T1_cold"] = {"us": round(per * 1e3, 1), "tokens/s": round(1 / (per * 1e-3), 1),
                      "GB/s": round(nb / (per * 1e-3) / 1e9, 1), "hbm_frac": round(nb / (per * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                      "experts_touched_per_cycle": touched,
                      "bytes_per_cycle_MB": round(touched * wbytes_expert / 1e6, 1),
                      "note": f"{R} distinct tokens per replay, {Kk} experts each; the cycle's experts exceed the "
                              "256 MB Infinity Cache when bytes_per_cycle_MB > 256"}
    log(f"MoE {tag} T=1 cold: {per * 1e3:.1f} us ({touched} experts, {touched * wbytes_expert / 1e6:.0f} MB per cycle)")
    # the drop-in host ABI: moe_forward_omp (host pointers) per call, on the
    # routing the layer itself computes for these tokens
    n_tok = 24
    idx_d = torch.empty(n_tok, Kk, dtype=torch.int32, device="cuda")
    w_d = torch.empty(n_tok, Kk, dtype=torch.float32, device="cuda")
    layer.forward(x[:n_tok].contiguous(), idx=idx_d, w=w_d)
    idx_h, w_h = idx_d.cpu().numpy(), w_d.cpu().numpy()
    need = sorted(set(int(e) for e in idx_h.ravel()))
    host = {e: (gates[e].cpu().numpy(), ups[e].cpu().numpy(), downs[e].cpu().numpy()) for e in need}
    dummy = host[need[0]]
    call = MoECall([[host.get(e, dummy)[i] for e in range(E)] for i in range(3)], M, N, qts, Kk)
    call.prepare(x_np[:n_tok], idx_h, w_h)
    for t in range(n_tok):
        call(dev.so, t)     # first calls upload the experts
    ts = []
    for t in range(n_tok):
        s0 = time.perf_counter()
        call(dev.so, t)
        ts.append(time.perf_counter() - s0)
    res["host_abi_moe_forward_omp_us"] = round(float(np.median(ts)) * 1e6, 1)
    log(f"host-ABI moe_forward_omp ({tag}): {res['host_abi_moe_forward_omp_us']} us per call")
    del layer
    torch.cuda.empty_cache()
    return res


def bench_attention(torch, dev, args):
    """Decode attention (gqa_attention.c semantics) at gpt-oss-20b's head layout
    (64 query / 8 KV heads of 64) over 4096 cached positions: B=1 on a
    contiguous cache and B=8 sequences on 64-row pages scattered by a random
    page table.  Bytes = the K and V rows read + q and out; each replay cycles
    over copies of the caches that together exceed the 256 MB Infinity Cache."""
    nh, nkh, hd, S = 64, 8, 64, 4096
    res = {}
    for B, page in ((1, 0), (8, 64)):
        row = nkh * hd
        per = B * S * row * 4 * 2
        R = max(2, -(-600_000_000 // per))
        kvs = []
        for _ in range(R):
            k = torch.randn(B * S, row, device="cuda")
            v = torch.randn(B * S, row, device="cuda")
            if page:
                n_pages = B * S // page
                tables = torch.randperm(n_pages, device="cuda").to(torch.int32).view(B, S // page).contiguous()
                kvs.append(dev.kv_view(k, v, block_tables=tables, page_size=page, n_pages=n_pages))
            else:
                kvs.append(dev.kv_view(k, v, seq_stride=S * row))
        lens = torch.full((B,), S, dtype=torch.int32, device="cuda")
        q = torch.randn(B, nh * hd, device="cuda")
        out = torch.empty(B, nh * hd, device="cuda")
        ws = torch.empty(dev.so.mllm_gqa_workspace_size(B, nh, hd, S), dtype=torch.uint8, device="cuda")
        ms = time_region(torch, lambda: [dev.gqa_decode(K.ATTN_GQA_C, q, kv, lens, S, nh, nkh, hd, out=out, ws=ws)
                                         for kv in kvs], max(5, args.steps // 2), args.warmup) / R
        nbytes = per + B * nh * hd * 8
        key = f"B{B}_{'paged' + str(page) if page else 'contiguous'}"
        res[key] = {"us": round(ms * 1e3, 2), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                    "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "seq": S}
        log(f"attention {key}: {ms * 1e3:.2f} us, {res[key]['GB/s']} GB/s")
        del kvs
        torch.cuda.empty_cache()
    return res


def bench_gptoss(torch, dev, args):
    """gptoss_forward's device step (mllm_gptoss_step) at gpt-oss-20b shapes:
    24 layers, N 2880, 64/8 heads of 64, MXFP4 q/k/v/o, 32 MXFP4 experts of
    2880 (top-4, expert e of layer l = matrix l + e as GO:179-181 index them),
    vocab 201088, with 512 positions already cached; one token per step,
    replayed from a captured graph (each replay appends a row)."""
    L, N, NH, NKH, HD, E, Kk, M, V, ctx = 24, 2880, 64, 8, 64, 32, 4, 2880, 201088, 1024
    inner, kvd = NH * HD, NKH * HD
    gen = torch.Generator(device="cuda").manual_seed(11)
    mx = lambda r, c: W.gen_weights_torch(gen, W.QT_MXFP4, r, c).cpu().numpy()  # noqa: E731
    f32 = lambda *sh, sc=1.0: (torch.randn(*sh, generator=gen, device="cuda") * sc).cpu().numpy()  # noqa: E731
    wq = [mx(inner, N) for _ in range(L)]
    wk = [mx(kvd, N) for _ in range(L)]
    wv = [mx(kvd, N) for _ in range(L)]
    wo = [mx(N, inner) for _ in range(L)]
    an = [1 + f32(N, sc=0.1) for _ in range(L)]
    fn = [1 + f32(N, sc=0.1) for _ in range(L)]
    router = [f32(E, N, sc=0.05) for _ in range(L)]
    ge = [mx(M, N) for _ in range(L - 1 + E)]
    ue = [mx(M, N) for _ in range(L - 1 + E)]
    de = [mx(N, M) for _ in range(L - 1 + E)]
    wout = mx(V, N)
    theta = f32(ctx, HD // 2)
    cos_t, sin_t = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
    arr_u = lambda xs: (K.cu * len(xs))(*[a.ctypes.data_as(K.cu) for a in xs])  # noqa: E731
    arr_f = lambda xs: (K.cf * len(xs))(*[a.ctypes.data_as(K.cf) for a in xs])  # noqa: E731
    keep = [arr_u(wq), arr_u(wk), arr_u(wv), arr_u(wo), arr_f(an), arr_f(fn), arr_f(router), arr_u(ge), arr_u(ue),
            arr_u(de)]
    d = K.GptOssDesc(L=L, N=N, NH=NH, NKH=NKH, HD=HD, E=E, K=Kk, M=M, max_ctx=ctx, rope_dim=HD, outNR=V, eps=1e-5,
                     wQ=keep[0], wK=keep[1], wV=keep[2], wO=keep[3], wAN=keep[4], wFN=keep[5],
                     wOut=wout.ctypes.data_as(K.cu), w_gate_inp=keep[6], w_gate_exps=keep[7], w_up_exps=keep[8],
                     w_down_exps=keep[9], qt_gate=39, qt_up=39, qt_down=39, cos_t=cos_t.ctypes.data_as(K.cf),
                     sin_t=sin_t.ctypes.data_as(K.cf))
    h = dev.so.mllm_gptoss_create(ctypes.byref(d))
    if not h:
        raise RuntimeError("mllm_gptoss_create: " + K.last_error(dev.so))
    try:
        n = dev.so.mllm_gptoss_kv_floats(h)
        kc = torch.randn(n, device="cuda")
        vc = torch.randn(n, device="cuda")
        lens = torch.full((L,), 512, dtype=torch.int32, device="cuda")
        pos = torch.full((1,), 512, dtype=torch.int32, device="cuda")
        x = torch.randn(N, device="cuda")
        logits = torch.empty(V, device="cuda")

        def step():
            rc = dev.so.mllm_gptoss_step(h, x.data_ptr(), pos.data_ptr(), lens.data_ptr(), kc.data_ptr(),
                                         vc.data_ptr(), logits.data_ptr(), dev._stream())
            if rc:
                raise RuntimeError("mllm_gptoss_step: " + K.last_error(dev.so))
        steps = min(20, max(5, args.steps))
        ms = time_region(torch, step, steps, 2)
        fin = bool(torch.isfinite(logits).all())
        seq = int(lens[0].item())
    finally:
        dev.so.mllm_gptoss_release(h)
    wb = (L * (W.row_bytes(39, N) * (inner + 2 * kvd) + W.row_bytes(39, inner) * N +
               Kk * (2 * W.row_bytes(39, N) * M + W.row_bytes(39, M) * N) + E * N * 4) + W.row_bytes(39, N) * V)
    kvb = L * 2 * 512 * kvd * 4
    res = {"ms_per_token": round(ms, 3), "tokens/s": round(1e3 / ms, 1),
           "GB/s": round((wb + kvb) / (ms * 1e-3) / 1e9, 1),
           "hbm_frac": round((wb + kvb) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "bytes_per_token_MB": round((wb + kvb) / 1e6, 1), "logits_finite": fin, "kv_len_after": seq,
           "note": "weights read per token: q/k/v/o, the 4 routed experts and the router of each layer, lm_head; "
                   "KV rows at ~512 positions"}
    log(f"gptoss step (24 layers, vocab {V}): {ms:.3f} ms/token, {res['GB/s']} GB/s, logits finite {fin}")
    return res


class MoECall:
    """moe_forward_omp (QK:2066) through a library's host ABI as the reference's
    caller makes it (TE:2031-2085): per-expert pointer arrays built once
    (TE:868-905), scratch sized as TE:954-960, caller-supplied routing."""

    def __init__(self, ptrs, M, N, qts, Kk):
        E = len(ptrs[0])
        arr = ctypes.POINTER(ctypes.c_uint8) * E
        self.keep = ptrs
        self.pg, self.pu, self.pd = (arr(*[a.ctypes.data_as(K.cu) for a in lst]) for lst in ptrs)
        self.M, self.N, self.qts, self.K = M, N, qts, Kk
        self.comb = np.zeros(N, np.float32)
        self.buf = np.zeros(3 * Kk * M, np.float32)
        self.q8 = np.zeros(Kk * M * 34 // 32 + 64, np.uint8)
        self.p = (self.comb.ctypes.data_as(K.cf), self.buf.ctypes.data_as(K.cf), self.q8.ctypes.data_as(K.cu))

    def prepare(self, xs, idx, w):
        """Per-token argument pointers, made before any timed call."""
        self.args = [(np.ascontiguousarray(x, np.float32), np.ascontiguousarray(i, np.int32),
                      np.ascontiguousarray(v, np.float32)) for x, i, v in zip(xs, idx, w)]
        self.cargs = [(x.ctypes.data_as(K.cf), i.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), v.ctypes.data_as(K.cf))
                      for x, i, v in self.args]

    def __call__(self, lib, t):
        x, ti, tw = self.cargs[t]
        lib.moe_forward_omp(self.pg, self.pu, self.pd, x, self.M, self.N, self.qts[0], self.qts[1], self.qts[2], ti,
                            tw, self.K, self.p[0], self.p[1], self.p[2])
        return self.comb


# ------------------------------------------------------------------ host CPU reference (child process)
CPU_LEGS = ("tinyllama", "q8", "prefill", "moe_gptoss", "moe_qwen3")


def cpu_leg(name, cores, model):
    """One leg of the reference's own C (oracle/_ref, AVX2 + OpenMP) on this
    host, in this (child) process: 3 warm-ups, then the median of >= 20 timed
    calls.  Inputs are drawn with numpy from the GPU legs' distributions (the
    MoE router and hidden states are the GPU legs' own: the same seeds)."""
    O, ref = ref_lib()
    if not ref:
        return None
    ref.so.set_num_threads(cores)
    tag = cpu_tag(cores, model)
    if name == "tinyllama":
        # 4 layers' 7 matrices + lm_head at B=1 (165 MB per pass, past the L3)
        r2 = np.random.default_rng(2)
        work = [(W.gen_weights(r2, qt, rows, cols), rows, cols, qt) for _ in range(4)
                for (_, rows, cols, qt) in W.TINYLLAMA_MATS]
        _, rows, cols, qt = W.TINYLLAMA_LM_HEAD
        work.append((W.gen_weights(r2, qt, rows, cols), rows, cols, qt))
        x = {c: W.gen_x(np.random.default_rng(5), 1, c) for c in (2048, 5632)}
        outs = {r: np.zeros(r, np.float32) for (_, r, _, _) in work}
        fns = {12: ref.so.q4_k_batch_matmul, 14: ref.so.q6_k_batch_matmul}
        nbytes = sum(w.size + (r + c) * 4 for (w, r, c, _) in work)

        def one():
            for (w, r, c, q) in work:
                fns[q](w.ctypes.data_as(K.cu), x[c].ctypes.data_as(K.cf), outs[r].ctypes.data_as(K.cf), r, c, 1)
        med = median_time(one, 20)
        return {"value": round(nbytes / med / 1e9, 2), "unit": "GB/s", **tag, "ms_per_pass": round(med * 1e3, 3),
                "sample": f"q4_k/q6_k_batch_matmul (oracle/_ref, AVX2+OpenMP, {cores} threads) over 4 TinyLlama "
                          f"layers (7 matrices each) + lm_head, B=1, {nbytes / 1e6:.1f} MB per pass, median of 20 "
                          "passes after 3 warm-ups"}
    if name == "q8":
        raws = [W.gen_weights(np.random.default_rng(100 + i), W.QT_Q8_0, 5632, 2048) for i in range(24)]
        xh = W.gen_x(np.random.default_rng(0), 1, 2048)
        oh = np.zeros(5632, np.float32)
        it = iter(range(10 ** 9))
        f = lambda: ref.so.q8_0_batch_matmul(raws[next(it) % 24].ctypes.data_as(K.cu), xh.ctypes.data_as(K.cf),  # noqa
                                             oh.ctypes.data_as(K.cf), 5632, 2048, 1)
        sec = median_time(f, 48)
        nb = raws[0].size + (2048 + 5632) * 4
        return {"value": round(nb / sec / 1e9, 2), "unit": "GB/s", **tag, "us": round(sec * 1e6, 1),
                "sample": f"q8_0_batch_matmul (oracle/_ref, AVX2+OpenMP, {cores} threads), B=1, median of 48 calls "
                          "over 24 rotating 12 MB matrices after 3 warm-ups"}
    if name == "prefill":
        out = {}
        for key, fname, qt, R, C in (("gate_q4k_M128", "q4_k_batch_matmul", W.QT_Q4_K, 5632, 2048),
                                     ("down_q6k_M128", "q6_k_batch_matmul", W.QT_Q6_K, 2048, 5632)):
            rn = W.gen_weights(np.random.default_rng(3), qt, R, C)
            xh = W.gen_x(np.random.default_rng(6), 128, C, bf16=True)
            oh = np.zeros(128 * R, np.float32)
            fn = getattr(ref.so, fname)
            sec = median_time(lambda: fn(rn.ctypes.data_as(K.cu), xh.ctypes.data_as(K.cf), oh.ctypes.data_as(K.cf),
                                         R, C, 128), 20)
            out[key] = {"value": round(2.0 * R * C * 128 / sec / 1e12, 4), "unit": "TFLOP/s", **tag,
                        "ms": round(sec * 1e3, 2),
                        "sample": f"{fname} (oracle/_ref, AVX2+OpenMP, {cores} threads), B=128, median of 20 after "
                                  "3 warm-ups"}
        return out
    # MoE layers: moe_forward_omp per token (renormalised C routing), and moe_ffn for GPT-OSS
    tag_moe = name.split("_")[1]
    c = dict(W.GPTOSS) if tag_moe == "gptoss" else dict(W.QWEN3)
    N, E, Kk, M = c["N"], c["E"], c["K"], c["M"]
    qts = (c["qt_gate"], c["qt_up"], c["qt_down"])
    rng = np.random.default_rng(7)
    router = W.gen_router(rng, E, N)
    n_tok = 24
    if tag_moe == "qwen3":
        x, router, _, _ = W.skewed_tokens(rng, router, 1280)
    else:
        x = W.gen_x(rng, 1280, N)
    rw = np.random.default_rng(11)
    gates = [W.gen_weights(rw, qts[0], M, N) for _ in range(E)]
    ups = [W.gen_weights(rw, qts[1], M, N) for _ in range(E)]
    downs = [W.gen_weights(rw, qts[2], N, M) for _ in range(E)]
    orc = O.Oracle()
    idx, w = orc.route(router, x[:n_tok], Kk, renorm=True)
    call = MoECall((gates, ups, downs), M, N, qts, Kk)
    call.prepare(x[:n_tok], idx, w)
    it = iter(range(10 ** 9))
    sec = median_time(lambda: call(ref.so, next(it) % n_tok), n_tok)
    res = {"moe_forward_omp": {
        "value": round(1 / sec, 2), "unit": "tokens/s", **tag, "ms": round(sec * 1e3, 2),
        "sample": f"moe_forward_omp (oracle/_ref) per token on {n_tok} tokens of the {tag_moe} workload (router and "
                  f"hidden states as the GPU leg), C routing (renormalised top-{Kk}) precomputed, median of {n_tok} "
                  "after 3 warm-ups"}}
    if tag_moe == "gptoss":
        # moe_ffn (CE:591-665) addresses each expert tensor contiguously at its own strides (CE:593-605)
        gate, upw, down = np.concatenate(gates), np.concatenate(ups), np.concatenate(downs)
        bc = W.BCView(N, E, Kk, M, router, gate, upw, down, qts)
        cf = ctypes.POINTER(ctypes.c_float)
        ref.so.moe_ffn.argtypes = [ctypes.c_void_p, ctypes.c_int, cf, cf, cf, cf, ctypes.c_int]
        ref.so.moe_ffn.restype = None
        gb, ub, o = np.zeros(8192, np.float32), np.zeros(8192, np.float32), np.zeros(N, np.float32)
        xs = [np.ascontiguousarray(x[t]).copy() for t in range(n_tok)]
        it2 = iter(range(10 ** 9))
        f = lambda: ref.so.moe_ffn(bc.ptr(), 0, xs[next(it2) % n_tok].ctypes.data_as(cf), gb.ctypes.data_as(cf),  # noqa
                                   ub.ctypes.data_as(cf), o.ctypes.data_as(cf), 1)
        sec = median_time(f, n_tok)
        res["moe_ffn"] = {"value": round(1 / sec, 2), "unit": "tokens/s", **tag, "ms": round(sec * 1e3, 2),
                          "sample": f"moe_ffn (oracle/_ref, its own C routing, un-renormalised top-{Kk}) per token, "
                                    f"B=1 calls, median of {n_tok} after 3 warm-ups"}
    return res


def run_cpu_leg(name):
    """A CPU leg in a child process with the OpenMP binding set from its start."""
    import subprocess
    env = dict(os.environ, OMP_PROC_BIND="close", OMP_PLACES="cores")
    try:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-leg", name], env=env,
                           capture_output=True, text=True, timeout=600)
    except subprocess.TimeoutExpired:
        log(f"CPU leg {name}: timed out")
        return None
    for line in (r.stderr or "").splitlines():
        if line.startswith("[bench]"):
            print(line, file=sys.stderr, flush=True)
    if r.returncode != 0:
        log(f"CPU leg {name} failed (rc {r.returncode}): {(r.stderr or '')[-400:]}")
        return None
    try:
        return json.loads(r.stdout.strip().splitlines()[-1])
    except (ValueError, IndexError):
        return None


def main():
    args = parse()
    if args.cpu_leg:
        print(json.dumps(cpu_leg(args.cpu_leg, CPU_THREADS, CPU_MODEL)), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported: the multi-GPU sharding "
              "(row-sharded GEMV, expert-parallel MoE) is designed, not built: every run here uses one GPU.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = K.DeviceOps()
    torch.cuda.set_device(0)
    if args.kernel:
        kernel_only(torch, dev, args.kernel)
        return
    cores, model = CPU_THREADS, CPU_MODEL
    use_cpu = not args.no_cpu
    log(f"host: {model}, {cores} threads for the CPU reference (run in a child process with OMP_PROC_BIND=close, "
        "OMP_PLACES=cores)")
    rng = np.random.default_rng(2)
    n_layers = W.TINYLLAMA_LAYERS
    log(f"building {n_layers} TinyLlama layers + lm_head on {gpu_info(torch)}")
    layers, lm, out_norm = build_tinyllama(dev, rng, n_layers)
    allm = [L[k] for L in layers for k in ("qkv", "o", "gate_up", "down")] + [lm]

    chains = {}
    for B in (1, 4, 8):
        ch = DecodeChain(torch, dev, layers, lm, out_norm, B)
        ms = time_region(torch, ch.run, args.steps if B == 1 else max(3, args.steps // 2), args.warmup)
        fin = bool(torch.isfinite(ch.logits).all())
        chains[B] = (ms, ch.bytes() / (ms * 1e-3) / 1e9, fin)
        log(f"decode chain B={B}: {ms:.3f} ms/pass, {chains[B][1]:.1f} GB/s, logits finite: {fin}")

    def independent_pass(B):
        xs = {c: torch.randn(B, c, device="cuda") for c in (2048, 5632)}
        outs = {m.rows: torch.empty(B, m.rows, device="cuda") for m in allm}
        return lambda: [dev.gemv(m.sem, m.packed, xs[m.cols], m.rows, m.cols, out=outs[m.rows]) for m in allm]
    ms_ind = time_region(torch, independent_pass(1), args.steps, args.warmup)
    gbs_ind = sum(algo_bytes(m, 1) for m in allm) / (ms_ind * 1e-3) / 1e9
    log(f"independent GEMV set B=1: {ms_ind:.3f} ms/pass, {gbs_ind:.1f} GB/s")

    kinds = bench_kinds(torch, dev, layers, lm, out_norm, args)
    # dominant kernel of the chain: the kind with the largest share of the pass
    share = {k: v["us"] * (1 if k == "lm_head" else n_layers) for k, v in kinds.items()}
    dom = max(share, key=share.get)
    kd = kinds[dom]
    dom_names = {"qkv": "k_gemv_p<Q4_K_GGML,B=1> fused RMSNorm + qkv 2560x2048",
                 "o": "k_gemv_p<Q4_K_GGML,B=1> o 2048x2048 + residual",
                 "gate_up": "k_gemv_p<Q4_K_GGML,B=1,pro+pair> fused RMSNorm + gate/up 11264x2048 + SiLU product",
                 "down": "k_gemv_p<Q6_K_SEQ,B=1> down 2048x5632 + residual",
                 "lm_head": "k_gemv_p<Q6_K_SEQ,B=1> fused RMSNorm + lm_head 32000x2048"}

    cpu = run_cpu_leg("tinyllama") if use_cpu else None
    if cpu:
        log(f"CPU reference TinyLlama set: {cpu['value']} GB/s on {cores} threads")

    extra = {}
    if not args.no_extra:
        extra["configs0_q8_0_gemv"] = bench_q8(torch, dev, args)
        extra["long_gemv_b1"] = bench_long_gemv(torch, dev, args)
        extra["configs2_prefill_gemm"] = bench_prefill(torch, dev, args)
        extra["configs3_gptoss_moe"] = bench_moe(torch, dev, args, "gptoss")
        extra["configs4_qwen3_moe"] = bench_moe(torch, dev, args, "qwen3")
        extra["decode_attention_gptoss_heads"] = bench_attention(torch, dev, args)
        extra["gptoss_forward_step"] = bench_gptoss(torch, dev, args)
        if use_cpu:
            for key, leg in (("configs0_q8_0_gemv", "q8"), ("configs2_prefill_gemm", "prefill"),
                             ("configs3_gptoss_moe", "moe_gptoss"), ("configs4_qwen3_moe", "moe_qwen3")):
                r = run_cpu_leg(leg)
                extra[key]["cpu_baseline"] = r
                log(f"CPU reference {leg}: {json.dumps(r)[:300]}")

    ms1, gbs1, fin1 = chains[1]
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
        "dtype": "f32 (fp32 activations as three int8 digit planes, int32 dot4 per 16-weight run, fp32 scales and "
                 "accumulation)",
        "data": "synthetic (BASELINE.json distributions, seeded)",
        "config": {"workload": "configs[1] TinyLlama-1.1B Q4_K_M matmul set (22 layers + lm_head) as a B=1 decode "
                               "chain: RMSNorm fused into qkv and gate/up, residual adds into o and down, SiLU "
                               "product in the gate/up epilogue (paired rows), each matrix fed by the previous one "
                               "(89 dependent launches); "
                               "*_batch_matmul semantics",
                   "hbm_frac": round(gbs1 / HBM_PEAK_GBS, 4), "logits_finite": fin1,
                   "B4": {"ms_per_pass": round(chains[4][0], 4), "GB/s": round(chains[4][1], 1)},
                   "B8": {"ms_per_pass": round(chains[8][0], 4), "GB/s": round(chains[8][1], 1)},
                   "independent_gemvs_B1": {"ms_per_pass": round(ms_ind, 4), "GB/s": round(gbs_ind, 1),
                                            "note": "the same 89 GEMVs with independent inputs, no prologue"},
                   "per_kind_B1": kinds},
        "roofline": {"bound": "hbm", "achieved": kd["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kd["GB/s"] / HBM_PEAK_GBS, 4), "traffic": ROOFLINE_TRAFFIC_BYTES.get(dom),
                     "kernel": f"{dom_names[dom]} ({kd['bytes']:,} algorithmic B/launch, {kd['us']} us/launch)",
                     "frac_of_plain_read": kd["frac_of_plain_read"]},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
