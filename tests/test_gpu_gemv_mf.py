"""GPU parity of the batch 2..8 decode GEMV on the matrix cores (gemv_mf.h)
at the TinyLlama decode shapes bench.py times (configs[1], B in {4, 8}) and
at odd batch widths, against the oracle's q4_k_batch_matmul (CE:255-313) /
q6_k_batch_matmul (CE:315-378) / q8_0 and q4_0 batch matmuls (CE:216-253,
CE:68-110) / mxfp4 (QK:683-720, clamped CE:427-534) on the activation formed
in float64 from the reference's formulas (RMSNorm TE:1516,1641; SiLU
product; residual adds).

Every output row and token is compared: the kernel's tiles (32 rows, or 16
gate + 16 up rows), its K splits across workgroups (short matrices) and the
four waves' K quarters all land in the checked outputs.  Reported: the
normalised error max|d| / max|ref| (bound GEMV_TOL) and the per-element
relative error over outputs with |ref| >= 1e-3 max|ref|.
"""
import zlib

import numpy as np
import pytest

import oracle as O
from helpers import GEMV_TOL
from mojollama_amd import kernels as K
from mojollama_amd import workloads as W

pytestmark = pytest.mark.gpu

QT = {K.Q4_K_GGML: W.QT_Q4_K, K.Q6_K_SEQ: W.QT_Q6_K, K.Q8_0: W.QT_Q8_0, K.Q4_0: W.QT_Q4_0, K.MXFP4: W.QT_MXFP4,
      K.MXFP4_CLAMP: W.QT_MXFP4}


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return K.DeviceOps(K.load_kernels())


def rms_np(v, w, eps):
    v = v.astype(np.float64)
    return v * (1.0 / np.sqrt(np.mean(v * v, axis=1, keepdims=True) + eps)) * w


def silu_np(g, u):
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g)) * u


def rel_err(got, ref):
    big = np.abs(ref) >= 1e-3 * np.abs(ref).max()
    return float(np.max(np.abs(got[big] - ref[big]) / np.abs(ref[big])))


def check(name, got, ref):
    err, rel = O.norm_err(got, ref), rel_err(got, ref)
    print(f"[parity] mfma gemv {name}: norm {err:.3e} max rel {rel:.3e}", flush=True)
    assert np.all(np.isfinite(got)), name
    assert err < GEMV_TOL, name


CASES = [
    # name, sem, rows (output), cols, mode
    ("qkv", K.Q4_K_GGML, 2560, 2048, "rms"),
    ("o", K.Q4_K_GGML, 2048, 2048, "add"),
    ("gate_up", K.Q4_K_GGML, 5632, 2048, "pair_rms"),
    ("down", K.Q6_K_SEQ, 2048, 5632, "add"),
    ("lm_head", K.Q6_K_SEQ, 32000, 2048, "rms"),
]


@pytest.mark.parametrize("B", [4, 8])
@pytest.mark.parametrize("name,sem,R,C,mode", CASES)
def test_mfma_decode_shapes(dev, orc, name, sem, R, C, mode, B):
    import torch
    rng = np.random.default_rng(zlib.crc32(f"{name}{B}".encode()))
    mrows = 2 * R if mode.startswith("pair") else R
    w = W.gen_weights(rng, QT[sem], mrows, C)
    x = W.gen_x(rng, B, C)
    g = (rng.standard_normal(C) * 0.5 + 1.0).astype(np.float32)
    add = W.gen_x(rng, B, R)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    packed = dev.pack(sem, cu(w), mrows, C)
    gt, addt = cu(g), cu(add)
    eps = 1e-5
    if mode == "rms":
        f, xe = dev.fusion(rms_w=gt, rms_eps=eps), rms_np(x, g, eps)
    elif mode == "pair_rms":
        f, xe = dev.fusion(rms_w=gt, rms_eps=eps, silu_pair=True, silu_clamp=False), rms_np(x, g, eps)
    else:
        f, xe = dev.fusion(out_add=addt), x
    got = dev.gemv_fused(sem, packed, cu(x), R, C, f).cpu().numpy()
    y = orc.gemv(sem, w, np.ascontiguousarray(xe, np.float32), mrows, C, B).astype(np.float64)
    if mode == "pair_rms":
        ref = silu_np(y[:, :R], y[:, R:])
    elif mode == "add":
        ref = y + add
    else:
        ref = y
    check(f"{name} {R}x{C} B={B} {mode}", got, ref)


@pytest.mark.parametrize("B", [2, 3, 5, 7])
@pytest.mark.parametrize("sem,R,C", [(K.Q4_K_GGML, 2560, 2048), (K.Q6_K_SEQ, 2048, 5632), (K.Q4_K_GGML, 45, 768),
                                     (K.Q8_0, 5632, 2048), (K.Q4_0, 300, 2080), (K.MXFP4, 2880, 2880),
                                     (K.MXFP4_CLAMP, 333, 800)])
def test_mfma_gemv_odd_batches(dev, orc, sem, R, C, B):
    """mllm_gemv at every batch-width class (tokens past B padded in the tile)."""
    import torch
    rng = np.random.default_rng(R + C + B)
    w = W.gen_weights(rng, QT[sem], R, C)
    x = W.gen_x(rng, B, C)
    packed = dev.pack(sem, torch.from_numpy(w).cuda(), R, C)
    got = dev.gemv(sem, packed, torch.from_numpy(x).cuda(), R, C).cpu().numpy()
    check(f"{K.SEM_NAMES[sem]} {R}x{C} B={B}", got, orc.gemv(sem, w, x, R, C, B))


@pytest.mark.parametrize("sem,R,C", [(K.Q4_K_GGML, 2048, 2048), (K.Q6_K_SEQ, 300, 1024)])
def test_mfma_gemv_without_workspace(dev, orc, sem, R, C):
    """No partials buffer: the K range is not split (one workgroup per row
    tile over all of K) and the result is the same to tolerance."""
    import torch
    rng = np.random.default_rng(5 + R)
    B = 8
    w = W.gen_weights(rng, QT[sem], R, C)
    x = W.gen_x(rng, B, C)
    packed = dev.pack(sem, torch.from_numpy(w).cuda(), R, C)
    out = torch.empty(B, R, device="cuda")
    xt = torch.from_numpy(x).cuda()
    dev._check(dev.so.mllm_gemv(sem, packed.data_ptr(), xt.data_ptr(), out.data_ptr(), R, C, B, None, dev._stream()),
               "mllm_gemv")
    check(f"{K.SEM_NAMES[sem]} {R}x{C} B={B} no workspace", out.cpu().numpy(), orc.gemv(sem, w, x, R, C, B))


def test_mfma_gemv_strided_x(dev, orc):
    """The o projection of bench.py's chain reads q from the qkv rows (x_ld 2560)."""
    import torch
    rng = np.random.default_rng(11)
    B, R, C = 8, 2048, 2048
    w = W.gen_weights(rng, W.QT_Q4_K, R, C)
    qkv = W.gen_x(rng, B, 2560)
    add = W.gen_x(rng, B, R)
    packed = dev.pack(K.Q4_K_GGML, torch.from_numpy(w).cuda(), R, C)
    qt, addt = torch.from_numpy(qkv).cuda(), torch.from_numpy(add).cuda()
    f = dev.fusion(out_add=addt, x_ld=2560)
    got = dev.gemv_fused(K.Q4_K_GGML, packed, qt.data_ptr(), R, C, f, B=B).cpu().numpy()
    ref = orc.gemv(K.Q4_K_GGML, w, np.ascontiguousarray(qkv[:, :C]), R, C, B) + add
    check("o strided x B=8", got, ref)


@pytest.mark.parametrize("B", [4, 8])
@pytest.mark.parametrize("sem,R,C", [(K.Q8_0, 5632, 2048), (K.MXFP4, 2880, 2880), (K.Q4_0, 1024, 2048)])
@pytest.mark.parametrize("mode", ["rms", "pair_rms", "add"])
def test_mfma_block32_fused(dev, orc, sem, R, C, mode, B):
    """The 32-element block formats (one unit = one block) with the fused
    prologue, paired rows and residual, as the decode chain uses them."""
    import torch
    rng = np.random.default_rng(zlib.crc32(f"{sem}{R}{mode}{B}".encode()))
    mrows = 2 * R if mode.startswith("pair") else R
    w = W.gen_weights(rng, QT[sem], mrows, C)
    x = W.gen_x(rng, B, C)
    g = (rng.standard_normal(C) * 0.5 + 1.0).astype(np.float32)
    add = W.gen_x(rng, B, R)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    packed = dev.pack(sem, cu(w), mrows, C)
    gt, addt = cu(g), cu(add)
    eps = 1e-5
    if mode == "rms":
        f, xe = dev.fusion(rms_w=gt, rms_eps=eps), rms_np(x, g, eps)
    elif mode == "pair_rms":
        f, xe = dev.fusion(rms_w=gt, rms_eps=eps, silu_pair=True, silu_clamp=True), rms_np(x, g, eps)
    else:
        f, xe = dev.fusion(out_add=addt), x
    got = dev.gemv_fused(sem, packed, cu(x), R, C, f).cpu().numpy()
    y = orc.gemv(sem, w, np.ascontiguousarray(xe, np.float32), mrows, C, B).astype(np.float64)
    if mode == "pair_rms":
        ref = silu_np(np.clip(y[:, :R], -80, 80), y[:, R:])
    elif mode == "add":
        ref = y + add
    else:
        ref = y
    check(f"{K.SEM_NAMES[sem]} {R}x{C} B={B} {mode}", got, ref)


@pytest.mark.parametrize("B", [4, 8])
def test_mfma_split_arrival_graph_replay(dev, orc, B):
    """K split over workgroups (the o and down projections at these shapes,
    their partials added by the reduction launch) and the unsplit paired
    gate/up sharing one workspace that starts as garbage, captured once in a
    graph and replayed with new activations written eagerly between replays:
    every replay equals the eager calls bit for bit, and the eager o
    projection matches the oracle."""
    import ctypes
    import torch
    rng = np.random.default_rng(77 + B)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    w_o = W.gen_weights(rng, W.QT_Q4_K, 2048, 2048)
    w_gu = W.gen_weights(rng, W.QT_Q4_K, 2 * 5632, 2048)
    w_d = W.gen_weights(rng, W.QT_Q6_K, 2048, 5632)
    p_o = dev.pack(K.Q4_K_GGML, cu(w_o), 2048, 2048)
    p_gu = dev.pack(K.Q4_K_GGML, cu(w_gu), 2 * 5632, 2048)
    p_d = dev.pack(K.Q6_K_SEQ, cu(w_d), 2048, 5632)
    g = cu((rng.standard_normal(2048) * 0.5 + 1.0).astype(np.float32))
    f_o, f_d = dev.fusion(), dev.fusion()
    f_gu = dev.fusion(rms_w=g, rms_eps=1e-5, silu_pair=True, silu_clamp=False)
    n = max(dev.so.mllm_gemv_fused_workspace_size(K.Q4_K_GGML, 2048, 2048, B, ctypes.byref(f_o)),
            dev.so.mllm_gemv_fused_workspace_size(K.Q4_K_GGML, 5632, 2048, B, ctypes.byref(f_gu)),
            dev.so.mllm_gemv_fused_workspace_size(K.Q6_K_SEQ, 2048, 5632, B, ctypes.byref(f_d)), 256)
    ws = torch.full((n,), 0xA5, dtype=torch.uint8, device="cuda")
    x = cu(W.gen_x(rng, B, 2048))
    y_o = torch.empty(B, 2048, device="cuda")
    h = torch.empty(B, 5632, device="cuda")
    y_d = torch.empty(B, 2048, device="cuda")

    def run():
        dev.gemv_fused(K.Q4_K_GGML, p_o, x, 2048, 2048, f_o, out=y_o, ws=ws)
        dev.gemv_fused(K.Q4_K_GGML, p_gu, y_o, 5632, 2048, f_gu, out=h, ws=ws)
        dev.gemv_fused(K.Q6_K_SEQ, p_d, h, 2048, 5632, f_d, out=y_d, ws=ws)

    run()
    torch.cuda.synchronize()
    check(f"o {2048}x{2048} B={B} split", y_o.cpu().numpy(), orc.gemv(K.Q4_K_GGML, w_o, x.cpu().numpy(), 2048, 2048, B))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for i in range(4):
        x.copy_(cu(W.gen_x(rng, B, 2048)))
        run()
        torch.cuda.synchronize()
        want = [t.clone() for t in (y_o, h, y_d)]
        for t in (y_o, h, y_d):
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for name, got, ref in zip(("o", "gate_up", "down"), (y_o, h, y_d), want):
            assert torch.equal(got, ref), f"replay {i} {name}"
