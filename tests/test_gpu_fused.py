"""GPU parity of the fused decode GEMV (mllm_gemv_fused): the RMSNorm /
residual prologue, the residual epilogue and the SiLU product, in one launch
where the decode kernel stages the whole activation, otherwise through the
standalone prologue kernel -- against the oracle's GEMV applied to the
activation formed in float64 from the reference's formulas:
  simd_ops rms_norm (TE:1516,1641):    v * (1 / sqrt(mean(v^2) + eps)) * w
  gptoss rms_norm (GO:29-34):          (v / sqrt(mean(v^2) + eps)) * w
  SiLU product (QK:2157-2164 clamped / moe_ffn CE:649-652 plain).

Tolerance: GEMV_TOL for fp32-activation semantics (the norm's reduction order
moves the activation by an fp32 ulp at most); MOE_Q8H_TOL for the Q8_0-
activation semantics, where such an ulp can move one Q8_0 rounding step.
"""
import numpy as np
import pytest

import oracle as O
from helpers import GEMV_TOL, MOE_Q8H_TOL
from mojollama_amd import kernels as K
from mojollama_amd import workloads as W

pytestmark = pytest.mark.gpu

QT = {K.Q4_K_GGML: 12, K.Q6_K_SEQ: 14, K.MXFP4: 39, K.Q8_0: 8, K.Q4_K_Q8: 12, K.MXFP4_Q8: 39, K.Q4_0: 2}


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return K.DeviceOps(K.load_kernels())


def silu_np(g, u, clamp):
    g = g.astype(np.float64)
    if clamp:
        g = np.clip(g, -80.0, 80.0)
    with np.errstate(over="ignore"):     # exp(-g) -> inf for large negative g: silu -> 0
        return g / (1.0 + np.exp(-g)) * u


def rms_np(v, w, eps, div):
    v = v.astype(np.float64)
    r = np.sqrt(np.mean(v * v, axis=1, keepdims=True) + eps)
    return (v / r if div else v * (1.0 / r)) * w


def run_case(dev, orc, sem, R, C, B, mode, seed):
    import torch
    rng = np.random.default_rng(seed)
    qt = QT[sem]
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, B, C)
    res = W.gen_x(rng, B, C)
    g = (rng.standard_normal(C) * 0.5 + 1.0).astype(np.float32)
    add = W.gen_x(rng, B, R)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    packed = dev.pack(sem, cu(w), R, C)
    xt, rt, gt = cu(x), cu(res), cu(g)
    out = torch.full((B, R), float("nan"), device="cuda")
    res_out = torch.full((B, C), float("nan"), device="cuda")
    want_res = None
    eps = 1e-5
    if mode == "rms":
        f = dev.fusion(rms_w=gt, rms_eps=eps)
        xe = rms_np(x, g, eps, False)
    elif mode == "rms_div_res":
        f = dev.fusion(x_res=rt, res_out=res_out, rms_w=gt, rms_eps=eps, rms_div=True)
        xe = rms_np(x.astype(np.float64) + res, g, eps, True)
        want_res = x + res
    elif mode == "res_add":
        addt = cu(add)    # kept alive: the fusion holds only its address
        f = dev.fusion(x_res=rt, out_add=addt)
        xe = x.astype(np.float64) + res
    elif mode == "add_inplace":
        out = cu(add)
        f = dev.fusion(out_add=out)
        xe = x
    elif mode in ("silu", "silu_noclamp"):
        clamp = mode == "silu"
        x = x * 40.0          # gates well past +-80 for some elements
        xt = cu(x)
        f = dev.fusion(x_up=rt, silu_clamp=clamp)
        xe = silu_np(x, res, clamp)
    got = dev.gemv_fused(sem, packed, xt, R, C, f, out=out).cpu().numpy()
    ref = orc.gemv(sem, w, np.ascontiguousarray(xe, np.float32), R, C, B)
    if mode in ("res_add", "add_inplace"):
        ref = ref + add
    tol = MOE_Q8H_TOL if mllm_q8(sem) else GEMV_TOL
    err = O.norm_err(got, ref)
    print(f"[parity] fused {K.SEM_NAMES[sem]} {R}x{C} B={B} {mode}: {err:.3e}", flush=True)
    assert err < tol, K.last_error(dev.so)
    if want_res is not None:
        assert np.array_equal(res_out.cpu().numpy(), want_res)


def mllm_q8(sem):
    return sem in (K.Q4_K_Q8, K.MXFP4_Q8, K.Q5_0_Q8)


@pytest.mark.parametrize("mode", ["rms", "rms_div_res", "res_add", "add_inplace"])
@pytest.mark.parametrize("sem", [K.Q4_K_GGML, K.Q6_K_SEQ, K.MXFP4, K.Q8_0, K.Q4_K_Q8, K.MXFP4_Q8])
@pytest.mark.parametrize("B", [1, 3, 8])
def test_fused_prologue_epilogue(dev, orc, sem, B, mode):
    """One launch: the whole activation is staged at these shapes."""
    R, C = 300, 2048 if QT[sem] in (12, 14) else 2880
    run_case(dev, orc, sem, R, C, B, mode, seed=sem * 10 + B + len(mode))


@pytest.mark.parametrize("mode", ["silu", "silu_noclamp"])
@pytest.mark.parametrize("sem,B", [(K.Q4_K_GGML, 1), (K.MXFP4, 1), (K.MXFP4_Q8, 4), (K.Q6_K_SEQ, 4), (K.Q4_K_Q8, 2)])
def test_fused_silu(dev, orc, sem, B, mode):
    """The SiLU product in the kernel's staging (fp32 at B = 1, the in-kernel
    Q8_0 quantiser at any B) or through the prologue kernel (fp32 at B > 1)."""
    run_case(dev, orc, sem, 200, 768 if QT[sem] in (12, 14) else 800, B, mode, seed=sem + B)


@pytest.mark.parametrize("mode", ["rms_div_res", "res_add", "add_inplace", "silu"])
@pytest.mark.parametrize("sem,R,C,B", [(K.Q6_K_SEQ, 2048, 5632, 8), (K.Q4_K_GGML, 256, 2048, 20),
                                       (K.MXFP4, 130, 2880, 12)])
def test_fused_fallback(dev, orc, sem, R, C, B, mode):
    """Shapes the decode kernel cannot stage at once (B = 8 with K = 5632) and
    B > 8 (the MFMA GEMM): the prologue kernel, then the GEMV / GEMM, then the
    residual (the in-place residual from a copy on the GEMM path)."""
    run_case(dev, orc, sem, R, C, B, mode, seed=R + C + B + len(mode))


def test_fused_res_out_overlap_rejected(dev):
    import torch
    rng = np.random.default_rng(1)
    w = torch.from_numpy(W.gen_weights(rng, 12, 64, 256)).cuda()
    packed = dev.pack(K.Q4_K_GGML, w, 64, 256)
    x = torch.randn(1, 256, device="cuda")
    f = dev.fusion(res_out=x, rms_w=torch.ones(256, device="cuda"))
    with pytest.raises(RuntimeError, match="overlaps"):
        dev.gemv_fused(K.Q4_K_GGML, packed, x, 64, 256, f)


@pytest.mark.parametrize("sem,C", [(K.Q4_K_GGML, 2048), (K.Q6_K_SEQ, 2048), (K.MXFP4, 2880), (K.Q4_K_Q8, 2048),
                                   (K.Q8_0, 1024)])
@pytest.mark.parametrize("B", [1, 3])
@pytest.mark.parametrize("mode", ["pair", "pair_rms", "pair_noclamp_add"])
def test_fused_silu_pair(dev, orc, sem, C, B, mode):
    """Stacked gate/up rows: out[r] = silu(gate_r . v) * (up_r . v) in the GEMV's
    epilogue (B = 1, one launch, with the RMSNorm prologue for 'pair_rms'), or
    the GEMV over both halves followed by the SiLU product (B = 3)."""
    import torch
    rng = np.random.default_rng(sem * 7 + C + B + len(mode))
    R = 300
    qt = QT[sem]
    w = W.gen_weights(rng, qt, 2 * R, C)
    x = W.gen_x(rng, B, C)
    g = (rng.standard_normal(C) * 0.5 + 1.0).astype(np.float32)
    add = W.gen_x(rng, B, R)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    packed = dev.pack(sem, cu(w), 2 * R, C)
    gt, addt = cu(g), cu(add)
    clamp = mode != "pair_noclamp_add"
    if mode == "pair_rms":
        f = dev.fusion(silu_pair=True, silu_clamp=clamp, rms_w=gt, rms_eps=1e-5)
        xe = rms_np(x, g, 1e-5, False)
    elif mode == "pair":
        f = dev.fusion(silu_pair=True, silu_clamp=clamp)
        xe = x
    else:
        f = dev.fusion(silu_pair=True, silu_clamp=clamp, out_add=addt)
        xe = x
    got = dev.gemv_fused(sem, packed, cu(x), R, C, f).cpu().numpy()
    y = orc.gemv(sem, w, np.ascontiguousarray(xe, np.float32), 2 * R, C, B).astype(np.float64)
    ref = silu_np(y[:, :R], y[:, R:], clamp)
    if mode == "pair_noclamp_add":
        ref = ref + add
    tol = MOE_Q8H_TOL if mllm_q8(sem) else GEMV_TOL
    err = O.norm_err(got, ref)
    print(f"[parity] fused pair {K.SEM_NAMES[sem]} {R}x{C} B={B} {mode}: {err:.3e}", flush=True)
    assert err < tol, K.last_error(dev.so)
