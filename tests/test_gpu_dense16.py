"""GPU parity of the prefill GEMM over a load-time fp16 weight copy
(mllm_dense16_make + mllm_gemm16) against the oracle.

Two bars per case:
  * the fp16 copy equals the oracle's dequantisation (the reference's
    *_dequantize_row arithmetic) rounded to fp16 by numpy, and the
    GEMM equals the float64 product of its own fp16 operands (the weights and
    the activations under the power-of-two scale) to D16_EXACT: any layout,
    scale or transpose mistake fails here;
  * against the oracle's fp32 *_batch_matmul the normalised max error stays
    below D16_TOL = 1e-3, the north star's bound for floating-point outputs
    (weights and activations each rounded to fp16, relative 2^-11 at most:
    ~3e-4 expected).
"""
import numpy as np
import pytest

import oracle as O
from mojollama_amd import kernels as K
from mojollama_amd import workloads as W

pytestmark = pytest.mark.gpu
D16_TOL = 1e-3
D16_EXACT = 2e-6

QT = {K.Q4_0: 2, K.Q4_1: 3, K.Q5_0_F32: 6, K.Q8_0: 8, K.Q4_K_GGML: 12, K.Q5_K_GGML: 13, K.Q5_K_CE: 13,
      K.Q6_K_GGML: 14, K.Q6_K_LOWNIB: 14, K.Q6_K_SEQ: 14, K.MXFP4: 39, K.MXFP4_CLAMP: 39}


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return K.DeviceOps(K.load_kernels())


def x16_of(x):
    """The activations as the GEMM sees them: fp16(x * 2^e) and 2^-e, e placing
    the largest finite |x| in [2^14, 2^15)."""
    a = np.abs(x[np.isfinite(x)])
    m = float(a.max()) if a.size else 0.0
    e = 0 if m == 0.0 else 15 - int(np.frexp(np.float32(m))[1])
    e = max(-120, min(120, e))
    return (x.astype(np.float32) * np.float32(2.0 ** e)).astype(np.float16), 2.0 ** -e


def exact_product(w16, x):
    xs, inv = x16_of(x)
    return (xs.astype(np.float64) @ w16.astype(np.float64).T) * inv


def make(dev, sem, w, R, C):
    import torch
    packed = dev.pack(sem, torch.from_numpy(w).cuda(), R, C)
    return dev.dense16(sem, packed, R, C)


def gemm(dev, w16_dev, x, R, C, **kw):
    import torch
    xt = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    out = torch.full((x.shape[0], R), float("nan"), device="cuda")   # beta = 0: out is never read
    dev.gemm16(w16_dev, xt, R, C, out=out, **kw)
    return out.cpu().numpy()


@pytest.mark.parametrize("sem", sorted(QT))
def test_dense16_copy_bit_exact(dev, orc, sem):
    qt = QT[sem]
    rng = np.random.default_rng(1600 + sem)
    R, C = 70, 768 if W.BLOCK[qt][0] == 256 else 800
    w = W.gen_weights(rng, qt, R, C)
    got = make(dev, sem, w, R, C).cpu().numpy()
    ref = orc.dequant(sem, w, R, C).astype(np.float16)
    assert np.array_equal(got, ref), K.SEM_NAMES[sem]   # by value: the GPU's fl(s*q) + 0 gives +0 for -0


@pytest.mark.parametrize("sem", sorted(QT))
@pytest.mark.parametrize("M", [9, 64, 300])
def test_gemm16_vs_oracle(dev, orc, sem, M):
    qt = QT[sem]
    rng = np.random.default_rng(1700 + 31 * sem + M)
    R, C = 200, 768 if W.BLOCK[qt][0] == 256 else 800
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, M, C)
    w16 = make(dev, sem, w, R, C)
    got = gemm(dev, w16, x, R, C)
    ref = orc.gemv(sem, w, x, R, C, M)
    err = O.norm_err(got, ref)
    print(f"{K.SEM_NAMES[sem]} M={M}: norm err {err:.2e}, elem rel {O.elem_rel_err(got, ref):.2e}")
    assert err < D16_TOL, K.SEM_NAMES[sem]
    assert O.norm_err(got, exact_product(w16.cpu().numpy(), x)) < D16_EXACT


@pytest.mark.parametrize("name,sem,qt,R,C,M", [("gate", K.Q4_K_GGML, 12, 5632, 2048, 128),
                                               ("gate", K.Q4_K_GGML, 12, 5632, 2048, 512),
                                               ("gate", K.Q4_K_GGML, 12, 5632, 2048, 1280),
                                               ("down", K.Q6_K_SEQ, 14, 2048, 5632, 1280)])
def test_gemm16_config_shapes(dev, orc, name, sem, qt, R, C, M):
    """configs[2] at full size (bf16-valued activations): every output against the
    float64 product of the fp16 operands, and a strided token x row sample (every
    output tile's rows and tokens touched) against the oracle."""
    import torch
    rng = np.random.default_rng(R + M + 5)
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, M, C, bf16=True)
    w16 = make(dev, sem, w, R, C)
    got = gemm(dev, w16, x, R, C)
    assert np.all(np.isfinite(got))
    xs, inv = x16_of(x)
    exact = (torch.from_numpy(xs).cuda().double() @ w16.double().T * inv).cpu().numpy()
    assert O.norm_err(got, exact) < D16_EXACT
    toks, rows = np.arange(M)[::max(1, M // 48)], np.arange(R)[::max(1, R // 200)]
    rb = W.row_bytes(qt, C)
    wr = np.ascontiguousarray(w.reshape(R, rb)[rows].ravel())
    ref = orc.gemv(sem, wr, x[toks], len(rows), C, len(toks))
    sub = got[np.ix_(toks, rows)]
    err = O.norm_err(sub, ref)
    print(f"{name} M={M}: norm err {err:.2e}, elem rel {O.elem_rel_err(sub, ref):.2e}")
    assert err < D16_TOL


def test_gemm16_strided(dev, orc):
    """x with a token stride above n_cols, out with a row stride above n_rows."""
    import torch
    rng = np.random.default_rng(1801)
    R, C, M, ldx, ldo = 150, 512, 40, 520, 160
    w = W.gen_weights(rng, 12, R, C)
    x = W.gen_x(rng, M, ldx)
    w16 = make(dev, K.Q4_K_GGML, w, R, C)
    xt = torch.from_numpy(x).cuda()
    out = torch.full((M, ldo), -7.0, device="cuda")
    dev.gemm16(w16, xt, R, C, out=out, M=M, ldx=ldx, ldo=ldo)
    o = out.cpu().numpy()
    assert np.all(o[:, R:] == -7.0)
    ref = orc.gemv(K.Q4_K_GGML, w, np.ascontiguousarray(x[:, :C]), R, C, M)
    assert O.norm_err(o[:, :R], ref) < D16_TOL


@pytest.mark.parametrize("qt,sem,C", [(12, K.Q4_K_GGML, 2048 + 32), (39, K.MXFP4, 800 + 4)])
def test_gemm16_ragged_columns(dev, orc, qt, sem, C):
    """Columns past the last whole block contribute nothing, as in the reference."""
    import torch
    rng = np.random.default_rng(1806 + qt)
    R, M = 80, 20
    be, bb = W.BLOCK[qt]
    nb = C // be
    w = W.gen_weights(rng, qt, R, nb * be)   # whole blocks only: the ragged tail has no bytes
    x = W.gen_x(rng, M, C)
    packed = dev.pack(sem, torch.from_numpy(w).cuda(), R, C)
    w16 = dev.dense16(sem, packed, R, C)
    assert np.all(w16.cpu().numpy()[:, nb * be:] == 0)
    got = gemm(dev, w16, x, R, C)
    ref = orc.gemv(sem, w, np.ascontiguousarray(x[:, :nb * be]), R, nb * be, M)
    assert O.norm_err(got, ref) < D16_TOL


def test_gemm16_nonfinite_activations(dev, orc):
    """inf / NaN activations give the oracle's inf / NaN outputs; the scale
    ignores them, so the other tokens keep their precision."""
    rng = np.random.default_rng(1802)
    R, C, M = 96, 512, 24
    w = W.gen_weights(rng, 14, R, C)
    x = W.gen_x(rng, M, C)
    x[3, 5] = np.inf
    x[7, 9] = np.nan
    x[11, 100] = -np.inf
    w16 = make(dev, K.Q6_K_SEQ, w, R, C)
    got = gemm(dev, w16, x, R, C)
    ref = orc.gemv(K.Q6_K_SEQ, w, x, R, C, M)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])
    fin = np.isfinite(ref).all(axis=1)
    assert O.norm_err(got[fin], ref[fin]) < D16_TOL


@pytest.mark.parametrize("scale", [1e-30, 0.02, 0.3, 6000.0, 1e6, 1e30])
def test_gemm16_activation_scale(dev, orc, scale):
    """Activations scaled far below and above fp16's range, and either side of
    the bounds [1/4, 2^15) of the largest element within which the one-pass
    conversion at scale 1 stands (else it is redone at a power-of-two scale),
    keep their precision; calls at different scales alternate on one copy."""
    rng = np.random.default_rng(1803)
    R, C, M = 64, 512, 16
    w = W.gen_weights(rng, 8, R, C)
    x0 = W.gen_x(rng, M, C)
    w16 = make(dev, K.Q8_0, w, R, C)
    for s in (scale, 1.0, scale):
        x = (x0 * np.float32(s)).astype(np.float32)
        got = gemm(dev, w16, x, R, C)
        assert O.norm_err(got, orc.gemv(K.Q8_0, w, x, R, C, M)) < D16_TOL, s


@pytest.mark.parametrize("qt,sem", [(8, K.Q8_0), (39, K.MXFP4)])
def test_dense16_rejects_unrepresentable(dev, qt, sem):
    """A weight beyond fp16's finite range (Q8_0 d = 60000, an E8M0 of 255) is
    refused: the matrix stays on the quantised path."""
    rng = np.random.default_rng(1804)
    R, C = 8, 256
    w = W.gen_weights(rng, qt, R, C).reshape(R * C // 32, -1)
    if qt == 8:
        w[5, 0:2] = np.frombuffer(np.float16(60000).tobytes(), np.uint8)
    else:
        w[5, 16] = 255
    with pytest.raises(RuntimeError, match="fp16"):
        make(dev, sem, np.ascontiguousarray(w.ravel()), R, C)


def test_gemm16_graph_replay(dev, orc):
    """Captured once, replayed with new activations written eagerly between
    replays: every replay matches the eager call."""
    import torch
    rng = np.random.default_rng(1805)
    R, C, M = 256, 1024, 96
    w = W.gen_weights(rng, 12, R, C)
    w16 = make(dev, K.Q4_K_GGML, w, R, C)
    xt = torch.from_numpy(W.gen_x(rng, M, C)).cuda()
    out = torch.empty(M, R, device="cuda")
    ws = dev.gemm16_workspace(R, C, M, xt.device)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        dev.gemm16(w16, xt, R, C, out=out, ws=ws)   # plan built outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dev.gemm16(w16, xt, R, C, out=out, ws=ws)
    for i in range(3):
        xt.copy_(torch.from_numpy(W.gen_x(rng, M, C) * np.float32(4.0 ** i)).cuda())
        eager = dev.gemm16(w16, xt, R, C, ws=dev.gemm16_workspace(R, C, M, xt.device))
        torch.cuda.synchronize()
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert O.norm_err(out.cpu().numpy(), eager.cpu().numpy()) < 1e-6, f"replay {i}"
