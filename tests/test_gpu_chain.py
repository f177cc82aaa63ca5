"""GPU parity of the headline's own launches: bench.py's TinyLlama decode pass
(mojollama_amd.decode_chain.DecodeChain, the same object bench.py times) at
the bench's shapes and fusion modes, against the oracle.

Per layer the pass runs (TE:1516-1716 with the *_batch_matmul semantics of
CE:255-378):
    qkv  = Wqkv . rmsnorm(x) * g_attn                       2560 x 2048 Q4_K, RMSNorm prologue
    xb   = x + Wo . qkv[:, :2048]                           2048 x 2048 Q4_K, residual epilogue
    h    = silu(Wg . v) * (Wu . v), v = rmsnorm(xb) * g_ffn   5632 paired rows x 2048 Q4_K
    x'   = xb + Wdown . h                                   2048 x 5632 Q6_K sequential, residual epilogue
and logits = Wlm . rmsnorm(x) * g_out (32000 x 2048 Q6_K sequential).  At B = 1
these are the bench's launches exactly: the paired gate/up selects 16 lanes per
row (its 11264 stacked rows give about two workgroups per CU), the lm_head the
RMS-prologue instantiation of the Q6_K kernel.

Checks:
  * stage by stage: each launch against the oracle applied to the GPU's own
    input of that launch (the activation formed in float64 from the
    reference's formulas), at GEMV_TOL -- the bound of every decode GEMV;
  * end to end: the oracle composition of the whole two-layer pass from the
    same x0 against the GPU logits, at CHAIN_TOL (below).
"""
import numpy as np
import pytest

import oracle as O
from helpers import GEMV_TOL
from mojollama_amd import kernels as K
from mojollama_amd import workloads as W
from mojollama_amd.decode_chain import EPS, DecodeChain, build_tinyllama

pytestmark = pytest.mark.gpu

# End to end, each stage's fp32 differences (summation order, the norm's
# rounding: ~1e-7 of a stage's output scale) feed the next stage.  Ten stages
# with RMSNorms between them keep that growth linear in practice; 1e-4 keeps a
# factor of ~50 over what ten such steps can add while a decode mistake in any
# matrix (> 3e-3 of its output) still fails.
CHAIN_TOL = 1e-4


def centered(rng, qt, rows, cols):
    """The chain's weights: zero-mean Q4_K blocks (workloads.gen_q4k_centered)
    and BASELINE's Q6_K.  With BASELINE's Q4_K scales and mins every row has a
    positive mean, the residual stream saturates after one layer and every
    gate of the SiLU product lies far below zero (h = 0 on both sides), which
    would leave the later stages unchecked.  The launches (shapes, batch,
    fusions) are the bench's either way."""
    return W.gen_q4k_centered(rng, rows, cols) if qt == W.QT_Q4_K else W.gen_weights(rng, qt, rows, cols)


@pytest.fixture(scope="module")
def chain_model():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    dev = K.DeviceOps(K.load_kernels())
    layers, lm, out_norm = build_tinyllama(dev, np.random.default_rng(2), 2, keep_raw=True, gen=centered)
    norms = [(L["attn_norm"].cpu().numpy(), L["ffn_norm"].cpu().numpy()) for L in layers]
    return dev, layers, lm, out_norm, norms, out_norm.cpu().numpy()


def rms_np(v, w):
    v = np.asarray(v, np.float64)
    return (v * (1.0 / np.sqrt(np.mean(v * v, axis=1, keepdims=True) + EPS)) * w).astype(np.float32)


def silu_mul(g, u):
    g = np.asarray(g, np.float64)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g)) * np.asarray(u, np.float64)


def stage_refs(orc, layers, lm, norms, g_out, x_in, B):
    """The oracle's value of every stage of the pass from x_in [B][2048], as
    (name, function of the GPU's input to that stage) pairs in launch order."""
    out = []
    for L, (ga, gf) in zip(layers, norms):
        out.append(("qkv", lambda x, L=L, ga=ga: orc.gemv(K.Q4_K_GGML, L["qkv"].raw, rms_np(x, ga), 2560, 2048, B)))
        out.append(("o", lambda qkv, xa, L=L: xa.astype(np.float64) +
                    orc.gemv(K.Q4_K_GGML, L["o"].raw, np.ascontiguousarray(qkv[:, :2048]), 2048, 2048, B)))
        out.append(("gate_up", lambda xb, L=L, gf=gf: silu_mul(*np.split(
            orc.gemv(K.Q4_K_GGML, L["gate_up"].raw, rms_np(xb, gf), 11264, 2048, B), 2, axis=1))))
        out.append(("down", lambda h, xb, L=L: xb.astype(np.float64) +
                    orc.gemv(K.Q6_K_SEQ, L["down"].raw, np.ascontiguousarray(h, np.float32), 2048, 5632, B)))
    out.append(("lm_head", lambda x: orc.gemv(K.Q6_K_SEQ, lm.raw, rms_np(x, g_out), 32000, 2048, B)))
    return out


def compose(orc, layers, lm, norms, g_out, x0, B):
    """The whole pass in the oracle from x0, every intermediate rounded to fp32
    as the GPU stores it."""
    f32 = lambda a: np.asarray(a, np.float32)  # noqa: E731
    xa = f32(x0)
    for L, (ga, gf) in zip(layers, norms):
        qkv = orc.gemv(K.Q4_K_GGML, L["qkv"].raw, rms_np(xa, ga), 2560, 2048, B)
        xb = f32(xa + orc.gemv(K.Q4_K_GGML, L["o"].raw, np.ascontiguousarray(qkv[:, :2048]), 2048, 2048, B))
        gu = orc.gemv(K.Q4_K_GGML, L["gate_up"].raw, rms_np(xb, gf), 11264, 2048, B)
        h = f32(silu_mul(gu[:, :5632], gu[:, 5632:]))
        xa = f32(xb + orc.gemv(K.Q6_K_SEQ, L["down"].raw, h, 2048, 5632, B))
    return orc.gemv(K.Q6_K_SEQ, lm.raw, rms_np(xa, g_out), 32000, 2048, B)


@pytest.mark.parametrize("B", [1, 4, 8])
def test_decode_chain_vs_oracle(chain_model, orc, B):
    import torch
    dev, layers, lm, out_norm, norms, g_out = chain_model
    x0 = torch.from_numpy(np.random.default_rng(100 + B).standard_normal((B, 2048)).astype(np.float32)).cuda()
    ch = DecodeChain(torch, dev, layers, lm, out_norm, B, x0=x0)
    rec = []
    ch.run(record=rec)
    torch.cuda.synchronize()
    got = [(n, t.cpu().numpy()) for n, t in rec]
    refs = stage_refs(orc, layers, lm, norms, g_out, None, B)
    assert [n for n, _ in got] == [n for n, _ in refs]
    xa = x0.cpu().numpy()
    worst = 0.0
    for i, ((name, g), (_, fn)) in enumerate(zip(got, refs)):
        if name == "qkv":
            ref = fn(xa)
            qkv = g
        elif name == "o":
            ref = fn(qkv, xa)
            xb = g
        elif name == "gate_up":
            ref = fn(xb)
            h = g
        elif name == "down":
            ref = fn(h, xb)
            xa = g
        else:
            ref = fn(xa)
        err = O.norm_err(g, ref)
        worst = max(worst, err)
        assert np.abs(ref).max() > 1e-3, f"stage {i} {name}: degenerate reference"
        print(f"[parity] chain B={B} stage {i} {name}: {err:.3e}", flush=True)
        assert np.isfinite(g).all(), f"stage {i} {name}: non-finite output"
        assert err < GEMV_TOL, f"stage {i} {name} B={B}: {err:.3e} ({K.last_error(dev.so)})"
    e2e = O.norm_err(got[-1][1], compose(orc, layers, lm, norms, g_out, x0.cpu().numpy(), B))
    print(f"[parity] chain B={B} end to end logits: {e2e:.3e} (worst stage {worst:.3e})", flush=True)
    assert e2e < CHAIN_TOL


def test_headline_launches_b1_standalone(chain_model, orc):
    """The B = 1 launches on their own, each from an independent N(0,1)
    activation (no chain), so a stage that only passes on its chain input's
    statistics still fails: fused RMSNorm + qkv, o + residual (x_ld = 2560),
    fused RMSNorm + paired gate/up + SiLU, down + residual, RMSNorm + lm_head."""
    import torch
    dev, layers, lm, out_norm, norms, g_out = chain_model
    L = layers[0]
    ga, gf = norms[0]
    rng = np.random.default_rng(7)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()  # noqa: E731
    ch = DecodeChain(torch, dev, layers, lm, out_norm, 1)
    x = rng.standard_normal((1, 2048)).astype(np.float32)
    res = rng.standard_normal((1, 2048)).astype(np.float32)
    qkvx = rng.standard_normal((1, 2560)).astype(np.float32)
    h = (rng.standard_normal((1, 5632)) * 50).astype(np.float32)
    cases = []
    out = dev.gemv_fused(L["qkv"].sem, L["qkv"].packed, cu(x), 2560, 2048, ch.f_qkv[0], ws=ch.ws)
    cases.append(("qkv", out, orc.gemv(K.Q4_K_GGML, L["qkv"].raw, rms_np(x, ga), 2560, 2048, 1)))
    ch.xa.copy_(cu(res))
    q = cu(qkvx)
    out = dev.gemv_fused(L["o"].sem, L["o"].packed, q.data_ptr(), 2048, 2048, ch.f_o, ws=ch.ws, B=1)
    cases.append(("o", out, res + orc.gemv(K.Q4_K_GGML, L["o"].raw, np.ascontiguousarray(qkvx[:, :2048]), 2048, 2048, 1)))
    out = dev.gemv_fused(L["gate_up"].sem, L["gate_up"].packed, cu(x), 5632, 2048, ch.f_gu[0], ws=ch.ws)
    gu = orc.gemv(K.Q4_K_GGML, L["gate_up"].raw, rms_np(x, gf), 11264, 2048, 1)
    cases.append(("gate_up", out, silu_mul(gu[:, :5632], gu[:, 5632:])))
    ch.xb.copy_(cu(res))
    out = dev.gemv_fused(L["down"].sem, L["down"].packed, cu(h), 2048, 5632, ch.f_down, ws=ch.ws)
    cases.append(("down", out, res + orc.gemv(K.Q6_K_SEQ, L["down"].raw, h, 2048, 5632, 1)))
    out = dev.gemv_fused(lm.sem, lm.packed, cu(x), 32000, 2048, ch.f_lm, ws=ch.ws)
    cases.append(("lm_head", out, orc.gemv(K.Q6_K_SEQ, lm.raw, rms_np(x, g_out), 32000, 2048, 1)))
    for name, got, ref in cases:
        err = O.norm_err(got.cpu().numpy(), ref)
        print(f"[parity] headline B=1 {name}: {err:.3e}", flush=True)
        assert err < GEMV_TOL, f"{name}: {err:.3e}"
