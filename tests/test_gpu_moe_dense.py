"""GPU tests of the MoE layer's load-time bf16 expert copies
(mllm_moe_dense_experts, the MXFP4 forms): the batched path over the copies
gives results bit-identical to the per-tile decode (same bf16 tile values,
same MFMA sequence), checked at small shapes against the oracle
(helpers.moe_tol: 1e-4, or 1e-3 where an MXFP4 down requantises h to Q8_0).
Matrices the fp16-plane GEMM takes (MXFP4 with whole 64-element steps, i.e.
a row length that is a multiple of 64, and exponents within its range) are
not copied: at configs[3]'s full shape nothing is."""
import numpy as np
import pytest

import oracle as O
from helpers import MOE_Q8H_TOL, moe_tol
from mojollama_amd import kernels as K
from mojollama_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return K.DeviceOps(K.load_kernels())


def _layers(dev, qts, N, M, E, Kk, gates, ups, downs, router, renorm):
    plain = dev.moe_prepare(qts, N, M, E, Kk, gates, ups, downs, router, renorm)
    dense = dev.moe_prepare(qts, N, M, E, Kk, gates, ups, downs, router, renorm)
    return plain, dense


def _copy_bytes(qts, N, M, E):
    """Bytes mllm_moe_dense_experts allocates: MXFP4 gate/up (one semantic)
    when N is not a multiple of 64, an MXFP4 down when M is not (the
    generated exponents always fit the fp16-plane GEMM)."""
    ld_gu, ld_d = (N + 63) // 64 * 64, (M + 63) // 64 * 64
    gu = qts[0] == 39 and qts[1] == 39 and N % 64 != 0
    dn = qts[2] == 39 and M % 64 != 0
    return (2 * E * M * ld_gu if gu else 0) * 2 + (E * N * ld_d * 2 if dn else 0)


def test_dense_experts_none_on_fp16_plane_gptoss(dev):
    """configs[3] (E=32, N=M=2880, top-4, MXFP4): both GEMMs run on the
    fp16-plane GEMM, so there is nothing to copy and the layer is unchanged."""
    import torch
    wl = W.moe_workload("gptoss", 1280)
    c = wl["cfg"]
    N, M, E, Kk = c["N"], c["M"], c["E"], c["K"]
    router = torch.from_numpy(wl["router"]).cuda()
    plain, dense = _layers(dev, wl["qts"], N, M, E, Kk, wl["gates"], wl["ups"], wl["downs"], router, 1)
    assert plain.info() == 3
    assert dense.dense_experts() == 0
    x = torch.from_numpy(wl["x"][:300]).cuda()
    a = plain.forward(x)
    b = dense.forward(x)
    torch.cuda.synchronize()
    assert torch.isfinite(a).all()
    assert torch.equal(a, b)


@pytest.mark.parametrize("N,M,E,Kk,T", [(256, 96, 8, 2, 40), (320, 160, 16, 4, 70), (288, 160, 8, 2, 50)])
def test_dense_experts_small_vs_oracle(dev, orc, N, M, E, Kk, T):
    """Odd block counts (N/32, M/32 odd: the copies' zero-padded last step;
    rows of 32 mod 64 blocks stay off the fp16-plane GEMM), vs the oracle and
    bit-equal to the decoding layer."""
    import torch
    qts = (39, 39, 39)
    rng = np.random.default_rng(2100 + N + T)
    gates = [W.gen_weights(rng, 39, M, N) for _ in range(E)]
    ups = [W.gen_weights(rng, 39, M, N) for _ in range(E)]
    downs = [W.gen_weights(rng, 39, N, M) for _ in range(E)]
    router = W.gen_router(rng, E, N)
    x = W.gen_x(rng, T, N)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    plain, dense = _layers(dev, qts, N, M, E, Kk, [cu(g) for g in gates], [cu(u) for u in ups],
                           [cu(d) for d in downs], cu(router), 1)
    assert dense.dense_experts() == _copy_bytes(qts, N, M, E) > 0
    a = plain.forward(cu(x))
    b = dense.forward(cu(x))
    assert torch.equal(a, b)
    ri, rw = orc.route(router, x, Kk, 1)
    ref = np.stack([orc.moe_forward_token(gates, ups, downs, x[t], M, N, qts, ri[t], rw[t]) for t in range(T)])
    assert O.norm_err(b.cpu().numpy(), ref) < MOE_Q8H_TOL


def test_dense_experts_qwen3_config(dev):
    """configs[4] (Q4_K x Q8_0 gate/up, Q6_K down: no one-plane form): no copy is
    made and the layer runs as before."""
    import torch
    wl = W.moe_workload("qwen3", 300)
    c = wl["cfg"]
    N, M, E, Kk = c["N"], c["M"], c["E"], c["K"]
    router = torch.from_numpy(wl["router"]).cuda()
    plain, dense = _layers(dev, wl["qts"], N, M, E, Kk, wl["gates"], wl["ups"], wl["downs"], router, 1)
    assert dense.dense_experts() == 0
    x = torch.from_numpy(wl["x"]).cuda()
    assert torch.equal(plain.forward(x), dense.forward(x))


@pytest.mark.parametrize("qts,N", [((39, 39, 39), 544), ((12, 12, 39), 512)])
def test_dense_experts_formats_vs_oracle(dev, orc, qts, N):
    """MXFP4 experts with and without MXFP4 gate/up (a down-only copy beside
    the Q4_K x Q8_0 gate/up on the fp16-plane GEMM), vs the oracle and
    bit-equal to the decoding layer.  (Gate/up products exact in both cases:
    at this small M a
    single one-step flip of a Q8_0 code of h already moves an output by
    3 / (127 sqrt(M)) ~ 1.5e-3 of its max.)"""
    import torch
    M, E, Kk, T = 288, 8, 2, 60
    rng = np.random.default_rng(2300 + sum(qts))
    gates = [W.gen_weights(rng, qts[0], M, N) for _ in range(E)]
    ups = [W.gen_weights(rng, qts[1], M, N) for _ in range(E)]
    downs = [W.gen_weights(rng, qts[2], N, M) for _ in range(E)]
    router = W.gen_router(rng, E, N)
    x = W.gen_x(rng, T, N)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    plain, dense = _layers(dev, qts, N, M, E, Kk, [cu(g) for g in gates], [cu(u) for u in ups],
                           [cu(d) for d in downs], cu(router), 0)
    assert dense.dense_experts() == _copy_bytes(qts, N, M, E) > 0
    a = plain.forward(cu(x))
    b = dense.forward(cu(x))
    assert torch.equal(a, b)
    ri, rw = orc.route(router, x, Kk, 0)
    ref = np.stack([orc.moe_forward_token(gates, ups, downs, x[t], M, N, qts, ri[t], rw[t]) for t in range(T)])
    assert O.norm_err(b.cpu().numpy(), ref) < moe_tol(qts)
