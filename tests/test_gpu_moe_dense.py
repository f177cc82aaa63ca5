"""GPU tests of the MoE layer's load-time bf16 expert copies
(mllm_moe_dense_experts): the batched path over the copies gives results
bit-identical to the per-tile decode (same bf16 tile values, same MFMA
sequence), checked at configs[3]'s full GPT-OSS shape and at small shapes
against the oracle, and layers whose weights are not exact in bf16 make no
copy."""
import numpy as np
import pytest

import oracle as O
from mojollama_amd import kernels as K
from mojollama_amd import workloads as W

pytestmark = pytest.mark.gpu
MOE_TOL_MX = 1e-3   # MXFP4 down: h requantised to Q8_0 (as in test_gpu_moe)


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return K.DeviceOps(K.load_kernels())


def _layers(dev, qts, N, M, E, Kk, gates, ups, downs, router, renorm):
    plain = dev.moe_prepare(qts, N, M, E, Kk, gates, ups, downs, router, renorm)
    dense = dev.moe_prepare(qts, N, M, E, Kk, gates, ups, downs, router, renorm)
    return plain, dense


@pytest.mark.parametrize("T", [25, 300, 1280])
def test_dense_experts_bit_identical_gptoss(dev, T):
    """configs[3] (E=32, N=M=2880, top-4, MXFP4): every output bit-equal."""
    import torch
    wl = W.moe_workload("gptoss", 1280)
    c = wl["cfg"]
    N, M, E, Kk = c["N"], c["M"], c["E"], c["K"]
    router = torch.from_numpy(wl["router"]).cuda()
    plain, dense = _layers(dev, wl["qts"], N, M, E, Kk, wl["gates"], wl["ups"], wl["downs"], router, 1)
    nbytes = dense.dense_experts()
    ld = (N + 63) // 64 * 64
    assert nbytes == 3 * E * M * ld * 2
    assert dense.dense_experts() == 0   # made once
    x = torch.from_numpy(wl["x"][:T]).cuda()
    a = plain.forward(x)
    b = dense.forward(x)
    torch.cuda.synchronize()
    assert torch.isfinite(a).all()
    assert torch.equal(a, b)


@pytest.mark.parametrize("N,M,E,Kk,T", [(256, 96, 8, 2, 40), (320, 160, 16, 4, 70)])
def test_dense_experts_small_vs_oracle(dev, orc, N, M, E, Kk, T):
    """Odd block counts (N/32, M/32 odd: the copies' zero-padded last step), vs
    the oracle and bit-equal to the decoding layer."""
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
    assert dense.dense_experts() > 0
    a = plain.forward(cu(x))
    b = dense.forward(cu(x))
    assert torch.equal(a, b)
    ri, rw = orc.route(router, x, Kk, 1)
    ref = np.stack([orc.moe_forward_token(gates, ups, downs, x[t], M, N, qts, ri[t], rw[t]) for t in range(T)])
    assert O.norm_err(b.cpu().numpy(), ref) < MOE_TOL_MX


def test_dense_experts_not_exact_formats(dev):
    """Q4_K / Q6_K experts are not exact in one bf16: no copy is made and the
    layer runs as before."""
    import torch
    qts = (12, 12, 14)
    N, M, E, Kk, T = 256, 256, 8, 2, 30
    rng = np.random.default_rng(2200)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    gates = [cu(W.gen_weights(rng, 12, M, N)) for _ in range(E)]
    ups = [cu(W.gen_weights(rng, 12, M, N)) for _ in range(E)]
    downs = [cu(W.gen_weights(rng, 14, N, M)) for _ in range(E)]
    router = cu(W.gen_router(rng, E, N))
    x = cu(W.gen_x(rng, T, N))
    plain, dense = _layers(dev, qts, N, M, E, Kk, gates, ups, downs, router, 0)
    assert dense.dense_experts() == 0
    assert torch.equal(plain.forward(x), dense.forward(x))
