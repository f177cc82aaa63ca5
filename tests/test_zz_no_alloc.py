"""mllm_moe_forward_noalloc (the MoE layer with its workspace in the library's
static device array) against mllm_moe_forward with a caller workspace,
through the C ABI: two calls in a row on one layer, the second with fewer
tokens, on the decode path (T <= 24) and on the grouped-GEMM path; routing
bit-exact and outputs bit-identical (same kernels, same inputs).  A T whose
workspace exceeds the static maximum is rejected and leaves the output alone.
"""
import numpy as np
import pytest

from mojollama_amd import kernels as K
from mojollama_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return K.DeviceOps(K.load_kernels())


def _layer(dev, qts, N, M, E, Kk, seed):
    import torch
    rng = np.random.default_rng(seed)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    gates = [cu(W.gen_weights(rng, qts[0], M, N)) for _ in range(E)]
    ups = [cu(W.gen_weights(rng, qts[1], M, N)) for _ in range(E)]
    downs = [cu(W.gen_weights(rng, qts[2], N, M)) for _ in range(E)]
    router = cu(W.gen_router(rng, E, N))
    return dev.moe_prepare(qts, N, M, E, Kk, gates, ups, downs, router, 1), rng


def _noalloc(dev, layer, x, T):
    import torch
    out = torch.full((T, layer.N), float("nan"), device="cuda")
    idx = torch.full((T, layer.K), -7, dtype=torch.int32, device="cuda")
    w = torch.empty((T, layer.K), dtype=torch.float32, device="cuda")
    rc = dev.so.mllm_moe_forward_noalloc(layer.h, x.data_ptr(), T, out.data_ptr(), idx.data_ptr(), w.data_ptr(),
                                         dev._stream())
    torch.cuda.synchronize()
    return rc, out, idx, w


@pytest.mark.parametrize("qts,N,M,E,Kk,Ts", [((12, 12, 14), 2048, 768, 32, 8, (20, 3)),
                                             ((39, 39, 39), 2880, 2880, 8, 4, (40, 30))])
def test_noalloc_matches_forward(dev, qts, N, M, E, Kk, Ts):
    import torch
    layer, rng = _layer(dev, qts, N, M, E, Kk, seed=N + E)
    for T in Ts:
        print(f"[case] noalloc {qts} N={N} M={M} E={E} K={Kk} T={T}", flush=True)
        x = torch.from_numpy(W.gen_x(rng, T, N)).cuda()
        idx = torch.empty((T, Kk), dtype=torch.int32, device="cuda")
        w = torch.empty((T, Kk), dtype=torch.float32, device="cuda")
        ref = layer.forward(x, idx=idx, w=w)
        rc, got, gidx, gw = _noalloc(dev, layer, x, T)
        assert rc == 0, K.last_error(dev.so)
        assert torch.equal(gidx, idx)
        assert torch.equal(gw, w)
        assert torch.equal(got, ref)


def test_noalloc_rejects_oversized_T(dev):
    import torch
    layer, rng = _layer(dev, (12, 12, 14), 2048, 768, 32, 8, seed=3)
    T = 256
    assert dev.so.mllm_moe_workspace_size(layer.h, T) > 32 * 1024 * 1024
    x = torch.from_numpy(W.gen_x(rng, T, 2048)).cuda()
    rc, out, idx, _ = _noalloc(dev, layer, x, T)
    assert rc == -1
    assert "static maximum" in K.last_error(dev.so)
    assert torch.isnan(out).all() and bool((idx == -7).all())
    # a smaller call on the same layer still works afterwards
    rc, out, _, _ = _noalloc(dev, layer, x[:2].contiguous(), 2)
    assert rc == 0 and torch.isfinite(out).all()
