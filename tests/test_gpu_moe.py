"""GPU parity of routing and the MoE entry points through the C ABI.

Routing: expert selection bit-exact with the reference (golden vectors from
its compiled moe_ffn at the real router shapes) and with the oracle; routing
weights within 1e-6 relative.  MoE outputs: MOE_TOL normalised max error.
"""
import ctypes
import zlib

import numpy as np
import pytest

import oracle as O
from helpers import MOE_TOL, BCView, fp, up
from mojollama_amd import kernels as K
from mojollama_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return K.load_kernels()


@pytest.fixture(scope="module")
def dev(lib):
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return K.DeviceOps(lib)


def crc(*arrays):
    c = 0
    for a in arrays:
        c = zlib.crc32(np.ascontiguousarray(a).view(np.uint8).tobytes(), c)
    return c


def moe_ffn(lib, bc, x, N):
    out = np.full(N, np.nan, np.float32)
    gate_buf = np.zeros(4096, np.float32)
    up_buf = np.zeros(4096, np.float32)
    xx = np.ascontiguousarray(x, np.float32).copy()
    lib.moe_ffn(bc.ptr(), 0, fp(xx), fp(gate_buf), fp(up_buf), fp(out), 1)
    return out


def moe_forward(lib, gates, ups, downs, x, n_ff, n_embd, qts, ti, tw, with_q8=True):
    arr = ctypes.POINTER(ctypes.c_uint8) * len(gates)
    g = arr(*[up(a) for a in gates])
    u = arr(*[up(a) for a in ups])
    d = arr(*[up(a) for a in downs])
    Kk = len(ti)
    out = np.full(n_embd, np.nan, np.float32)
    buf = np.zeros(3 * Kk * n_ff, np.float32)
    q8 = np.zeros(Kk * n_ff * 34 // 32 + 64, np.uint8)
    ti = np.ascontiguousarray(ti, np.int32)
    tw = np.ascontiguousarray(tw, np.float32)
    lib.moe_forward_omp(g, u, d, fp(np.ascontiguousarray(x, np.float32)), n_ff, n_embd, qts[0], qts[1], qts[2],
                        ti.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), fp(tw), Kk, fp(out), fp(buf),
                        up(q8) if with_q8 else ctypes.cast(None, ctypes.POINTER(ctypes.c_uint8)))
    return out


@pytest.mark.parametrize("tag", ["gptoss", "qwen3"])
def test_golden_route_selection_bitexact(lib, golden, tag):
    """moe_ffn at the real router shapes (2880x32 top-4, 2048x128 top-8) picks
    exactly the experts the reference's compiled moe_ffn picked."""
    g = golden(f"route_sel_{tag}.npz")
    N, E, Kk, T, M = (int(g[k]) for k in ("N", "E", "K", "T", "M"))
    r2 = np.random.default_rng(int(g["seed"]))
    router = W.gen_router(r2, E, N)
    xs = W.gen_x(r2, T, N)
    assert crc(router, xs) == int(g["crc"]), "numpy RNG stream changed: regenerate fixtures"
    g1 = W.gen_weights(r2, 12, M, N).reshape(-1, 144)
    g1[:, 0:4] = np.array([1e-6, 1e-6], np.float16).view(np.uint8)
    g1 = np.ascontiguousarray(g1.ravel())
    gate = np.concatenate([g1] * E)
    blk = np.zeros(210, np.uint8)
    blk[0:128] = 0xFF
    blk[128:192] = 0xFF
    blk[192:208] = 1
    blk[208:210] = np.array([1.0], np.float16).view(np.uint8)
    down = np.zeros((E, N, (M // 256) * 210), np.uint8)
    for e in range(E):
        down[e, e, :] = blk
    down = np.ascontiguousarray(down.ravel())
    bc = BCView(N, E, Kk, M, router, gate, gate, down, (12, 12, 14))
    ffn = np.stack([moe_ffn(lib, bc, xs[t], N)[:E] for t in range(T)])
    sel = (ffn != 0).astype(np.uint8)
    assert np.array_equal(sel, g["sel"])
    assert O.norm_err(ffn, g["ffn"]) < MOE_TOL


@pytest.mark.parametrize("E,N,Kk,renorm", [(32, 2880, 4, 0), (128, 2048, 8, 1), (8, 256, 2, 0)])
def test_device_route_vs_oracle(dev, orc, E, N, Kk, renorm):
    import torch
    rng = np.random.default_rng(E + N)
    T = 300
    rw = W.gen_router(rng, E, N)
    x = W.gen_x(rng, T, N)
    ri, rwt = orc.route(rw, x, Kk, renorm)
    idx, wt = dev.route(torch.from_numpy(np.ascontiguousarray(rw.T)).cuda(), torch.from_numpy(x).cuda(), Kk, renorm)
    assert np.array_equal(idx.cpu().numpy(), ri)
    assert np.max(np.abs(wt.cpu().numpy() - rwt) / rwt) < 1e-6


@pytest.mark.parametrize("tag", ["qwen", "gptoss"])
def test_golden_moe_forward(lib, golden, tag):
    g = golden(f"moe_forward_{tag}.npz")
    got = moe_forward(lib, list(g["gates"]), list(g["ups"]), list(g["downs"]), g["x"], int(g["n_ff"]),
                      int(g["n_embd"]), tuple(int(v) for v in g["qts"]), g["top_idx"], g["top_w"])
    assert O.norm_err(got, g["out"]) < MOE_TOL, K.last_error(lib)


@pytest.mark.parametrize("tag", ["q4k", "mxfp4"])
def test_golden_moe_ffn(lib, golden, tag):
    g = golden(f"moe_ffn_{tag}.npz")
    N, E, Kk, M = (int(g[k]) for k in ("N", "E", "K", "M"))
    bc = BCView(N, E, Kk, M, g["router"], g["gate"], g["up"], g["down"], tuple(int(v) for v in g["qts"]))
    for t in range(g["x"].shape[0]):
        got = moe_ffn(lib, bc, g["x"][t], N)
        assert O.norm_err(got, g["out"][t]) < MOE_TOL


def test_moe_ffn_batch_keeps_last_token(lib, golden):
    """With B > 1 the reference's moe_ffn clears ffn_buf per token (CE:643)."""
    g = golden("moe_ffn_q4k.npz")
    N, E, Kk, M = (int(g[k]) for k in ("N", "E", "K", "M"))
    bc = BCView(N, E, Kk, M, g["router"], g["gate"], g["up"], g["down"], tuple(int(v) for v in g["qts"]))
    xs = np.ascontiguousarray(g["x"][:3])
    out = np.zeros(N, np.float32)
    gb, ub = np.zeros(4096, np.float32), np.zeros(4096, np.float32)
    lib.moe_ffn(bc.ptr(), 0, fp(xs), fp(gb), fp(ub), fp(out), 3)
    assert O.norm_err(out, g["out"][2]) < MOE_TOL


@pytest.mark.parametrize("qts,n_embd,n_ff", [((39, 39, 39), 2880, 2880), ((12, 12, 14), 2048, 768),
                                              ((14, 14, 2), 512, 256)])
def test_moe_forward_vs_oracle_real_shapes(lib, orc, qts, n_embd, n_ff):
    """moe_forward_omp at the GPT-OSS (MXFP4) and Qwen3 (Q4_K/Q6_K) expert shapes."""
    rng = np.random.default_rng(sum(qts) + n_embd)
    E, Kk = 6, 4
    gates = [W.gen_weights(rng, qts[0], n_ff, n_embd) for _ in range(E)]
    ups = [W.gen_weights(rng, qts[1], n_ff, n_embd) for _ in range(E)]
    downs = [W.gen_weights(rng, qts[2], n_embd, n_ff) for _ in range(E)]
    x = W.gen_x(rng, 1, n_embd)[0]
    ti = np.array([4, 1, 5, 0], np.int32)
    tw = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    got = moe_forward(lib, gates, ups, downs, x, n_ff, n_embd, qts, ti, tw)
    ref = orc.moe_forward_token(gates, ups, downs, x, n_ff, n_embd, qts, ti, tw)
    assert O.norm_err(got, ref) < MOE_TOL


def test_moe_forward_null_q8_mxfp4_down_is_guarded(lib, orc):
    rng = np.random.default_rng(9)
    n_embd, n_ff = 256, 128
    gates = [W.gen_weights(rng, 39, n_ff, n_embd) for _ in range(2)]
    downs = [W.gen_weights(rng, 39, n_embd, n_ff) for _ in range(2)]
    x = W.gen_x(rng, 1, n_embd)[0]
    ti, tw = np.array([1, 0], np.int32), np.array([0.6, 0.4], np.float32)
    got = moe_forward(lib, gates, gates, downs, x, n_ff, n_embd, (39, 39, 39), ti, tw, with_q8=False)
    assert np.all(got == 0.0)
    assert "prealloc_q8" in K.last_error(lib)
