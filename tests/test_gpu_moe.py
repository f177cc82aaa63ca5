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
from helpers import MOE_TOL, BCView, fp, moe_tol, up
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


@pytest.mark.parametrize("T,slices", [(3, True), (3, False), (300, True)])
@pytest.mark.parametrize("E,N,Kk,renorm", [(32, 2880, 4, 0), (128, 2048, 8, 1), (8, 256, 2, 0), (256, 512, 16, 1),
                                           (6, 250, 2, 1), (36, 2884, 4, 0), (30, 1000, 3, 0), (64, 2880, 4, 1)])
def test_device_route_vs_oracle(dev, orc, E, N, Kk, renorm, T, slices):
    """The streamed variants (T <= 8 per token or over 32-expert slices, token
    groups), the any-shape fallback (N not a multiple of 4) and a ragged last
    chunk (N % 8 == 4)."""
    import torch
    rng = np.random.default_rng(E + N + T)
    rw = W.gen_router(rng, E, N)
    x = W.gen_x(rng, T, N)
    ri, rwt = orc.route(rw, x, Kk, renorm)
    idx, wt = dev.route(torch.from_numpy(rw).cuda(), torch.from_numpy(x).cuda(), Kk, renorm, slices=slices)
    assert np.array_equal(idx.cpu().numpy(), ri)
    assert np.max(np.abs(wt.cpu().numpy() - rwt) / rwt) < 1e-6


@pytest.mark.parametrize("E,N,Kk,renorm", [(128, 2048, 8, 1), (144, 1000, 6, 0), (130, 2884, 8, 1)])
def test_device_route_many_tokens_vs_oracle(dev, orc, E, N, Kk, renorm):
    """T = 1100 (a ragged last token group) through the many-token routing
    kernel, with N % 16 != 0 (a 16-step group that straddles the end of the
    rows) and E not a multiple of 16."""
    import torch
    T = 1100
    rng = np.random.default_rng(E + N)
    rw = W.gen_router(rng, E, N)
    x = W.gen_x(rng, T, N)
    ri, rwt = orc.route(rw, x, Kk, renorm)
    idx, wt = dev.route(torch.from_numpy(rw).cuda(), torch.from_numpy(x).cuda(), Kk, renorm)
    assert np.array_equal(idx.cpu().numpy(), ri)
    assert np.max(np.abs(wt.cpu().numpy() - rwt) / rwt) < 1e-6


@pytest.mark.parametrize("tag", ["qwen", "gptoss", "q5down", "q5down_all"])
def test_golden_moe_forward(lib, golden, tag):
    """q5down*: a Q5_0 down projection with n_embd < n_ff, whose rows the
    reference addresses with a stride from n_embd (QK:2216, 2230)."""
    g = golden(f"moe_forward_{tag}.npz")
    got = moe_forward(lib, list(g["gates"]), list(g["ups"]), list(g["downs"]), g["x"], int(g["n_ff"]),
                      int(g["n_embd"]), tuple(int(v) for v in g["qts"]), g["top_idx"], g["top_w"])
    assert O.norm_err(got, g["out"]) < MOE_TOL, K.last_error(lib)


@pytest.mark.parametrize("tag", ["qwen", "gptoss"])
def test_golden_moe_forward_nonfinite(lib, golden, tag):
    """Tokens holding a NaN or an inf: NaN / inf outputs where the reference
    has them (its Q8_0 amax order, the +-80 clamp passing NaN), finite ones
    within tolerance."""
    g = golden(f"moe_forward_nonfinite_{tag}.npz")
    qts = tuple(int(v) for v in g["qts"])
    for i, (x, ref) in enumerate(zip(g["x"], g["out"])):
        got = moe_forward(lib, list(g["gates"]), list(g["ups"]), list(g["downs"]), x, int(g["n_ff"]),
                          int(g["n_embd"]), qts, g["top_idx"], g["top_w"])
        assert np.array_equal(np.isnan(got), np.isnan(ref)), (tag, i)
        assert np.array_equal(np.isinf(got), np.isinf(ref)), (tag, i)
        fin = np.isfinite(ref)
        if fin.any():
            assert O.norm_err(got[fin], ref[fin]) < moe_tol(qts), (tag, i)


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
    assert O.norm_err(got, ref) < moe_tol(qts)


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


# ------------------------------------------------------------- batched MoE

def test_bucketing_stable_and_exact(dev):
    """GPU bucketing of (token, slot) entries by expert equals a stable sort by expert."""
    import torch
    rng = np.random.default_rng(31)
    E, TK = 128, 10240
    idx = rng.integers(0, E, TK).astype(np.int32)
    idx[rng.choice(TK, TK // 4, replace=False)] = rng.integers(0, 8, TK // 4)   # hot experts
    off, perm, pos_of, (te, tb, tend) = dev.moe_bucket(torch.from_numpy(idx).cuda(), E)
    order = np.argsort(idx, kind="stable")
    assert np.array_equal(perm.cpu().numpy(), order)
    pos = np.empty(TK, np.int64)
    pos[order] = np.arange(TK)
    assert np.array_equal(pos_of.cpu().numpy(), pos)
    counts = np.bincount(idx, minlength=E)
    assert np.array_equal(off.cpu().numpy(), np.concatenate([[0], np.cumsum(counts)]))
    te, tb, tend = te.cpu().numpy(), tb.cpu().numpy(), tend.cpu().numpy()
    assert np.all(tend - tb <= 64) and np.all(tend > tb)
    cover = np.zeros(TK, np.int32)
    for e, b, x in zip(te, tb, tend):
        assert np.all(idx[order[b:x]] == e)
        cover[b:x] += 1
    assert np.all(cover == 1)


def _moe_case(dev, orc, qts, N, M, E, Kk, T, renorm, seed, skew=False, plant=None, info=None):
    import torch
    rng = np.random.default_rng(seed)
    gates = [W.gen_weights(rng, qts[0], M, N) for _ in range(E)]
    ups = [W.gen_weights(rng, qts[1], M, N) for _ in range(E)]
    downs = [W.gen_weights(rng, qts[2], N, M) for _ in range(E)]
    if plant:
        plant(gates, ups, downs)
    router = W.gen_router(rng, E, N)
    if skew:
        x, router, _, _ = W.skewed_tokens(rng, router, T)
    else:
        x = W.gen_x(rng, T, N)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    layer = dev.moe_prepare(qts, N, M, E, Kk, [cu(g) for g in gates], [cu(u) for u in ups], [cu(d) for d in downs],
                            cu(router), renorm)
    idx = torch.empty((T, Kk), dtype=torch.int32, device="cuda")
    w = torch.empty((T, Kk), dtype=torch.float32, device="cuda")
    got = layer.forward(cu(x), idx=idx, w=w).cpu().numpy()
    ri, rw = orc.route(router, x, Kk, renorm)
    assert np.array_equal(idx.cpu().numpy(), ri), "routing differs"
    assert np.max(np.abs(w.cpu().numpy() - rw) / np.abs(rw)) < 1e-6
    ref = np.stack([orc.moe_forward_token(gates, ups, downs, x[t], M, N, qts, ri[t], rw[t]) for t in range(T)])
    if info is not None:
        info.append(layer.info())
    return got, ref


def _plant_mxfp4_span(span, zero_blocks, big=147):
    """Every MXFP4 block of every expert matrix at E = big - span, except blocks 3, 40
    and 77 of each: E = big with all-zero codes (they set the largest exponent and add
    nothing), and with zero_blocks blocks 5 and 6 at E = 0 (a zero scale)."""
    def plant(gates, ups, downs):
        for a in gates + ups + downs:
            b = a.reshape(-1, 17)
            b[:, 16] = big - span
            b[[3, 40, 77], :16] = 0
            b[[3, 40, 77], 16] = big
            if zero_blocks:
                b[[5, 6], 16] = 0
    return plant


@pytest.mark.parametrize("span,zero_blocks,fits", [(22, True, True), (25, False, True), (26, True, False)])
def test_moe_layer_mxfp4_exponent_span(dev, orc, span, zero_blocks, fits):
    """T = 40 MXFP4 layers whose weights sit 22, 25 and 26 binades below the largest
    exponent.  Up to 25 the grouped GEMMs run on the fp16 plane (the weights fp16
    subnormals, down to 2^-24 at 25; E = 0 blocks zero); at 26 they keep the bf16
    tiles.  Either way the outputs match the oracle."""
    qts = (39, 39, 39)
    info = []
    got, ref = _moe_case(dev, orc, qts, N=512, M=2880, E=8, Kk=2, T=40, renorm=0, seed=span,
                         plant=_plant_mxfp4_span(span, zero_blocks), info=info)
    assert info[0] == (3 if fits else 0), info
    assert np.all(np.isfinite(ref)) and np.mean(np.abs(ref)) > 1.0
    assert O.norm_err(got, ref) < moe_tol(qts)


def _plant_mxfp4_exponents(tensor, e_byte):
    """Set the E8M0 byte of a few MXFP4 blocks in every expert of one tensor."""
    def plant(gates, ups, downs):
        for a in {"gate": gates, "down": downs}[tensor]:
            a.reshape(-1, 17)[[3, 40, 77], 16] = e_byte
    return plant


@pytest.mark.parametrize("tensor,e_byte", [("down", 200), ("down", 255), ("gate", 255)])
def test_moe_layer_batched_extreme_exponents(dev, orc, tensor, e_byte):
    """T = 40 (the grouped-GEMM range) with MXFP4 exponents the GEMMs would not
    reproduce: an inf scale (255), or a down-projection exponent where
    mxfp4_row_dot_q8 clamps 2^(E-127) * d8 to +-1e20 (QK:648-650).  The layer's
    setup-time scale scan keeps it on the per-token GEMV path: NaN / inf where
    the oracle has them, finite outputs within tolerance."""
    qts = (39, 39, 39)
    # M = 2880 (GPT-OSS): one Q8_0 flip of h moves an output by ~3 / (127 sqrt(M)) of its max
    got, ref = _moe_case(dev, orc, qts, N=256, M=2880, E=8, Kk=2, T=40, renorm=0, seed=e_byte,
                         plant=_plant_mxfp4_exponents(tensor, e_byte))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    inf = np.isinf(ref)
    assert np.array_equal(got[inf], ref[inf])
    fin = np.isfinite(ref)
    big = np.abs(ref) > 1e18
    assert O.norm_err(got[fin & ~big], ref[fin & ~big]) < moe_tol(qts)
    if (fin & big).any():
        assert np.max(np.abs(got[fin & big] / ref[fin & big] - 1)) < 1e-3


@pytest.mark.parametrize("qts", [(12, 12, 14), (39, 39, 39), (14, 14, 2)])
@pytest.mark.parametrize("T", [1, 5, 37])
def test_moe_layer_small_vs_oracle(dev, orc, qts, T):
    got, ref = _moe_case(dev, orc, qts, N=256, M=256, E=8, Kk=2, T=T, renorm=int(qts[0] == 12), seed=T + sum(qts))
    assert O.norm_err(got, ref) < moe_tol(qts)


@pytest.mark.parametrize("qts", [(12, 14, 6), (2, 3, 12), (6, 6, 2), (39, 39, 39), (14, 14, 14)])
@pytest.mark.parametrize("T", [2, 8, 24])
def test_moe_layer_decode_vs_oracle(dev, orc, qts, T):
    """Decode path (T <= 24): one launch over all T*K (token, slot) jobs, gate and up fused when their
    semantics agree ((2, 3) and (12, 14) run two launches), the SiLU product formed by the down
    projection's staging (fp32 activations) or its Q8_0 quantiser (MXFP4), Q4_K down left at zero."""
    got, ref = _moe_case(dev, orc, qts, N=512, M=256, E=16, Kk=4, T=T, renorm=T % 2, seed=11 * T + sum(qts))
    if qts[2] == 12:
        assert not np.any(got) and not np.any(ref)
        return
    assert O.norm_err(got, ref) < moe_tol(qts)


@pytest.mark.parametrize("qts,N,M,Kk,T", [((39, 39, 39), 2880, 2880, 4, 1), ((12, 12, 14), 2048, 768, 8, 8)])
def test_moe_layer_decode_real_shapes(dev, orc, qts, N, M, Kk, T):
    """GPT-OSS-20B (batch 1) and Qwen3-30B-A3B (batch 8) expert shapes on the decode path."""
    got, ref = _moe_case(dev, orc, qts, N=N, M=M, E=16, Kk=Kk, T=T, renorm=int(qts[0] == 12), seed=T + N)
    assert O.norm_err(got, ref) < moe_tol(qts)


def test_moe_layer_repeated_decode_calls(dev, orc):
    """Decode routing's arrival counters are left at zero by every call: alternating T = 1, 5, 8, 1
    calls on one layer keep matching the oracle's routing."""
    import torch
    rng = np.random.default_rng(21)
    qts, N, M, E, Kk = (12, 12, 14), 512, 256, 32, 4
    gates = [W.gen_weights(rng, qts[0], M, N) for _ in range(E)]
    ups = [W.gen_weights(rng, qts[1], M, N) for _ in range(E)]
    downs = [W.gen_weights(rng, qts[2], N, M) for _ in range(E)]
    router = W.gen_router(rng, E, N)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    layer = dev.moe_prepare(qts, N, M, E, Kk, [cu(g) for g in gates], [cu(u) for u in ups], [cu(d) for d in downs],
                            cu(router), 1)
    for T in (1, 5, 8, 1, 8):
        x = W.gen_x(rng, T, N)
        idx = torch.empty((T, Kk), dtype=torch.int32, device="cuda")
        w = torch.empty((T, Kk), dtype=torch.float32, device="cuda")
        got = layer.forward(cu(x), idx=idx, w=w).cpu().numpy()
        ri, rw = orc.route(router, x, Kk, 1)
        assert np.array_equal(idx.cpu().numpy(), ri), f"routing differs at T={T}"
        ref = np.stack([orc.moe_forward_token(gates, ups, downs, x[t], M, N, qts, ri[t], rw[t]) for t in range(T)])
        assert O.norm_err(got, ref) < MOE_TOL


def test_moe_layer_gptoss_shape(dev, orc):
    """GPT-OSS-20B expert shapes (N = M = 2880, MXFP4, top-4), batched path."""
    info = []
    got, ref = _moe_case(dev, orc, (39, 39, 39), N=2880, M=2880, E=8, Kk=4, T=32, renorm=1, seed=4, info=info)
    assert info[0] == 3, info   # gate/up and down on the fp16-plane GEMM
    assert O.norm_err(got, ref) < moe_tol((39, 39, 39))


def test_moe_layer_qwen3_shape_skewed(dev, orc):
    """Qwen3-30B-A3B expert shapes (N = 2048, M = 768, Q4_K/Q6_K, top-8 renormalised), skewed routing."""
    got, ref = _moe_case(dev, orc, (12, 12, 14), N=2048, M=768, E=32, Kk=8, T=40, renorm=1, seed=5, skew=True)
    assert O.norm_err(got, ref) < MOE_TOL


@pytest.mark.parametrize("E,N", [(32, 2880), (5, 9)])
def test_router_pack_layout(dev, E, N):
    """mllm_router_pack: element (i, e) at ((i/4)*E + e)*4 + i%4, rows from N up
    to a multiple of 32 zero."""
    import torch
    rng = np.random.default_rng(N)
    rw = W.gen_router(rng, E, N)
    got = dev.router_pack(torch.from_numpy(rw).cuda()).cpu().numpy()
    N4 = (N + 31) // 32 * 32
    want = np.zeros((N4, E), np.float32)
    want[:N] = rw.T
    want = want.reshape(N4 // 4, 4, E).transpose(0, 2, 1).reshape(-1)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("T", [2, 40])
@pytest.mark.parametrize("renorm", [0, 1])
def test_device_route_exact_ties(dev, orc, T, renorm):
    """Experts with identical router rows have bit-identical probabilities; the
    reference's strict '>' insertion keeps the lower index first, and so must
    the device routing."""
    import torch
    rng = np.random.default_rng(11 + T)
    E, N, Kk = 32, 512, 4
    rw = W.gen_router(rng, E, N)
    rw[3] *= 6.0
    rw[7] = rw[3]
    rw[20] = rw[3]
    rw[9] = rw[1]
    x = W.gen_x(rng, T, N)
    ri, rwt = orc.route(rw, x, Kk, renorm)
    assert any((1 in r and 9 in r) or (3 in r and 7 in r) for r in ri.tolist()), "fixture lost its ties"
    idx, wt = dev.route(torch.from_numpy(rw).cuda(), torch.from_numpy(x).cuda(), Kk, renorm)
    assert np.array_equal(idx.cpu().numpy(), ri)
    assert np.max(np.abs(wt.cpu().numpy() - rwt) / rwt) < 1e-6


def _moe_ffn_case(qts, N, M, E, Kk, T, seed):
    rng = np.random.default_rng(seed)
    gate = np.concatenate([W.gen_weights(rng, qts[0], M, N) for _ in range(E)])
    upw = np.concatenate([W.gen_weights(rng, qts[1], M, N) for _ in range(E)])
    down = np.concatenate([W.gen_weights(rng, qts[2], N, M) for _ in range(E)])
    router = W.gen_router(rng, E, N)
    x = W.gen_x(rng, T, N)
    return gate, upw, down, router, x


@pytest.mark.parametrize("tag", ["q4k", "mxfp4"])
def test_golden_moe_ffn_batched(lib, golden, tag):
    """moe_ffn_batched keeps every token's moe_ffn result (B <= 8: the token path)."""
    g = golden(f"moe_ffn_{tag}.npz")
    N, E, Kk, M = (int(g[k]) for k in ("N", "E", "K", "M"))
    bc = BCView(N, E, Kk, M, g["router"], g["gate"], g["up"], g["down"], tuple(int(v) for v in g["qts"]))
    T = g["x"].shape[0]
    out = np.full((T, N), np.nan, np.float32)
    lib.moe_ffn_batched(bc.ptr(), 0, fp(np.ascontiguousarray(g["x"], np.float32)), fp(out), T)
    assert O.norm_err(out, g["out"]) < MOE_TOL, K.last_error(lib)


@pytest.mark.parametrize("qts", [(12, 12, 14), (39, 39, 39), (14, 14, 14)])
@pytest.mark.parametrize("T", [37, 160])
def test_moe_ffn_batched_vs_oracle(lib, orc, qts, T):
    """B > 8: the grouped-GEMM layer with moe_ffn's semantics (quant_matmul_omp per
    projection, unclamped SiLU, no renormalisation) against the oracle's moe_ffn
    token by token, and against this library's own moe_ffn at B = 1."""
    N, M, E, Kk = 256, 256, 8, 2
    gate, upw, down, router, x = _moe_ffn_case(qts, N, M, E, Kk, T, seed=T + sum(qts))
    bc = BCView(N, E, Kk, M, router, gate, upw, down, qts)
    out = np.full((T, N), np.nan, np.float32)
    lib.moe_ffn_batched(bc.ptr(), 0, fp(np.ascontiguousarray(x)), fp(out), T)
    ref = np.stack([orc.moe_ffn_token(router, gate, upw, down, qts, N, E, Kk, M, x[t]) for t in range(T)])
    assert O.norm_err(out, ref) < MOE_TOL, K.last_error(lib)
    one = np.stack([moe_ffn(lib, bc, x[t], N) for t in range(0, T, 7)])
    assert O.norm_err(out[::7], one) < MOE_TOL


def test_moe_ffn_batched_large_gate(lib, orc):
    """Gate values past +-80 take moe_ffn's unclamped SiLU on the batched path."""
    qts, N, M, E, Kk, T = (39, 39, 39), 256, 256, 8, 2, 24
    gate, upw, down, router, x = _moe_ffn_case(qts, N, M, E, Kk, T, seed=5)
    x = x * 60.0   # gate outputs well beyond 80 in magnitude
    bc = BCView(N, E, Kk, M, router, gate, upw, down, qts)
    out = np.full((T, N), np.nan, np.float32)
    lib.moe_ffn_batched(bc.ptr(), 0, fp(np.ascontiguousarray(x, np.float32)), fp(out), T)
    ref = np.stack([orc.moe_ffn_token(router, gate, upw, down, qts, N, E, Kk, M, x[t]) for t in range(T)])
    assert O.norm_err(out, ref) < MOE_TOL, K.last_error(lib)


def test_moe_ffn_router_rewritten_in_place(lib, orc):
    """A router whose host contents change at the same address is packed again
    (the device cache keys on the address and checks the contents)."""
    qts, N, M, E, Kk, T = (14, 14, 14), 256, 256, 8, 2, 3
    gate, upw, down, router, x = _moe_ffn_case(qts, N, M, E, Kk, T, seed=11)
    bc = BCView(N, E, Kk, M, router, gate, upw, down, qts)
    for step in range(2):
        got = np.stack([moe_ffn(lib, bc, x[t], N) for t in range(T)])
        ref = np.stack([orc.moe_ffn_token(router, gate, upw, down, qts, N, E, Kk, M, x[t]) for t in range(T)])
        assert O.norm_err(got, ref) < MOE_TOL, step
        router[:] = router[::-1].copy()   # other experts win, same buffer


@pytest.mark.parametrize("qts,N,M", [((39, 39, 39), 224, 96), ((2, 2, 2), 160, 96), ((39, 39, 2), 96, 160)])
@pytest.mark.parametrize("E,Kk,T", [(12, 3, 29), (12, 3, 50), (5, 1, 27)])
def test_moe_layer_batched_odd_shapes(dev, orc, qts, N, M, E, Kk, T):
    """Batched path (T > 24) at shapes off every power of two: K not a multiple
    of 64 (padded activation rows), rows not a multiple of the weight tile,
    expert counts whose tiles spread unevenly over the XCDs, odd top-K."""
    got, ref = _moe_case(dev, orc, qts, N=N, M=M, E=E, Kk=Kk, T=T, renorm=int(Kk > 1), seed=T * 7 + E + N)
    assert O.norm_err(got, ref) < moe_tol(qts), K.last_error(dev.so)


@pytest.mark.parametrize("bad", [np.nan, np.inf])
def test_moe_ffn_nonfinite_token_gives_zeros(lib, orc, bad):
    """moe_ffn on a token whose logits hold an inf or NaN: no expert is
    selected and the output is zero, as the reference's moe_ffn gives
    (CE:640-641); the other tokens are unchanged."""
    qts, N, M, E, Kk, T = (12, 12, 14), 256, 256, 8, 2, 3
    gate, upw, down, router, x = _moe_ffn_case(qts, N, M, E, Kk, T, seed=41)
    x[1, 37] = bad
    bc = BCView(N, E, Kk, M, router, gate, upw, down, qts)
    for t in range(T):
        got = moe_ffn(lib, bc, x[t], N)
        ref = orc.moe_ffn_token(router, gate, upw, down, qts, N, E, Kk, M, x[t])
        if t == 1:
            assert np.all(got == 0.0) and np.all(ref == 0.0)
        else:
            assert O.norm_err(got, ref) < MOE_TOL
    out = np.full((T, N), np.nan, np.float32)
    lib.moe_ffn_batched(bc.ptr(), 0, fp(np.ascontiguousarray(x)), fp(out), T)
    assert np.all(out[1] == 0.0) and np.all(np.isfinite(out))


@pytest.mark.parametrize("T", [4, 30])
def test_moe_layer_nonfinite_token_gives_zeros(dev, orc, T):
    """mllm_moe_forward at T = 4 (decode GEMVs) and T = 30 (grouped GEMMs): a
    token with a NaN element is routed to no expert (idx -1) and its output
    row is zero on both paths; every other token matches the oracle."""
    import torch
    rng = np.random.default_rng(50 + T)
    qts, N, M, E, Kk = (12, 12, 14), 512, 256, 16, 4
    gates = [W.gen_weights(rng, qts[0], M, N) for _ in range(E)]
    ups = [W.gen_weights(rng, qts[1], M, N) for _ in range(E)]
    downs = [W.gen_weights(rng, qts[2], N, M) for _ in range(E)]
    router = W.gen_router(rng, E, N)
    x = W.gen_x(rng, T, N)
    x[1, 5] = np.nan
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    layer = dev.moe_prepare(qts, N, M, E, Kk, [cu(g) for g in gates], [cu(u) for u in ups], [cu(d) for d in downs],
                            cu(router), 1)
    idx = torch.empty((T, Kk), dtype=torch.int32, device="cuda")
    got = layer.forward(cu(x), idx=idx).cpu().numpy()
    ri, rw = orc.route(router, x, Kk, 1)
    assert np.array_equal(idx.cpu().numpy(), ri) and np.all(ri[1] == -1)
    assert np.all(got[1] == 0.0)
    keep = [t for t in range(T) if t != 1]
    ref = np.stack([orc.moe_forward_token(gates, ups, downs, x[t], M, N, qts, ri[t], rw[t]) for t in keep])
    assert O.norm_err(got[keep], ref) < MOE_TOL


def test_moe_forward_omp_empty_slots(lib, orc):
    """moe_forward_omp with a slot whose expert id is -1 (a routing that left it
    empty) adds nothing for it; top_k = 0 clears combined (QK:2179)."""
    rng = np.random.default_rng(61)
    qts, n_embd, n_ff, E = (12, 12, 14), 512, 256, 4
    gates = [W.gen_weights(rng, qts[0], n_ff, n_embd) for _ in range(E)]
    ups = [W.gen_weights(rng, qts[1], n_ff, n_embd) for _ in range(E)]
    downs = [W.gen_weights(rng, qts[2], n_embd, n_ff) for _ in range(E)]
    x = W.gen_x(rng, 1, n_embd)[0]
    got = moe_forward(lib, gates, ups, downs, x, n_ff, n_embd, qts, np.array([2, -1, 0], np.int32),
                      np.array([0.5, 0.3, 0.2], np.float32))
    ref = orc.moe_forward_token(gates, ups, downs, x, n_ff, n_embd, qts, np.array([2, 0], np.int32),
                                np.array([0.5, 0.2], np.float32))
    assert O.norm_err(got, ref) < MOE_TOL
    arr = ctypes.POINTER(ctypes.c_uint8) * E
    out = np.full(n_embd, 3.0, np.float32)
    ti = np.zeros(1, np.int32)
    tw = np.zeros(1, np.float32)
    lib.moe_forward_omp(arr(*[up(a) for a in gates]), arr(*[up(a) for a in ups]), arr(*[up(a) for a in downs]),
                        fp(x), n_ff, n_embd, 12, 12, 14, ti.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), fp(tw), 0,
                        fp(out), fp(np.zeros(16, np.float32)), up(np.zeros(64, np.uint8)))
    assert np.all(out == 0.0)
