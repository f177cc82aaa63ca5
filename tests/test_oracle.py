"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Three independent pins:
  1. golden vectors written by the reference's own compiled C (tests/golden);
  2. the live reference build oracle/_ref/libref.so on fresh inputs, where it
     was built (skipped otherwise);
  3. properties the mathematics fixes (closed forms, linearity, batching,
     zero scales, semantic distinctness, quantisation bounds).
"""
import zlib

import math

import numpy as np
import pytest

import oracle as O
from mojollama_amd import workloads as W

TOL = 1e-5       # oracle (double accumulation) vs reference (fp32 AVX2)


def crc(*arrays):
    c = 0
    for a in arrays:
        c = zlib.crc32(np.ascontiguousarray(a).view(np.uint8).tobytes(), c)
    return c


# ------------------------------------------------------------ 1. golden

@pytest.mark.parametrize("qt", [0, 2, 3, 6, 8, 12, 13, 14, 39])
def test_golden_quant_matmul(orc, golden, qt):
    g = golden(f"qmm_{qt}.npz")
    sem = orc.sem_for(0, qt)
    got = orc.gemv(sem, g["W"], g["x"], int(g["n_rows"]), int(g["n_cols"]), 1)[0]
    assert O.norm_err(got, g["out"]) < TOL


@pytest.mark.parametrize("name,qt", [("q4_0", 2), ("q8_0", 8), ("q4_k", 12), ("q6_k", 14),
                                     ("q5_k", 13), ("mxfp4", 39)])
@pytest.mark.parametrize("B", [1, 3, 5])
def test_golden_batch_matmul(orc, golden, name, qt, B):
    g = golden(f"bmm_{name}_B{B}.npz")
    sem = orc.sem_for(1, qt)
    got = orc.gemv(sem, g["W"], g["x"], int(g["n_rows"]), int(g["n_cols"]), B)
    assert O.norm_err(got, g["out"]) < TOL


def test_golden_mxfp4_scale_edges(orc, golden):
    g = golden("edge_mxfp4.npz")
    R, C = int(g["n_rows"]), int(g["n_cols"])
    got = orc.gemv(O.MXFP4_CLAMP, g["W"], g["x"], R, C, 1)[0]
    assert np.all(np.isfinite(g["out_clamp"]))
    assert O.norm_err(got, g["out_clamp"]) < TOL
    got = orc.gemv(O.MXFP4, g["W"], g["x"], R, C, 1)[0]
    ref = g["out_noclamp"]
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = np.isfinite(ref)
    if fin.any():
        assert O.norm_err(got[fin], ref[fin]) < TOL


def test_golden_quantize_q8_0_bitexact(orc, golden):
    g = golden("q8_0.npz")
    assert np.array_equal(orc.quantize_q8_0(g["x"]), g["q8"])


@pytest.mark.parametrize("name,sem", [("q4_k", O.Q4_K_GGML), ("q6_k", O.Q6_K_GGML),
                                      ("q5_k", O.Q5_K_GGML), ("q8_0", O.Q8_0)])
def test_golden_dequantize_row(orc, golden, name, sem):
    g = golden(f"deq_{name}.npz")
    got = orc.dequant(sem, g["W"], 1, 1024)[0]
    assert O.norm_err(got, g["out"]) < 1e-6


def test_golden_batch_qkv_and_gate_up(orc, golden):
    g = golden("batch_qkv.npz")
    for w, o, rows, qt in ((g["Wq"], g["oq"], 32, 12), (g["Wk"], g["ok"], 16, 14), (g["Wv"], g["ov"], 16, 8)):
        got = orc.gemv(orc.sem_for(2, qt), w, g["x"], rows, 512, 1)[0]
        assert O.norm_err(got, o) < TOL
    g = golden("batch_gate_up.npz")
    for w, o, qt in ((g["Wg"], g["og"], 39), (g["Wu"], g["ou"], 2)):
        got = orc.gemv(orc.sem_for(2, qt), w, g["x"], 32, 512, 1)[0]
        assert O.norm_err(got, o) < TOL


def test_golden_quantize_q8_0_nonfinite_bitexact(orc, golden):
    """NaN / +-inf at every block position: amax turns NaN only where the
    reference's vmaxps order lets it (QK:1417-1425)."""
    g = golden("q8_0_nonfinite.npz")
    assert np.array_equal(orc.quantize_q8_0(g["x"]), g["q8"])


def same_nonfinite(got, ref, tol):
    """NaN and inf at the same places, finite values within tol (normalised)."""
    if not (np.array_equal(np.isnan(got), np.isnan(ref)) and np.array_equal(np.isinf(got), np.isinf(ref))):
        return False
    fin = np.isfinite(ref)
    return not fin.any() or O.norm_err(got[fin], ref[fin]) < tol


@pytest.mark.parametrize("tag", ["qwen", "gptoss"])
def test_golden_moe_forward_nonfinite(orc, golden, tag):
    g = golden(f"moe_forward_nonfinite_{tag}.npz")
    for x, out in zip(g["x"], g["out"]):
        got = orc.moe_forward_token(list(g["gates"]), list(g["ups"]), list(g["downs"]), x, int(g["n_ff"]),
                                    int(g["n_embd"]), tuple(int(v) for v in g["qts"]), g["top_idx"], g["top_w"])
        assert same_nonfinite(got, out, TOL)


@pytest.mark.parametrize("tag", ["qwen", "gptoss", "q5down", "q5down_all"])
def test_golden_moe_forward(orc, golden, tag):
    g = golden(f"moe_forward_{tag}.npz")
    got = orc.moe_forward_token(list(g["gates"]), list(g["ups"]), list(g["downs"]), g["x"],
                                int(g["n_ff"]), int(g["n_embd"]), tuple(int(v) for v in g["qts"]),
                                g["top_idx"], g["top_w"])
    assert O.norm_err(got, g["out"]) < 1e-4


@pytest.mark.parametrize("tag", ["q5down", "q5down_all"])
def test_golden_moe_forward_q5_down_stride_matters(orc, golden, tag):
    """The Q5_0 down fixtures pin the reference's row stride: the same token
    through down matrices read with their own (contiguous) row stride misses
    the reference's output by far more than the tolerance."""
    g = golden(f"moe_forward_{tag}.npz")
    N, F = int(g["n_embd"]), int(g["n_ff"])
    qg, qu, qd = (int(v) for v in g["qts"])
    assert qd == 6 and N < F
    x = g["x"]
    naive = np.zeros(N, np.float32)
    for e, wk in zip(g["top_idx"], g["top_w"]):
        gv = orc.gemv(orc.sem_for(3, qg), g["gates"][e], x[None], F, N, 1)[0]
        uv = orc.gemv(orc.sem_for(3, qu), g["ups"][e], x[None], F, N, 1)[0]
        gc = np.clip(gv, -80, 80)
        h = (gc / (1 + np.exp(-gc)) * uv).astype(np.float32)
        naive += wk * orc.gemv(orc.sem_for(4, qd), g["downs"][e], h[None], N, F, 1)[0]
    assert O.norm_err(naive, g["out"]) > 0.1


@pytest.mark.parametrize("tag", ["q4k", "mxfp4"])
def test_golden_moe_ffn(orc, golden, tag):
    g = golden(f"moe_ffn_{tag}.npz")
    N, E, K, M = (int(g[k]) for k in ("N", "E", "K", "M"))
    for t in range(g["x"].shape[0]):
        got = orc.moe_ffn_token(g["router"], g["gate"], g["up"], g["down"], tuple(int(v) for v in g["qts"]),
                                N, E, K, M, g["x"][t])
        assert O.norm_err(got, g["out"][t]) < 1e-4


@pytest.mark.parametrize("tag", ["gptoss", "qwen3"])
def test_golden_route_selection_bitexact(orc, golden, tag):
    g = golden(f"route_sel_{tag}.npz")
    N, E, K, T = (int(g[k]) for k in ("N", "E", "K", "T"))
    r2 = np.random.default_rng(int(g["seed"]))
    router = W.gen_router(r2, E, N)
    xs = W.gen_x(r2, T, N)
    assert crc(router, xs) == int(g["crc"]), "numpy RNG stream changed: regenerate fixtures"
    idx, w = orc.route(router, xs, K, renorm=False)
    sel = np.zeros((T, E), np.uint8)
    for t in range(T):
        sel[t, idx[t]] = 1
    assert np.array_equal(sel, g["sel"])
    # the probe's output is p_e * D_t at the selected experts (same D_t for all e)
    ratio = g["ffn"][np.arange(T)[:, None], idx] / w
    assert np.all(np.abs(ratio / ratio[:, :1] - 1.0) < 1e-5)


@pytest.mark.parametrize("qt", [12, 14, 1])
def test_golden_requant_q8_0(orc, golden, qt):
    """TE's lm_head requantisation (TE:620-666) as the fixture generator ran it:
    the reference's own dequantize_row per row (F16: TE:643-645's conversion),
    then TE's numpy statements."""
    g = golden(f"requant_q8_{qt}.npz")
    got = orc.requant_q8_0(qt, g["W"], int(g["n_rows"]), int(g["n_cols"]))
    assert np.array_equal(got, g["out"])


def test_requant_f16_takes_bit_patterns_as_integers():
    """TE:643-645 turns each fp16 pattern into its integer value, not its fp16
    value: a block of the pattern 0x3C00 (fp16 1.0) is 32 values 15360, so
    d = fp16(15360 / 127) and every quant is 127; a block whose patterns are
    0..31 has amax 31, d = fp16(31 / 127) and quants rint(k * 127 / 31)
    (half to even); a row of fp16 -0.0 patterns (0x8000 = 32768) is not zero.
    Reading the patterns as fp16 fails all three."""
    orc = O.Oracle()
    C = 96
    u = np.zeros((2, C), np.uint16)
    u[0, :32] = 0x3C00
    u[0, 32:64] = np.arange(32)
    u[0, 64:] = 0x8000
    got = orc.requant_q8_0(1, u.view(np.uint8).ravel(), 1, C).reshape(-1, 34)
    d = got[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    q = got[:, 2:].view(np.int8)
    assert d[0] == np.float16(np.float32(15360.0) / np.float32(127.0)) and np.all(q[0] == 127)
    d1 = np.float32(31.0) / np.float32(127.0)
    assert d[1] == np.float16(d1)
    assert np.array_equal(q[1], np.clip(np.round(np.arange(32, dtype=np.float32) / d1), -127, 127).astype(np.int8))
    assert d[2] == np.float16(np.float32(32768.0) / np.float32(127.0)) and np.all(q[2] == 127)
    with pytest.raises(ValueError):
        orc.requant_q8_0(1, u.view(np.uint8).ravel(), 1, 80)   # not whole 32-element blocks


def test_requant_q8_0_differs_from_quantize_row():
    """TE's rule (x / d, amax floored at 1e-10) is not quantize_row_q8_0's
    (x * (1/d), d = 1 for an all-zero block): the restatement keeps them apart
    and stays within half a step of its input."""
    orc = O.Oracle()
    rng = np.random.default_rng(5)
    R, C = 64, 512
    w = W.gen_weights(rng, 14, R, C)
    req = orc.requant_q8_0(14, w, R, C).reshape(R * C // 32, 34)
    deq = orc.dequant(10, w, R, C).reshape(-1, 32)
    d = req[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    q = req[:, 2:].view(np.int8).astype(np.float32)
    # half a step, plus the stored scale's fp16 rounding (2^-11 relative) times |q| <= 127
    step = np.abs(deq).max(1, keepdims=True) / 127
    assert np.all(np.abs(q * d[:, None] - deq) <= step * (0.5 + 127 * 2.0 ** -11) * 1.001 + 1e-6)
    row = orc.quantize_q8_0(deq.reshape(-1)).reshape(-1, 34)
    assert not np.array_equal(row, req)


# ----------------------------------------------------- 2. live reference

@pytest.fixture(scope="module")
def ref():
    if not O.ref_available():
        pytest.skip("oracle/_ref/libref.so not built (reference tree absent)")
    r = O.RefLib()
    r.so.set_num_threads(2)
    return r


@pytest.mark.parametrize("qt", [0, 2, 3, 6, 8, 12, 13, 14, 39])
def test_live_quant_matmul(orc, ref, qt):
    rng = np.random.default_rng(100 + qt)
    R, C = 40, 2048
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, 1, C)
    assert O.norm_err(orc.gemv(orc.sem_for(0, qt), w, x, R, C, 1)[0], ref.quant_matmul(w, x, R, C, qt)) < TOL


@pytest.mark.parametrize("name,qt", [("q4_0", 2), ("q8_0", 8), ("q4_k", 12), ("q6_k", 14),
                                     ("q5_k", 13), ("mxfp4", 39)])
def test_live_batch_matmul(orc, ref, name, qt):
    rng = np.random.default_rng(200 + qt)
    R, C, B = 24, 2816 if qt not in (12, 13, 14) else 2816 // 256 * 256, 4
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, B, C)
    got = orc.gemv(orc.sem_for(1, qt), w, x, R, C, B)
    assert O.norm_err(got, ref.batch_matmul(name + "_batch_matmul", w, x, R, C, B)) < TOL


def test_live_quantize_q8_0(orc, ref):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(1 << 16) * np.exp(rng.uniform(-8, 8, 1 << 16))).astype(np.float32)
    assert np.array_equal(orc.quantize_q8_0(x), ref.quantize_q8_0(x))


def test_live_quantize_q8_0_nonfinite(orc, ref):
    rng = np.random.default_rng(8)
    x = W.gen_x(rng, 1, 32 * 2048)[0].copy()
    pos = rng.choice(x.size, size=3000, replace=False)
    x[pos] = rng.choice([np.nan, np.inf, -np.inf, 0.0, 3e38], size=pos.size)
    assert np.array_equal(orc.quantize_q8_0(x), ref.quantize_q8_0(x))


@pytest.mark.parametrize("qt", [2, 3, 6, 8, 12, 13, 14, 39])
def test_live_nonfinite_block_scales(orc, ref, qt):
    """inf / NaN fp16 scales and mins (E8M0 255 for MXFP4) through
    quant_matmul_omp (B = 1) and *_batch_matmul (B = 3): NaN / inf at the same
    outputs as the reference, finite outputs within tolerance."""
    rng = np.random.default_rng(5 + qt)
    be, bb = W.BLOCK[qt]
    R, C = 24, 768 if be == 256 else 800
    w = W.gen_weights(rng, qt, R, C).reshape(R, C // be, bb)
    if qt == 39:
        w[3, 1, 16] = w[6, 0, 16] = 255
    else:
        d_off = 208 if qt == W.QT_Q6_K else 0
        for row, blk, bits in ((3, 1, 0x7C00), (6, 0, 0x7E00), (9, 2, 0xFC00)):
            w[row, blk, d_off:d_off + 2] = np.frombuffer(np.uint16(bits).tobytes(), np.uint8)
        if qt in (3, 12, 13):
            w[12, 1, 2:4] = np.frombuffer(np.uint16(0x7C00).tobytes(), np.uint8)
    w = np.ascontiguousarray(w.ravel())
    x = W.gen_x(rng, 3, C)
    for b in range(3):
        assert same_nonfinite(orc.gemv(orc.sem_for(0, qt), w, x[b], R, C, 1)[0],
                              ref.quant_matmul(w, x[b], R, C, qt), 1e-5), b
    name = {2: "q4_0", 8: "q8_0", 12: "q4_k", 14: "q6_k", 13: "q5_k", 39: "mxfp4"}.get(qt)
    if name:
        assert same_nonfinite(orc.gemv(orc.sem_for(1, qt), w, x, R, C, 3).ravel(),
                              ref.batch_matmul(name + "_batch_matmul", w, x, R, C, 3).ravel(), 1e-5)


@pytest.mark.parametrize("qt", [0, 2, 3, 6, 8, 12, 13, 14, 39])
def test_live_quant_matmul_nonfinite_activations(orc, ref, qt):
    """inf / NaN activations: every quant_matmul_omp code (B = 1) and
    *_batch_matmul (B = 3) give NaN / inf at the same outputs as the reference."""
    rng = np.random.default_rng(60 + qt)
    R, C = 32, 512
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, 3, C).copy()
    x[0, 5], x[1, 200], x[1, 301], x[2, 17] = np.inf, -np.inf, np.inf, np.nan
    for b in range(3):
        got = orc.gemv(orc.sem_for(0, qt), w, x[b], R, C, 1)[0]
        want = ref.quant_matmul(w, x[b], R, C, qt)
        assert same_nonfinite(got, want, 1e-5), b
    name = {2: "q4_0", 8: "q8_0", 12: "q4_k", 14: "q6_k", 13: "q5_k", 39: "mxfp4"}.get(qt)
    if name:
        got = orc.gemv(orc.sem_for(1, qt), w, x, R, C, 3)
        want = ref.batch_matmul(name + "_batch_matmul", w, x, R, C, 3)
        assert same_nonfinite(got.ravel(), want.ravel(), 1e-5)


@pytest.mark.parametrize("qts", [(39, 39, 39), (12, 12, 14), (14, 14, 14), (39, 39, 14), (2, 2, 2), (6, 6, 14)])
def test_live_moe_forward_nonfinite(orc, ref, qts):
    rng = np.random.default_rng(sum(qts))
    n_embd, n_ff = 512, 256
    gates = [W.gen_weights(rng, qts[0], n_ff, n_embd) for _ in range(3)]
    ups = [W.gen_weights(rng, qts[1], n_ff, n_embd) for _ in range(3)]
    downs = [W.gen_weights(rng, qts[2], n_embd, n_ff) for _ in range(3)]
    ti = np.array([2, 0], np.int32)
    for pos in (0, 31, 100, 511):
        for val in (np.nan, np.inf, -np.inf):
            x = W.gen_x(rng, 1, n_embd)[0].copy()
            x[pos] = val
            for tw in (np.array([0.6, 0.4], np.float32), np.array([np.nan, np.nan], np.float32)):
                a = ref.moe_forward(gates, ups, downs, x, n_ff, n_embd, qts, ti, tw)
                b = orc.moe_forward_token(gates, ups, downs, x, n_ff, n_embd, qts, ti, tw)
                assert same_nonfinite(b, a, 1e-4), (pos, val, tw)


def test_live_moe_forward_null_q8_scratch_differs_only_for_mxfp4_down(orc, ref):
    # With prealloc_q8 == NULL the reference still runs a Q6_K down projection.
    rng = np.random.default_rng(9)
    n_embd, n_ff = 256, 256
    gates = [W.gen_weights(rng, 12, n_ff, n_embd) for _ in range(2)]
    ups = [W.gen_weights(rng, 12, n_ff, n_embd) for _ in range(2)]
    downs = [W.gen_weights(rng, 14, n_embd, n_ff) for _ in range(2)]
    x = W.gen_x(rng, 1, n_embd)[0]
    ti, tw = np.array([1, 0], np.int32), np.array([0.6, 0.4], np.float32)
    a = ref.moe_forward(gates, ups, downs, x, n_ff, n_embd, (12, 12, 14), ti, tw, with_q8=False)
    b = orc.moe_forward_token(gates, ups, downs, x, n_ff, n_embd, (12, 12, 14), ti, tw, has_q8=False)
    assert O.norm_err(b, a) < 1e-4


@pytest.mark.parametrize("qt,nc", [(8, 16), (12, 128), (14, 128), (39, 16), (2, 16), (13, 200)])
def test_live_short_rows_give_zeros(orc, ref, qt, nc):
    """Rows shorter than one quant block: the reference's dot runs over
    n_cols / block = 0 blocks and writes 0; so does the oracle."""
    rng = np.random.default_rng(qt + nc)
    w = rng.integers(0, 256, 64, dtype=np.uint8)
    x = W.gen_x(rng, 1, nc)
    out = np.full(4, 7.0, np.float32)
    ref.quant_matmul(w, x, 4, nc, qt, out=out)
    assert np.all(out == 0.0)
    assert np.all(orc.gemv(orc.sem_for(0, qt), w, x, 4, nc, 1) == 0.0)


@pytest.mark.parametrize("bad", [np.nan, np.inf])
def test_live_moe_ffn_nonfinite_token_gives_zeros(orc, ref, bad):
    """A token whose router logits hold an inf or NaN: the reference's moe_ffn
    inserts no expert (strict '>' against NaN probabilities), skips the empty
    slots (CE:640-641) and returns zeros; the oracle routes it to no expert."""
    import ctypes
    from helpers import BCView, fp
    rng = np.random.default_rng(17)
    N, E, Kk, M, qts = 256, 8, 2, 256, (12, 12, 14)
    gate = np.concatenate([W.gen_weights(rng, 12, M, N) for _ in range(E)])
    upw = np.concatenate([W.gen_weights(rng, 12, M, N) for _ in range(E)])
    down = np.concatenate([W.gen_weights(rng, 14, N, M) for _ in range(E)])
    router = W.gen_router(rng, E, N)
    x = W.gen_x(rng, 2, N)
    x[1, 37] = bad
    bc = BCView(N, E, Kk, M, router, gate, upw, down, qts)
    ref.so.moe_ffn.argtypes = [ctypes.c_void_p, ctypes.c_int] + [ctypes.POINTER(ctypes.c_float)] * 4 + [ctypes.c_int]
    ref.so.moe_ffn.restype = None
    for t in range(2):
        out = np.full(N, 5.0, np.float32)
        gb, ub = np.zeros(4096, np.float32), np.zeros(4096, np.float32)
        xx = x[t].copy()
        ref.so.moe_ffn(bc.ptr(), 0, fp(xx), fp(gb), fp(ub), fp(out), 1)
        mine = orc.moe_ffn_token(router, gate, upw, down, qts, N, E, Kk, M, x[t])
        if t == 1:
            assert np.all(out == 0.0) and np.all(mine == 0.0)
            idx, _ = orc.route(router, x[1:2], Kk, 0)
            assert np.all(idx == -1)
        else:
            assert O.norm_err(mine, out) < 1e-4


# ------------------------------------------------ 3. mathematical pins

def _np_decode_q8_0(w, R, C):
    b = w.reshape(R, C // 32, 34)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float32)
    q = b[:, :, 2:].view(np.int8).astype(np.float32)
    return (q * d).reshape(R, C)


def _np_decode_mxfp4(w, R, C, clamp):
    b = w.reshape(R, C // 32, 17)
    s = (b[:, :, 16].astype(np.uint32) << 23).view(np.float32)
    if clamp:
        s = np.minimum(s, np.float32(1e20))
    lo = (b[:, :, :16] & 15).astype(np.int32)
    hi = (b[:, :, :16] >> 4).astype(np.int32)
    v = np.stack([lo, hi], axis=-1).reshape(R, C // 32, 32)
    v = np.where(v >= 8, v - 16, v).astype(np.float32)
    return (v * s[:, :, None]).reshape(R, C)


def test_closed_form_q8_0_and_mxfp4_are_dense_gemv(orc):
    rng = np.random.default_rng(1)
    R, C, B = 33, 640, 3
    x = W.gen_x(rng, B, C)
    w = W.gen_weights(rng, 8, R, C)
    dense = x.astype(np.float64) @ _np_decode_q8_0(w, R, C).T.astype(np.float64)
    assert O.norm_err(orc.gemv(O.Q8_0, w, x, R, C, B), dense) < 1e-6
    w = W.gen_weights(rng, 39, R, C)
    for sem, clamp in ((O.MXFP4, False), (O.MXFP4_CLAMP, True)):
        dense = x.astype(np.float64) @ _np_decode_mxfp4(w, R, C, clamp).T.astype(np.float64)
        assert O.norm_err(orc.gemv(sem, w, x, R, C, B), dense) < 1e-6


FP32_SEMS = [O.F32, O.Q4_0, O.Q4_1, O.Q5_0_F32, O.Q8_0, O.Q4_K_GGML, O.Q5_K_GGML, O.Q5_K_CE,
             O.Q6_K_GGML, O.Q6_K_LOWNIB, O.Q6_K_SEQ, O.MXFP4, O.MXFP4_CLAMP]
SEM_QT = {O.F32: 0, O.Q4_0: 2, O.Q4_1: 3, O.Q5_0_F32: 6, O.Q5_0_Q8: 6, O.Q8_0: 8, O.Q4_K_GGML: 12,
          O.Q4_K_Q8: 12, O.Q5_K_GGML: 13, O.Q5_K_CE: 13, O.Q6_K_GGML: 14, O.Q6_K_LOWNIB: 14,
          O.Q6_K_SEQ: 14, O.MXFP4: 39, O.MXFP4_CLAMP: 39, O.MXFP4_Q8: 39}


@pytest.mark.parametrize("sem", FP32_SEMS)
def test_linearity_and_batching(orc, sem):
    rng = np.random.default_rng(50 + sem)
    R, C = 20, 512
    w = W.gen_weights(rng, SEM_QT[sem], R, C)
    x = W.gen_x(rng, 4, C)
    y = orc.gemv(sem, w, x, R, C, 4)
    for b in range(4):
        assert np.array_equal(orc.gemv(sem, w, x[b], R, C, 1)[0], y[b])
    y01 = orc.gemv(sem, w, x[0] + 2.0 * x[1], R, C, 1)[0]
    assert O.norm_err(y01, y[0] + 2.0 * y[1]) < 1e-5


@pytest.mark.parametrize("sem", [s for s in range(16) if s != O.F32])
def test_zero_scales_give_zero(orc, sem):
    rng = np.random.default_rng(5)
    R, C = 8, 512
    qt = SEM_QT[sem]
    w = W.gen_weights(rng, qt, R, C)
    be, bb = W.BLOCK[qt]
    blk = w.reshape(-1, bb)
    zero_fields = {2: [(0, 2)], 3: [(0, 4)], 6: [(0, 2)], 8: [(0, 2)], 12: [(0, 4)], 13: [(0, 4)],
                   14: [(208, 210)], 39: [(16, 17)]}[qt]
    for a, b in zero_fields:
        blk[:, a:b] = 0
    if qt == 3:
        pass  # Q4_1: w = n*d + m with d = m = 0
    y = orc.gemv(sem, w, W.gen_x(rng, 1, C), R, C, 1)
    assert np.all(y == 0.0)


@pytest.mark.parametrize("family", [(O.Q6_K_GGML, O.Q6_K_LOWNIB, O.Q6_K_SEQ), (O.Q5_K_GGML, O.Q5_K_CE),
                                    (O.Q4_K_GGML, O.Q4_K_Q8), (O.MXFP4, O.MXFP4_Q8), (O.Q5_0_F32, O.Q5_0_Q8)])
def test_semantic_variants_are_distinguishable(orc, family):
    """A variant mix-up must fail a parity check: variants of one quant type
    disagree by far more than any tolerance on random data (the Q8-x variants
    differ by the activation quantisation, still well above 1e-3)."""
    rng = np.random.default_rng(3)
    R, C = 16, 512
    w = W.gen_weights(rng, SEM_QT[family[0]], R, C)
    x = W.gen_x(rng, 1, C)
    ys = [orc.gemv(s, w, x, R, C, 1)[0] for s in family]
    for i in range(len(ys)):
        for j in range(i + 1, len(ys)):
            assert O.norm_err(ys[i], ys[j]) > 3e-3


def test_quantize_q8_0_bounds(orc):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(4096) * 5).astype(np.float32)
    q = orc.quantize_q8_0(x).reshape(-1, 34)
    d = q[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    v = q[:, 2:].view(np.int8).astype(np.float32)
    assert np.max(np.abs(v)) <= 127
    amax = np.abs(x.reshape(-1, 32)).max(1)
    dd = amax / np.float32(127.0)
    # values are quantised with the fp32 scale; the stored fp16 scale is that rounded
    err = np.abs(x.reshape(-1, 32) - v * dd[:, None])
    assert np.all(err <= dd[:, None] * 0.5 * (1 + 1e-5))
    assert np.all(np.abs(d - dd) <= np.abs(dd) * 2.0 ** -11)


def test_route_properties(orc):
    rng = np.random.default_rng(6)
    E, N, K, T = 32, 256, 4, 16
    rw = W.gen_router(rng, E, N)
    x = W.gen_x(rng, T, N)
    i0, w0 = orc.route(rw, x, K, renorm=False)
    i1, w1 = orc.route(rw, x, K, renorm=True)
    assert np.array_equal(i0, i1)                       # renorm does not change the selection
    assert np.all(np.diff(w0, axis=1) <= 0)             # descending
    assert np.allclose(w1.sum(1), 1.0, atol=1e-6)
    logits = x.astype(np.float64) @ rw.T.astype(np.float64)
    top = np.argsort(-logits, axis=1, kind="stable")[:, :K]
    assert np.array_equal(np.sort(top, 1), np.sort(i0, 1))
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert np.allclose(np.take_along_axis(p, i0, 1), w0, rtol=1e-5)


# ------------------------------------------------- decode attention, RoPE

def _textbook_attention(q, k, v, nh, nkh, hd):
    """Softmax attention in double precision (one query token)."""
    S = k.shape[0]
    kk = k.reshape(S, nkh, hd).astype(np.float64)
    vv = v.reshape(S, nkh, hd).astype(np.float64)
    out = np.zeros((nh, hd))
    for h in range(nh):
        j = h // (nh // nkh)
        sc = (kk[:, j] @ q.reshape(nh, hd)[h].astype(np.float64)) / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        out[h] = (p / p.sum()) @ vv[:, j]
    return out.ravel()


@pytest.mark.parametrize("nh,nkh,hd,S", [(8, 2, 32, 1), (8, 2, 32, 40), (16, 4, 64, 300), (4, 4, 16, 7)])
def test_attention_ce_is_textbook_softmax(orc, nh, nkh, hd, S):
    """CE:141-158 is plain softmax attention with expf: the double-precision
    closed form pins it (scores scaled by 1/sqrt(hd), GQA head grouping h // (nh/nkh))."""
    rng = np.random.default_rng(S + hd)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal((S, nkh * hd)).astype(np.float32)
    v = rng.standard_normal((S, nkh * hd)).astype(np.float32)
    got = orc.gqa_decode(O.ATTN_CE, q, k, v, S, nh, nkh, hd)
    assert O.norm_err(got, _textbook_attention(q, k, v, nh, nkh, hd)) < 1e-6


@pytest.mark.parametrize("S", [1, 3, 7])
def test_attention_gqa_c_below_eight_positions_is_textbook(orc, S):
    """softmax_simd's vector loop covers floor(S/8)*8 positions: below 8 every
    weight is the scalar tail's expf, so gqa_attention_decode is softmax attention."""
    rng = np.random.default_rng(S)
    nh, nkh, hd = 8, 2, 32
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal((S, nkh * hd)).astype(np.float32)
    v = rng.standard_normal((S, nkh * hd)).astype(np.float32)
    got = orc.gqa_decode(O.ATTN_GQA_C, q, k, v, S, nh, nkh, hd)
    assert O.norm_err(got, _textbook_attention(q, k, v, nh, nkh, hd)) < 1e-6


@pytest.mark.parametrize("S", [8, 13, 64, 100])
def test_attention_gqa_c_equal_scores_closed_form(orc, S):
    """q = 0 makes every score 0 = the maximum: the vector loop's weights are
    exp_ps_simd(0), which the source's polynomial evaluates to its last
    coefficient 0.0013333558146428f (t = 0, n = rne(0.5) = 0, f = 0), the tail's
    expf(0) = 1, and out = (c sum_{s < 8k} v + sum_tail v) / (8k c + r + 1e-10).
    A textbook exponential (weight 1 everywhere), a Horner order that yields
    2^0 = 1, or a different vector/tail split all fail this."""
    rng = np.random.default_rng(S)
    nh, nkh, hd = 4, 2, 16
    q = np.zeros(nh * hd, np.float32)
    k = rng.standard_normal((S, nkh * hd)).astype(np.float32)
    v = rng.standard_normal((S, nkh * hd)).astype(np.float32)
    got = orc.gqa_decode(O.ATTN_GQA_C, q, k, v, S, nh, nkh, hd)
    c = float(np.float32(0.0013333558146428))
    vec = S // 8 * 8
    vv = v.reshape(S, nkh, hd).astype(np.float64)
    num = c * vv[:vec].sum(0) + vv[vec:].sum(0)
    den = c * vec + (S - vec) + 1e-10
    want = np.repeat(num / den, nh // nkh, axis=0).ravel()
    assert O.norm_err(got, want) < 1e-5
    assert orc.exp_ps_simd(0.0) == np.float32(0.0013333558146428)


def _exp_ps_simd_exact(x):
    """exp_ps_simd (gqa_attention.c:32-48) for one float32 x, evaluated with
    exact rational arithmetic and one rounding to float32 per operation: the
    fp32 multiply by log2e, t + 0.5 rounded to an integer with ties to even
    (cvtps_epi32 under the default MXCSR), f = t - n, five fused multiply-adds
    starting from p = 1, the clamped biased exponent.  The five coefficients
    are not copied from any source: they are (ln 2)^k / k! for k = 1..5 (the
    Taylor coefficients of 2^f the source's literals spell to 16 digits),
    rounded to float32 as a float literal is."""
    from fractions import Fraction as F

    def r32(q):
        # round the exact rational q to the nearest float32 (ties to even)
        v = np.float32(float(q))             # within an ulp; then fix up exactly
        lo, hi = np.nextafter(v, np.float32(-np.inf)), np.nextafter(v, np.float32(np.inf))
        best = min((lo, v, hi), key=lambda c: (abs(F(float(c)) - q), int(np.float32(c).view(np.uint32)) & 1))
        return np.float32(best)

    coef = [r32(F(math.log(2) ** k) / math.factorial(k)) for k in range(1, 6)]
    log2e = np.float32(1.4426950408889634)
    t = r32(F(float(np.float32(x))) * F(float(log2e)))
    h = r32(F(float(t)) + F(1, 2))
    n = int(np.rint(np.float64(h)))          # ties to even
    f = r32(F(float(t)) - n)
    p = np.float32(1.0)
    for c in coef:
        p = r32(F(float(p)) * F(float(f)) + F(float(c)))
    b = min(max(n + 127, 0), 255)
    two_n = np.array([b << 23], np.uint32).view(np.float32)[0]
    return r32(F(float(p)) * F(float(two_n)))


def test_exp_ps_simd_pinned_over_its_range(orc):
    """The oracle's exp_ps_simd bit for bit against an exact-arithmetic
    evaluation of the source's steps with coefficients derived from the
    Taylor series of 2^f (not typed from the source) over many arguments:
    scores of a softmax (<= 0) down to the underflow of 2^n, small positive
    ones, every half-integer t (where the rounding of t + 0.5 decides n) and
    signed zeros.  A wrong coefficient, a different Horner order or a
    different rounding of n changes thousands of these."""
    rng = np.random.default_rng(33)
    xs = list(rng.uniform(-110.0, 0.0, 3000).astype(np.float32))
    xs += list(rng.uniform(-2.0, 2.0, 1500).astype(np.float32))
    xs += list(rng.uniform(0.0, 60.0, 500).astype(np.float32))
    ln2 = np.float32(math.log(2))
    xs += [np.float32(k * 0.5 * ln2) for k in range(-60, 61)]   # t near k / 2
    xs += [np.float32(0.0), np.float32(-0.0), np.float32(-87.3), np.float32(-1e-30)]
    bad = []
    for x in xs:
        want = _exp_ps_simd_exact(x)
        got = np.float32(orc.exp_ps_simd(float(x)))
        if not (got == want or (np.isnan(got) and np.isnan(want))):
            bad.append((float(x), float(got), float(want)))
    assert not bad, f"{len(bad)} mismatches, e.g. {bad[:4]}"
    # and the closed form where f = 0: exp_ps_simd(0) is the last coefficient, (ln 2)^5 / 120
    assert np.float32(orc.exp_ps_simd(0.0)) == np.float32(math.log(2) ** 5 / 120)


def test_attention_modes_differ_from_eight_positions(orc):
    rng = np.random.default_rng(5)
    nh, nkh, hd, S = 4, 1, 16, 16
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal((S, nkh * hd)).astype(np.float32)
    v = rng.standard_normal((S, nkh * hd)).astype(np.float32)
    a = orc.gqa_decode(O.ATTN_CE, q, k, v, S, nh, nkh, hd)
    b = orc.gqa_decode(O.ATTN_GQA_C, q, k, v, S, nh, nkh, hd)
    assert O.norm_err(a, b) > 1e-2


def test_rope_is_a_rotation(orc):
    """rope_apply (GO:37-51): each pair (j, j + r/2) rotated by angle theta_pj,
    i.e. the complex product (a0 + i a1) e^{i theta}; lanes past rope_dim untouched."""
    rng = np.random.default_rng(3)
    nh, hd, r, P = 4, 64, 48, 9
    theta = rng.uniform(-3, 3, (P, r // 2))
    cos_t, sin_t = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
    buf = rng.standard_normal(nh * hd).astype(np.float32)
    for pos in (0, 5, 8):
        got = orc.rope(buf, nh, hd, pos, cos_t, sin_t, r).reshape(nh, hd)
        b = buf.reshape(nh, hd).astype(np.float64)
        z = (b[:, :r // 2] + 1j * b[:, r // 2:r]) * np.exp(1j * theta[pos].astype(np.float32).astype(np.float64))
        assert np.max(np.abs(got[:, :r // 2] - z.real)) < 1e-5
        assert np.max(np.abs(got[:, r // 2:r] - z.imag)) < 1e-5
        assert np.array_equal(got[:, r:], buf.reshape(nh, hd)[:, r:])
