"""GPU parity of the decode GEMVs, the Q8_0 quantiser and the dequantisers,
through the C ABI, against the golden vectors written by the reference's own
C and against the oracle on seeded inputs.

Tolerance: GEMV_TOL (tests/helpers.py) normalised max error for every GEMV
semantic; bit-exact for quantize_row_q8_0 and the *_dequantize_row outputs.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from helpers import GEMV_TOL, fp, up
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


def qmm(lib, w, x, R, C, qt):
    out = np.full(R, np.nan, np.float32)
    lib.quant_matmul_omp(up(w), fp(np.ascontiguousarray(x, np.float32)), fp(out), R, C, qt)
    return out


def bmm(lib, name, w, x, R, C, B):
    out = np.full(B * R, np.nan, np.float32)
    getattr(lib, name + "_batch_matmul")(up(w), fp(np.ascontiguousarray(x, np.float32)), fp(out), R, C, B)
    return out.reshape(B, R)


# ------------------------------------------------------------ golden vectors

@pytest.mark.parametrize("qt", [0, 2, 3, 6, 8, 12, 13, 14, 39])
def test_golden_quant_matmul(lib, golden, qt):
    g = golden(f"qmm_{qt}.npz")
    got = qmm(lib, g["W"], g["x"], int(g["n_rows"]), int(g["n_cols"]), qt)
    assert O.norm_err(got, g["out"]) < GEMV_TOL, K.last_error(lib)


@pytest.mark.parametrize("name", ["q4_0", "q8_0", "q4_k", "q6_k", "q5_k", "mxfp4"])
@pytest.mark.parametrize("B", [1, 3, 5])
def test_golden_batch_matmul(lib, golden, name, B):
    g = golden(f"bmm_{name}_B{B}.npz")
    got = bmm(lib, name, g["W"], g["x"], int(g["n_rows"]), int(g["n_cols"]), B)
    assert O.norm_err(got, g["out"]) < GEMV_TOL


def test_golden_mxfp4_scale_edges(lib, golden):
    g = golden("edge_mxfp4.npz")
    R, C = int(g["n_rows"]), int(g["n_cols"])
    got = bmm(lib, "mxfp4", g["W"], g["x"], R, C, 1)[0]
    assert np.all(np.isfinite(got))
    assert O.norm_err(got, g["out_clamp"]) < GEMV_TOL
    got = qmm(lib, g["W"], g["x"], R, C, 39)
    ref = g["out_noclamp"]
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = np.isfinite(ref)
    assert np.array_equal(got[~fin & ~np.isnan(ref)], ref[~fin & ~np.isnan(ref)])
    assert O.norm_err(got[fin], ref[fin]) < GEMV_TOL


def test_golden_quantize_q8_0_bitexact(lib, golden):
    g = golden("q8_0.npz")
    q = np.zeros_like(g["q8"])
    nb = lib.quantize_row_q8_0(fp(g["x"]), up(q), g["x"].size)
    assert nb == g["x"].size // 32
    assert np.array_equal(q, g["q8"])


def test_golden_quantize_q8_0_nonfinite_bitexact(lib, golden):
    """NaN / +-inf activations: bit-exact with the reference, including the
    blocks whose amax its vmaxps order turns NaN."""
    g = golden("q8_0_nonfinite.npz")
    q = np.zeros_like(g["q8"])
    lib.quantize_row_q8_0(fp(g["x"]), up(q), g["x"].size)
    assert np.array_equal(q, g["q8"])


@pytest.mark.parametrize("name", ["q4_k", "q6_k", "q5_k", "q8_0"])
def test_golden_dequantize_row_bitexact(lib, golden, name):
    g = golden(f"deq_{name}.npz")
    out = np.zeros(1024, np.float32)
    getattr(lib, name + "_dequantize_row")(up(g["W"]), fp(out), 1024)
    assert np.array_equal(out, g["out"])


def test_golden_batch_qkv_and_gate_up(lib, golden):
    g = golden("batch_qkv.npz")
    oq, ok, ov = np.zeros(32, np.float32), np.zeros(16, np.float32), np.zeros(16, np.float32)
    lib.batch_qkv_omp(up(g["Wq"]), up(g["Wk"]), up(g["Wv"]), fp(g["x"]), fp(oq), fp(ok), fp(ov), 32, 16, 16, 512,
                      12, 14, 8)
    for got, ref in ((oq, g["oq"]), (ok, g["ok"]), (ov, g["ov"])):
        assert O.norm_err(got, ref) < GEMV_TOL
    g = golden("batch_gate_up.npz")
    og, ou = np.zeros(32, np.float32), np.zeros(32, np.float32)
    lib.batch_gate_up_omp(up(g["Wg"]), up(g["Wu"]), fp(g["x"]), fp(og), fp(ou), 32, 32, 512, 39, 2)
    assert O.norm_err(og, g["og"]) < GEMV_TOL
    assert O.norm_err(ou, g["ou"]) < GEMV_TOL


def test_unknown_quant_type_leaves_output_untouched(lib):
    w = np.zeros(64 * 34, np.uint8)
    x = np.ones(64, np.float32)
    out = np.full(2, 7.0, np.float32)
    lib.quant_matmul_omp(up(w), fp(x), fp(out), 2, 64, 7)   # 7 is not a code the dispatch knows (QK:1385)
    assert np.all(out == 7.0)
    assert "unknown quant type" in K.last_error(lib)


# --------------------------------------------- oracle on seeded inputs

SEM_QT = {K.F32: 0, K.Q4_0: 2, K.Q4_1: 3, K.Q5_0_F32: 6, K.Q5_0_Q8: 6, K.Q8_0: 8, K.Q4_K_GGML: 12,
          K.Q4_K_Q8: 12, K.Q5_K_GGML: 13, K.Q5_K_CE: 13, K.Q6_K_GGML: 14, K.Q6_K_LOWNIB: 14,
          K.Q6_K_SEQ: 14, K.MXFP4: 39, K.MXFP4_CLAMP: 39, K.MXFP4_Q8: 39}


@pytest.mark.parametrize("sem", list(range(16)))
@pytest.mark.parametrize("B", [1, 2, 3, 5, 8, 11])
def test_device_gemv_vs_oracle(dev, orc, sem, B):
    """Every semantic, every batch width class, ragged row counts, via mllm_gemv."""
    import torch
    rng = np.random.default_rng(1000 + 16 * B + sem)
    qt = SEM_QT[sem]
    R, C = 131, (768 if W.BLOCK[qt][0] == 256 else 800)
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, B, C)
    ref = orc.gemv(sem, w, x, R, C, B)
    raw = torch.from_numpy(w).cuda()
    packed = dev.pack(sem, raw, R, C)
    got = dev.gemv(sem, packed, torch.from_numpy(x).cuda(), R, C).cpu().numpy()
    assert O.norm_err(got, ref) < GEMV_TOL, (K.SEM_NAMES[sem], B)


@pytest.mark.parametrize("sem", [K.Q4_0, K.Q8_0, K.Q4_K_GGML, K.Q5_K_GGML, K.Q6_K_SEQ])
@pytest.mark.parametrize("B", [1, 4, 8])
def test_device_gemv_nonfinite_scales(dev, orc, sem, B):
    """Blocks whose fp16 scale is inf or NaN take the per-element path (w = s*q, then w*x, as
    the reference weighs them): the NaN/inf pattern matches the oracle exactly, and rows
    decoded beside them in the same lane group stay within tolerance."""
    import torch
    rng = np.random.default_rng(77 + 16 * B + sem)
    qt = SEM_QT[sem]
    be, bb = W.BLOCK[qt]
    R, C = 24, 768 if be == 256 else 800
    w = W.gen_weights(rng, qt, R, C).reshape(R, C // be, bb)
    d_off = 208 if qt == W.QT_Q6_K else 0   # the block's fp16 d
    for row, blk, bits in ((3, 1, 0x7C00), (6, 0, 0x7E00), (9, 2, 0xFC00)):
        w[row, blk, d_off:d_off + 2] = np.frombuffer(np.uint16(bits).tobytes(), np.uint8)
    w = w.ravel()
    x = W.gen_x(rng, B, C)
    ref = orc.gemv(sem, w, x, R, C, B).reshape(B, R)
    packed = dev.pack(sem, torch.from_numpy(w).cuda(), R, C)
    got = dev.gemv(sem, packed, torch.from_numpy(x).cuda(), R, C).cpu().numpy().reshape(B, R)
    assert not np.all(np.isfinite(ref)), "the planted scales must reach the output"
    assert np.array_equal(np.isnan(got), np.isnan(ref)), (K.SEM_NAMES[sem], B)
    inf = np.isinf(ref)
    assert np.array_equal(got[inf], ref[inf])
    fin = np.isfinite(ref)
    assert O.norm_err(got[fin], ref[fin]) < GEMV_TOL, (K.SEM_NAMES[sem], B)


@pytest.mark.parametrize("sem", [K.F32, K.Q4_0, K.Q4_1, K.Q5_0_F32, K.Q8_0, K.Q4_K_GGML, K.Q5_K_GGML, K.Q5_K_CE,
                                 K.Q6_K_GGML, K.Q6_K_LOWNIB, K.Q6_K_SEQ, K.MXFP4, K.MXFP4_CLAMP])
@pytest.mark.parametrize("B", [1, 3, 8])
def test_device_gemv_nonfinite_activations(dev, orc, sem, B):
    """fp32-activation semantics on tokens holding +-inf / NaN: a staged
    16-element group keeps each element's class, and the per-element path
    weighs it as the reference does (Q5_K ggml with its min term factored
    out, QK:300,338), so NaN / inf land on the same outputs as the oracle's."""
    import torch
    rng = np.random.default_rng(95 + 16 * B + sem)
    qt = SEM_QT[sem]
    R, C = 40, 1024
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, B, C).copy()
    for b in range(B):
        if b % 3 == 0:
            x[b, 5 + 64 * b] = np.inf
        elif b % 3 == 1:
            x[b, 200 + b] = -np.inf
            x[b, 301] = np.inf
        else:
            x[b, 17] = np.nan
    ref = orc.gemv(sem, w, x, R, C, B).reshape(B, R)
    packed = dev.pack(sem, torch.from_numpy(w).cuda(), R, C)
    got = dev.gemv(sem, packed, torch.from_numpy(x).cuda(), R, C).cpu().numpy().reshape(B, R)
    if sem != K.Q5_K_GGML:   # there d1 * inf - m1 * inf is NaN whenever d1, m1 > 0
        assert not np.all(np.isnan(ref)), "an inf token must give +-inf somewhere for the test to mean something"
    assert np.array_equal(np.isnan(got), np.isnan(ref)), (K.SEM_NAMES[sem], B)
    inf = np.isinf(ref)
    assert np.array_equal(got[inf], ref[inf]), (K.SEM_NAMES[sem], B)


@pytest.mark.parametrize("sem", [K.Q4_K_Q8, K.Q5_0_Q8, K.MXFP4_Q8])
@pytest.mark.parametrize("B", [1, 4])
def test_device_gemv_q8_activation_nonfinite(dev, orc, sem, B):
    """Q8_0-activation semantics on activations holding NaN / +-inf at block
    positions 0, 7, 24 and 31 (the vmaxps order makes only some of them reach
    amax): NaN / inf pattern exact, finite outputs within tolerance."""
    import torch
    rng = np.random.default_rng(91 + 16 * B + sem)
    qt = SEM_QT[sem]
    R, C = 40, 1024
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, B, C).copy()
    for b in range(B):
        for blk, pos, val in ((1, 0, np.nan), (3, 31, np.nan), (5, 24, np.inf), (8, 7, -np.inf), (12, 31, np.inf)):
            if (blk + b) % 3:
                x[b, 32 * (blk + 4 * b) + pos] = val
    ref = orc.gemv(sem, w, x, R, C, B).reshape(B, R)
    packed = dev.pack(sem, torch.from_numpy(w).cuda(), R, C)
    got = dev.gemv(sem, packed, torch.from_numpy(x).cuda(), R, C).cpu().numpy().reshape(B, R)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), (K.SEM_NAMES[sem], B)
    inf = np.isinf(ref)
    assert np.array_equal(got[inf], ref[inf])
    fin = np.isfinite(ref)
    if fin.any():
        assert O.norm_err(got[fin], ref[fin]) < GEMV_TOL, (K.SEM_NAMES[sem], B)


@pytest.mark.parametrize("sem", [K.Q4_0, K.Q4_1, K.Q5_0_F32, K.Q8_0, K.Q4_K_GGML, K.Q5_K_GGML, K.Q5_K_CE,
                                 K.Q6_K_GGML, K.Q6_K_LOWNIB, K.Q6_K_SEQ, K.MXFP4, K.MXFP4_CLAMP])
def test_device_dequant_vs_oracle(dev, orc, sem):
    import torch
    rng = np.random.default_rng(77 + sem)
    qt = SEM_QT[sem]
    R, C = 9, 512
    w = W.gen_weights(rng, qt, R, C)
    ref = orc.dequant(sem, w, R, C)
    got = dev.dequant(sem, dev.pack(sem, torch.from_numpy(w).cuda(), R, C), R, C).cpu().numpy()
    assert O.norm_err(got, ref) < 1e-6


def test_quantize_q8_0_bitexact_wide_range(dev, orc):
    import torch
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(1 << 16) * np.exp(rng.uniform(-8, 8, 1 << 16))).astype(np.float32)
    x[:32] = 0.0
    got = dev.quantize_q8_0(torch.from_numpy(x).cuda(), 1 << 16).cpu().numpy()
    assert np.array_equal(got, orc.quantize_q8_0(x))


# ------------------------------------------------ full benchmark shapes

@pytest.mark.parametrize("name,R,C,qt,B", [("q8_0_ffn_up", 5632, 2048, 8, 1),
                                           ("q4k_gate", 5632, 2048, 12, 4),
                                           ("q4k_k", 256, 2048, 12, 8),
                                           ("q6k_down", 2048, 5632, 14, 8),
                                           ("q6k_lm_head", 32000, 2048, 14, 1)])
def test_benchmark_shapes_batch_entry(lib, orc, name, R, C, qt, B):
    """configs[0]/[1] shapes through the *_batch_matmul entry points vs the oracle."""
    rng = np.random.default_rng(hash(name) % 2**32)
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, B, C)
    fname = {8: "q8_0", 12: "q4_k", 14: "q6_k"}[qt]
    got = bmm(lib, fname, w, x, R, C, B)
    ref = orc.gemv(orc.sem_for(1, qt), w, x, R, C, B)
    assert O.norm_err(got, ref) < GEMV_TOL


@pytest.mark.parametrize("B,R", [(7, 9000), (8, 9000), (8, 8192)])
def test_batch_entry_output_paths(lib, orc, B, R):
    """The host-buffer entry points write results up to 256 KB straight into
    pinned memory from the kernels and copy larger ones back from HBM: B = 7
    (252 KB) and B = 8 at 8192 rows (256 KB) take the first path, B = 8 at
    9000 rows (288 KB) the second; consecutive calls alternate the paths."""
    rng = np.random.default_rng(1000 * B + R)
    C = 2048
    w = W.gen_weights(rng, 12, R, C)
    x = W.gen_x(rng, B, C)
    ref = orc.gemv(orc.sem_for(1, 12), w, x, R, C, B)
    for _ in range(2):
        got = bmm(lib, "q4_k", w, x, R, C, B)
        assert O.norm_err(got, ref) < GEMV_TOL
        small = bmm(lib, "q4_k", w[: 64 * (C // 256) * 144], x[:1], 64, C, 1)
        assert O.norm_err(small, ref[0, :64]) < GEMV_TOL


def test_q4k_q8_path_full_shape(lib, orc):
    """TurboEngine's Q4_K path (quant_matmul_omp -> dot_q4_k_q8_0) at the gate shape."""
    rng = np.random.default_rng(12)
    w = W.gen_weights(rng, 12, 5632, 2048)
    x = W.gen_x(rng, 1, 2048)
    got = qmm(lib, w, x, 5632, 2048, 12)
    assert O.norm_err(got, orc.gemv(K.Q4_K_Q8, w, x, 5632, 2048, 1)[0]) < GEMV_TOL


@pytest.mark.parametrize("sem,qt,C", [(K.Q4_K_GGML, 12, 9984), (K.MXFP4, 39, 9952), (K.Q8_0, 8, 9920),
                                      (K.Q6_K_SEQ, 14, 9984)])
def test_long_row_ring_vs_oracle(dev, orc, sem, qt, C):
    """The batch-1 path for long rows (64 lanes per row, the four-step weight ring,
    eight-wave workgroups, buffer-resource fetch): rows of 5-10 KB, 4100 of them, so
    waves run one or two row groups of five ring steps, the last step with lanes
    past the row's end, and the last row group ragged."""
    import torch
    rng = np.random.default_rng(qt + C)
    R = 4100
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, 1, C)
    packed = dev.pack(sem, torch.from_numpy(w).cuda(), R, C)
    got = dev.gemv(sem, packed, torch.from_numpy(x).cuda(), R, C).cpu().numpy()
    assert O.norm_err(got, orc.gemv(sem, w, x, R, C, 1)) < GEMV_TOL, K.SEM_NAMES[sem]


def test_gemv_linearity_full_shape(dev):
    """Size-independent property at the lm_head shape: W(a x + b y) = a Wx + b Wy."""
    import torch
    rng = np.random.default_rng(3)
    R, C = 32000, 2048
    w = W.gen_weights(rng, 14, R, C)
    x = W.gen_x(rng, 2, C)
    packed = dev.pack(K.Q6_K_SEQ, torch.from_numpy(w).cuda(), R, C)
    xs = torch.from_numpy(x).cuda()
    y = dev.gemv(K.Q6_K_SEQ, packed, xs, R, C)
    comb = (xs[0] * 0.5 + xs[1] * 2.0).contiguous()
    yc = dev.gemv(K.Q6_K_SEQ, packed, comb, R, C)[0]
    ref = y[0] * 0.5 + y[1] * 2.0
    assert O.norm_err(yc.cpu().numpy(), ref.cpu().numpy()) < 1e-5


@pytest.mark.parametrize("qt,nc", [(8, 16), (12, 128), (14, 128), (39, 16), (2, 16), (13, 200)])
def test_short_rows_give_zeros(lib, qt, nc):
    """Rows shorter than one quant block: zeros, as the reference writes
    (no kernel reads a block that is not there)."""
    rng = np.random.default_rng(qt + nc)
    w = rng.integers(0, 256, 64, dtype=np.uint8)
    x = W.gen_x(rng, 12, nc)
    assert np.all(qmm(lib, w, x[0], 4, nc, qt) == 0.0), K.last_error(lib)
    name = {8: "q8_0", 12: "q4_k", 14: "q6_k", 39: "mxfp4", 2: "q4_0", 13: "q5_k"}[qt]
    for B in (1, 5, 12):          # B = 12 would take the MFMA GEMM with whole blocks
        assert np.all(bmm(lib, name, w, x[:B], 4, nc, B) == 0.0)


@pytest.mark.parametrize("qt", [12, 14, 8, 39])
def test_batch_qkv_gate_up_one_launch(lib, orc, qt):
    """batch_qkv_omp / batch_gate_up_omp with matrices of one type (stacked into
    one packed matrix, one GEMV launch) at the TinyLlama shapes, against the
    oracle's row-path semantics (QK:1095-1222); rewriting a matrix in place
    re-packs the stack."""
    rng = np.random.default_rng(400 + qt)
    C = 2048
    Wq, Wk, Wv = (W.gen_weights(rng, qt, r, C) for r in (2048, 256, 256))
    x = W.gen_x(rng, 1, C)[0]
    sem = orc.sem_for(2, qt)
    for step in range(2):
        oq, ok, ov = (np.full(r, np.nan, np.float32) for r in (2048, 256, 256))
        lib.batch_qkv_omp(up(Wq), up(Wk), up(Wv), fp(x), fp(oq), fp(ok), fp(ov), 2048, 256, 256, C, qt, qt, qt)
        for got, w, r in ((oq, Wq, 2048), (ok, Wk, 256), (ov, Wv, 256)):
            assert O.norm_err(got, orc.gemv(sem, w, x, r, C, 1)[0]) < GEMV_TOL, (step, r)
        Wk[:] = W.gen_weights(rng, qt, 256, C)   # same buffer, new contents
    Wg, Wu = (W.gen_weights(rng, qt, 5632, C) for _ in range(2))
    og, ou = np.full(5632, np.nan, np.float32), np.full(5632, np.nan, np.float32)
    lib.batch_gate_up_omp(up(Wg), up(Wu), fp(x), fp(og), fp(ou), 5632, 5632, C, qt, qt)
    assert O.norm_err(og, orc.gemv(sem, Wg, x, 5632, C, 1)[0]) < GEMV_TOL
    assert O.norm_err(ou, orc.gemv(sem, Wu, x, 5632, C, 1)[0]) < GEMV_TOL


def test_batch_qkv_unknown_type_leaves_output(lib, orc):
    rng = np.random.default_rng(5)
    C = 512
    Wq, Wv = W.gen_weights(rng, 12, 32, C), W.gen_weights(rng, 12, 16, C)
    x = W.gen_x(rng, 1, C)[0]
    oq, ok, ov = np.full(32, np.nan, np.float32), np.full(16, 7.0, np.float32), np.full(16, np.nan, np.float32)
    lib.batch_qkv_omp(up(Wq), up(Wq), up(Wv), fp(x), fp(oq), fp(ok), fp(ov), 32, 16, 16, C, 12, 7, 12)
    assert np.all(ok == 7.0)
    assert O.norm_err(ov, orc.gemv(orc.sem_for(2, 12), Wv, x, 16, C, 1)[0]) < GEMV_TOL


@pytest.mark.parametrize("qt", [12, 14, 1])
def test_golden_requantize_output_q8_0(lib, golden, qt):
    """TE's lm_head requantisation (TE:620-666) through the C ABI: bit-exact
    with the fixture (the reference's dequantize_row, or for F16 TE:643-645's
    conversion of the patterns, + TE's numpy statements)."""
    g = golden(f"requant_q8_{qt}.npz")
    R, C = int(g["n_rows"]), int(g["n_cols"])
    out = np.full(R * (C // 32) * 34, 0xAB, np.uint8)
    assert lib.requantize_output_q8_0(up(g["W"]), R, C, qt, up(out)) == 0, K.last_error(lib)
    assert np.array_equal(out, g["out"])


def test_requantize_lm_head_full_shape(lib, orc):
    """The TinyLlama lm_head (Q6_K 32000x2048): bit-exact with the oracle, and the
    requantised Q8_0 head's logits within a Q8_0 step of the Q6_K head's."""
    rng = np.random.default_rng(88)
    R, C = 32000, 2048
    w = W.gen_weights(rng, 14, R, C)
    out = np.zeros(R * (C // 32) * 34, np.uint8)
    assert lib.requantize_output_q8_0(up(w), R, C, 14, up(out)) == 0, K.last_error(lib)
    assert np.array_equal(out, orc.requant_q8_0(14, w, R, C))
    x = W.gen_x(rng, 1, C)[0]
    q8_logits = qmm(lib, out, x, R, C, 8)
    q6_logits = orc.gemv(K.Q6_K_GGML, w, x, R, C, 1)[0]   # the ggml order the requantisation decodes
    assert O.norm_err(q8_logits, q6_logits) < 2e-2
    assert lib.requantize_output_q8_0(up(w), R, C, 13, up(out)) == -1
    assert lib.requantize_output_q8_0(up(w), 2, 80, 1, up(out)) == -1   # F16: whole 32-element blocks only


# ------------------------------------------------ activations with outliers

@pytest.mark.parametrize("name,qt,C", [("q4_k", 12, 2048), ("q6_k", 14, 2048), ("mxfp4", 39, 2880), ("q8_0", 8, 2048)])
@pytest.mark.parametrize("B", [1, 8])
def test_digit_staging_outliers(lib, orc, name, qt, C, B):
    """fp32 activations with an outlier 10^3-10^4 x its neighbours in every
    16-element group (real LLM activations have such channels).  The decode
    GEMVs stage x as three int8 digit planes under one power of two per group
    of 16 (B = 1) or 32 (the MFMA form at B = 8) elements, exact up to a
    remainder below 2^-20 of the group's largest element, so the small
    neighbours of an outlier carry an absolute error of up to 2^-20 x the
    outlier.  Checked element by element against that bound: for output r,
    |got - ref| <= 4 * 2^-20 * sum_g max_{i in g}|x_i| * sum_{i in g}|w_ri|
    + 2^-20 * sum_i |w_ri x_i| (fp32 summation), ref = the dot of the
    oracle's fp32 weights and x in float64 (groups of 32)."""
    rng = np.random.default_rng(qt * 31 + B)
    R = 256
    w = W.gen_weights(rng, qt, R, C)
    x = rng.standard_normal((B, C)).astype(np.float32)
    pos = rng.integers(0, 16, size=(B, C // 16))
    mag = (10.0 ** rng.uniform(3, 4, size=(B, C // 16)) * rng.choice([-1, 1], size=(B, C // 16))).astype(np.float32)
    for b in range(B):
        x[b, np.arange(C // 16) * 16 + pos[b]] *= mag[b]
    sem = orc.sem_for(1, qt)
    wf = orc.dequant(sem, w, R, C).astype(np.float64)
    ref = x.astype(np.float64) @ wf.T                                       # [B][R]
    gmax = np.abs(x.astype(np.float64)).reshape(B, C // 32, 32).max(axis=2)   # [B][G]
    wabs = np.abs(wf).reshape(R, C // 32, 32).sum(axis=2)                     # [R][G]
    bound = 4 * 2.0 ** -20 * (gmax @ wabs.T) + 2.0 ** -20 * (np.abs(x.astype(np.float64)) @ np.abs(wf).T)
    got = bmm(lib, name, w, x, R, C, B)
    excess = np.abs(got - ref) / bound
    print(f"[parity] outliers {name} B={B}: worst |err|/bound {excess.max():.3f}, "
          f"normalised err {O.norm_err(got, ref):.2e}", flush=True)
    assert np.isfinite(got).all()
    assert excess.max() <= 1.0, K.last_error(lib)
