"""GPU parity of the quantised-weight MFMA GEMM (prefill / batched path of
*_batch_matmul and mllm_gemv for B > 8) against the oracle.

Tolerance GEMM_TOL: weights and fp32 activations enter the MFMA as bf16
hi+lo pairs (about 16 significant bits each, products accumulated in fp32),
so the normalised max error is ~1e-5; any decode or layout mistake costs
> 3e-3.
"""
import numpy as np
import pytest

import oracle as O
from helpers import fp, up
from mojollama_amd import kernels as K
from mojollama_amd import workloads as W

pytestmark = pytest.mark.gpu
GEMM_TOL = 5e-5


@pytest.fixture(scope="module")
def lib():
    return K.load_kernels()


@pytest.fixture(scope="module")
def dev(lib):
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return K.DeviceOps(lib)


def bmm(lib, name, w, x, R, C, B):
    out = np.full(B * R, np.nan, np.float32)
    getattr(lib, name + "_batch_matmul")(up(w), fp(np.ascontiguousarray(x, np.float32)), fp(out), R, C, B)
    return out.reshape(B, R)


@pytest.mark.parametrize("name,qt", [("q4_0", 2), ("q8_0", 8), ("q4_k", 12), ("q6_k", 14), ("q5_k", 13),
                                     ("mxfp4", 39)])
@pytest.mark.parametrize("B", [9, 64, 130])
def test_batch_matmul_gemm_vs_oracle(lib, orc, name, qt, B):
    rng = np.random.default_rng(300 + qt + B)
    R, C = 200, 512
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, B, C)
    got = bmm(lib, name, w, x, R, C, B)
    assert O.norm_err(got, orc.gemv(orc.sem_for(1, qt), w, x, R, C, B)) < GEMM_TOL


def same_nonfinite(got, ref, tol):
    if not (np.array_equal(np.isnan(got), np.isnan(ref)) and np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])):
        return False
    fin = np.isfinite(ref)
    return not fin.any() or O.norm_err(got[fin], ref[fin]) < tol


@pytest.mark.parametrize("name,qt", [("q4_0", 2), ("q8_0", 8), ("q4_k", 12), ("q6_k", 14), ("q5_k", 13),
                                     ("mxfp4", 39)])
def test_batch_matmul_large_B_nonfinite_scales(lib, orc, name, qt):
    """B = 16 with inf / NaN block scales (E8M0 255, or 194 where
    mxfp4_batch_matmul's 1e20 clamp bites): the weight cache's scale scan keeps
    such a matrix off the MFMA GEMM, whose bf16 weights would turn inf * 0
    into NaN and would not apply the clamp; outputs match the oracle's
    per-element weighting exactly in their NaN / inf pattern."""
    rng = np.random.default_rng(930 + qt)
    be, bb = W.BLOCK[qt]
    R, C, B = 24, 768 if be == 256 else 800, 16
    w = W.gen_weights(rng, qt, R, C).reshape(R, C // be, bb)
    if qt == 39:
        for row, blk, e in ((3, 1, 255), (6, 0, 194), (9, 2, 230)):
            w[row, blk, 16] = e
    else:
        d_off = 208 if qt == W.QT_Q6_K else 0
        for row, blk, bits in ((3, 1, 0x7C00), (6, 0, 0x7E00), (9, 2, 0xFC00)):
            w[row, blk, d_off:d_off + 2] = np.frombuffer(np.uint16(bits).tobytes(), np.uint8)
    w = np.ascontiguousarray(w.ravel())
    x = W.gen_x(rng, B, C)
    got = bmm(lib, name, w, x, R, C, B)
    ref = orc.gemv(orc.sem_for(1, qt), w, x, R, C, B)
    assert same_nonfinite(got, ref, GEMM_TOL)


@pytest.mark.parametrize("sem", [K.Q4_0, K.Q4_1, K.Q5_0_F32, K.Q8_0, K.Q4_K_GGML, K.Q4_K_Q8, K.Q5_K_GGML, K.Q5_K_CE,
                                 K.Q6_K_GGML, K.Q6_K_LOWNIB, K.Q6_K_SEQ, K.MXFP4, K.MXFP4_CLAMP, K.MXFP4_Q8])
def test_device_gemm_every_semantic(dev, orc, sem):
    import torch
    qt = {K.Q4_0: 2, K.Q4_1: 3, K.Q5_0_F32: 6, K.Q8_0: 8, K.Q4_K_GGML: 12, K.Q4_K_Q8: 12, K.Q5_K_GGML: 13,
          K.Q5_K_CE: 13, K.Q6_K_GGML: 14, K.Q6_K_LOWNIB: 14, K.Q6_K_SEQ: 14, K.MXFP4: 39, K.MXFP4_CLAMP: 39,
          K.MXFP4_Q8: 39}[sem]
    rng = np.random.default_rng(700 + sem)
    R, C, B = 130, 768 if W.BLOCK[qt][0] == 256 else 800, 70
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, B, C)
    packed = dev.pack(sem, torch.from_numpy(w).cuda(), R, C)
    got = dev.gemv(sem, packed, torch.from_numpy(x).cuda(), R, C).cpu().numpy()
    assert O.norm_err(got, orc.gemv(sem, w, x, R, C, B)) < GEMM_TOL, K.SEM_NAMES[sem]


@pytest.mark.parametrize("name,qt,R,C,M", [("q4_k", 12, 5632, 2048, 128), ("q6_k", 14, 2048, 5632, 128),
                                           ("q4_k", 12, 5632, 2048, 1280)])
def test_prefill_config_shapes(lib, orc, name, qt, R, C, M):
    """the full matrices with bf16-valued activations, checked on a row subset."""
    rng = np.random.default_rng(R + M)
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, M, C, bf16=True)
    got = bmm(lib, name, w, x, R, C, M)
    rows = 256
    rb = W.row_bytes(qt, C)
    ref = orc.gemv(orc.sem_for(1, qt), w[:rows * rb], x[:64], rows, C, 64)
    assert O.norm_err(got[:64, :rows], ref) < GEMM_TOL
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("sem,qt", [(K.Q4_K_GGML, 12), (K.Q6_K_SEQ, 14), (K.MXFP4, 39)])
@pytest.mark.parametrize("bf16_rows", ["all", "some"])
def test_gemm_bf16_exact_activations(dev, orc, sem, qt, bf16_rows):
    """Rows whose activations are exact in bf16 (configs[2]'s prefill inputs) let a
    tile skip its lower activation planes; a tile holding one fp32 row must not."""
    import torch
    rng = np.random.default_rng(900 + qt + len(bf16_rows))
    R, C, B = 300, 1024, 600          # B >= 512: 128-entry tiles, and split-K off
    w = W.gen_weights(rng, qt, R, C)
    x = torch.from_numpy(W.gen_x(rng, B, C)).bfloat16().float().numpy()
    if bf16_rows == "some":
        x[::97] = W.gen_x(rng, x[::97].shape[0], C)   # a full-precision row in most tiles
    raw = torch.from_numpy(w).cuda()
    packed = dev.pack(sem, raw, R, C)
    got = dev.gemv(sem, packed, torch.from_numpy(np.ascontiguousarray(x)).cuda(), R, C).cpu().numpy()
    assert O.norm_err(got, orc.gemv(sem, w, x, R, C, B)) < GEMM_TOL


@pytest.mark.parametrize("B", [16, 100])
def test_gemm_split_k_vs_oracle(dev, orc, B):
    """Few output tiles and a long K: the launch splits K across workgroups and
    adds the partials in order (deterministic: two runs agree bit for bit)."""
    import torch
    rng = np.random.default_rng(950 + B)
    R, C = 256, 5632
    w = W.gen_weights(rng, 14, R, C)
    x = W.gen_x(rng, B, C)
    raw = torch.from_numpy(w).cuda()
    packed = dev.pack(K.Q6_K_SEQ, raw, R, C)
    xt = torch.from_numpy(x).cuda()
    got1 = dev.gemv(K.Q6_K_SEQ, packed, xt, R, C).cpu().numpy()
    got2 = dev.gemv(K.Q6_K_SEQ, packed, xt, R, C).cpu().numpy()
    assert np.array_equal(got1, got2)
    assert O.norm_err(got1, orc.gemv(K.Q6_K_SEQ, w, x, R, C, B)) < GEMM_TOL
