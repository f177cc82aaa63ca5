"""GPU parity of the Qwen3.6 hybrid drivers through the C ABI against fixtures
written by the reference's own C (oracle/_ref/libref.so, compiled from CE;
tests/golden/make_golden.py gen_qwen36):

  * qwen36_batch_forward (CE:859-1231) on a small seeded model that takes
    every path of the driver (workloads.qwen36_case: SSM and attention
    layers, fused QKV with V read from the workspace slice, MoE with Q4_K /
    MXFP4 experts, shared experts of two types, a layer without MoE, fp32 and
    Q4_K embeddings), two calls in a row with kv_lens advanced in between;
    checked: logits, the SSM state, the KV rows each call writes and the
    fused-QKV workspace slice the reference leaves (its second call reads V
    from what the first left there);
  * ssm_layer_fused (CE:803-849), including N > inner, where a token's result
    overwrites later tokens' intermediates before they are used;
  * ssm_decode_step (CE:736-802).

Tolerances (normalised max error, max|got - ref| / max|ref|):
  * SSM drop-ins: GEMV_TOL -- elementwise SiLU / exp / log (within an ulp of
    glibc's) and the decode GEMVs' fp32 summation order;
  * qwen36_batch_forward: QWEN36_TOL for logits, KV rows and slice, and the
    SSM state.  Every Q4_K matmul of quant_matmul_omp requantises its input
    to Q8_0 (dot_q4_k_q8_0, QK:1647-1735) and every MXFP4 expert down
    projection requantises h (mxfp4_row_dot_q8): an fp32 ulp of difference
    upstream can move a Q8_0 code by one step, ~4e-4 of that matmul's output
    (MOE_Q8H_TOL's reasoning): 1e-3 allows a few such steps.  The top-K
    selection itself is exact (the router's fp32 sums run in
    f32_matmul_omp's order); a flipped selection would move the logits by
    far more.  The fixture's case is checked at generation not to sit on such
    an edge: a few ulps of change in any norm weight moves the reference's
    own logits by <= 1.3e-6 (`ulp_sensitivity` in the fixture).
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from helpers import GEMV_TOL
from mojollama_amd import kernels as K
from mojollama_amd import workloads as W

pytestmark = pytest.mark.gpu

QWEN36_TOL = 1e-3

SSM_CASES = [("a", 91, 3, 256, 256, W.QT_Q8_0, W.QT_Q6_K), ("b", 92, 3, 512, 256, W.QT_Q4_K, W.QT_MXFP4),
             ("c", 93, 2, 256, 384, W.QT_MXFP4, W.QT_Q8_0)]


@pytest.fixture(scope="module")
def lib():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return K.load_kernels()


def crc(*arrays):
    import zlib
    c = 0
    for a in arrays:
        c = zlib.crc32(np.ascontiguousarray(a).view(np.uint8).tobytes(), c)
    return c


@pytest.mark.parametrize("emb_quant", [0, 12])
def test_qwen36_batch_forward_vs_reference(lib, golden, emb_quant):
    g = golden(f"qwen36_emb{emb_quant}.npz")
    c = W.qwen36_case(0, 2, emb_quant)
    assert W.qwen36_arrays_crc(c) == int(g["crc"]), "regenerated inputs differ from the fixture's"
    call = W.Qwen36Call(c)
    for i in range(2):
        logits = call.call(lib, c["tokens"][i])
        assert np.abs(logits).max() > 0, K.last_error(lib)
        kv = np.stack([call.kv[:, l, call.kv_lens[l]] for l in range(c["L"])])
        errs = {"logits": O.norm_err(logits, g[f"logits{i}"]), "state": O.norm_err(call.state, g[f"state{i}"]),
                "kv": O.norm_err(kv, g[f"kv{i}"]), "slice": O.norm_err(call.qkv_slice(), g[f"slice{i}"])}
        print(f"[parity] qwen36 emb{emb_quant} call {i}: " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()),
              flush=True)
        assert np.isfinite(logits).all()
        for k, v in errs.items():
            assert v < QWEN36_TOL, f"call {i} {k}: {v:.3e}"
        call.kv_lens += 1


def test_qwen36_kv_mirror_follows_the_caller(lib, golden):
    """The device keeps mirrors of the caller's KV caches.  The same first
    call again over caches whose cached rows all changed (the reference's
    logits move by > 1%) must give the reference's logits for those caches
    (the sampled seal sees the change without mllm_cache_clear); then the
    original caches, after mllm_cache_clear() (what the header asks of a
    caller that rewrites rows below kv_lens), give the first result bit for
    bit; and a repeated identical call also gives it bit for bit."""
    g = golden("qwen36_emb0.npz")
    c = W.qwen36_case(0, 2, 0)
    call = W.Qwen36Call(c)

    def restore(kv):
        call.state[:] = c["state0"]
        call.ws[:] = c["ws0"]
        call.kv[:] = kv
        call.kv_lens[:] = c["kv_lens0"]
    a = call.call(lib, c["tokens"][0])
    restore(g["kv_mod"])
    m = call.call(lib, c["tokens"][0])
    err = O.norm_err(m, g["logits_mod"])
    print(f"[parity] qwen36 rewritten KV rows: {err:.2e}", flush=True)
    assert err < QWEN36_TOL
    restore(c["kv0"])
    lib.mllm_cache_clear()
    b = call.call(lib, c["tokens"][0])
    assert np.array_equal(a, b)
    restore(c["kv0"])
    d = call.call(lib, c["tokens"][0])
    assert np.array_equal(a, d)


@pytest.mark.parametrize("case", SSM_CASES, ids=[c[0] for c in SSM_CASES])
def test_ssm_drop_ins_vs_reference(lib, golden, case):
    tag, seed, B, N, inner, gq, sq = case
    g = golden(f"ssm_{tag}.npz")
    c = W.ssm_case(seed, B, N, inner, gate_qt=gq, so_qt=sq)
    assert crc(c["x"], c["gate"], c["so"], c["state"]) == int(g["crc"])
    out_f, st_f = W.ssm_call(lib, c, True)
    out_d, st_d = W.ssm_call(lib, c, False)
    errs = {"fused": O.norm_err(out_f, g["fused"]), "fused_state": O.norm_err(st_f, g["fused_state"]),
            "step": O.norm_err(out_d, g["step"]), "step_state": O.norm_err(st_d, g["step_state"])}
    print(f"[parity] ssm {tag} B={B} N={N} inner={inner}: " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()),
          flush=True)
    for k, v in errs.items():
        assert v < GEMV_TOL, f"{k}: {v:.3e}"
