"""GPU parity of gptoss_forward (GO:96-189), the whole-model decode driver.

A small gpt-oss-shaped model (MXFP4 attention and experts, fp32 norms and
routers, GQA, partial RoPE) runs token by token through the drop-in
gptoss_forward (the reference's argument list and host buffers) and through
the oracle's restatement; logits, the K/V rows each step writes and kv_len
are compared.  The oracle's driver composes functions pinned elsewhere
(MXFP4 GEMV, rope_apply, gqa_attention_decode, the renormalised router, the
moe_forward_omp restatement); its own glue (order of steps, the residual
quirk of GO:186, the [l + e] expert indexing of GO:179-181, logits from the
last xn) is restated from the source, not run: gptoss_batch_forward.c links
gqa_attention.c, which needs cblas (absent here).

Tolerance GPTOSS_TOL of max|logits|: every layer's down projection
requantises h to Q8_0 (one code flip moves a layer output by ~3/(127 sqrt M)
of its max, MOE_Q8H_TOL) and the RMS norms, attention and residuals carry
fp32 summation-order differences through the layers.  Sequences stay below
8 positions so gqa_attention.c's scalar expf tail gives every weight (its
exp_ps_simd steps, where one ulp of a score can move a weight by a step, are
compared kernel to kernel in tests/test_gpu_attn.py).
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from helpers import MOE_Q8H_TOL, fp
from mojollama_amd import kernels as K
from mojollama_amd import workloads as W

pytestmark = pytest.mark.gpu
GPTOSS_TOL = 4 * MOE_Q8H_TOL


@pytest.fixture(scope="module")
def lib():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return K.load_kernels()


class ToyGptOss:
    """Random gpt-oss-shaped weights in the reference's host layout."""

    def __init__(self, seed, L=2, N=256, NH=8, NKH=2, HD=32, E=6, Kk=2, M=128, V=96, max_ctx=16, rope_dim=24):
        rng = np.random.default_rng(seed)
        self.L, self.N, self.NH, self.NKH, self.HD, self.E, self.K, self.M = L, N, NH, NKH, HD, E, Kk, M
        self.V, self.max_ctx, self.rope_dim, self.eps = V, max_ctx, rope_dim, 1e-5
        inner, kvd = NH * HD, NKH * HD
        mx = lambda r, c: W.gen_weights(rng, W.QT_MXFP4, r, c)  # noqa: E731
        self.emb = rng.standard_normal((V, N)).astype(np.float32)
        self.wq = [mx(inner, N) for _ in range(L)]
        self.wk = [mx(kvd, N) for _ in range(L)]
        self.wv = [mx(kvd, N) for _ in range(L)]
        self.wo = [mx(N, inner) for _ in range(L)]
        self.an = [(1 + 0.1 * rng.standard_normal(N)).astype(np.float32) for _ in range(L)]
        self.fn = [(1 + 0.1 * rng.standard_normal(N)).astype(np.float32) for _ in range(L)]
        self.router = [(rng.standard_normal((E, N)) * 0.05).astype(np.float32) for _ in range(L)]
        n_exp = L - 1 + E                                  # GO:179-181 read w_*_exps[l + e]
        self.gate = [mx(M, N) for _ in range(n_exp)]
        self.up = [mx(M, N) for _ in range(n_exp)]
        self.down = [mx(N, M) for _ in range(n_exp)]
        self.wout = mx(V, N)
        theta = rng.uniform(-3, 3, (max_ctx, rope_dim // 2))
        self.cos_t, self.sin_t = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
        # ctypes pointer arrays (kept alive with the model)
        cu, cf = K.cu, K.cf
        arr_u = lambda xs: (cu * len(xs))(*[x.ctypes.data_as(cu) for x in xs])  # noqa: E731
        arr_f = lambda xs: (cf * len(xs))(*[x.ctypes.data_as(cf) for x in xs])  # noqa: E731
        self.p = dict(wQ=arr_u(self.wq), wK=arr_u(self.wk), wV=arr_u(self.wv), wO=arr_u(self.wo), wAN=arr_f(self.an),
                      wFN=arr_f(self.fn), gin=arr_f(self.router), ge=arr_u(self.gate), ue=arr_u(self.up),
                      de=arr_u(self.down))
        self.rows = {k: np.full(L, v, np.int32) for k, v in (("q", inner), ("k", kvd), ("v", kvd), ("o", N))}
        self.qts = np.full(L, 39, np.int32)

    def oracle_struct(self):
        p = self.p
        cast = ctypes.cast
        return O.GptOss(L=self.L, N=self.N, NH=self.NH, NKH=self.NKH, HD=self.HD, V=self.V, E=self.E, K=self.K,
                        M=self.M, max_ctx=self.max_ctx, rope_dim=self.rope_dim, outNR=self.V, eps=self.eps,
                        emb=fp(self.emb), wQ=cast(p["wQ"], O.GptOss._pp), wK=cast(p["wK"], O.GptOss._pp),
                        wV=cast(p["wV"], O.GptOss._pp), wO=cast(p["wO"], O.GptOss._pp),
                        wAN=cast(p["wAN"], O.GptOss._pf), wFN=cast(p["wFN"], O.GptOss._pf),
                        wOut=self.wout.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
                        w_gate_inp=cast(p["gin"], O.GptOss._pf), w_gate_exps=cast(p["ge"], O.GptOss._pp),
                        w_up_exps=cast(p["ue"], O.GptOss._pp), w_down_exps=cast(p["de"], O.GptOss._pp),
                        qt_gate=39, qt_up=39, qt_down=39, cos_t=fp(self.cos_t), sin_t=fp(self.sin_t))

    def new_cache(self):
        z = np.zeros((self.L, self.max_ctx, self.NKH * self.HD), np.float32)
        return z, z.copy(), np.zeros(self.L, np.int32)

    def drop_in(self, lib, token, pos, kc, vc, kv_len, logits):
        p, pi = self.p, lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_int))  # noqa: E731
        tok = np.array([token], np.int32)
        ws = np.zeros(64, np.float32)
        lib.gptoss_forward(pi(tok), pos, fp(self.emb), self.V, p["wQ"], p["wK"], p["wV"], p["wO"], p["wAN"],
                           p["wFN"], pi(self.rows["q"]), pi(self.rows["k"]), pi(self.rows["v"]), pi(self.rows["o"]),
                           pi(self.qts), pi(self.qts), pi(self.qts), pi(self.qts),
                           self.wout.ctypes.data_as(K.cu), self.V, self.N, 39, fp(kc), fp(vc), pi(kv_len),
                           fp(self.cos_t), fp(self.sin_t), self.max_ctx, self.rope_dim, fp(ws), ws.size, self.L,
                           self.N, self.NH, self.NKH, self.HD, 4 * self.N, self.eps, self.E, self.K, self.M,
                           p["gin"], p["ge"], p["ue"], p["de"], 39, 39, 39, fp(logits), fp(ws),
                           ws.view(np.uint8).ctypes.data_as(K.cu), fp(ws))


def close(got, ref, tol=GPTOSS_TOL):
    return np.max(np.abs(got - ref)) <= tol * np.max(np.abs(ref))


def test_gptoss_forward_decode_vs_oracle(lib, orc):
    m = ToyGptOss(1)
    st = m.oracle_struct()
    kc, vc, kl = m.new_cache()
    rk, rv, rl = m.new_cache()
    tokens = [5, 17, 5, 90, 33, 2]
    for pos, t in enumerate(tokens):
        got = np.full(m.V, np.nan, np.float32)
        ref = np.zeros(m.V, np.float32)
        m.drop_in(lib, t, pos, kc, vc, kl, got)
        orc.gptoss_forward(st, t, pos, rk, rv, rl, ref)
        assert np.array_equal(kl, rl) and np.all(kl == pos + 1), K.last_error(lib)
        assert close(got, ref), (pos, np.max(np.abs(got - ref)), np.max(np.abs(ref)), K.last_error(lib))
        for l in range(m.L):
            assert close(kc[l, pos], rk[l, pos]) and close(vc[l, pos], rv[l, pos]), (pos, l)
    assert np.all(kc[:, len(tokens):] == 0)


def test_gptoss_forward_prefilled_and_rewritten_caches(lib, orc):
    """A caller that filled rows itself (the mirror uploads them), restarts at
    kv_len 0, or rewrites rows it had (sampled rows differ: uploaded again)."""
    m = ToyGptOss(2)
    st = m.oracle_struct()
    rng = np.random.default_rng(9)
    kc, vc, kl = m.new_cache()
    kc[:, :3] = rng.standard_normal(kc[:, :3].shape)
    vc[:, :3] = rng.standard_normal(vc[:, :3].shape)
    kl[:] = 3
    rk, rv, rl = kc.copy(), vc.copy(), kl.copy()

    def step(t, pos):
        got = np.zeros(m.V, np.float32)
        ref = np.zeros(m.V, np.float32)
        m.drop_in(lib, t, pos, kc, vc, kl, got)
        orc.gptoss_forward(st, t, pos, rk, rv, rl, ref)
        assert np.array_equal(kl, rl), K.last_error(lib)
        assert close(got, ref), (pos, np.max(np.abs(got - ref)), np.max(np.abs(ref)))

    step(7, 3)
    step(8, 4)
    kc[:, :2] = rng.standard_normal(kc[:, :2].shape)      # the caller rewrites rows it already had
    rk[:, :2] = kc[:, :2]
    step(9, 5)
    kl[:] = 0                                              # a new sequence in the same buffers
    rl[:] = 0
    step(11, 0)
    step(12, 1)


def test_gptoss_forward_refuses_a_full_cache(lib):
    m = ToyGptOss(3, max_ctx=4)
    kc, vc, kl = m.new_cache()
    kl[:] = 4
    out = np.full(m.V, 7.0, np.float32)
    m.drop_in(lib, 1, 4, kc, vc, kl, out)
    assert np.all(out == 7.0) and np.all(kl == 4) and "max_ctx" in K.last_error(lib)


def test_gptoss_device_step_matches_drop_in(lib):
    """mllm_gptoss_step on device buffers (no host synchronisation inside)
    gives the drop-in's logits bit for bit: the same kernels in the same order."""
    import torch
    m = ToyGptOss(4)
    kc, vc, kl = m.new_cache()
    ref = np.zeros(m.V, np.float32)
    m.drop_in(lib, 3, 0, kc, vc, kl, ref)
    p = m.p
    d = K.GptOssDesc(L=m.L, N=m.N, NH=m.NH, NKH=m.NKH, HD=m.HD, E=m.E, K=m.K, M=m.M, max_ctx=m.max_ctx,
                     rope_dim=m.rope_dim, outNR=m.V, eps=m.eps, wQ=p["wQ"], wK=p["wK"], wV=p["wV"], wO=p["wO"],
                     wAN=p["wAN"], wFN=p["wFN"], wOut=m.wout.ctypes.data_as(K.cu), w_gate_inp=p["gin"],
                     w_gate_exps=p["ge"], w_up_exps=p["ue"], w_down_exps=p["de"], qt_gate=39, qt_up=39, qt_down=39,
                     cos_t=fp(m.cos_t), sin_t=fp(m.sin_t))
    h = lib.mllm_gptoss_create(ctypes.byref(d))
    assert h, K.last_error(lib)
    try:
        n = lib.mllm_gptoss_kv_floats(h)
        kd = torch.zeros(n, device="cuda")
        vd = torch.zeros(n, device="cuda")
        lens = torch.zeros(m.L, dtype=torch.int32, device="cuda")
        pos = torch.zeros(1, dtype=torch.int32, device="cuda")
        x = torch.from_numpy(m.emb[3]).cuda()
        logits = torch.empty(m.V, device="cuda")
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        assert lib.mllm_gptoss_step(h, x.data_ptr(), pos.data_ptr(), lens.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                    logits.data_ptr(), s) == 0
        assert np.array_equal(logits.cpu().numpy(), ref)
        assert np.all(lens.cpu().numpy() == 1)
    finally:
        lib.mllm_gptoss_release(h)


def test_gptoss_forward_real_layer_shapes(lib, orc):
    """gpt-oss-20b layer shapes (N 2880, 64 query / 8 KV heads of 64, 32
    experts of 2880, top-4, full RoPE), two layers, three tokens."""
    m = ToyGptOss(5, L=2, N=2880, NH=64, NKH=8, HD=64, E=32, Kk=4, M=2880, V=256, max_ctx=8, rope_dim=64)
    st = m.oracle_struct()
    kc, vc, kl = m.new_cache()
    rk, rv, rl = m.new_cache()
    for pos, t in enumerate([3, 200, 3]):
        got = np.zeros(m.V, np.float32)
        ref = np.zeros(m.V, np.float32)
        m.drop_in(lib, t, pos, kc, vc, kl, got)
        orc.gptoss_forward(st, t, pos, rk, rv, rl, ref)
        assert np.array_equal(kl, rl), K.last_error(lib)
        assert close(got, ref), (pos, np.max(np.abs(got - ref)), np.max(np.abs(ref)))
