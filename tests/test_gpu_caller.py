"""Replays the reference's Python caller of the MoE FFN against the HIP
library: TurboEngine._forward_moe (TE:2031-2085) as it drives
combined_engine.so, with the buffers TurboEngine allocates for it
(TE:945-960) and the per-expert pointer arrays it builds at load
(TE:851-900), through the ctypes argtypes it binds (TE:273-311).

Per layer and token the caller
  1. computes router logits, either through quant_matmul_omp on the raw
     router tensor (TE:2039-2042, F32 code 0 here) or in numpy
     (TE:2043-2045);
  2. takes softmax, argpartition top-k and renormalises in numpy
     (TE:2047-2055);
  3. clears _moe_combined and calls moe_forward_omp with the full expert
     pointer arrays, its prealloc buffers and the int32/float32 index and
     weight arrays (TE:2062-2076);
  4. copies the result out and zeroes NaNs when combined[0] is NaN
     (TE:2078-2085).
The library's result is checked against the oracle's moe_forward_omp
restatement on the same routing (MOE_TOL, MOE_Q8H_TOL with an MXFP4 down
projection), the routing set against the oracle's fp32 router logits, and
the NaN guard's outcome against the same guard applied to the oracle.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from helpers import moe_tol
from mojollama_amd import kernels as K
from mojollama_amd import workloads as W

pytestmark = pytest.mark.gpu

cu = ctypes.POINTER(ctypes.c_uint8)
cf = ctypes.POINTER(ctypes.c_float)


@pytest.fixture(scope="module")
def kern():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return K.load_kernels()


class ExpertPointers:
    """One MoE layer as TurboEngine holds it (TE:851-900): the router as a
    raw tensor (code 0) or an fp32 matrix, and per expert tensor one raw
    buffer with an n_experts pointer array into it."""

    def __init__(self, rng, qts, n_embd, n_ff, n_experts, router_raw):
        self.n_experts, self.n_ff_expert, self.n_embd = n_experts, n_ff, n_embd
        self.gate_qt, self.up_qt, self.down_qt = (ctypes.c_int(q) for q in qts)
        self.qts = qts
        router = (rng.standard_normal((n_experts, n_embd)) * 0.02).astype(np.float32)
        self.router_f32 = None if router_raw else router
        self._router_host = router
        if router_raw:
            self._router_bytes = np.ascontiguousarray(router).view(np.uint8).ravel()
            self.router_raw = self._router_bytes.ctypes.data_as(cu)
            self.router_nr, self.router_nc, self.router_qt = (ctypes.c_int(v) for v in (n_experts, n_embd, 0))
        else:
            self.router_raw = None
        self.raw = {}
        for attr, qt, rows, cols in (("gate", qts[0], n_ff, n_embd), ("up", qts[1], n_ff, n_embd),
                                     ("down", qts[2], n_embd, n_ff)):
            raw = W.gen_weights(rng, qt, n_experts * rows, cols)
            expert_bytes = raw.size // n_experts
            base = ctypes.addressof(raw.ctypes.data_as(cu).contents)
            arr = (cu * n_experts)(*[ctypes.cast(base + e * expert_bytes, cu) for e in range(n_experts)])
            self.raw[attr] = [raw[e * expert_bytes:(e + 1) * expert_bytes] for e in range(n_experts)]
            setattr(self, f"{attr}_ptrs_arr", arr)
            setattr(self, f"_{attr}_buf", raw)


class MoECaller:
    """TurboEngine's MoE buffers (TE:945-960) and _forward_moe (TE:2031-2085)."""

    def __init__(self, kern, n_embd, n_ff, n_experts, top_k):
        self._kern = kern
        self.n_experts_per_tok = top_k
        self._moe_router_scores = np.zeros(max(128, n_experts), dtype=np.float32)
        self._moe_combined = np.zeros(n_embd, dtype=np.float32)
        max_top_k = max(8, top_k)
        self._moe_prealloc_buf = np.zeros(3 * max_top_k * n_ff, dtype=np.float32)
        self._moe_prealloc_q8 = np.zeros(top_k * n_ff * 34 // 32, dtype=np.uint8)
        self._x_norm = np.zeros(n_embd, dtype=np.float32)
        self._p_moe_router = self._moe_router_scores.ctypes.data_as(cf)
        self._p_moe_combined = self._moe_combined.ctypes.data_as(cf)
        self.last_routing = None

    def forward_moe(self, me, x_norm, b_ffn_out, N):
        np.copyto(self._x_norm, x_norm)
        p_xn = self._x_norm.ctypes.data_as(cf)
        n_exp, top_k, FF, kern = me.n_experts, self.n_experts_per_tok, me.n_ff_expert, self._kern
        if me.router_raw is not None:
            kern.quant_matmul_omp(me.router_raw, p_xn, self._p_moe_router, me.router_nr, me.router_nc, me.router_qt)
        else:
            np.copyto(self._moe_router_scores[:n_exp], (me.router_f32 @ self._x_norm)[:n_exp])
        scores = self._moe_router_scores[:n_exp]
        self.last_logits = scores.copy()
        with np.errstate(invalid="ignore"):
            scores -= np.max(scores)
            np.exp(scores, out=scores)
            scores /= np.sum(scores)
            top_indices = np.argpartition(scores, -top_k)[-top_k:]
            top_weights = scores[top_indices]
            top_weights /= np.sum(top_weights)
        top_idx_arr = np.ascontiguousarray(top_indices.astype(np.int32))
        top_wt_arr = np.ascontiguousarray(top_weights.astype(np.float32))
        self.last_routing = (top_idx_arr.copy(), top_wt_arr.copy())
        self._moe_combined[:] = 0.0
        kern.moe_forward_omp(
            me.gate_ptrs_arr, me.up_ptrs_arr, me.down_ptrs_arr, p_xn,
            ctypes.c_int(FF), ctypes.c_int(N), me.gate_qt, me.up_qt, me.down_qt,
            top_idx_arr.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
            top_wt_arr.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
            ctypes.c_int(top_k), self._p_moe_combined,
            self._moe_prealloc_buf.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
            self._moe_prealloc_q8.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)))
        b_ffn_out[:N] = self._moe_combined[:N]
        nan_guard(self._moe_combined, b_ffn_out, N)


def nan_guard(combined, out, N):
    """TE:2080-2085: zero NaN outputs when combined[0] is NaN."""
    if np.isnan(combined[0]):
        mask = np.isnan(out[:N])
        if np.any(mask):
            out[:N][mask] = 0.0


def expected(orc, me, x, routing, N):
    ti, tw = routing
    ref = orc.moe_forward_token(me.raw["gate"], me.raw["up"], me.raw["down"], x, me.n_ff_expert, N, me.qts, ti, tw)
    out = ref.copy()
    nan_guard(ref, out, N)
    return out


def check_routing(orc, me, x, logits, routing, top_k):
    """The caller's logits agree with the oracle's fp32 router GEMV, and its
    top-k set is the top-k of those logits (a swap only across a gap below
    the logits' own rounding)."""
    ref = orc.gemv(O.F32, np.ascontiguousarray(me._router_host).view(np.uint8).ravel(), x, me.n_experts,
                   me.n_embd, 1)[0]
    assert np.max(np.abs(logits - ref)) <= 1e-5 * max(1.0, np.max(np.abs(ref)))
    want = set(np.argsort(-ref, kind="stable")[:top_k].tolist())
    got = set(routing[0].tolist())
    if got != want:
        kth = np.sort(ref)[-top_k]
        assert all(abs(ref[e] - kth) < 1e-5 for e in got ^ want), (got, want)


@pytest.mark.parametrize("tag,qts,N,M,E,k,router_raw", [
    ("gptoss", (39, 39, 39), 2880, 2880, 32, 4, True),
    ("qwen3", (12, 12, 14), 2048, 768, 128, 8, False),
])
def test_forward_moe_replay(kern, orc, tag, qts, N, M, E, k, router_raw):
    rng = np.random.default_rng(4100 + E)
    layers = [ExpertPointers(rng, qts, N, M, E, router_raw) for _ in range(2)]
    caller = MoECaller(kern, N, M, E, k)
    xs = W.gen_x(rng, 3, N)
    b_ffn_out = np.full(N + 64, -7.0, np.float32)        # TE's per-token output view is wider than N
    for t in range(3):
        for li, me in enumerate(layers):
            caller.forward_moe(me, xs[t], b_ffn_out, N)
            assert np.all(b_ffn_out[N:] == -7.0), "moe output wrote past N"
            check_routing(orc, me, xs[t], caller.last_logits, caller.last_routing, k)
            ref = expected(orc, me, xs[t], caller.last_routing, N)
            assert np.all(np.isfinite(b_ffn_out[:N]))
            assert O.norm_err(b_ffn_out[:N], ref) < moe_tol(qts), (tag, t, li, K.last_error(kern))
            # the library keeps no state between calls beyond its weight cache:
            # the scratch buffers the caller passes are not read back
            assert caller._moe_prealloc_q8.size == k * M * 34 // 32


@pytest.mark.parametrize("tag,qts,N,M,E,k,router_raw", [
    ("gptoss", (39, 39, 39), 2880, 2880, 32, 4, True),
    ("qwen3", (12, 12, 14), 2048, 768, 128, 8, False),
])
@pytest.mark.parametrize("bad", [np.nan, np.inf])
def test_forward_moe_replay_nan_guard(kern, orc, tag, qts, N, M, E, k, router_raw, bad):
    """A non-finite token: the router's softmax gives NaN weights, the layer
    NaN outputs, and TE's guard zeroes them; the next token is unaffected."""
    rng = np.random.default_rng(4200 + E)
    me = ExpertPointers(rng, qts, N, M, E, router_raw)
    caller = MoECaller(kern, N, M, E, k)
    xs = W.gen_x(rng, 2, N).copy()
    xs[0, N // 3] = bad
    b_ffn_out = np.full(N, -7.0, np.float32)
    caller.forward_moe(me, xs[0], b_ffn_out, N)
    ref = expected(orc, me, xs[0], caller.last_routing, N)
    assert np.array_equal(np.isnan(b_ffn_out), np.isnan(ref))
    fin = np.isfinite(ref)
    assert np.array_equal(b_ffn_out[~fin], ref[~fin])
    if np.all(ref[fin] == 0.0):
        assert np.all(b_ffn_out[fin] == 0.0)
    else:
        assert O.norm_err(b_ffn_out[fin], ref[fin]) < moe_tol(qts)
    caller.forward_moe(me, xs[1], b_ffn_out, N)
    ref = expected(orc, me, xs[1], caller.last_routing, N)
    assert O.norm_err(b_ffn_out, ref) < moe_tol(qts)
