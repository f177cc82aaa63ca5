"""ctypes bindings for the test oracle.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py import this module, and only as the checker.

Two libraries:
  * ``Oracle``   — liboracle.so, our scalar C restatement (oracle.c).
  * ``RefLib``   — _ref/libref.so, the reference's own C compiled in place
                   from /root/reference by oracle/Makefile (absent when the
                   reference tree is absent and nothing was built).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")

# Semantic ids (enum orc_sem in oracle.h; the GPU library uses the same numbers).
F32, Q4_0, Q4_1, Q5_0_F32, Q5_0_Q8, Q8_0, Q4_K_GGML, Q4_K_Q8 = range(8)
Q5_K_GGML, Q5_K_CE, Q6_K_GGML, Q6_K_LOWNIB, Q6_K_SEQ, MXFP4, MXFP4_CLAMP, MXFP4_Q8 = range(8, 16)
SEM_NAMES = ["F32", "Q4_0", "Q4_1", "Q5_0_F32", "Q5_0_Q8", "Q8_0", "Q4_K_GGML", "Q4_K_Q8",
             "Q5_K_GGML", "Q5_K_CE", "Q6_K_GGML", "Q6_K_LOWNIB", "Q6_K_SEQ", "MXFP4",
             "MXFP4_CLAMP", "MXFP4_Q8"]

_cf = ctypes.POINTER(ctypes.c_float)
_cu = ctypes.POINTER(ctypes.c_uint8)
_ci = ctypes.c_int


def fp(a):
    return a.ctypes.data_as(_cf)


def up(a):
    return a.ctypes.data_as(_cu)


def ip(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int))


def build():
    """Compile liboracle.so (and _ref/libref.so where the reference is present)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


ATTN_CE, ATTN_GQA_C = 0, 1


class GptOss(ctypes.Structure):
    """orc_gptoss (oracle.h): the weights and shapes orc_gptoss_forward reads."""
    _pp = ctypes.POINTER(ctypes.POINTER(ctypes.c_uint8))
    _pf = ctypes.POINTER(ctypes.POINTER(ctypes.c_float))
    _fields_ = [(n, ctypes.c_int) for n in ("L", "N", "NH", "NKH", "HD", "V", "E", "K", "M", "max_ctx", "rope_dim",
                                            "outNR")] + [
        ("eps", ctypes.c_float), ("emb", ctypes.POINTER(ctypes.c_float)),
        ("wQ", _pp), ("wK", _pp), ("wV", _pp), ("wO", _pp), ("wAN", _pf), ("wFN", _pf),
        ("wOut", ctypes.POINTER(ctypes.c_uint8)), ("w_gate_inp", _pf),
        ("w_gate_exps", _pp), ("w_up_exps", _pp), ("w_down_exps", _pp),
        ("qt_gate", ctypes.c_int), ("qt_up", ctypes.c_int), ("qt_down", ctypes.c_int),
        ("cos_t", ctypes.POINTER(ctypes.c_float)), ("sin_t", ctypes.POINTER(ctypes.c_float))]


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            build()
        lib = ctypes.CDLL(path)
        lib.orc_gemv.argtypes = [_ci, _cu, _cf, _cf, _ci, _ci, _ci]
        lib.orc_gemv.restype = None
        lib.orc_dequant_row.argtypes = [_ci, _cu, _cf, _ci]
        lib.orc_dequant_row.restype = _ci
        lib.orc_quantize_row_q8_0.argtypes = [_cf, _cu, _ci]
        lib.orc_quantize_row_q8_0.restype = _ci
        lib.orc_block_elems.argtypes = [_ci]
        lib.orc_block_elems.restype = _ci
        lib.orc_block_bytes.argtypes = [_ci]
        lib.orc_block_bytes.restype = _ci
        lib.orc_sem_for.argtypes = [_ci, _ci]
        lib.orc_sem_for.restype = _ci
        lib.orc_route.argtypes = [_cf, _cf, _ci, _ci, _ci, _ci, _ci, ctypes.POINTER(ctypes.c_int), _cf]
        lib.orc_route.restype = None
        lib.orc_requant_q8_0.argtypes = [_ci, _cu, _ci, _ci, _cu]
        lib.orc_requant_q8_0.restype = _ci
        lib.orc_moe_ffn_stride.argtypes = [_ci, _ci, _ci, _ci]
        lib.orc_moe_ffn_stride.restype = ctypes.c_long
        lib.orc_moe_ffn_token.argtypes = [_cf, _cu, _cu, _cu, _ci, _ci, _ci, _ci, _ci, _ci, _ci, _cf, _cf]
        lib.orc_moe_ffn_token.restype = None
        lib.orc_moe_forward_token.argtypes = [ctypes.POINTER(_cu)] * 3 + [_cf, _ci, _ci, _ci, _ci, _ci,
                                              ctypes.POINTER(ctypes.c_int), _cf, _ci, _ci, _cf]
        lib.orc_moe_forward_token.restype = None
        lib.orc_gqa_decode.argtypes = [_ci, _cf, _cf, _cf, ctypes.c_long, _ci, _ci, _ci, _ci, _cf]
        lib.orc_gqa_decode.restype = None
        lib.orc_exp_ps_simd.argtypes = [ctypes.c_float]
        lib.orc_exp_ps_simd.restype = ctypes.c_float
        lib.orc_rope.argtypes = [_cf, _ci, _ci, _ci, _cf, _cf, _ci]
        lib.orc_rope.restype = None
        lib.orc_gptoss_forward.argtypes = [ctypes.POINTER(GptOss), _ci, _ci, _cf, _cf, ctypes.POINTER(ctypes.c_int), _cf]
        lib.orc_gptoss_forward.restype = None
        lib.orc_f32_to_f16.argtypes = [ctypes.c_float]
        lib.orc_f32_to_f16.restype = ctypes.c_uint16
        lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_f16_to_f32.restype = ctypes.c_float
        self.lib = lib

    def block_elems(self, sem):
        return self.lib.orc_block_elems(sem)

    def block_bytes(self, sem):
        return self.lib.orc_block_bytes(sem)

    def row_bytes(self, sem, n_cols):
        return n_cols // self.block_elems(sem) * self.block_bytes(sem)

    def sem_for(self, entry, qt):
        return self.lib.orc_sem_for(entry, qt)

    def gemv(self, sem, W, x, n_rows, n_cols, B=1):
        W = np.ascontiguousarray(W, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros(B * n_rows, dtype=np.float32)
        self.lib.orc_gemv(sem, up(W), fp(x), fp(out), n_rows, n_cols, B)
        return out.reshape(B, n_rows)

    def dequant(self, sem, W, n_rows, n_cols):
        W = np.ascontiguousarray(W, dtype=np.uint8)
        rb = self.row_bytes(sem, n_cols)
        out = np.zeros((n_rows, n_cols), dtype=np.float32)
        for r in range(n_rows):
            rc = self.lib.orc_dequant_row(sem, up(W[r * rb:(r + 1) * rb]), fp(out[r]), n_cols)
            if rc != 0:
                raise ValueError(f"semantic {SEM_NAMES[sem]} has no fp32 weight")
        return out

    def quantize_q8_0(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        q = np.zeros(x.size // 32 * 34, dtype=np.uint8)
        self.lib.orc_quantize_row_q8_0(fp(x), up(q), x.size)
        return q

    def route(self, router_w, x, K, renorm):
        router_w = np.ascontiguousarray(router_w, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        E, N = router_w.shape
        T = x.size // N
        idx = np.zeros((T, K), dtype=np.int32)
        w = np.zeros((T, K), dtype=np.float32)
        self.lib.orc_route(fp(router_w), fp(x), T, N, E, K, int(renorm), ip(idx), fp(w))
        return idx, w

    def requant_q8_0(self, qt, W, n_rows, n_cols):
        """TE:620-666: a Q4_K / Q6_K matrix, or F16 bit patterns taken as
        integers (TE:643-645), requantised to raw Q8_0 blocks."""
        out = np.zeros(n_rows * (n_cols // 32) * 34, dtype=np.uint8)
        rc = self.lib.orc_requant_q8_0(qt, up(np.ascontiguousarray(W, dtype=np.uint8)), n_rows, n_cols, up(out))
        if rc != 0:
            raise ValueError(f"no requantisation for type {qt}")
        return out

    def gqa_decode(self, mode, q, k, v, seq_len, nh, nkh, hd):
        """Decode attention (ATTN_CE: CE:141-158, ATTN_GQA_C: gqa_attention.c:93) of one
        query [nh*hd] over k, v [>= seq_len][nkh*hd]; returns [nh*hd]."""
        q = np.ascontiguousarray(q, np.float32)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        out = np.zeros(nh * hd, np.float32)
        self.lib.orc_gqa_decode(mode, fp(q), fp(k), fp(v), nkh * hd, seq_len, nh, nkh, hd, fp(out))
        return out

    def exp_ps_simd(self, x):
        return self.lib.orc_exp_ps_simd(float(x))

    def rope(self, buf, nh, hd, pos, cos_t, sin_t, rope_dim):
        """rope_apply (GO:37-51) on a copy of buf [nh*hd]."""
        b = np.array(buf, np.float32, copy=True)
        self.lib.orc_rope(fp(b), nh, hd, pos, fp(np.ascontiguousarray(cos_t, np.float32)),
                          fp(np.ascontiguousarray(sin_t, np.float32)), rope_dim)
        return b

    def gptoss_forward(self, model, token, pos, k_cache, v_cache, kv_len, logits):
        """orc_gptoss_forward on a GptOss struct; caches, kv_len and logits updated in place."""
        self.lib.orc_gptoss_forward(ctypes.byref(model), token, pos, fp(k_cache), fp(v_cache),
                                    kv_len.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), fp(logits))

    def moe_ffn_stride(self, which, qt, N, M):
        return self.lib.orc_moe_ffn_stride(which, qt, N, M)

    def moe_ffn_token(self, router_w, gate, upw, down, qts, N, E, K, M, x):
        out = np.zeros(N, dtype=np.float32)
        self.lib.orc_moe_ffn_token(fp(np.ascontiguousarray(router_w, dtype=np.float32)), up(gate), up(upw),
                                   up(down), qts[0], qts[1], qts[2], N, E, K, M,
                                   fp(np.ascontiguousarray(x, dtype=np.float32)), fp(out))
        return out

    def moe_forward_token(self, gates, ups, downs, x, n_ff, n_embd, qts, top_idx, top_w, has_q8=True):
        arr = ctypes.POINTER(ctypes.c_uint8) * len(gates)
        g = arr(*[up(a) for a in gates])
        u = arr(*[up(a) for a in ups])
        d = arr(*[up(a) for a in downs])
        out = np.zeros(n_embd, dtype=np.float32)
        ti = np.ascontiguousarray(top_idx, dtype=np.int32)
        tw = np.ascontiguousarray(top_w, dtype=np.float32)
        self.lib.orc_moe_forward_token(g, u, d, fp(np.ascontiguousarray(x, dtype=np.float32)), n_ff, n_embd,
                                       qts[0], qts[1], qts[2], ip(ti), fp(tw), len(ti), int(has_q8), fp(out))
        return out


class RefLib:
    """The reference's own C (combined like combined_engine.so), by its exported names."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        so = ctypes.CDLL(path)
        # Signatures as bound by the reference's caller (TE:251-392) and declared in CE/QK.
        so.quant_matmul_omp.argtypes = [_cu, _cf, _cf, _ci, _ci, _ci]
        so.quant_matmul_omp.restype = None
        for name in ("q4_0_batch_matmul", "q8_0_batch_matmul", "q4_k_batch_matmul",
                     "q6_k_batch_matmul", "q5_k_batch_matmul", "mxfp4_batch_matmul"):
            f = getattr(so, name)
            f.argtypes = [_cu, _cf, _cf, _ci, _ci, _ci]
            f.restype = None
        so.f32_matmul_omp.argtypes = [_cf, _cf, _cf, _ci, _ci]
        so.f32_matmul_omp.restype = None
        so.quantize_row_q8_0.argtypes = [_cf, _cu, _ci]
        so.quantize_row_q8_0.restype = _ci
        for name in ("q4_k_dequantize_row", "q6_k_dequantize_row", "q5_k_dequantize_row",
                     "q8_0_dequantize_row"):
            f = getattr(so, name)
            f.argtypes = [_cu, _cf, _ci]
            f.restype = None
        so.batch_qkv_omp.argtypes = [_cu, _cu, _cu, _cf, _cf, _cf, _cf, _ci, _ci, _ci, _ci, _ci, _ci, _ci]
        so.batch_qkv_omp.restype = None
        so.batch_gate_up_omp.argtypes = [_cu, _cu, _cf, _cf, _cf, _ci, _ci, _ci, _ci, _ci]
        so.batch_gate_up_omp.restype = None
        so.moe_forward_omp.argtypes = [ctypes.POINTER(_cu)] * 3 + [_cf, _ci, _ci, _ci, _ci, _ci,
                                       ctypes.POINTER(ctypes.c_int), _cf, _ci, _cf, _cf, _cu]
        so.moe_forward_omp.restype = None
        so.set_num_threads.argtypes = [_ci]
        so.set_num_threads.restype = None
        so.get_max_threads.argtypes = []
        so.get_max_threads.restype = _ci
        self.so = so

    def quant_matmul(self, W, x, n_rows, n_cols, qt, out=None):
        out = np.zeros(n_rows, dtype=np.float32) if out is None else out
        self.so.quant_matmul_omp(up(W), fp(np.ascontiguousarray(x, dtype=np.float32)), fp(out), n_rows, n_cols, qt)
        return out

    def batch_matmul(self, name, W, x, n_rows, n_cols, B):
        out = np.zeros(B * n_rows, dtype=np.float32)
        getattr(self.so, name)(up(W), fp(np.ascontiguousarray(x, dtype=np.float32)), fp(out), n_rows, n_cols, B)
        return out.reshape(B, n_rows)

    def quantize_q8_0(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        q = np.zeros(x.size // 32 * 34, dtype=np.uint8)
        self.so.quantize_row_q8_0(fp(x), up(q), x.size)
        return q

    def moe_forward(self, gates, ups, downs, x, n_ff, n_embd, qts, top_idx, top_w, with_q8=True):
        arr = ctypes.POINTER(ctypes.c_uint8) * len(gates)
        g = arr(*[up(a) for a in gates])
        u = arr(*[up(a) for a in ups])
        d = arr(*[up(a) for a in downs])
        K = len(top_idx)
        out = np.zeros(n_embd, dtype=np.float32)
        buf = np.zeros(3 * K * n_ff, dtype=np.float32)
        q8 = np.zeros(K * n_ff * 34 // 32 + 64, dtype=np.uint8)
        ti = np.ascontiguousarray(top_idx, dtype=np.int32)
        tw = np.ascontiguousarray(top_w, dtype=np.float32)
        self.so.moe_forward_omp(g, u, d, fp(np.ascontiguousarray(x, dtype=np.float32)), n_ff, n_embd,
                                qts[0], qts[1], qts[2], ip(ti), fp(tw), K, fp(out), fp(buf),
                                up(q8) if with_q8 else ctypes.cast(None, _cu))
        return out


def ref_available():
    return os.path.exists(REF_SO)


def norm_err(got, ref):
    """max|got-ref| / max|ref|: the normalised max error used for every tolerance."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref)) if ref.size else 0.0
    num = np.max(np.abs(got - ref)) if ref.size else 0.0
    if den == 0.0:
        return float(num)
    return float(num / den)


def elem_rel_err(got, ref, floor=1e-3):
    """Per-element relative error max |got-ref| / |ref| over the elements with
    |ref| >= floor * max|ref| (nearer zero a relative error only measures fp32
    summation noise against a vanishing reference)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if not ref.size:
        return 0.0
    big = np.abs(ref) >= floor * np.max(np.abs(ref))
    if not np.any(big):
        return 0.0
    return float(np.max(np.abs(got[big] - ref[big]) / np.abs(ref[big])))
