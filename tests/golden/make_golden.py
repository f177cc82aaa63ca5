"""Write golden vectors for the hot path by running the reference's own C
(oracle/_ref/libref.so, compiled in place from /root/reference by
oracle/Makefile) on small seeded inputs.

Usage:  python tests/golden/make_golden.py [group]   (from the repo root;
        group = gen_requant, gen_nonfinite or gen_q5_down writes that group only)

Outputs (committed): tests/golden/*.npz.  Each file holds the inputs and the
reference's outputs, so the tests need neither the reference tree nor
libref.so.  Large inputs are regenerated from their seed in the test and
checked against a stored CRC first.
"""
import ctypes
import os
import sys
import zlib

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

from oracle import RefLib, fp, up  # noqa: E402
from mojollama_amd import kernels as K  # noqa: E402
from mojollama_amd import workloads as W  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

# entry points of the reference, by (name, GGUF code)
QMM_TYPES = [0, 2, 3, 6, 8, 12, 13, 14, 39]
BMM = [("q4_0", 2), ("q8_0", 8), ("q4_k", 12), ("q6_k", 14), ("q5_k", 13), ("mxfp4", 39)]

# moe_ffn reads these BC fields (offsets from CE:536-589 on x86-64).
BC_SIZE, BC_N, BC_NE, BC_NK, BC_M = 736, 4, 224, 228, 232
BC_ROUTER, BC_GATE, BC_UP, BC_DOWN, BC_QG, BC_QU, BC_QD = 240, 248, 256, 264, 272, 276, 280


def crc(*arrays):
    c = 0
    for a in arrays:
        c = zlib.crc32(np.ascontiguousarray(a).view(np.uint8).tobytes(), c)
    return c


class BCView:
    """A zeroed BC-sized buffer with the moe_ffn fields filled in."""

    def __init__(self, N, E, K, M, router, gate, upw, down, qts):
        self.buf = (ctypes.c_uint64 * (BC_SIZE // 8))()
        base = ctypes.addressof(self.buf)
        self.keep = [router, gate, upw, down]
        self.pr = (ctypes.c_void_p * 1)(router.ctypes.data)
        self.pg = (ctypes.c_void_p * 1)(gate.ctypes.data)
        self.pu = (ctypes.c_void_p * 1)(upw.ctypes.data)
        self.pd = (ctypes.c_void_p * 1)(down.ctypes.data)
        for off, v in ((BC_N, N), (BC_NE, E), (BC_NK, K), (BC_M, M),
                       (BC_QG, qts[0]), (BC_QU, qts[1]), (BC_QD, qts[2])):
            ctypes.c_int.from_address(base + off).value = v
        for off, p in ((BC_ROUTER, self.pr), (BC_GATE, self.pg), (BC_UP, self.pu), (BC_DOWN, self.pd)):
            ctypes.c_void_p.from_address(base + off).value = ctypes.addressof(p)

    def ptr(self):
        return ctypes.byref(self.buf)


def moe_ffn_ref(ref, bc, x, N, M):
    so = ref.so
    so.moe_ffn.argtypes = [ctypes.c_void_p, ctypes.c_int] + [ctypes.POINTER(ctypes.c_float)] * 4 + [ctypes.c_int]
    so.moe_ffn.restype = None
    gate_buf = np.zeros(M, np.float32)
    up_buf = np.zeros(max(M, N), np.float32)
    out = np.zeros(N, np.float32)
    xx = np.ascontiguousarray(x, np.float32).copy()
    so.moe_ffn(bc.ptr(), 0, fp(xx), fp(gate_buf), fp(up_buf), fp(out), 1)
    return out


def expert_tensor(rng, qt, E, rows, cols):
    return np.concatenate([W.gen_weights(rng, qt, rows, cols) for _ in range(E)])


def te_requantize(ref, W, qt, n_rows, n_cols):
    """The reference caller's _requantize_output (TE:620-666) as it runs: each
    row through the reference's own C dequantize_row, then TE's numpy Q8_0
    quantisation, statement for statement."""
    f32 = np.zeros((n_rows, n_cols), dtype=np.float32)
    if qt == 1:
        # TE:643-645 statement for statement (the integer value of each 16-bit pattern)
        raw_u16 = np.frombuffer(W[:n_rows * n_cols * 2], dtype=np.uint16).copy().reshape(n_rows, n_cols)
        f32 = raw_u16.astype(np.float32).view(np.float32)
    else:
        rb = n_cols // 256 * (144 if qt == 12 else 210)
        fn = ref.so.q4_k_dequantize_row if qt == 12 else ref.so.q6_k_dequantize_row
        for r in range(n_rows):
            row = np.ascontiguousarray(W[r * rb:(r + 1) * rb])
            fn(up(row), fp(f32[r]), n_cols)
    n_blocks = n_cols // 32
    blocks = f32.reshape(n_rows, n_blocks, 32)
    amax = np.max(np.abs(blocks), axis=2, keepdims=True)
    amax = np.clip(amax, 1e-10, None)
    d = amax / 127.0
    qs = np.clip(np.round(blocks / d), -127, 127).astype(np.int8)
    d_u16 = d[:, :, 0].astype(np.float16).view(np.uint16)
    q8 = np.zeros((n_rows, n_blocks, 34), dtype=np.uint8)
    q8[:, :, 0] = d_u16 & 0xFF
    q8[:, :, 1] = (d_u16 >> 8) & 0xFF
    q8[:, :, 2:] = qs.view(np.uint8)
    return q8.reshape(-1)


def gen_requant(ref):
    """lm_head requantisation fixtures: Q4_K and Q6_K matrices (one row's
    super-blocks zeroed to exercise the amax floor) and an F16 matrix (random
    16-bit patterns, one row zero) -> Q8_0."""
    for qt, R, C, seed in ((12, 24, 768, 71), (14, 24, 768, 72), (1, 24, 800, 74)):
        rng = np.random.default_rng(seed)
        if qt == 1:
            w = rng.integers(0, 256, size=R * C * 2, dtype=np.uint8)
            rb = 2 * C
        else:
            w = W.gen_weights(rng, qt, R, C)
            rb = C // 256 * (144 if qt == 12 else 210)
        w[3 * rb:4 * rb] = 0          # row 3: all-zero blocks (the amax floor)
        out = te_requantize(ref, w, qt, R, C)
        np.savez_compressed(os.path.join(OUT, f"requant_q8_{qt}.npz"), W=w, out=out, qt=qt, n_rows=R, n_cols=C)


def gen_nonfinite(ref):
    """Non-finite activations: quantize_row_q8_0 with NaN / +-inf at every
    block position (its vmaxps order decides when amax itself turns NaN),
    and moe_forward_omp on tokens holding a NaN or an inf."""
    rng = np.random.default_rng(73)
    x = W.gen_x(rng, 1, 4096)[0].copy()
    for b in range(96):
        x[32 * b + b % 32] = (np.nan, np.inf, -np.inf)[b // 32]
    for b in range(96, 128):
        pos = rng.choice(32, size=int(rng.integers(2, 6)), replace=False)
        x[32 * b + pos] = rng.choice([np.nan, np.inf, -np.inf], size=pos.size)
    np.savez_compressed(os.path.join(OUT, "q8_0_nonfinite.npz"), x=x, q8=ref.quantize_q8_0(x))

    for tag, qts, n_embd, n_ff in (("gptoss", (39, 39, 39), 192, 160), ("qwen", (12, 12, 14), 256, 256)):
        E = 2
        gates = [W.gen_weights(rng, qts[0], n_ff, n_embd) for _ in range(E)]
        ups = [W.gen_weights(rng, qts[1], n_ff, n_embd) for _ in range(E)]
        downs = [W.gen_weights(rng, qts[2], n_embd, n_ff) for _ in range(E)]
        xs, outs = [], []
        for pos, val in ((0, np.nan), (31, np.nan), (n_embd - 1, np.nan), (5, np.inf), (n_embd // 2, -np.inf)):
            xt = W.gen_x(rng, 1, n_embd)[0].copy()
            xt[pos] = val
            xs.append(xt)
            outs.append(ref.moe_forward(gates, ups, downs, xt, n_ff, n_embd, qts, np.array([1, 0], np.int32),
                                        np.array([0.625, 0.375], np.float32)))
        np.savez_compressed(os.path.join(OUT, f"moe_forward_nonfinite_{tag}.npz"), gates=np.stack(gates),
                            ups=np.stack(ups), downs=np.stack(downs), x=np.stack(xs), out=np.stack(outs),
                            top_idx=np.array([1, 0], np.int32), top_w=np.array([0.625, 0.375], np.float32),
                            n_embd=n_embd, n_ff=n_ff, qts=np.array(qts))


def gen_q5_down(ref):
    """moe_forward_omp with a Q5_0 down projection where n_embd != n_ff: the
    reference addresses down row r at r * ((n_embd+31)/32)*22 bytes (QK:2216,
    2230), a stride from n_embd; n_embd < n_ff keeps every row it reads inside
    the n_embd x n_ff matrix (its rows then overlap)."""
    rng = np.random.default_rng(74)
    for tag, qts, n_embd, n_ff in (("q5down", (12, 12, 6), 256, 288), ("q5down_all", (6, 6, 6), 96, 320)):
        E = 3
        gates = [W.gen_weights(rng, qts[0], n_ff, n_embd) for _ in range(E)]
        ups = [W.gen_weights(rng, qts[1], n_ff, n_embd) for _ in range(E)]
        downs = [W.gen_weights(rng, qts[2], n_embd, n_ff) for _ in range(E)]
        x = W.gen_x(rng, 1, n_embd)[0]
        ti = np.array([2, 0, 1], np.int32)
        tw = np.array([0.5, 0.3, 0.2], np.float32)
        out = ref.moe_forward(gates, ups, downs, x, n_ff, n_embd, qts, ti, tw)
        np.savez_compressed(os.path.join(OUT, f"moe_forward_{tag}.npz"), gates=np.stack(gates), ups=np.stack(ups),
                            downs=np.stack(downs), x=x, top_idx=ti, top_w=tw, out=out,
                            n_embd=n_embd, n_ff=n_ff, qts=np.array(qts))


# the ssm_* / qwen36 cases: (tag, seed, B, N, inner, gate_qt, ssm_out_qt); N > inner makes
# ssm_layer_fused's later tokens read intermediates the earlier ones overwrote (CE:829-846)
SSM_CASES = [("a", 91, 3, 256, 256, W.QT_Q8_0, W.QT_Q6_K), ("b", 92, 3, 512, 256, W.QT_Q4_K, W.QT_MXFP4),
             ("c", 93, 2, 256, 384, W.QT_MXFP4, W.QT_Q8_0)]


def gen_qwen36(ref):
    """qwen36_batch_forward (CE:859-1231), ssm_layer_fused and ssm_decode_step
    as the reference's own C computes them.  The inputs are regenerated in the
    test from their seeds (workloads.qwen36_case / ssm_case) and checked by
    CRC; the fixtures hold the outputs: for two consecutive qwen36 calls
    (kv_lens + 1 between them, as TE:1880 does) the logits, SSM state, the KV
    rows written and the fused-QKV workspace slice."""
    K.bind_model_entry_points(ref.so)

    def two_calls(c):
        call = W.Qwen36Call(c)
        res = {}
        for i in range(2):
            res[f"logits{i}"] = call.call(ref.so, c["tokens"][i])
            res[f"state{i}"] = call.state.copy()
            res[f"kv{i}"] = np.stack([call.kv[:, l, call.kv_lens[l]] for l in range(c["L"])])
            res[f"slice{i}"] = call.qkv_slice()
            call.kv_lens += 1
        return res
    rng = np.random.default_rng(94)
    for emb_quant in (0, 12):
        c = W.qwen36_case(0, 2, emb_quant)
        res = two_calls(c)
        # the case must not sit on a discrete edge (a top-K near-tie, a clip): a
        # few ulps of change in any norm weight may move the logits only by
        # fp32-rounding amounts, else another summation order could flip it
        worst = 0.0
        for trial in range(12):
            c2 = dict(c)
            which = ("attn_norm", "ffn_norm", "out_norm")[trial % 3]
            pert = lambda v: np.nextafter(v, v + np.float32(np.inf) * rng.choice([-1, 1], v.shape).astype(np.float32))  # noqa: E731
            c2[which] = [pert(v) for v in c[which]] if which != "out_norm" else pert(c[which])
            r2 = two_calls(c2)
            worst = max(worst, max(float(np.max(np.abs(r2[k] - res[k])) / np.max(np.abs(res[k])))
                                   for k in ("logits0", "logits1")))
        assert worst < 1e-4, f"qwen36 case emb{emb_quant} is ulp-sensitive ({worst:.2e})"
        # the first call again over KV caches whose cached rows all changed: must differ
        call = W.Qwen36Call(c)
        nkv = c["n_kv_h"] * c["HD"]
        for l in range(c["L"]):
            n = c["kv_lens0"][l]
            call.kv[:, l, :n] = rng.standard_normal((2, n, nkv)) * 8.0
        res["kv_mod"] = call.kv.copy()
        res["logits_mod"] = call.call(ref.so, c["tokens"][0])
        moved = float(np.max(np.abs(res["logits_mod"] - res["logits0"])) / np.max(np.abs(res["logits0"])))
        print(f"qwen36 emb{emb_quant}: ulp sensitivity {worst:.2e}, rewritten KV rows move the logits by {moved:.2e}")
        assert moved > 1e-2
        np.savez_compressed(os.path.join(OUT, f"qwen36_emb{emb_quant}.npz"), crc=W.qwen36_arrays_crc(c),
                            ulp_sensitivity=worst, **res)
    for tag, seed, B, N, inner, gq, sq in SSM_CASES:
        c = W.ssm_case(seed, B, N, inner, gate_qt=gq, so_qt=sq)
        out_f, st_f = W.ssm_call(ref.so, c, True)
        out_d, st_d = W.ssm_call(ref.so, c, False)
        np.savez_compressed(os.path.join(OUT, f"ssm_{tag}.npz"), crc=crc(c["x"], c["gate"], c["so"], c["state"]),
                            fused=out_f, fused_state=st_f, step=out_d, step_state=st_d)


def main():
    ref = RefLib()
    ref.so.set_num_threads(1)
    rng = np.random.default_rng(20261201)
    R, C = 16, 512

    # quant_matmul_omp (B=1) for every code it dispatches
    for qt in QMM_TYPES:
        w = W.gen_weights(rng, qt, R, C)
        x = W.gen_x(rng, 1, C)
        out = ref.quant_matmul(w, x, R, C, qt)
        np.savez_compressed(os.path.join(OUT, f"qmm_{qt}.npz"), W=w, x=x, out=out, n_rows=R, n_cols=C)

    # *_batch_matmul with B = 1 and 3, plus a ragged B=5 on 24 rows
    for name, qt in BMM:
        for B, rows in ((1, R), (3, R), (5, 24)):
            w = W.gen_weights(rng, qt, rows, C)
            x = W.gen_x(rng, B, C)
            out = ref.batch_matmul(name + "_batch_matmul", w, x, rows, C, B)
            np.savez_compressed(os.path.join(OUT, f"bmm_{name}_B{B}.npz"), W=w, x=x, out=out,
                                n_rows=rows, n_cols=C, B=B)

    # MXFP4 scale edge cases: E = 0 (zero scale) and 255 (+inf, clamped in CE)
    w = W.gen_weights(rng, 39, R, C).reshape(-1, 17)
    w[::5, 16] = 255
    w[1::7, 16] = 0
    w = np.ascontiguousarray(w.ravel())
    x = W.gen_x(rng, 1, C)
    np.savez_compressed(os.path.join(OUT, "edge_mxfp4.npz"), W=w, x=x, n_rows=R, n_cols=C,
                        out_clamp=ref.batch_matmul("mxfp4_batch_matmul", w, x, R, C, 1),
                        out_noclamp=ref.quant_matmul(w, x, R, C, 39))

    # quantize_row_q8_0, including zero and large blocks
    x = (W.gen_x(rng, 1, 4096)[0] * 3.0).astype(np.float32)
    x[:32] = 0.0
    x[32:64] *= 1e4
    x[64:96] *= 1e-6
    np.savez_compressed(os.path.join(OUT, "q8_0.npz"), x=x, q8=ref.quantize_q8_0(x))

    # *_dequantize_row
    so = ref.so
    for name, qt in (("q4_k", 12), ("q6_k", 14), ("q5_k", 13), ("q8_0", 8)):
        w = W.gen_weights(rng, qt, 1, 1024)
        out = np.zeros(1024, np.float32)
        getattr(so, name + "_dequantize_row")(up(w), fp(out), 1024)
        np.savez_compressed(os.path.join(OUT, f"deq_{name}.npz"), W=w, out=out)

    # batch_qkv_omp with mixed types (Q4_K, Q6_K, Q8_0)
    C2 = 512
    wq, wk, wv = (W.gen_weights(rng, qt, r, C2) for qt, r in ((12, 32), (14, 16), (8, 16)))
    x = W.gen_x(rng, 1, C2)[0]
    oq, ok, ov = np.zeros(32, np.float32), np.zeros(16, np.float32), np.zeros(16, np.float32)
    so.batch_qkv_omp(up(wq), up(wk), up(wv), fp(x), fp(oq), fp(ok), fp(ov), 32, 16, 16, C2, 12, 14, 8)
    np.savez_compressed(os.path.join(OUT, "batch_qkv.npz"), Wq=wq, Wk=wk, Wv=wv, x=x, oq=oq, ok=ok, ov=ov)
    wg, wu = W.gen_weights(rng, 39, 32, C2), W.gen_weights(rng, 2, 32, C2)
    og, ou = np.zeros(32, np.float32), np.zeros(32, np.float32)
    so.batch_gate_up_omp(up(wg), up(wu), fp(x), fp(og), fp(ou), 32, 32, C2, 39, 2)
    np.savez_compressed(os.path.join(OUT, "batch_gate_up.npz"), Wg=wg, Wu=wu, x=x, og=og, ou=ou)

    # moe_forward_omp: Qwen3-like (Q4_K gate/up, Q6_K down) and GPT-OSS-like (MXFP4)
    for tag, (qg, qu, qd), n_embd, n_ff in (("qwen", (12, 12, 14), 256, 256),
                                            ("gptoss", (39, 39, 39), 192, 160)):
        E, K = 3, 3
        gates = [W.gen_weights(rng, qg, n_ff, n_embd) for _ in range(E)]
        ups = [W.gen_weights(rng, qu, n_ff, n_embd) for _ in range(E)]
        downs = [W.gen_weights(rng, qd, n_embd, n_ff) for _ in range(E)]
        x = W.gen_x(rng, 1, n_embd)[0]
        ti = np.array([2, 0, 1], np.int32)
        tw = np.array([0.5, 0.3, 0.2], np.float32)
        out = ref.moe_forward(gates, ups, downs, x, n_ff, n_embd, (qg, qu, qd), ti, tw)
        np.savez_compressed(os.path.join(OUT, f"moe_forward_{tag}.npz"), gates=np.stack(gates), ups=np.stack(ups),
                            downs=np.stack(downs), x=x, top_idx=ti, top_w=tw, out=out,
                            n_embd=n_embd, n_ff=n_ff, qts=np.array([qg, qu, qd]))

    # moe_ffn (C routing, no renorm) on small experts, two quant mixes
    for tag, qts, N, M in (("q4k", (12, 12, 14), 256, 256), ("mxfp4", (39, 39, 39), 128, 96)):
        E, K = 4, 2
        router = W.gen_router(rng, E, N)
        gate = expert_tensor(rng, qts[0], E, M, N)
        upw = expert_tensor(rng, qts[1], E, M, N)
        down = expert_tensor(rng, qts[2], E, N, M)
        xs = W.gen_x(rng, 4, N)
        bc = BCView(N, E, K, M, router, gate, upw, down, qts)
        outs = np.stack([moe_ffn_ref(ref, bc, xs[t], N, M) for t in range(4)])
        np.savez_compressed(os.path.join(OUT, f"moe_ffn_{tag}.npz"), router=router, gate=gate, up=upw, down=down,
                            x=xs, out=outs, N=N, E=E, K=K, M=M, qts=np.array(qts))

    # Routing at the real router shapes.  All experts share one gate = up
    # tensor with tiny scales (so h = silu(g)*g = g^2*sigmoid(g) > 0), and
    # expert e's down projection is zero except row e, whose Q6_K codes are
    # all +31 with scale +1.  moe_ffn's output is then p_e * D (D > 0, the
    # same for every expert) at each selected e and 0 elsewhere: it pins the
    # selected set bit-exactly and the routing weights up to the factor D.
    for tag, N, E, K, T, seed in (("gptoss", 2880, 32, 4, 48, 11), ("qwen3", 2048, 128, 8, 48, 12)):
        r2 = np.random.default_rng(seed)
        router = W.gen_router(r2, E, N)
        xs = W.gen_x(r2, T, N)
        M = 256
        g1 = W.gen_weights(r2, 12, M, N).reshape(-1, 144)
        g1[:, 0:4] = np.array([1e-6, 1e-6], np.float16).view(np.uint8)      # d, dmin
        g1 = np.ascontiguousarray(g1.ravel())
        gate = np.concatenate([g1] * E)
        blk = np.zeros(210, np.uint8)
        blk[0:128] = 0xFF                                                    # ql: nibble 15
        blk[128:192] = 0xFF                                                  # qh: 3 in every slot
        blk[192:208] = 1                                                     # int8 scales +1
        blk[208:210] = np.array([1.0], np.float16).view(np.uint8)            # d = 1
        down = np.zeros((E, N, (M // 256) * 210), np.uint8)
        for e in range(E):
            down[e, e, :] = blk
        down = np.ascontiguousarray(down.ravel())
        bc = BCView(N, E, K, M, router, gate, gate, down, (12, 12, 14))
        ffn = np.zeros((T, E), np.float32)
        for t in range(T):
            ffn[t] = moe_ffn_ref(ref, bc, xs[t], N, M)[:E]
        sel = (ffn != 0).astype(np.uint8)
        assert np.all(sel.sum(1) == K)
        np.savez_compressed(os.path.join(OUT, f"route_sel_{tag}.npz"), seed=seed, N=N, E=E, K=K, T=T, M=M,
                            crc=crc(router, xs), sel=sel, ffn=ffn)
    gen_requant(ref)
    gen_nonfinite(ref)
    gen_q5_down(ref)
    gen_qwen36(ref)
    print("golden vectors written to", OUT)


if __name__ == "__main__":
    if len(sys.argv) > 1:
        # one group only, e.g. `make_golden.py gen_nonfinite`
        _ref = RefLib()
        _ref.so.set_num_threads(1)
        globals()[sys.argv[1]](_ref)
    else:
        main()
