"""Seeded synthetic weights and activations with the distributions and
shapes of the benchmark configurations (raw GGUF block bytes, as the
reference's caller hands them over: TE:459-480).

Distributions:
  * fp16 block scales d / dmin: |N(0,1)| * 0.01, rounded to fp16 (RNE)
  * Q8_0 quants: int8 uniform in [-127, 127]
  * Q4_K / Q5_K / Q4_0 / Q4_1 / Q5_0 packed fields: uniform random bytes
    (iid uniform 6-bit scales/mins and 4-bit quants)
  * Q6_K: uniform ql/qh bytes, int8 sub-scales uniform in [-32, 31]
  * MXFP4: uniform nibble bytes, E8M0 exponent 127 + U{-8..0}
  * fp32 routers N(0, 0.02^2); activations N(0, 1)
"""
import ctypes

import numpy as np

QT_F32, QT_Q4_0, QT_Q4_1, QT_Q5_0, QT_Q8_0 = 0, 2, 3, 6, 8
QT_Q4_K, QT_Q5_K, QT_Q6_K, QT_MXFP4 = 12, 13, 14, 39

# GGUF code -> (elements per block, bytes per block)   (QK:26-37, TE:24-25)
BLOCK = {QT_F32: (1, 4), QT_Q4_0: (32, 18), QT_Q4_1: (32, 20), QT_Q5_0: (32, 22),
         QT_Q8_0: (32, 34), QT_Q4_K: (256, 144), QT_Q5_K: (256, 176), QT_Q6_K: (256, 210),
         QT_MXFP4: (32, 17)}


def row_bytes(qt, n_cols):
    be, bb = BLOCK[qt]
    return n_cols // be * bb


def _f16_scales(rng, n):
    return (np.abs(rng.standard_normal(n)) * 0.01).astype(np.float16).view(np.uint8).reshape(n, 2)


def gen_weights(rng, qt, n_rows, n_cols):
    """Raw GGUF-order bytes for an n_rows x n_cols matrix of type qt."""
    if qt == QT_F32:
        return (rng.standard_normal((n_rows, n_cols)) * 0.02).astype(np.float32).view(np.uint8).ravel()
    be, bb = BLOCK[qt]
    nb = n_rows * (n_cols // be)
    blk = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    if qt == QT_Q8_0:
        blk[:, 0:2] = _f16_scales(rng, nb)
        blk[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    elif qt in (QT_Q4_0, QT_Q5_0):
        blk[:, 0:2] = _f16_scales(rng, nb)
    elif qt in (QT_Q4_1, QT_Q4_K, QT_Q5_K):
        blk[:, 0:2] = _f16_scales(rng, nb)
        blk[:, 2:4] = _f16_scales(rng, nb)
    elif qt == QT_Q6_K:
        blk[:, 192:208] = rng.integers(-32, 32, size=(nb, 16), dtype=np.int8).view(np.uint8)
        blk[:, 208:210] = _f16_scales(rng, nb)
    elif qt == QT_MXFP4:
        blk[:, 16] = (127 + rng.integers(-8, 1, size=nb)).astype(np.uint8)
    return np.ascontiguousarray(blk.ravel())


def gen_q4k_centered(rng, n_rows, n_cols):
    """Q4_K blocks whose weights have mean ~0: sub-block scales sc in [0, 8],
    mins m = round(7.5 sc) and dmin = d, so w = d sc (q - 7.5) up to the
    rounding of m.  BASELINE's uniform [0, 63] scales and mins give every row a
    positive mean, which makes a chain of such matrices saturate (every gate of
    a SiLU product far below zero after one layer); a parity test of a chain
    uses these instead.  The scale/min pairs are packed as get_scale_min_k4
    reads them (QK:62-71)."""
    nb = n_rows * (n_cols // 256)
    blk = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    blk[:, 0:2] = _f16_scales(rng, nb)
    blk[:, 2:4] = blk[:, 0:2]
    sc = rng.integers(0, 9, size=(nb, 8)).astype(np.uint8)
    m = np.rint(7.5 * sc).astype(np.uint8)
    q = np.zeros((nb, 12), np.uint8)
    q[:, 0:4] = sc[:, 0:4] | ((sc[:, 4:8] >> 4) << 6)
    q[:, 4:8] = m[:, 0:4] | ((m[:, 4:8] >> 4) << 6)
    q[:, 8:12] = (sc[:, 4:8] & 15) | ((m[:, 4:8] & 15) << 4)
    blk[:, 4:16] = q
    return np.ascontiguousarray(blk.ravel())


def gen_x(rng, B, n_cols, bf16=False):
    """fp32 activations ~ N(0,1); bf16=True rounds them to bf16 (RNE) and back."""
    x = rng.standard_normal((B, n_cols)).astype(np.float32)
    if bf16:
        u = x.view(np.uint32).astype(np.uint64)
        u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
        x = u.astype(np.uint32).view(np.float32)
    return np.ascontiguousarray(x)


def gen_router(rng, E, N):
    return (rng.standard_normal((E, N)) * 0.02).astype(np.float32)


# ---------------------------------------------------------- configurations

# TinyLlama-1.1B Q4_K_M matmul set (per layer) + lm_head.
TINYLLAMA_LAYERS = 22
TINYLLAMA_MATS = [  # name, rows, cols, qt
    ("q", 2048, 2048, QT_Q4_K), ("k", 256, 2048, QT_Q4_K), ("v", 256, 2048, QT_Q4_K),
    ("o", 2048, 2048, QT_Q4_K), ("gate", 5632, 2048, QT_Q4_K), ("up", 5632, 2048, QT_Q4_K),
    ("down", 2048, 5632, QT_Q6_K)]
TINYLLAMA_LM_HEAD = ("lm_head", 32000, 2048, QT_Q6_K)

# MoE layer shapes.
GPTOSS = dict(N=2880, E=32, K=4, M=2880, qt_gate=QT_MXFP4, qt_up=QT_MXFP4, qt_down=QT_MXFP4)
QWEN3 = dict(N=2048, E=128, K=8, M=768, qt_gate=QT_Q4_K, qt_up=QT_Q4_K, qt_down=QT_Q6_K)


def skewed_tokens(rng, router_w, T, n_hot=8, frac=0.25):
    """Hidden states for the Qwen3 skewed-routing case: a seeded unit direction
    u is added (x0.5) to the router rows of n_hot seeded experts, and (x16) to
    a seeded `frac` of the tokens, which pushes those tokens onto the hot set.
    Returns (x [T,N], router_w_skewed [E,N], hot_experts, hot_tokens)."""
    E, N = router_w.shape
    u = rng.standard_normal(N).astype(np.float32)
    u /= np.linalg.norm(u)
    hot = np.sort(rng.choice(E, size=n_hot, replace=False))
    rw = router_w.copy()
    rw[hot] += 0.5 * u
    x = rng.standard_normal((T, N)).astype(np.float32)
    hot_tok = np.sort(rng.choice(T, size=int(T * frac), replace=False))
    x[hot_tok] += 16.0 * u
    return np.ascontiguousarray(x), np.ascontiguousarray(rw), hot, hot_tok


def gen_weights_torch(gen, qt, n_rows, n_cols, device="cuda"):
    """gen_weights' distributions drawn on the GPU with a torch Generator (for
    the large benchmark tensors; the parity tests use the numpy generator)."""
    import torch
    be, bb = BLOCK[qt]
    nb = n_rows * (n_cols // be)
    blk = torch.randint(0, 256, (nb, bb), dtype=torch.uint8, device=device, generator=gen)

    def f16_scales(n):
        return (torch.randn(n, device=device, generator=gen).abs() * 0.01).half().view(torch.uint8).view(n, 2)
    if qt == QT_Q8_0:
        blk[:, 0:2] = f16_scales(nb)
        blk[:, 2:] = torch.randint(-127, 128, (nb, 32), dtype=torch.int8, device=device, generator=gen).view(torch.uint8)
    elif qt in (QT_Q4_0, QT_Q5_0):
        blk[:, 0:2] = f16_scales(nb)
    elif qt in (QT_Q4_1, QT_Q4_K, QT_Q5_K):
        blk[:, 0:2] = f16_scales(nb)
        blk[:, 2:4] = f16_scales(nb)
    elif qt == QT_Q6_K:
        blk[:, 192:208] = torch.randint(-32, 32, (nb, 16), dtype=torch.int8, device=device, generator=gen).view(torch.uint8)
        blk[:, 208:210] = f16_scales(nb)
    elif qt == QT_MXFP4:
        blk[:, 16] = (127 + torch.randint(-8, 1, (nb,), device=device, generator=gen)).to(torch.uint8)
    return blk.reshape(-1)


def moe_workload(tag, T=1280, device="cuda"):
    """The configs[3] ("gptoss") / configs[4] ("qwen3") MoE workload exactly as
    bench.py times it: per-expert raw GGUF weights drawn on the GPU with a
    seeded torch Generator (GPT-OSS: one fused 5760-row gate/up tensor per
    expert, gate = rows [0, M), up = rows [M, 2M), as the reference's caller
    addresses it, TE:868-905), the fp32 router [E][N] and T tokens of hidden
    states from numpy (Qwen3: the skewed case of `skewed_tokens`).
    Returns a dict: cfg, qts, gates/ups/downs (lists of uint8 device tensors),
    router (numpy [E][N]), x (numpy [T][N]), hot_experts, hot_tokens."""
    import torch
    c = dict(GPTOSS) if tag == "gptoss" else dict(QWEN3)
    N, E, M = c["N"], c["E"], c["M"]
    qts = (c["qt_gate"], c["qt_up"], c["qt_down"])
    gen = torch.Generator(device=device)
    gen.manual_seed(4 if tag == "gptoss" else 5)
    if tag == "gptoss":
        rb = row_bytes(qts[0], N)
        fused = [gen_weights_torch(gen, qts[0], 2 * M, N, device) for _ in range(E)]
        gates = [f[:M * rb] for f in fused]
        ups = [f[M * rb:] for f in fused]
    else:
        gates = [gen_weights_torch(gen, qts[0], M, N, device) for _ in range(E)]
        ups = [gen_weights_torch(gen, qts[1], M, N, device) for _ in range(E)]
    downs = [gen_weights_torch(gen, qts[2], N, M, device) for _ in range(E)]
    rng = np.random.default_rng(7)
    router = gen_router(rng, E, N)
    hot, hot_tok = np.zeros(0, np.int64), np.zeros(0, np.int64)
    if tag == "qwen3":
        x, router, hot, hot_tok = skewed_tokens(rng, router, T)
    else:
        x = gen_x(rng, T, N)
    return dict(cfg=c, qts=qts, gates=gates, ups=ups, downs=downs, router=router, x=x, hot_experts=hot,
                hot_tokens=hot_tok)


# moe_ffn reads these BC fields (x86-64 offsets of the engine's struct, CE:536-589).
BC_SIZE, BC_N, BC_NE, BC_NK, BC_M = 736, 4, 224, 228, 232
BC_ROUTER, BC_GATE, BC_UP, BC_DOWN, BC_QG, BC_QU, BC_QD = 240, 248, 256, 264, 272, 276, 280


class BCView:
    """A zeroed BC-sized buffer with the moe_ffn fields of layer 0 filled in."""

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
        return ctypes.addressof(self.buf)


# ------------------------------------------------- qwen36_batch_forward case
def rope_tables(max_ctx, hd, rope_dim):
    """cos/sin tables as rope_init builds them (CE:674-685): [max_ctx][rope_dim/2]."""
    rd = rope_dim if rope_dim > 0 else hd
    j = np.arange(rd // 2, dtype=np.float64)
    pos = np.arange(max_ctx, dtype=np.float64)[:, None]
    theta = pos / np.power(10000.0, 2.0 * j / hd)
    return np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)


def scale_weights(raw, qt, log2):
    """raw GGUF blocks with every block scale multiplied by 2**log2 (fp16 d /
    dmin fields exactly; the MXFP4 E8M0 exponent shifted)."""
    out = raw.copy()
    be, bb = BLOCK[qt]
    blk = out.reshape(-1, bb)
    f = np.float32(2.0 ** log2)

    def rescale(lo):
        h = blk[:, lo:lo + 2].copy().view(np.float16)
        blk[:, lo:lo + 2] = (h.astype(np.float32) * f).astype(np.float16).view(np.uint8)
    if qt == QT_MXFP4:
        blk[:, 16] = np.clip(blk[:, 16].astype(np.int32) + log2, 1, 254).astype(np.uint8)
    elif qt == QT_Q6_K:
        rescale(208)
    elif qt in (QT_Q4_K, QT_Q5_K, QT_Q4_1):
        rescale(0)
        rescale(2)
    elif qt != QT_F32:
        rescale(0)
    return np.ascontiguousarray(out)


def qwen36_case(seed=0, B=2, emb_quant=0):
    """A small seeded Qwen3.6-style hybrid model for qwen36_batch_forward
    (CE:859-1231), every path of the driver exercised.  Weights keep the
    residual stream well inside RMS_NORM_SIMD's +-1000 clip (CE:958-960):
    zero-mean Q4_K blocks (gen_q4k_centered) and block scales chosen per
    type so that each matmul's outputs stay O(1-10); with BASELINE's
    positive-mean Q4_K the stream passes the clip after one layer and the
    normalised input keeps only the signs.  Paths:
      layer 0  SSM (Q8_0 gate, Q4_K ssm_out), MoE Q4_K/Q4_K/Q6_K, shared expert MXFP4
      layer 1  attention, fused QKV of inner + 2*n_kv rows (so V at inner + N
               is read from the workspace, CE:1002-1009), Q6_K QKV, Q8_0 o,
               MoE MXFP4 x3, shared expert Q8_0
      layer 2  SSM (MXFP4 gate, Q6_K ssm_out), no MoE (the FFN is skipped)
      layer 3  attention, QKV of inner + 2*N rows (the caller's layout,
               TE:1533-1543), Q4_K QKV, MXFP4 o, MoE Q4_K/Q4_K/Q6_K, no
               shared expert
    output head Q6_K; fp32 routers (code 0).  Returns a dict of arrays and
    scalars; the per-call state (KV caches, SSM state, workspace) is created
    by Qwen36Call."""
    rng = np.random.default_rng(seed)
    SHIFT = {QT_Q4_K: 0, QT_Q8_0: -3, QT_Q6_K: -4, QT_MXFP4: -2}   # block-scale shift (log2) per type

    def gen(r, qt, rows, cols):
        raw = gen_q4k_centered(r, rows, cols) if qt == QT_Q4_K else gen_weights(r, qt, rows, cols)
        return scale_weights(raw, qt, SHIFT.get(qt, 0))
    c = dict(B=B, L=4, N=256, NH=4, n_kv_h=2, HD=64, FF=512, n_experts=8, top_k=2, n_ff_expert=256, eps=1e-6,
             rope_dim=0, max_ctx=8, ssm_inner=256, ssm_groups=4, ssm_state_size=16, ssm_conv_kernel=4,
             ssm_dt_rank=8, V=300, emb_quant=emb_quant)
    N, L, E, M = c["N"], c["L"], c["n_experts"], c["n_ff_expert"]
    inner, nkv, si = c["NH"] * c["HD"], c["n_kv_h"] * c["HD"], c["ssm_inner"]
    G, Sz, dtr = c["ssm_groups"], c["ssm_state_size"], c["ssm_dt_rank"]
    c["layer_types"] = np.array([1, 0, 1, 0], np.int32)
    if emb_quant == 12:
        c["emb"] = gen(rng, QT_Q4_K, c["V"], N)
    else:
        c["emb"] = rng.standard_normal((c["V"], N)).astype(np.float32)
    c["attn_norm"] = [(1 + 0.1 * rng.standard_normal(N)).astype(np.float32) for _ in range(L)]
    c["ffn_norm"] = [(1 + 0.1 * rng.standard_normal(N)).astype(np.float32) for _ in range(L)]
    mats = {}   # name -> per-layer (raw, nr, nc, qt) or None
    mats["qkv"] = [None, (inner + 2 * nkv, N, QT_Q6_K), None, (inner + 2 * N, N, QT_Q4_K)]
    mats["gate"] = [(si, N, QT_Q8_0), None, (si, N, QT_MXFP4), None]
    mats["ssm_out"] = [(N, si, QT_Q4_K), None, (N, si, QT_Q6_K), None]
    mats["out"] = [None, (N, inner, QT_Q8_0), None, (N, inner, QT_MXFP4)]
    for name, per in mats.items():
        c[name] = [None if p is None else (gen(rng, p[2], p[0], p[1]),) + p for p in per]
    exp_qts = [(QT_Q4_K, QT_Q4_K, QT_Q6_K), (QT_MXFP4, QT_MXFP4, QT_MXFP4), None, (QT_Q4_K, QT_Q4_K, QT_Q6_K)]
    c["experts"] = []
    for l in range(L):
        q = exp_qts[l]
        if q is None:
            c["experts"].append(None)
            continue
        gate = np.concatenate([gen(rng, q[0], M, N) for _ in range(E)])
        upw = np.concatenate([gen(rng, q[1], M, N) for _ in range(E)])
        down = np.concatenate([gen(rng, q[2], N, M) for _ in range(E)])
        router = (rng.standard_normal((E, N)) * 0.05).astype(np.float32)
        c["experts"].append(dict(qts=q, gate=gate, up=upw, down=down, router=router))
    sh_qts = [(QT_MXFP4,) * 3, (QT_Q8_0,) * 3, None, None]
    c["shexp"] = []
    for l in range(L):
        q = sh_qts[l]
        if q is None or c["experts"][l] is None:
            c["shexp"].append(None)
            continue
        c["shexp"].append(dict(qts=q, si=128, gate=gen(rng, q[0], 128, N), up=gen(rng, q[1], 128, N),
                               down=gen(rng, q[2], N, 128),
                               router=(rng.standard_normal(N) * 0.05).astype(np.float32)))
    c["ssm"] = []
    for l in range(L):
        if c["layer_types"][l] != 1:
            c["ssm"].append(None)
            continue
        c["ssm"].append(dict(conv1d=(rng.standard_normal(2 * si) * 0.5).astype(np.float32),
                             a=(-rng.uniform(0.5, 2.0, G)).astype(np.float32),
                             dt_bias=(rng.standard_normal(G) * 0.5).astype(np.float32),
                             alpha=(rng.standard_normal(G * dtr) * 0.2).astype(np.float32),
                             beta=(rng.standard_normal(G * dtr) * 0.2).astype(np.float32),
                             norm=np.ones(Sz, np.float32)))
    c["out_norm"] = (1 + 0.1 * rng.standard_normal(N)).astype(np.float32)
    c["out_w"] = (gen(rng, QT_Q6_K, c["V"], N), c["V"], N, QT_Q6_K)
    c["cos"], c["sin"] = rope_tables(c["max_ctx"], c["HD"], c["rope_dim"])
    shexp_int0 = c["shexp"][0]["si"] if c["shexp"][0] else 512
    S = max(N, inner, c["FF"], nkv, inner + 2 * nkv, M, shexp_int0, 8192)
    c["S"] = S
    # initial per-call state: KV rows before kv_len, SSM state, workspace (stale values the driver may read)
    c["kv_lens0"] = np.array([0, 3, 0, 5], np.int32)
    kv = np.zeros((2, L, c["max_ctx"], nkv), np.float32)
    for l in range(L):
        n = c["kv_lens0"][l]
        kv[:, l, :n] = rng.standard_normal((2, n, nkv))
    c["kv0"] = kv
    c["state0"] = (rng.standard_normal((L, G, Sz)) * 0.1).astype(np.float32)
    c["ws0"] = rng.standard_normal(B * S * 12).astype(np.float32)
    c["tokens"] = [rng.integers(0, c["V"], B).astype(np.int32) for _ in range(2)]
    return c


def qwen36_arrays_crc(c):
    """CRC32 over every generated array of a qwen36_case (the fixture checks it
    before trusting the regenerated inputs)."""
    import zlib
    h = 0

    def add(a):
        nonlocal h
        h = zlib.crc32(np.ascontiguousarray(a).view(np.uint8).tobytes(), h)
    add(c["emb"]); add(c["out_w"][0]); add(c["out_norm"]); add(c["cos"]); add(c["kv0"]); add(c["state0"]); add(c["ws0"])
    for l in range(c["L"]):
        add(c["attn_norm"][l]); add(c["ffn_norm"][l])
        for name in ("qkv", "gate", "ssm_out", "out"):
            if c[name][l] is not None:
                add(c[name][l][0])
        for key in ("experts", "shexp"):
            d = c[key][l]
            if d is not None:
                for k in ("gate", "up", "down", "router"):
                    add(d[k])
        if c["ssm"][l] is not None:
            for v in c["ssm"][l].values():
                add(v)
    for t in c["tokens"]:
        add(t)
    return h


class Qwen36Call:
    """ctypes arguments of qwen36_batch_forward (CE:859-1231) for a
    qwen36_case, with the per-call state the caller owns (KV caches, kv_lens,
    SSM state, workspace): call(so, tokens) runs one forward on `so` (the
    reference's C or this library) and returns the logits [B][V]."""

    def __init__(self, c, ws_null_q8=False):
        cf_, cu_, ci_ = ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_uint8), ctypes.c_int
        self.c = c
        L, B = c["L"], c["B"]
        self.keep = []

        def fptr(a):
            if a is None:
                return None
            self.keep.append(a)
            return a.ctypes.data_as(cf_)

        def uptr(a):
            if a is None:
                return None
            self.keep.append(a)
            return a.ctypes.data_as(cu_)

        def arr(t, vals):
            a = (t * len(vals))(*vals)
            self.keep.append(a)
            return a

        def iarr(vals):
            a = np.ascontiguousarray(np.array(vals, np.int32))
            self.keep.append(a)
            return a.ctypes.data_as(ctypes.POINTER(ci_))
        self.kv = c["kv0"].copy()
        self.kv_lens = c["kv_lens0"].copy()
        self.state = c["state0"].copy()
        self.ws = c["ws0"].copy()
        self.q8 = np.zeros(1 << 16, np.uint8)
        self.logits = np.zeros((B, c["V"]), np.float32)
        self.tok = np.zeros(B, np.int32)
        mat = lambda name: ([uptr(m[0]) if m else None for m in c[name]],  # noqa: E731
                            [m[1] if m else 0 for m in c[name]], [m[2] if m else 0 for m in c[name]],
                            [m[3] if m else 0 for m in c[name]])
        ex, sh, ss = c["experts"], c["shexp"], c["ssm"]
        a = [ci_(B), ci_(L), ci_(c["N"]), ci_(c["NH"]), ci_(c["n_kv_h"]), ci_(c["HD"]), ci_(c["FF"]),
             ci_(c["n_experts"]), ci_(c["top_k"]), ci_(c["n_ff_expert"]), ctypes.c_float(c["eps"]),
             ci_(c["rope_dim"]), ci_(c["max_ctx"]), ci_(c["ssm_inner"]), ci_(c["ssm_groups"]),
             ci_(c["ssm_state_size"]), ci_(c["ssm_conv_kernel"]), ci_(c["ssm_dt_rank"]),
             fptr(c["emb"]) if c["emb_quant"] == 0 else ctypes.cast(uptr(c["emb"]), cf_), ci_(c["emb_quant"]),
             iarr(c["layer_types"]), self.tok.ctypes.data_as(ctypes.POINTER(ci_)), self.logits.ctypes.data_as(cf_),
             arr(cf_, [fptr(v) for v in c["attn_norm"]]), arr(cf_, [fptr(v) for v in c["ffn_norm"]])]
        for name in ("qkv", "gate", "ssm_out", "out"):
            raws, nr, nc, qt = mat(name)
            a += [arr(cu_, raws), iarr(nr), iarr(nc), iarr(qt)]
        for k, i in (("gate", 0), ("up", 1), ("down", 2)):
            a += [arr(cu_, [uptr(d[k]) if d else None for d in ex]), iarr([d["qts"][i] if d else 0 for d in ex])]
        for k in ("gate", "up", "down", "router"):
            a.append(arr(cf_, [ctypes.cast(uptr(d[k]), cf_) if d else None for d in sh]))
        a.append(iarr([d["si"] if d else 512 for d in sh]))
        a += [arr(cu_, [ctypes.cast(fptr(d["router"]), cu_) if d else None for d in ex]), iarr([0] * L)]
        for i in range(3):
            a.append(iarr([d["qts"][i] if d else 39 for d in sh]))
        a += [fptr(c["out_norm"]), uptr(c["out_w"][0]), ci_(c["out_w"][1]), ci_(c["out_w"][2]), ci_(c["out_w"][3])]
        for k in ("conv1d", "a", "dt_bias", "alpha", "beta", "norm"):
            a.append(arr(cf_, [fptr(d[k]) if d else None for d in ss]))
        a.append(self.state.ctypes.data_as(cf_))
        a += [self.kv[0].ctypes.data_as(cf_), self.kv[1].ctypes.data_as(cf_),
              self.kv_lens.ctypes.data_as(ctypes.POINTER(ci_)), fptr(c["cos"]), fptr(c["sin"]),
              self.ws.ctypes.data_as(cf_), None if ws_null_q8 else self.q8.ctypes.data_as(cu_)]
        self.args = a

    def call(self, so, tokens):
        self.tok[:] = tokens
        so.qwen36_batch_forward(*self.args)
        return self.logits.copy()

    def qkv_slice(self):
        """The fused-QKV slice of the workspace (ws + 3*B*S, CE:915), first 1024 floats."""
        o = 3 * self.c["B"] * self.c["S"]
        return self.ws[o:o + 1024].copy()


def ssm_case(seed, B, N, inner, G=4, Sz=16, dtr=8, gate_qt=QT_Q8_0, so_qt=QT_Q6_K):
    """Seeded inputs of ssm_decode_step / ssm_layer_fused (CE:736-849): x and
    the residual [B][N] ~ N(0,1), conv weights [2*inner], per-group A < 0,
    dt_bias, alpha / beta [G*dtr], state [G][Sz], the gate (inner x N) and
    ssm_out (N x inner) matrices of the given GGUF types."""
    rng = np.random.default_rng(seed)
    return dict(B=B, N=N, inner=inner, G=G, Sz=Sz, dtr=dtr, gate_qt=gate_qt, so_qt=so_qt,
                x=rng.standard_normal((B, N)).astype(np.float32),
                res=rng.standard_normal((B, N)).astype(np.float32),
                conv=(rng.standard_normal(2 * inner) * 0.5).astype(np.float32),
                a=(-rng.uniform(0.5, 2.0, G)).astype(np.float32),
                dtb=(rng.standard_normal(G) * 2.0).astype(np.float32),
                alpha=(rng.standard_normal(G * dtr) * 0.5).astype(np.float32),
                beta=(rng.standard_normal(G * dtr) * 0.5).astype(np.float32),
                norm=np.ones(max(Sz, 1), np.float32),
                state=(rng.standard_normal((G, Sz)) * 0.1).astype(np.float32),
                gate=gen_weights(rng, gate_qt, inner, N), so=gen_weights(rng, so_qt, N, inner))


def ssm_call(so, c, fused, gate_nc=None):
    """Run ssm_layer_fused (fused) or ssm_decode_step on `so` for an
    ssm_case; returns (output, state after).  gate_nc overrides the gate
    matrix's column count passed to ssm_layer_fused."""
    cf_, cu_ = ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_uint8)
    f = lambda a: np.ascontiguousarray(a).ctypes.data_as(cf_)  # noqa: E731
    B, N, inner = c["B"], c["N"], c["inner"]
    state = c["state"].copy()
    x, res = np.ascontiguousarray(c["x"]), np.ascontiguousarray(c["res"])
    keep = (x, res)
    if fused:
        out = np.full(max(B * N, B * inner), np.nan, np.float32)
        so.ssm_layer_fused(f(x), f(res), f(out), f(c["conv"]), f(c["a"]), f(c["dtb"]), f(c["alpha"]), f(c["beta"]),
                           f(c["norm"]), f(state), c["gate"].ctypes.data_as(cu_), inner, N if gate_nc is None else gate_nc, c["gate_qt"],
                           c["so"].ctypes.data_as(cu_), N, inner, c["so_qt"], B, N, inner, c["G"], c["Sz"], 4,
                           c["dtr"])
    else:
        out = np.full(B * inner, np.nan, np.float32)
        so.ssm_decode_step(f(x), f(out), f(c["conv"]), f(c["a"]), f(c["dtb"]), f(c["alpha"]), f(c["beta"]),
                           f(c["norm"]), f(state), B, N, inner, c["G"], c["Sz"], 4, c["dtr"])
    del keep
    return out, state
