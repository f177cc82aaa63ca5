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
