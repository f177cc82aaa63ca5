"""The TinyLlama decode pass of BASELINE configs[1] on device data, shared by
bench.py (its headline) and the GPU tests that pin the headline's launches.

A pass runs each layer's matrices through mllm_gemv_fused, every matrix fed by
the previous one's output:
    qkv  = Wqkv . rmsnorm(x) * g_attn              (simd_ops rms_norm, TE:1516)
    xb   = x + Wo . q                               (TE:1628-1633; q stands in for attention)
    h    = silu(Wg . v) * (Wu . v), v = rmsnorm(xb) * g_ffn   (TE:1641, 1660-1710; paired gate/up rows)
    x'   = xb + Wdown . h
for each layer, then logits = Wlm . rmsnorm(x) * g_out (TE:1716); matrices use
the *_batch_matmul semantics (Q4_K ggml CE:255-313, Q6_K sequential CE:315-378).
"""
import ctypes

import numpy as np

from . import kernels as K
from . import workloads as W

EPS = 1e-5


class Matrix:
    """A packed device matrix; keep_raw also keeps the raw GGUF bytes (host)."""

    def __init__(self, dev, sem, raw, rows, cols, keep_raw=False):
        import torch
        self.sem, self.rows, self.cols = sem, rows, cols
        self.raw_bytes = raw.size if isinstance(raw, np.ndarray) else raw.numel()
        self.raw = raw if keep_raw else None
        src = torch.from_numpy(raw).cuda() if isinstance(raw, np.ndarray) else raw
        self.packed = dev.pack(sem, src, rows, cols)


def norm_weight(rng, n):
    return (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)


def build_tinyllama(dev, rng, n_layers, keep_raw=False, gen=None):
    """Per layer, the device copies as a decode engine runs them: q/k/v rows
    stacked into one 2560x2048 matrix (one launch, as batch_qkv_omp), o,
    gate/up rows stacked into one 11264x2048 matrix (batch_gate_up_omp), down;
    the RMSNorm weights of the attention and FFN norms (1 + 0.1 N(0,1)).
    gen(rng, qt, rows, cols) makes the raw weights (default: BASELINE's
    distributions, workloads.gen_weights)."""
    import torch
    gen = gen or W.gen_weights
    layers = []
    for _ in range(n_layers):
        raw = {name: gen(rng, qt, rows, cols) for name, rows, cols, qt in W.TINYLLAMA_MATS}
        qkv = np.concatenate([raw["q"], raw["k"], raw["v"]])
        gu = np.concatenate([raw["gate"], raw["up"]])
        an, fn = norm_weight(rng, 2048), norm_weight(rng, 2048)
        layers.append({"qkv": Matrix(dev, K.Q4_K_GGML, qkv, 2560, 2048, keep_raw),
                       "o": Matrix(dev, K.Q4_K_GGML, raw["o"], 2048, 2048, keep_raw),
                       "gate_up": Matrix(dev, K.Q4_K_GGML, gu, 11264, 2048, keep_raw),
                       "down": Matrix(dev, K.Q6_K_SEQ, raw["down"], 2048, 5632, keep_raw),
                       "attn_norm": torch.from_numpy(an).cuda(),
                       "ffn_norm": torch.from_numpy(fn).cuda()})
    name, rows, cols, qt = W.TINYLLAMA_LM_HEAD
    lm = Matrix(dev, K.Q6_K_SEQ, gen(rng, qt, rows, cols), rows, cols, keep_raw)
    out_norm = torch.from_numpy(norm_weight(rng, 2048)).cuda()
    return layers, lm, out_norm


def algo_bytes(m, B):
    return m.raw_bytes + B * (m.cols + m.rows) * 4


class DecodeChain:
    """The decode pass at batch B (see the module docstring).  run() is a
    sequence of launches on the current stream (capturable); with `record`
    (a list) it appends a copy of every stage's output after its launch."""

    def __init__(self, torch, dev, layers, lm, out_norm, B, x0=None):
        self.torch, self.dev, self.layers, self.lm, self.out_norm, self.B = torch, dev, layers, lm, out_norm, B
        z = lambda *s: torch.zeros(*s, device="cuda")  # noqa: E731
        self.x0 = torch.randn(B, 2048, device="cuda") if x0 is None else x0
        self.xa, self.xb = z(B, 2048), z(B, 2048)
        self.qkv, self.h, self.logits = z(B, 2560), z(B, 5632), z(B, 32000)
        F = dev.fusion
        self.f_qkv = [F(rms_w=L["attn_norm"], rms_eps=EPS) for L in layers]
        self.f_o = F(out_add=self.xa, x_ld=2560)
        self.f_gu = [F(rms_w=L["ffn_norm"], rms_eps=EPS, silu_pair=True, silu_clamp=False) for L in layers]
        self.f_down = F(out_add=self.xb)
        self.f_lm = F(rms_w=out_norm, rms_eps=EPS)
        wsz = lambda m, f, rows=None: dev.so.mllm_gemv_fused_workspace_size(  # noqa: E731
            m.sem, rows or m.rows, m.cols, B, ctypes.byref(f))
        n = max([wsz(layers[0]["qkv"], self.f_qkv[0]), wsz(layers[0]["o"], self.f_o),
                 wsz(layers[0]["gate_up"], self.f_gu[0], 5632), wsz(layers[0]["down"], self.f_down),
                 wsz(lm, self.f_lm), 256])
        self.ws = torch.empty(n, dtype=torch.uint8, device="cuda")
        self.mats = [m for L in layers for m in (L["qkv"], L["o"], L["gate_up"], L["down"])] + [lm]

    def run(self, record=None):
        d, B, ws = self.dev, self.B, self.ws
        rec = (lambda name, t: record.append((name, t.clone()))) if record is not None else (lambda name, t: None)
        self.xa.copy_(self.x0)
        for i, L in enumerate(self.layers):
            d.gemv_fused(L["qkv"].sem, L["qkv"].packed, self.xa, 2560, 2048, self.f_qkv[i], out=self.qkv, ws=ws)
            rec("qkv", self.qkv)
            d.gemv_fused(L["o"].sem, L["o"].packed, self.qkv.data_ptr(), 2048, 2048, self.f_o, out=self.xb, ws=ws, B=B)
            rec("o", self.xb)
            d.gemv_fused(L["gate_up"].sem, L["gate_up"].packed, self.xb, 5632, 2048, self.f_gu[i], out=self.h, ws=ws)
            rec("gate_up", self.h)
            d.gemv_fused(L["down"].sem, L["down"].packed, self.h, 2048, 5632, self.f_down, out=self.xa, ws=ws)
            rec("down", self.xa)
        d.gemv_fused(self.lm.sem, self.lm.packed, self.xa, 32000, 2048, self.f_lm, out=self.logits, ws=ws)
        rec("lm_head", self.logits)

    def bytes(self):
        return sum(algo_bytes(m, self.B) for m in self.mats)
