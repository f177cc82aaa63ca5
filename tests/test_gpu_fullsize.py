"""GPU parity at the benchmark's full configuration sizes, on the exact kernel
instantiations bench.py times.

* configs[3] (GPT-OSS MoE, E=32, MXFP4, fused gate/up tensors) and configs[4]
  (Qwen3 MoE, E=128, Q4_K/Q6_K, skewed routing) at T=1280 tokens, with the
  bench's own seeds (workloads.moe_workload): every token's routing bit-exact
  with the oracle's C routing chain, the layer's bucketing (same kernels) equal
  to a stable sort, every output finite, and a stratified token subset --
  hot-expert tokens, the last tile of many experts, the first and last token,
  random ones -- within tolerance of the oracle's moe_forward_omp per token.
* The decode GEMVs at the bench's fused shapes (Q4_K 11264x2048 gate+up and
  2560x2048 qkv, which select 16 lanes per row at B=1; Q6_K 2048x5632 down;
  the 32000x2048 lm_head) at B = 1, 4, 8.
* The prefill GEMM at M = 512 and M = 1280 on the full Q4_K
  5632x2048 and Q6_K 2048x5632 matrices, on a strided sample of rows (every
  128-row weight tile) and tokens (every 64/128-entry tile); each output sums
  every split-K slice.

Alongside the normalised max error (the assertion) each check prints the
per-element relative error max |got - ref| / |ref| over elements with
|ref| >= 1e-3 * max|ref| (elements nearer zero have no meaningful relative
error at fp32 summation noise).
"""
import numpy as np
import pytest

import oracle as O
from helpers import GEMV_TOL, MOE_TOL, moe_tol
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


def report(tag, got, ref):
    ne = O.norm_err(got, ref)
    re = O.elem_rel_err(got, ref)
    print(f"[parity] {tag}: normalised max error {ne:.3e}, per-element max relative error {re:.3e}", flush=True)
    return ne


def last_tile_tokens(idx, E, K, n_experts, rng):
    """Tokens whose entry is the last one of an expert's last 64-entry tile
    (the bucketing's part-filled tiles), for up to n_experts experts picked
    across the count range."""
    flat = idx.ravel()
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat[flat >= 0], minlength=E)
    off = np.concatenate([[0], np.cumsum(counts)])
    live = np.nonzero(counts)[0]
    pick = live[np.argsort(counts[live], kind="stable")]
    pick = pick[np.linspace(0, len(pick) - 1, min(n_experts, len(pick))).astype(int)]
    toks = []
    for e in pick:
        c = counts[e]
        first_last_tile = off[e] + 64 * ((c - 1) // 64)
        toks.append(int(order[off[e + 1] - 1]) // K)          # last entry of the expert
        toks.append(int(order[first_last_tile]) // K)         # first entry of its last tile
    return toks


@pytest.mark.parametrize("tag", ["gptoss", "qwen3"])
def test_moe_layer_config_size(dev, orc, tag):
    """configs[3] / configs[4] at T = 1280 through mllm_moe_forward, as bench.py runs it."""
    import torch
    T = 1280
    wl = W.moe_workload(tag, T)
    c, qts = wl["cfg"], wl["qts"]
    N, E, Kk, M = c["N"], c["E"], c["K"], c["M"]
    print(f"[case] MoE {tag} N={N} E={E} K={Kk} M={M} T={T}", flush=True)
    router = torch.from_numpy(wl["router"]).cuda()
    layer = dev.moe_prepare(qts, N, M, E, Kk, wl["gates"], wl["ups"], wl["downs"], router, 1)
    x = torch.from_numpy(wl["x"]).cuda()
    idx = torch.empty((T, Kk), dtype=torch.int32, device="cuda")
    w = torch.empty((T, Kk), dtype=torch.float32, device="cuda")
    got = layer.forward(x, idx=idx, w=w).cpu().numpy()
    idx, w = idx.cpu().numpy(), w.cpu().numpy()
    assert np.all(np.isfinite(got)), "non-finite MoE outputs"
    # routing of every token, bit-exact
    ri, rw = orc.route(wl["router"], wl["x"], Kk, 1)
    assert np.array_equal(idx, ri), f"routing differs for {int(np.sum(np.any(idx != ri, axis=1)))} tokens"
    assert np.max(np.abs(w - rw) / np.abs(rw)) < 1e-6
    # the layer's bucketing kernels on these entries: a stable sort by expert
    off, perm, pos_of, (te, tb, tend) = dev.moe_bucket(torch.from_numpy(idx.ravel().copy()).cuda(), E)
    order = np.argsort(idx.ravel(), kind="stable")
    assert np.array_equal(perm.cpu().numpy(), order)
    counts = np.bincount(idx.ravel(), minlength=E)
    assert np.array_equal(off.cpu().numpy(), np.concatenate([[0], np.cumsum(counts)]))
    assert int(np.sum(tend.cpu().numpy() - tb.cpu().numpy())) == T * Kk
    # stratified token subset against the oracle's moe_forward_omp
    rng = np.random.default_rng(123)
    toks = [0, T - 1] + last_tile_tokens(idx, E, Kk, 12, rng)
    if len(wl["hot_tokens"]):
        toks += list(rng.choice(wl["hot_tokens"], 8, replace=False))
    toks += list(rng.choice(T, 10, replace=False))
    toks = sorted(set(int(t) for t in toks))
    need = sorted(set(int(e) for t in toks for e in ri[t]))
    host = {e: (wl["gates"][e].cpu().numpy(), wl["ups"][e].cpu().numpy(), wl["downs"][e].cpu().numpy())
            for e in need}
    dummy = host[need[0]]
    gs = [host.get(e, dummy)[0] for e in range(E)]
    us = [host.get(e, dummy)[1] for e in range(E)]
    ds = [host.get(e, dummy)[2] for e in range(E)]
    ref = np.stack([orc.moe_forward_token(gs, us, ds, wl["x"][t], M, N, qts, ri[t], rw[t]) for t in toks])
    if len(wl["hot_experts"]):
        hot_share = np.mean(np.isin(idx, wl["hot_experts"]))
        print(f"[case] share of entries on the {len(wl['hot_experts'])} hot experts: {hot_share:.3f}", flush=True)
    assert report(f"MoE {tag} T={T} ({len(toks)} tokens)", got[toks], ref) < moe_tol(qts)


@pytest.mark.parametrize("sem,qt,R,C", [(K.Q4_K_GGML, 12, 11264, 2048), (K.Q4_K_GGML, 12, 2560, 2048),
                                        (K.Q6_K_SEQ, 14, 2048, 5632), (K.Q4_K_GGML, 12, 2048, 2048)])
@pytest.mark.parametrize("B", [1, 4, 8])
def test_decode_gemv_bench_shapes(dev, orc, sem, qt, R, C, B):
    """The fused qkv / gate+up matrices, o and down of the TinyLlama set."""
    import torch
    print(f"[case] GEMV {K.SEM_NAMES[sem]} {R}x{C} B={B}", flush=True)
    rng = np.random.default_rng(R + C + B)
    w = W.gen_weights(rng, qt, R, C)
    x = W.gen_x(rng, B, C)
    packed = dev.pack(sem, torch.from_numpy(w).cuda(), R, C)
    got = dev.gemv(sem, packed, torch.from_numpy(x).cuda(), R, C).cpu().numpy()
    assert report(f"GEMV {K.SEM_NAMES[sem]} {R}x{C} B={B}", got, orc.gemv(sem, w, x, R, C, B)) < GEMV_TOL


def test_decode_gemv_lm_head(dev, orc):
    """The Q6_K 32000x2048 lm_head at B = 1 (the pass's largest matrix)."""
    import torch
    R, C = 32000, 2048
    rng = np.random.default_rng(77)
    w = W.gen_weights(rng, 14, R, C)
    x = W.gen_x(rng, 1, C)
    packed = dev.pack(K.Q6_K_SEQ, torch.from_numpy(w).cuda(), R, C)
    got = dev.gemv(K.Q6_K_SEQ, packed, torch.from_numpy(x).cuda(), R, C).cpu().numpy()
    assert report("GEMV lm_head Q6_K_SEQ 32000x2048 B=1", got, orc.gemv(K.Q6_K_SEQ, w, x, R, C, 1)) < GEMV_TOL


@pytest.mark.parametrize("sem,qt,R,C,M", [(K.Q4_K_GGML, 12, 5632, 2048, 512), (K.Q6_K_SEQ, 14, 2048, 5632, 512),
                                          (K.Q4_K_GGML, 12, 5632, 2048, 1280), (K.Q6_K_SEQ, 14, 2048, 5632, 1280)])
def test_prefill_every_tile(dev, orc, sem, qt, R, C, M):
    """the full weights with bf16-valued activations, as bench.py draws
    them; rows sampled with stride 7 (every 128-row tile, every row offset mod 7)
    and tokens with stride 5 (every 64- and 128-token tile)."""
    import torch
    print(f"[case] prefill {K.SEM_NAMES[sem]} {R}x{C} M={M}", flush=True)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    raw = W.gen_weights_torch(gen, qt, R, C)
    x = torch.randn(M, C, device="cuda", generator=gen).bfloat16().float()
    packed = dev.pack(sem, raw, R, C)
    got = dev.gemv(sem, packed, x, R, C, ws=dev.workspace(sem, C, M, x.device, R)).cpu().numpy()
    assert np.all(np.isfinite(got))
    rows = np.arange(3, R, 7)
    toks = np.arange(2, M, 5)
    rb = W.row_bytes(qt, C)
    wh = raw.cpu().numpy().reshape(R, rb)[rows].ravel()
    ref = orc.gemv(sem, np.ascontiguousarray(wh), np.ascontiguousarray(x.cpu().numpy()[toks]), len(rows), C, len(toks))
    assert report(f"prefill {K.SEM_NAMES[sem]} {R}x{C} M={M}", got[np.ix_(toks, rows)], ref) < GEMM_TOL
