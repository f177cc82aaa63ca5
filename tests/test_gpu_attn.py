"""GPU parity of decode attention, the KV cache and RoPE through the C ABI.

* mllm_gqa_decode, both softmaxes (CE:141-158 gqa, gqa_attention.c:93), at the
  head layouts of GPT-OSS (64/8 x 64), Qwen3-30B-A3B (32/4 x 128) and
  TinyLlama (32/4 x 64), against the oracle.  Tolerance ATTN_TOL of max|ref|
  for the expf softmax.  gqa_attention.c's exp_ps_simd gives weights of both
  signs whose sum can nearly cancel, so there the bound is also scaled by the
  oracle's own sensitivity to a 2^-20 relative change of V.
* The paged view equals the contiguous one bit for bit (same kernels, same
  order), with pages scattered by a random page table.
* mllm_kv_append writes rows where CE:1363-1381 / GO:158-161 put them.
* The drop-in gqa_attention_decode with TE's argtypes and workspace.
* mllm_rope against the oracle's rope_apply (GO:37-51).
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from helpers import fp
from mojollama_amd import kernels as K

pytestmark = pytest.mark.gpu
ATTN_TOL = 2e-5


@pytest.fixture(scope="module")
def lib():
    return K.load_kernels()


@pytest.fixture(scope="module")
def dev(lib):
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return K.DeviceOps(lib)


def attn_tol(orc, mode, q, k, v, S, nh, nkh, hd, ref):
    if mode == O.ATTN_CE:
        return ATTN_TOL * np.max(np.abs(ref))
    rng = np.random.default_rng(1)
    v2 = (v * (1 + 2.0 ** -20 * rng.standard_normal(v.shape))).astype(np.float32)
    sens = np.max(np.abs(orc.gqa_decode(mode, q, k, v2, S, nh, nkh, hd) - ref))
    return ATTN_TOL * np.max(np.abs(ref)) + 64 * sens


def make_case(rng, B, S_list, nh, nkh, hd, scale=1.0):
    Smax = max(S_list)
    q = (rng.standard_normal((B, nh * hd)) * scale).astype(np.float32)
    k = rng.standard_normal((B, Smax, nkh * hd)).astype(np.float32)
    v = rng.standard_normal((B, Smax, nkh * hd)).astype(np.float32)
    return q, k, v


SHAPES = [(64, 8, 64), (32, 4, 128), (32, 4, 64), (8, 8, 32), (12, 3, 80)]


@pytest.mark.parametrize("mode", [O.ATTN_CE, O.ATTN_GQA_C])
@pytest.mark.parametrize("nh,nkh,hd", SHAPES)
@pytest.mark.parametrize("S_list", [[1], [7], [8], [9], [64], [65], [200], [4096], [5, 130, 64]])
def test_gqa_decode_contiguous_vs_oracle(dev, orc, mode, nh, nkh, hd, S_list):
    import torch
    rng = np.random.default_rng(sum(S_list) + nh + hd + 7 * mode)
    B = len(S_list)
    q, k, v = make_case(rng, B, S_list, nh, nkh, hd)
    Smax = k.shape[1]
    kv = dev.kv_view(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), seq_stride=Smax * nkh * hd)
    lens = torch.tensor(S_list, dtype=torch.int32, device="cuda")
    qd = torch.from_numpy(q).cuda()
    got = dev.gqa_decode(mode, qd, kv, lens, Smax, nh, nkh, hd).cpu().numpy()
    for b, S in enumerate(S_list):
        ref = orc.gqa_decode(mode, q[b], k[b], v[b], S, nh, nkh, hd)
        err = np.max(np.abs(got[b] - ref))
        assert err <= attn_tol(orc, mode, q[b], k[b], v[b], S, nh, nkh, hd, ref), (b, S, err, np.max(np.abs(ref)))


def paged_copy(rng, k, v, S_list, page_size, nkh, hd):
    """Scatter each sequence's rows over a shared pool of pages (CE:164 layout
    for one layer) through a random page table; returns pools and tables."""
    B = len(S_list)
    need = [(S + page_size - 1) // page_size for S in S_list]
    n_pages = sum(need) + 3
    perm = rng.permutation(n_pages)
    max_blocks = max(need) + 2
    tables = np.full((B, max_blocks), -1, np.int32)
    kp = rng.standard_normal((n_pages, page_size, nkh * hd)).astype(np.float32)   # stale data everywhere else
    vp = rng.standard_normal((n_pages, page_size, nkh * hd)).astype(np.float32)
    at = 0
    for b, S in enumerate(S_list):
        for blk in range(need[b]):
            pg = perm[at]
            at += 1
            tables[b, blk] = pg
            rows = min(page_size, S - blk * page_size)
            kp[pg, :rows] = k[b, blk * page_size:blk * page_size + rows]
            vp[pg, :rows] = v[b, blk * page_size:blk * page_size + rows]
    return kp, vp, tables, n_pages


@pytest.mark.parametrize("mode", [O.ATTN_CE, O.ATTN_GQA_C])
@pytest.mark.parametrize("page_size", [16, 64, 100])
def test_gqa_decode_paged_equals_contiguous(dev, mode, page_size):
    import torch
    rng = np.random.default_rng(page_size + mode)
    nh, nkh, hd = 64, 8, 64
    S_list = [1, 333, 64, 1000]
    q, k, v = make_case(rng, len(S_list), S_list, nh, nkh, hd)
    Smax = k.shape[1]
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    lens = torch.tensor(S_list, dtype=torch.int32, device="cuda")
    kv_c = dev.kv_view(cu(k), cu(v), seq_stride=Smax * nkh * hd)
    kp, vp, tables, n_pages = paged_copy(rng, k, v, S_list, page_size, nkh, hd)
    kpd, vpd, td = cu(kp), cu(vp), cu(tables)
    kv_p = dev.kv_view(kpd, vpd, block_tables=td, page_size=page_size, n_pages=n_pages)
    a = dev.gqa_decode(mode, cu(q), kv_c, lens, Smax, nh, nkh, hd).cpu().numpy()
    b = dev.gqa_decode(mode, cu(q), kv_p, lens, Smax, nh, nkh, hd).cpu().numpy()
    assert np.array_equal(a, b)


def test_gqa_decode_unmapped_page_reads_zeros(dev, orc):
    """A logical page with no physical page (-1) contributes zero rows."""
    import torch
    rng = np.random.default_rng(11)
    nh, nkh, hd, ps, S = 8, 2, 32, 16, 48
    q, k, v = make_case(rng, 1, [S], nh, nkh, hd)
    kp, vp, tables, n_pages = paged_copy(rng, k, v, [S], ps, nkh, hd)
    tables[0, 1] = -1
    k0, v0 = k[0].copy(), v[0].copy()
    k0[16:32] = 0
    v0[16:32] = 0
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    kv_p = dev.kv_view(cu(kp), cu(vp), block_tables=cu(tables), page_size=ps, n_pages=n_pages)
    got = dev.gqa_decode(O.ATTN_CE, cu(q), kv_p, torch.tensor([S], dtype=torch.int32, device="cuda"), S, nh, nkh,
                         hd).cpu().numpy()[0]
    ref = orc.gqa_decode(O.ATTN_CE, q[0], k0, v0, S, nh, nkh, hd)
    assert np.max(np.abs(got - ref)) <= ATTN_TOL * np.max(np.abs(ref))


def test_gqa_decode_empty_sequence_gives_zeros(dev):
    import torch
    nh, nkh, hd = 8, 2, 32
    q = torch.randn(2, nh * hd, device="cuda")
    k = torch.randn(2, 16, nkh * hd, device="cuda")
    kv = dev.kv_view(k, k.clone(), seq_stride=16 * nkh * hd)
    out = dev.gqa_decode(O.ATTN_GQA_C, q, kv, torch.tensor([0, 5], dtype=torch.int32, device="cuda"), 16, nh, nkh,
                         hd).cpu().numpy()
    assert np.all(out[0] == 0) and np.all(np.isfinite(out[1])) and np.any(out[1] != 0)


@pytest.mark.parametrize("paged", [False, True])
def test_kv_append_then_attend(dev, orc, paged):
    """Decode steps as GO:146-166 / CE:1354-1402 run them: RoPE on q and k at the
    position, K/V row appended, attention over position + 1 rows; three tokens
    of a batch of two sequences at different positions."""
    import torch
    rng = np.random.default_rng(21 + paged)
    nh, nkh, hd, ps, cap = 16, 4, 64, 32, 256
    B = 2
    pos0 = [37, 100]
    theta = rng.uniform(-3, 3, (cap, hd // 2))
    cos_t, sin_t = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
    k = rng.standard_normal((B, cap, nkh * hd)).astype(np.float32)
    v = rng.standard_normal((B, cap, nkh * hd)).astype(np.float32)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    if paged:
        n_pages = 2 * cap // ps
        perm = rng.permutation(n_pages)
        tables = perm.reshape(B, cap // ps).astype(np.int32)
        kp = np.zeros((n_pages, ps, nkh * hd), np.float32)
        vp = np.zeros_like(kp)
        for b in range(B):
            for s in range(pos0[b]):
                kp[tables[b, s // ps], s % ps] = k[b, s]
                vp[tables[b, s // ps], s % ps] = v[b, s]
        kd, vd = cu(kp), cu(vp)
        kv = dev.kv_view(kd, vd, block_tables=cu(tables), page_size=ps, n_pages=n_pages)
    else:
        kc, vc = k.copy(), v.copy()
        for b in range(B):
            kc[b, pos0[b]:] = 0
            vc[b, pos0[b]:] = 0
        kd, vd = cu(kc), cu(vc)
        kv = dev.kv_view(kd, vd, seq_stride=cap * nkh * hd)
    ct, st = cu(cos_t), cu(sin_t)
    for step in range(3):
        pos = [p + step for p in pos0]
        qn = rng.standard_normal((B, nh * hd)).astype(np.float32)
        kn = rng.standard_normal((B, nkh * hd)).astype(np.float32)
        vn = rng.standard_normal((B, nkh * hd)).astype(np.float32)
        posd = torch.tensor(pos, dtype=torch.int32, device="cuda")
        qd, knd = cu(qn), cu(kn)
        dev.rope(qd, nh, hd, posd, ct, st)
        dev.rope(knd, nkh, hd, posd, ct, st)
        dev.kv_append(kv, posd, knd, cu(vn), nkh, hd)
        lens = posd + 1
        got = dev.gqa_decode(O.ATTN_GQA_C, qd, kv, lens, cap, nh, nkh, hd).cpu().numpy()
        q_gpu, k_gpu = qd.cpu().numpy(), knd.cpu().numpy()
        for b in range(B):
            qr = orc.rope(qn[b], nh, hd, pos[b], cos_t, sin_t, hd)
            kr = orc.rope(kn[b], nkh, hd, pos[b], cos_t, sin_t, hd)
            assert np.max(np.abs(q_gpu[b] - qr)) <= 1e-6 * np.max(np.abs(qr))
            assert np.max(np.abs(k_gpu[b] - kr)) <= 1e-6 * np.max(np.abs(kr))
            # attention checked on the GPU's own rotated q, k (RoPE is checked just above)
            qr = q_gpu[b]
            k[b, pos[b]], v[b, pos[b]] = k_gpu[b], vn[b]
            S = pos[b] + 1
            ref = orc.gqa_decode(O.ATTN_GQA_C, qr, k[b], v[b], S, nh, nkh, hd)
            assert np.max(np.abs(got[b] - ref)) <= attn_tol(orc, O.ATTN_GQA_C, qr, k[b], v[b], S, nh, nkh, hd, ref)
    if paged:
        kp_after = kd.cpu().numpy()
        for b in range(B):
            for s in range(pos0[b], pos0[b] + 3):
                assert np.max(np.abs(kp_after[tables[b, s // ps], s % ps] - k[b, s])) <= 1e-5 * np.max(np.abs(k[b, s]))


@pytest.mark.parametrize("S", [1, 8, 1000, 4096])
def test_drop_in_gqa_attention_decode(lib, orc, S):
    """gqa_attention_decode through TE's argtypes (TE:383-385, 1600-1606): GPT-OSS
    head layout, host buffers, workspace of n_head * 4096 floats (TE:962-963)
    left as it was."""
    rng = np.random.default_rng(S)
    nh, nkh, hd = 64, 8, 64
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal((4096, nkh * hd)).astype(np.float32)
    v = rng.standard_normal((4096, nkh * hd)).astype(np.float32)
    out = np.full(nh * hd, np.nan, np.float32)
    ws = np.full(nh * 4096, 3.0, np.float32)
    lib.gqa_attention_decode(fp(q), fp(k), fp(v), fp(out), S, nh, nkh, hd, fp(ws))
    ref = orc.gqa_decode(O.ATTN_GQA_C, q, k, v, S, nh, nkh, hd)
    assert np.max(np.abs(out - ref)) <= attn_tol(orc, O.ATTN_GQA_C, q, k, v, S, nh, nkh, hd, ref), K.last_error(lib)
    assert np.all(ws == 3.0)


def test_drop_in_gqa_attention_decode_edges(lib):
    nh, nkh, hd = 8, 2, 32
    q = np.ones(nh * hd, np.float32)
    k = np.ones((4, nkh * hd), np.float32)
    out = np.full(nh * hd, 5.0, np.float32)
    lib.gqa_attention_decode(fp(q), fp(k), fp(k), fp(out), 0, nh, nkh, hd, fp(out))
    assert np.all(out == 0)
    out[:] = 5.0
    lib.gqa_attention_decode(fp(q), fp(k), fp(k), fp(out), 4, nh, 3, hd, fp(out))   # 8 % 3: not served
    assert np.all(out == 5.0) and "n_kv_head" in K.last_error(lib)


@pytest.mark.parametrize("nh,hd,r", [(64, 64, 64), (32, 128, 64), (8, 80, 80)])
def test_rope_vs_oracle(dev, orc, nh, hd, r):
    import torch
    rng = np.random.default_rng(nh + r)
    P, T = 50, 3
    theta = rng.uniform(-3, 3, (P, r // 2))
    cos_t, sin_t = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
    x = rng.standard_normal((T, nh * hd)).astype(np.float32)
    pos = [0, 17, 49]
    xd = torch.from_numpy(x).cuda()
    dev.rope(xd, nh, hd, torch.tensor(pos, dtype=torch.int32, device="cuda"), torch.from_numpy(cos_t).cuda(),
             torch.from_numpy(sin_t).cuda(), r)
    got = xd.cpu().numpy()
    for t in range(T):
        ref = orc.rope(x[t], nh, hd, pos[t], cos_t, sin_t, r)
        assert np.max(np.abs(got[t] - ref)) <= 1e-6 * np.max(np.abs(ref))
