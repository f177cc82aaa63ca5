// moe.hip — the MoE FFN layer for T tokens on device data.
//
// Semantics per token are those of moe_forward_omp (QK:2066-2250) fed by the
// C routing of moe_ffn (CE:606-638), renormalised as GO:88-92 /
// CE:1148-1152 when asked: gate/up per quant type (an MXFP4 pair in fp32,
// Q4_K through the Q8_0-activation dot), SiLU with the gate clamped to +-80,
// down per type (MXFP4 through Q8_0(h)), combined[n] = sum_k w_k * down_k in
// k order.
//
// Batched flow (T > kMoeDecodeMaxT = 24 tokens):
//   route -> stable bucketing of the T*K (token, slot) entries by expert on
//   the GPU -> grouped MFMA GEMM gate+up with the SiLU product in its
//   epilogue (bucket order) -> grouped MFMA GEMM down -> per-token combine
//   in k order through the inverse permutation.
// Decode flow (T <= 24): the same stages with the decode GEMV kernels, one job
// per (token, slot), no bucketing.
#include <stdio.h>
#include <string.h>
#include <algorithm>
#include <mutex>
#include <vector>
#include "gemm.h"
#include "gemv.h"
#include "mllm.h"
#include "moe.h"
#include "gemm16.h"

namespace {

constexpr int kTileEntries = 64;   // entries per grouped-GEMM work tile (gemm.hip TM)

// Stable bucketing of entries i = t*K + k by expert idx[i]: entry i lands at
// pos = off[e] + #{j < i : idx[j] == e}, so each bucket keeps index order
// (no atomics decide an order).  Two launches over blocks of 1024 entries:
//   k_bucket_rank: per block, an entry's rank among the block's entries of
//     its expert (its rank among its wave's equal lanes below it -- a 64-step
//     scan of the wave -- plus that expert's count in the block's earlier
//     waves) and the block's histogram hist[b][e];
//   k_bucket_place: per block, the bucket offsets off[0..E] (an exclusive
//     scan over experts of the histogram totals) plus the earlier blocks'
//     counts give each entry its position: perm[pos] = i, pos_of[i] = pos
//     (-1 for an expert id outside [0, E)), tok[pos] = i / K when tok is
//     given; block 0 also writes off[] and the work-tile list (<=
//     kTileEntries consecutive positions of one expert).
constexpr int kBucketThreads = 1024, kBucketWaves = kBucketThreads / 64;

__global__ __launch_bounds__(1024) void k_bucket_rank(const int *__restrict__ idx, int TK, int E,
                                                      int *__restrict__ hist, int *__restrict__ rank)
{
    __shared__ int wcnt[kBucketWaves][256];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int q = tid; q < kBucketWaves * 256; q += kBucketThreads) (&wcnt[0][0])[q] = 0;
    const int i = blockIdx.x * kBucketThreads + tid;
    int e = i < TK ? idx[i] : -1;
    const bool valid = e >= 0 && e < E;
    if (!valid) e = -1;
    int r = 0, tot = 0;
    for (int j = 0; j < 64; j++) {
        const int ej = __builtin_amdgcn_readlane(e, j);
        const int m = ej == e;
        tot += m;
        r += m & (j < lane);
    }
    __syncthreads();
    if (valid && r == 0) wcnt[wave][e] = tot;
    __syncthreads();
    if (valid) {
        for (int w = 0; w < wave; w++) r += wcnt[w][e];
        rank[i] = r;
    }
    if (tid < E) {
        int h = 0;
        for (int w = 0; w < kBucketWaves; w++) h += wcnt[w][tid];
        hist[(long)blockIdx.x * E + tid] = h;
    }
}

__global__ __launch_bounds__(1024) void k_bucket_place(const int *__restrict__ idx, int TK, int E, int K, int nblk,
                                                       const int *__restrict__ hist, const int *__restrict__ rank,
                                                       int *__restrict__ off, int *__restrict__ perm,
                                                       int *__restrict__ pos_of, int *__restrict__ tok,
                                                       int *__restrict__ tile_expert, int *__restrict__ tile_begin,
                                                       int *__restrict__ tile_end, int *__restrict__ n_tiles)
{
    __shared__ int base[256], scan[256], tbase[256];
    const int tid = threadIdx.x;
    // per expert: its total, and the entries of it in earlier blocks
    int c = 0, before = 0, nt = 0;
    if (tid < 256) {
        if (tid < E)
            for (int b = 0; b < nblk; b++) {
                const int h = hist[(long)b * E + tid];
                c += h;
                before += b < (int)blockIdx.x ? h : 0;
            }
        nt = (c + kTileEntries - 1) / kTileEntries;
        scan[tid] = c;
        tbase[tid] = nt;
    }
    __syncthreads();
    // inclusive scans over experts (Hillis-Steele, 256 wide)
    for (int d = 1; d < 256; d <<= 1) {
        int v = 0, w = 0;
        if (tid < 256 && tid >= d) { v = scan[tid - d]; w = tbase[tid - d]; }
        __syncthreads();
        if (tid < 256 && tid >= d) { scan[tid] += v; tbase[tid] += w; }
        __syncthreads();
    }
    if (tid < E) {
        const int b = scan[tid] - c;   // exclusive
        base[tid] = b + before;
        if (blockIdx.x == 0) {
            off[tid] = b;
            const int tb = tbase[tid] - nt;
            for (int t = 0; t < nt; t++) {
                tile_expert[tb + t] = tid;
                tile_begin[tb + t] = b + t * kTileEntries;
                tile_end[tb + t] = b + min(c, (t + 1) * kTileEntries);
            }
        }
    }
    if (blockIdx.x == 0 && tid == E - 1) {
        off[E] = scan[tid];
        *n_tiles = tbase[tid];
    }
    __syncthreads();
    const int i = blockIdx.x * kBucketThreads + tid;
    if (i >= TK) return;
    const int e = idx[i];
    if (e >= 0 && e < E) {
        const int pos = base[e] + rank[i];
        perm[pos] = i;
        pos_of[i] = pos;
        if (tok) tok[pos] = i / K;
    } else {
        pos_of[i] = -1;
    }
}

// Both bucketing launches; hist needs (TK/1024 + 1) * E ints and rank TK ints of scratch.
hipError_t launch_bucket(const int *idx, int TK, int E, int K, int *hist, int *rank, int *off, int *perm,
                         int *pos_of, int *tok, int *tile_expert, int *tile_begin, int *tile_end, int *n_tiles,
                         hipStream_t st)
{
    const int nblk = (TK + kBucketThreads - 1) / kBucketThreads;
    hipLaunchKernelGGL(k_bucket_rank, dim3(nblk), dim3(kBucketThreads), 0, st, idx, TK, E, hist, rank);
    hipLaunchKernelGGL(k_bucket_place, dim3(nblk), dim3(kBucketThreads), 0, st, idx, TK, E, K, nblk, hist, rank,
                       off, perm, pos_of, tok, tile_expert, tile_begin, tile_end, n_tiles);
    return hipGetLastError();
}

size_t bucket_scratch_ints(int TK, int E) { return (size_t)(TK / kBucketThreads + 1) * E + TK; }

// out[t][n] = sum over k (in order) of w[t][k] * dn[pos_of[t*K+k]][n], as
// moe_forward_omp's combined[row] += top_weight * dot (QK:2243-2244); every dn
// term is 0 when dn is null (a down type the reference leaves at zero).
__global__ void k_combine_pos(const float *__restrict__ dn, const float *__restrict__ w,
                              const int *__restrict__ pos_of, int K, int N, float *__restrict__ out)
{
    // four consecutive n per thread (N % 4 == 0: 16-byte loads), the same
    // per-element arithmetic as one n per thread
    const int t = blockIdx.y;
    const int n = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
    if (n >= N) return;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int k = 0; k < K; k++) {
        const int pos = pos_of[t * K + k];
        if (pos < 0) continue;
        const float wk = w[t * K + k];
        const float4 v = dn ? *reinterpret_cast<const float4 *>(dn + (long)pos * N + n) : make_float4(0.f, 0.f, 0.f, 0.f);
        acc.x += wk * v.x; acc.y += wk * v.y; acc.z += wk * v.z; acc.w += wk * v.w;
    }
    *reinterpret_cast<float4 *>(out + (long)t * N + n) = acc;
}

__global__ void k_combine_pos1(const float *__restrict__ dn, const float *__restrict__ w,
                               const int *__restrict__ pos_of, int K, int N, float *__restrict__ out)
{
    const int t = blockIdx.y;
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    float acc = 0.0f;
    for (int k = 0; k < K; k++) {
        const int pos = pos_of[t * K + k];
        if (pos >= 0) acc += w[t * K + k] * (dn ? dn[(long)pos * N + n] : 0.0f);
    }
    out[(long)t * N + n] = acc;
}

size_t a256(size_t n) { return (n + 255) / 256 * 256; }

size_t xq_size(long rows, int n_cols)
{
    const long nb = n_cols / 32;
    return a256(rows * nb * 32) + 3 * a256(rows * nb * 4);
}

mllm_xq xq_at(uint8_t *p, long rows, int n_cols, int8_t **q, float **d, float **s4, int **sq)
{
    const long nb = n_cols / 32;
    *q = (int8_t *)p; p += a256(rows * nb * 32);
    *d = (float *)p; p += a256(rows * nb * 4);
    *s4 = (float *)p; p += a256(rows * nb * 4);
    *sq = (int *)p;
    return mllm_xq{*q, *d, *s4, *sq};
}

int sem_gu_of(int qt_gate, int qt_up, int which)
{
    if (qt_gate == 39 && qt_up == 39) return SEM_MXFP4;          // QK:2094
    const int qt = which == 0 ? qt_gate : qt_up;
    switch (qt) {                                                 // QK:2114-2152
    case 12: return SEM_Q4_K_Q8; case 14: return SEM_Q6_K_LOWNIB; case 2: return SEM_Q4_0;
    case 3: return SEM_Q4_1; case 6: return SEM_Q5_0_Q8;
    }
    return -1;
}

int sem_down_of(int qt)
{
    switch (qt) {                                                 // QK:2192-2245
    case 39: return SEM_MXFP4_Q8; case 14: return SEM_Q6_K_LOWNIB; case 2: return SEM_Q4_0; case 6: return SEM_Q5_0_F32;
    }
    return -1;
}

int xmode_of(int sem)
{
    return sem == SEM_Q4_K_Q8 ? XM_Q8 : sem == SEM_MXFP4_Q8 ? XM_Q8D : XM_PLANES;
}

} // namespace

struct mllm_moe_layer {
    int N, M, E, K, renorm;
    int sem_g, sem_u, sem_d;
    int clamp;          // SiLU with the gate clamped to +-80 (moe_forward_omp) or not (moe_ffn)
    int gemv_only;      // weights the grouped GEMMs would not reproduce (mllm_moe_needs_gemv)
    int owns_router, owns_tab;
    float *router_p;    // device, routing layout (mllm_router_pack); freed with the layer when owned
    mllm_packed *tab;   // device: [E] gate, [E] up, [E] down; freed with the layer when owned
    // load-time bf16 copies of the bf16-exact expert matrices (mllm_moe_dense_experts):
    // dtab as tab with p[0] = bf16 rows of stride ld_gu (gate/up) or ld_d (down);
    // dense_gu / dense_d: the batched path reads them
    mllm_packed *dtab = nullptr;
    void *dmem = nullptr;
    int dense_gu = 0, dense_d = 0, ld_gu = 0, ld_d = 0;
    // MXFP4 on the fp16-plane GEMM (mllm_q16_mx_shift of the matrices' exponent range):
    // gate/up (both MXFP4) and down, with their exponent offsets and result scales
    int mx_gu = 0, mx_d = 0, eoff_gu = 0, eoff_d = 0;
    float ws_gu = 1.0f, ws_d = 1.0f;
    // step-major metadata (mllm_launch_q16_smeta) of the matrices the fp16-plane GEMM
    // multiplies: gate / up / down of expert e at sm_g / sm_u / sm_d + e * stride
    uint8_t *smem = nullptr, *sm_g = nullptr, *sm_u = nullptr, *sm_d = nullptr;
    long sms_gu = 0, sms_d = 0, smd_gu = 0, smd_d = 0;
};

struct moe_ws {
    int *idx, *off, *perm, *pos_of, *tok, *tile_expert, *tile_begin, *tile_end, *n_tiles, *bscr;
    float *w, *g, *u, *h, *dn;
    uint8_t *xq_x, *xq_h;
    __bf16 *xp_x, *xp_h;      // split planes of x [T][N] and h [T*K][M] (batched path)
    int *lo_x, *lo_h;
    float *logits;            // routing logits [T][E] (decode path, expert slices)
    uint8_t *a16_x, *a16_h;   // fp16-plane GEMM activations of x and h (batched path), or null
};

// Whether the batched path runs gate/up and down on the fp16-plane GEMM (gemm16.h):
// K-quant semantics over whole super-blocks, on the packed experts (not the dense copies);
// MXFP4 over whole 64-element steps when the exponent ranges fit (moe_q16_setup).
static bool moe_q16_gu(const mllm_moe_layer &L)
{
    return (L.sem_g == L.sem_u && mllm_q16_supported(L.sem_g) && !L.dense_gu && L.N % 256 == 0) ||
           (L.mx_gu && L.N % 64 == 0);
}
static bool moe_q16_d(const mllm_moe_layer &L)
{
    return (L.sem_d >= 0 && mllm_q16_supported(L.sem_d) && !L.dense_d && L.M % 256 == 0) || (L.mx_d && L.M % 64 == 0);
}

// The fp16-plane GEMM's per-layer state: the MXFP4 exponent ranges (mx_gu / mx_d where
// they fit) and the step-major metadata of the matrices it multiplies.  Returns 0, or -1
// on a HIP error.
static int moe_q16_setup(mllm_moe_layer *L)
{
    if (L->gemv_only) return 0;
    const int E = L->E, N = L->N, M = L->M;
    const bool gmx = L->sem_g == SEM_MXFP4 && L->sem_u == SEM_MXFP4, dmx = L->sem_d == SEM_MXFP4_Q8;
    if (gmx || dmx) {
        int h[4] = {255, 0, 255, 0};
        int *f = nullptr;
        if (hipMalloc(&f, sizeof h) != hipSuccess) return -1;
        hipError_t r = hipMemcpy(f, h, sizeof h, hipMemcpyHostToDevice);
        if (r == hipSuccess && gmx) r = mllm_launch_mx_erange(L->tab, 2 * E, M, N, f, nullptr);
        if (r == hipSuccess && dmx) r = mllm_launch_mx_erange(L->tab + 2 * E, E, N, M, f + 2, nullptr);
        if (r == hipSuccess) r = hipMemcpy(h, f, sizeof h, hipMemcpyDeviceToHost);
        (void)hipFree(f);
        if (r != hipSuccess) return -1;
        if (gmx) L->mx_gu = mllm_q16_mx_shift(h[0], h[1], &L->eoff_gu, &L->ws_gu);
        if (dmx) L->mx_d = mllm_q16_mx_shift(h[2], h[3], &L->eoff_d, &L->ws_d);
    }
    // gate and up in Q6_K run without it (mllm_launch_q16)
    const bool gu = moe_q16_gu(*L) && L->sem_g != SEM_Q6_K_SEQ && L->sem_g != SEM_Q6_K_LOWNIB, dn = moe_q16_d(*L);
    if (!gu && !dn) return 0;
    const long sg = gu ? mllm_q16_smeta_bytes(L->sem_g, M, N, &L->smd_gu) : 0;
    const long sd = dn ? mllm_q16_smeta_bytes(L->sem_d, N, M, &L->smd_d) : 0;
    uint8_t *m = nullptr;
    if (hipMalloc(&m, (size_t)(2 * E * sg + E * sd)) != hipSuccess) return -1;
    if ((gu && (mllm_launch_q16_smeta(L->sem_g, L->tab, E, M, N, m, sg, nullptr) != hipSuccess ||
                mllm_launch_q16_smeta(L->sem_u, L->tab + E, E, M, N, m + E * sg, sg, nullptr) != hipSuccess)) ||
        (dn && mllm_launch_q16_smeta(L->sem_d, L->tab + 2 * E, E, N, M, m + 2 * E * sg, sd, nullptr) != hipSuccess) ||
        hipStreamSynchronize(nullptr) != hipSuccess) {
        (void)hipFree(m);
        return -1;
    }
    L->smem = m;
    if (gu) { L->sm_g = m; L->sm_u = m + E * sg; }
    if (dn) L->sm_d = m + 2 * E * sg;
    L->sms_gu = sg; L->sms_d = sd;
    return 0;
}

// Tokens up to which the layer runs the decode GEMVs (one job per (token,
// slot); an expert picked by several tokens is streamed once per token) rather
// than the bucketed grouped GEMMs.  Measured on MI355X: GPT-OSS shape 225 vs
// 388 us at T = 16, 407 vs 385 us at T = 32; Qwen3 shape 119 vs 256 us at
// T = 16, 219 vs 312 us at T = 32, 358 vs 342 us at T = 64.
constexpr int kMoeDecodeMaxT = 24;

static size_t moe_ws_layout(const mllm_moe_layer &L, int T, moe_ws *w, uint8_t *base)
{
    const size_t TK = (size_t)T * L.K;
    const size_t max_tiles = TK / kTileEntries + L.E + 1;
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t at = o; o += a256(bytes); return base ? base + at : nullptr; };
    moe_ws s;
    s.idx = (int *)take(TK * 4);
    s.w = (float *)take(TK * 4);
    s.off = (int *)take((L.E + 1) * 4);
    s.perm = (int *)take(TK * 4);
    s.pos_of = (int *)take(TK * 4);
    s.tok = (int *)take(TK * 4);
    s.bscr = (int *)take(bucket_scratch_ints((int)TK, L.E) * 4);
    s.tile_expert = (int *)take(max_tiles * 4);
    s.tile_begin = (int *)take(max_tiles * 4);
    s.tile_end = (int *)take(max_tiles * 4);
    s.n_tiles = (int *)take(4);
    s.g = (float *)take(TK * L.M * 4);
    s.u = (float *)take(TK * L.M * 4);
    s.h = (float *)take(TK * L.M * 4);
    s.dn = (float *)take(TK * L.N * 4);
    s.xq_x = take(xq_size(T, L.N));
    s.xq_h = take(xq_size((long)TK, L.M));
    s.xp_x = (__bf16 *)take(3 * act_planes_elems(T, L.N) * 2);
    s.xp_h = (__bf16 *)take(3 * act_planes_elems((long)TK, L.M) * 2);
    s.lo_x = (int *)take((size_t)T * 4);
    s.lo_h = (int *)take(TK * 4);
    s.logits = (float *)take((size_t)mllm_route_workspace_floats(T, L.E) * 4);
    s.a16_x = moe_q16_gu(L) ? take(mllm_act16_bytes(L.sem_g, T, L.N)) : nullptr;
    s.a16_h = moe_q16_d(L) ? take(mllm_act16_bytes(L.sem_d, (long)TK, L.M)) : nullptr;
    if (w) *w = s;
    return o;
}

extern "C" {

MLLM_API mllm_moe_layer *mllm_moe_prepare(int qt_gate, int qt_up, int qt_down, int N, int M, int E, int K,
                                          const void *const *gate_packed, const void *const *up_packed,
                                          const void *const *down_packed, const float *router_dev, int renorm)
{
    if (E <= 0 || E > 256 || K <= 0 || K > 16 || K > E || N <= 0 || M <= 0) return nullptr;
    mllm_moe_layer *L = new mllm_moe_layer;
    L->N = N; L->M = M; L->E = E; L->K = K; L->renorm = renorm;
    L->clamp = 1;
    L->owns_router = 1;
    L->owns_tab = 1;
    L->sem_g = sem_gu_of(qt_gate, qt_up, 0);
    L->sem_u = sem_gu_of(qt_gate, qt_up, 1);
    L->sem_d = qt_down == 12 ? -2 : sem_down_of(qt_down);     // Q4_K down: the reference adds zeros
    L->router_p = nullptr;
    L->tab = nullptr;
    L->gemv_only = 0;
    std::vector<mllm_packed> tab(3 * (size_t)E);
    for (int e = 0; e < E; e++) {
        if (L->sem_g >= 0) tab[e] = mllm_packed_view(mllm_sem_layout(L->sem_g), (const uint8_t *)gate_packed[e], M, N);
        if (L->sem_u >= 0) tab[E + e] = mllm_packed_view(mllm_sem_layout(L->sem_u), (const uint8_t *)up_packed[e], M, N);
        if (L->sem_d >= 0) tab[2 * E + e] = mllm_packed_view(mllm_sem_layout(L->sem_d), (const uint8_t *)down_packed[e], N, M);
    }
    const size_t rbytes = (size_t)mllm_router_packed_floats(N, E) * sizeof(float);
    if (hipMalloc(&L->tab, tab.size() * sizeof(mllm_packed)) != hipSuccess ||
        hipMemcpy(L->tab, tab.data(), tab.size() * sizeof(mllm_packed), hipMemcpyHostToDevice) != hipSuccess ||
        hipMalloc(&L->router_p, rbytes) != hipSuccess ||
        mllm_launch_router_pack(router_dev, N, E, L->router_p, nullptr) != hipSuccess ||
        hipStreamSynchronize(nullptr) != hipSuccess ||
        (L->gemv_only = mllm_moe_needs_gemv(L->tab, L->sem_g, L->sem_u, L->sem_d, N, M, E)) < 0 ||
        moe_q16_setup(L) != 0) {
        mllm_moe_release(L);
        return nullptr;
    }
    return L;
}

MLLM_API void mllm_moe_release(mllm_moe_layer *L)
{
    if (!L) return;
    if (L->tab && L->owns_tab) (void)hipFree(L->tab);
    if (L->dtab) (void)hipFree(L->dtab);
    if (L->dmem) (void)hipFree(L->dmem);
    if (L->smem) (void)hipFree(L->smem);
    if (L->router_p && L->owns_router) (void)hipFree(L->router_p);
    delete L;
}

// Load-time bf16 plane copies of the expert matrices (mllm_launch_dense_planes:
// the values put_w would write into the tiles, so results are bit-identical);
// gate and up take them when they share a semantic.  Only matrices the batched
// path runs on the bf16-tile GEMM are copied: those on the fp16-plane GEMM
// (moe_q16_gu / moe_q16_d) never read a copy.
MLLM_API long mllm_moe_dense_experts(mllm_moe_layer *L, void *stream)
{
    if (!L) return -1;
    if (L->dmem) return 0;
    const int pg = L->sem_g >= 0 ? mllm_dense_planes(L->sem_g) : 0;
    const int pd = L->sem_d >= 0 ? mllm_dense_planes(L->sem_d) : 0;
    const bool gu = !L->gemv_only && pg > 0 && L->sem_g == L->sem_u && !moe_q16_gu(*L);
    const bool dn = !L->gemv_only && pd > 0 && !moe_q16_d(*L);
    if (!gu && !dn) return 0;
    hipStream_t st = (hipStream_t)stream;
    const int E = L->E, N = L->N, M = L->M;
    const int ld_gu = (N + 63) / 64 * 64, ld_d = (M + 63) / 64 * 64;
    const size_t mgu = (size_t)pg * M * ld_gu, md = (size_t)pd * N * ld_d;   // elements per matrix copy
    const size_t total = (gu ? 2 * E * mgu : 0) + (dn ? E * md : 0);
    std::vector<mllm_packed> tab(3 * (size_t)E), dtab(3 * (size_t)E);
    __bf16 *mem = nullptr;
    if (hipMemcpy(tab.data(), L->tab, tab.size() * sizeof(mllm_packed), hipMemcpyDeviceToHost) != hipSuccess ||
        hipMalloc(&mem, total * 2) != hipSuccess)
        return -1;
    bool ok = hipMemsetAsync(mem, 0, total * 2, st) == hipSuccess;
    size_t at = 0;
    auto copy = [&](int which, int sem, int rows, int cols, int ld, size_t elems) {
        for (int e = 0; e < E && ok; e++) {
            __bf16 *dst = mem + at;
            at += elems;
            ok = mllm_launch_dense_planes(sem, tab[(size_t)which * E + e], rows, cols, ld, dst, st) == hipSuccess;
            dtab[(size_t)which * E + e].p[0] = reinterpret_cast<const uint8_t *>(dst);
        }
    };
    if (gu) { copy(0, L->sem_g, M, N, ld_gu, mgu); copy(1, L->sem_u, M, N, ld_gu, mgu); }
    if (dn) copy(2, L->sem_d, N, M, ld_d, md);
    ok = ok && hipStreamSynchronize(st) == hipSuccess;
    if (ok && (hipMalloc(&L->dtab, dtab.size() * sizeof(mllm_packed)) != hipSuccess ||
               hipMemcpy(L->dtab, dtab.data(), dtab.size() * sizeof(mllm_packed), hipMemcpyHostToDevice) != hipSuccess))
        ok = false;
    if (!ok) {
        (void)hipFree(mem);
        if (L->dtab) (void)hipFree(L->dtab);
        L->dtab = nullptr;
        return -1;
    }
    L->dmem = mem;
    L->dense_gu = gu;
    L->dense_d = dn;
    L->ld_gu = ld_gu;
    L->ld_d = ld_d;
    return (long)(total * 2);
}

MLLM_API long mllm_moe_workspace_size(const mllm_moe_layer *L, int T)
{
    return L ? (long)moe_ws_layout(*L, T, nullptr, nullptr) : -1;
}

MLLM_API int mllm_moe_layer_info(const mllm_moe_layer *L)
{
    if (!L) return -1;
    return (moe_q16_gu(*L) ? 1 : 0) | (moe_q16_d(*L) ? 2 : 0) | (L->gemv_only ? 4 : 0);
}

} // extern "C"

// x [T][N] fp32 -> out [T][N].  Routing from the layer's router, or, with
// idx_in / w_in (device [T][K]), the caller's (moe_forward_omp's own contract,
// QK:2066-2071).  idx_out / w_out (optional) receive the routing used.
static int moe_forward_impl(const mllm_moe_layer *L, const float *x, int T, float *out, void *workspace,
                            long ws_bytes, int *idx_out, float *w_out, const int *idx_in, const float *w_in,
                            hipStream_t st)
{
    if (!L || T <= 0) return -1;
    if (ws_bytes < (long)moe_ws_layout(*L, T, nullptr, nullptr)) return -1;
    moe_ws s;
    moe_ws_layout(*L, T, &s, (uint8_t *)workspace);
    const int N = L->N, M = L->M, E = L->E, K = L->K, TK = T * K;
#define CK(e) do { if ((e) != hipSuccess) return -1; } while (0)
    if (idx_in && w_in) {
        s.idx = const_cast<int *>(idx_in);
        s.w = const_cast<float *>(w_in);
    } else {
        if (!L->router_p) return -1;
        CK(mllm_launch_route(L->router_p, x, T, N, E, K, L->renorm, s.idx, s.w, s.logits, st));
    }
    if (L->sem_g < 0 || L->sem_u < 0) return -1;   // reference-zero gate/up types are not served here
    int8_t *q; float *d, *s4; int *sq;
    const mllm_xq xqx = xq_at(s.xq_x, T, N, &q, &d, &s4, &sq);
    int8_t *hq; float *hd, *hs4; int *hsq;
    const mllm_xq xqh = xq_at(s.xq_h, TK, M, &hq, &hd, &hs4, &hsq);

    // the grouped GEMMs need at least one quant block per row (else the decode
    // GEMVs write the reference's zeros)
    const bool batched = !L->gemv_only && T > kMoeDecodeMaxT && mllm_qgemm_supported(L->sem_g) && mllm_qgemm_supported(L->sem_u) &&
                         (L->sem_d < 0 || mllm_qgemm_supported(L->sem_d)) &&
                         N >= mllm_sem_block_elems(L->sem_g) && N >= mllm_sem_block_elems(L->sem_u) &&
                         (L->sem_d < 0 || M >= mllm_sem_block_elems(L->sem_d));
    if (batched) {
        if (mllm_sem_uses_q8(L->sem_g) || mllm_sem_uses_q8(L->sem_u))
            CK(mllm_launch_quantize_q8_0(x, T, N, nullptr, q, d, s4, sq, st));
        CK(launch_bucket(s.idx, TK, E, K, s.bscr, s.bscr + (TK / kBucketThreads + 1) * E, s.off, s.perm, s.pos_of,
                         s.tok, s.tile_expert, s.tile_begin, s.tile_end, s.n_tiles, st));
        const int max_tiles = TK / kTileEntries + E + 1;
        static_assert(kTileEntries == 64, "the bucketing's tiles are the grouped GEMMs' 64-entry tiles");
        if (moe_q16_gu(*L)) {
            // gate + up + SiLU in bucket order on the fp16-plane GEMM
            const act16 ax = mllm_act16_carve(L->sem_g, s.a16_x, T, N);
            CK(mllm_launch_act16(L->sem_g, x, N, &xqx, T, N, ax, st));
            q16_args a{};
            a.table = L->tab; a.table2 = L->tab + E;
            a.sm = L->sm_g; a.sm2 = L->sm_u; a.sm_stride = L->sms_gu; a.sm_doff = L->smd_gu;
            a.x = ax;
            a.row_of = s.tok;
            a.out = s.h; a.ldo = M;
            a.n_rows = M; a.n_cols = N; a.n_entries = TK;
            a.tile_expert = s.tile_expert; a.tile_begin = s.tile_begin; a.tile_end = s.tile_end; a.n_tiles = s.n_tiles;
            a.clamp_silu = L->clamp;
            a.ksplit = 1;
            a.eoff = L->eoff_gu; a.wscale = L->ws_gu;
            CK(mllm_launch_q16(L->sem_g, true, a, max_tiles, st));
        } else {
        // gate + up (+ SiLU) in bucket order
        qgemm_args a{};
        a.table = L->tab; a.table2 = L->tab + E;
        if (L->dense_gu) { a.table = L->dtab; a.table2 = L->dtab + E; a.dense_ld = L->ld_gu; }
        a.xq = xqx;
        if (xmode_of(L->sem_g) == XM_PLANES || xmode_of(L->sem_u) == XM_PLANES) {
            const long pe = act_planes_elems(T, N);
            const int np = std::max(xmode_of(L->sem_g) == XM_PLANES ? act_nplanes(L->sem_g) : 2,
                                    xmode_of(L->sem_u) == XM_PLANES ? act_nplanes(L->sem_u) : 2);
            CK(mllm_launch_act_split(x, N, T, N, np, s.xp_x, pe, s.lo_x, st));
            a.xp = {s.xp_x, pe, act_planes_ld(N), s.lo_x};
        }
        a.row_of = s.tok;
        a.n_rows = M; a.n_cols = N;
        a.tile_expert = s.tile_expert; a.tile_begin = s.tile_begin; a.tile_end = s.tile_end; a.n_tiles = s.n_tiles;
        a.clamp_silu = L->clamp;
        if (L->sem_g == L->sem_u) {
            a.out = s.h; a.ldo = M;
            CK(mllm_launch_qgemm(L->sem_g, xmode_of(L->sem_g), true, a, max_tiles, st));
        } else {
            a.out = s.g; a.ldo = M;
            CK(mllm_launch_qgemm(L->sem_g, xmode_of(L->sem_g), false, a, max_tiles, st));
            a.table = (L->dense_gu ? L->dtab : L->tab) + E; a.out = s.u;
            CK(mllm_launch_qgemm(L->sem_u, xmode_of(L->sem_u), false, a, max_tiles, st));
            CK(mllm_launch_silu_mul(s.g, s.u, s.h, (long)TK * M, L->clamp, st));
        }
        }
        // down, rows of h already in bucket order
        if (moe_q16_d(*L)) {
            const act16 ah = mllm_act16_carve(L->sem_d, s.a16_h, TK, M);
            // (MXFP4 x Q8_0: the activation kernel quantises h to Q8_0 itself)
            CK(mllm_launch_act16(L->sem_d, s.h, M, &xqh, TK, M, ah, st));
            q16_args b{};
            b.table = L->tab + 2 * E;
            b.sm = L->sm_d; b.sm_stride = L->sms_d; b.sm_doff = L->smd_d;
            b.x = ah;
            b.out = s.dn; b.ldo = N;
            b.n_rows = N; b.n_cols = M; b.n_entries = TK;
            b.tile_expert = s.tile_expert; b.tile_begin = s.tile_begin; b.tile_end = s.tile_end; b.n_tiles = s.n_tiles;
            b.ksplit = 1;
            b.eoff = L->eoff_d; b.wscale = L->ws_d;
            CK(mllm_launch_q16(L->sem_d, false, b, max_tiles, st));
        } else if (L->sem_d >= 0) {
            if (mllm_sem_uses_q8(L->sem_d)) CK(mllm_launch_quantize_q8_0(s.h, TK, M, nullptr, hq, hd, hs4, hsq, st));
            qgemm_args b{};
            b.table = L->tab + 2 * E;
            if (L->dense_d) { b.table = L->dtab + 2 * E; b.dense_ld = L->ld_d; }
            b.xq = xqh;
            if (xmode_of(L->sem_d) == XM_PLANES) {
                const long pe = act_planes_elems((long)TK, M);
                CK(mllm_launch_act_split(s.h, M, TK, M, act_nplanes(L->sem_d), s.xp_h, pe, s.lo_h, st));
                b.xp = {s.xp_h, pe, act_planes_ld(M), s.lo_h};
            }
            b.out = s.dn; b.ldo = N;
            b.n_rows = N; b.n_cols = M;
            b.tile_expert = s.tile_expert; b.tile_begin = s.tile_begin; b.tile_end = s.tile_end; b.n_tiles = s.n_tiles;
            CK(mllm_launch_qgemm(L->sem_d, xmode_of(L->sem_d), false, b, max_tiles, st));
        }
        if (N % 4 == 0 && ((uintptr_t)out & 15) == 0)
            hipLaunchKernelGGL(k_combine_pos, dim3((N / 4 + 255) / 256, T), dim3(256), 0, st,
                               L->sem_d >= 0 ? s.dn : nullptr, s.w, s.pos_of, K, N, out);
        else
            hipLaunchKernelGGL(k_combine_pos1, dim3((N + 255) / 256, T), dim3(256), 0, st,
                               L->sem_d >= 0 ? s.dn : nullptr, s.w, s.pos_of, K, N, out);
        CK(hipGetLastError());
    } else {
        // decode: one GEMV launch per projection over all T*K (token, slot)
        // jobs, the expert picked on the device; gate and up share a launch
        // when their semantics agree; Q8_0 activations are quantised by the
        // GEMV workgroups themselves, and the SiLU product is formed while
        // the down projection stages (or quantises) its activations
        mllm_gemv_args a{};
        a.table = L->tab; a.idx = s.idx; a.job_div = K;
        a.x = x; a.x_job_stride = N; a.ldx = N;
        a.out = s.g; a.out_job_stride = M; a.ldo = M;
        a.n_rows = M; a.n_cols = N; a.B = 1;
        if (L->sem_g == L->sem_u && L->sem_d >= 0 && mllm_gemv_fused_fits(L->sem_g, N, 1, false)) {
            // gate, up and the SiLU product in one launch (paired rows: the expert's
            // gate row from table, its up row from table2), h written directly
            a.table2 = L->tab + E; a.silu_pair = 1; a.silu_noclamp = !L->clamp;
            a.out = s.h;
            CK(mllm_launch_gemv(L->sem_g, a, TK, st));
            mllm_gemv_args b{};
            b.table = L->tab + 2 * (size_t)E; b.idx = s.idx;
            b.x = s.h; b.x_job_stride = M; b.ldx = M;
            b.out = s.dn; b.out_job_stride = N; b.ldo = N;
            b.n_rows = N; b.n_cols = M; b.B = 1;
            CK(mllm_launch_gemv(L->sem_d, b, TK, st));
            CK(mllm_launch_combine(s.dn, s.w, s.idx, T, K, N, out, 0, st));
            if (idx_out) CK(hipMemcpyAsync(idx_out, s.idx, (size_t)TK * 4, hipMemcpyDeviceToDevice, st));
            if (w_out) CK(hipMemcpyAsync(w_out, s.w, (size_t)TK * 4, hipMemcpyDeviceToDevice, st));
            return 0;
        }
        if (L->sem_g == L->sem_u) {
            a.job_split = TK; a.table2 = L->tab + E; a.out2 = s.u;
            CK(mllm_launch_gemv(L->sem_g, a, 2 * TK, st));
        } else {
            CK(mllm_launch_gemv(L->sem_g, a, TK, st));
            a.table = L->tab + E; a.out = s.u;
            CK(mllm_launch_gemv(L->sem_u, a, TK, st));
        }
        if (L->sem_d >= 0) {
            mllm_gemv_args b{};
            b.table = L->tab + 2 * (size_t)E; b.idx = s.idx;
            b.x = s.g; b.x_job_stride = M; b.ldx = M;
            b.out = s.dn; b.out_job_stride = N; b.ldo = N;
            b.n_rows = N; b.n_cols = M; b.B = 1;
            if (L->sem_d == SEM_F32 || !L->clamp) {
                // the down GEMV forms the clamped SiLU product itself; a separate
                // product for fp32 rows and for the unclamped SiLU
                CK(mllm_launch_silu_mul(s.g, s.u, s.h, (long)TK * M, L->clamp, st));
                b.x = s.h;
            } else {
                b.x_up = s.u;
            }
            CK(mllm_launch_gemv(L->sem_d, b, TK, st));
        }
        CK(mllm_launch_combine(L->sem_d >= 0 ? s.dn : nullptr, s.w, s.idx, T, K, N, out, 0, st));
    }
    if (idx_out) CK(hipMemcpyAsync(idx_out, s.idx, (size_t)TK * 4, hipMemcpyDeviceToDevice, st));
    if (w_out) CK(hipMemcpyAsync(w_out, s.w, (size_t)TK * 4, hipMemcpyDeviceToDevice, st));
#undef CK
    return 0;
}

int mllm_moe_forward_routed(const mllm_moe_layer *L, const float *x, int T, float *out, void *workspace,
                            long ws_bytes, const int *idx, const float *w, hipStream_t st)
{
    if (!idx || !w) return -1;
    return moe_forward_impl(L, x, T, out, workspace, ws_bytes, nullptr, nullptr, idx, w, st);
}

mllm_moe_layer *mllm_moe_layer_for_codes(int qt_gate, int qt_up, int qt_down, int N, int M, int E, int K,
                                         const mllm_packed *tab_dev)
{
    if (E <= 0 || E > 256 || K <= 0 || K > 16 || K > E || N <= 0 || M <= 0 || !tab_dev) return nullptr;
    mllm_moe_layer *L = new mllm_moe_layer;
    L->N = N; L->M = M; L->E = E; L->K = K; L->renorm = 0;
    L->clamp = 1;
    L->owns_router = 0;
    L->owns_tab = 0;
    L->sem_g = sem_gu_of(qt_gate, qt_up, 0);
    L->sem_u = sem_gu_of(qt_gate, qt_up, 1);
    L->sem_d = qt_down == 12 ? -2 : sem_down_of(qt_down);
    L->router_p = nullptr;
    L->tab = const_cast<mllm_packed *>(tab_dev);
    L->gemv_only = mllm_moe_needs_gemv(tab_dev, L->sem_g, L->sem_u, L->sem_d, N, M, E);
    if (L->sem_g < 0 || L->sem_u < 0 || L->gemv_only < 0 || moe_q16_setup(L) != 0) {
        delete L;
        return nullptr;
    }
    return L;
}

void mllm_moe_codes_sems(int qt_gate, int qt_up, int qt_down, int *sem_g, int *sem_u, int *sem_d)
{
    *sem_g = sem_gu_of(qt_gate, qt_up, 0);
    *sem_u = sem_gu_of(qt_gate, qt_up, 1);
    *sem_d = qt_down == 12 ? -2 : sem_down_of(qt_down);
}

extern "C" {

MLLM_API int mllm_moe_forward(const mllm_moe_layer *L, const float *x, int T, float *out, void *workspace,
                              long ws_bytes, int *idx_out, float *w_out, void *stream)
{
    return moe_forward_impl(L, x, T, out, workspace, ws_bytes, idx_out, w_out, nullptr, nullptr, (hipStream_t)stream);
}

} // extern "C"

// ------------------------------------------------ no-allocation forward
// mllm_moe_forward_noalloc's workspace: a file-scope device array that every
// GPU the library runs on holds until the process ends.  In host code its
// name is a host-side stand-in, not a device address: the device address is
// taken once per device with hipGetSymbolAddress (with that device current)
// and only that address is handed to kernels.
static __device__ __align__(256) uint8_t scratch[MLLM_MOE_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// The current device's copy of `scratch`, looked up on the first call on that device.
int scratch_for_current_device(void **out)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        mllm_set_error("mllm_moe_forward_noalloc: no current HIP device");
        return -1;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (r != hipSuccess || !p) {
            char msg[160];
            snprintf(msg, sizeof msg, "mllm_moe_forward_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                     hipGetErrorString(r));
            mllm_set_error(msg);
            return -1;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}
} // namespace

extern "C" {

MLLM_API int mllm_moe_forward_noalloc(const mllm_moe_layer *L, const float *x, int T, float *out, int *idx_out,
                                      float *w_out, void *stream)
{
    if (!L || T <= 0) { mllm_set_error("mllm_moe_forward_noalloc: no layer or T <= 0"); return -1; }
    const size_t need = moe_ws_layout(*L, T, nullptr, nullptr);
    if (need > (size_t)MLLM_MOE_NOALLOC_SCRATCH_BYTES) {
        char msg[200];
        snprintf(msg, sizeof msg,
                 "mllm_moe_forward_noalloc: T=%d needs %zu bytes of workspace, above the %d-byte static maximum",
                 T, need, (int)MLLM_MOE_NOALLOC_SCRATCH_BYTES);
        mllm_set_error(msg);
        return -1;
    }
    void *ws = nullptr;
    if (scratch_for_current_device(&ws)) return -1;
    return mllm_moe_forward(L, x, T, out, ws, (long)need, idx_out, w_out, stream);
}

// Bucketing alone (for tests): perm/pos_of/off of the entries idx [TK] over E experts.
MLLM_API int mllm_moe_bucket(const int *idx, int TK, int E, int *off, int *perm, int *pos_of, int *tiles, void *stream)
{
    if (E <= 0 || E > 256 || TK <= 0) return -1;
    const int max_tiles = TK / kTileEntries + E + 1;
    // scratch for this test entry point, allocated here (it is not a hot path)
    int *scr = nullptr;
    if (hipMalloc(&scr, bucket_scratch_ints(TK, E) * sizeof(int)) != hipSuccess) return -1;
    const hipError_t r = launch_bucket(idx, TK, E, 1, scr, scr + (TK / kBucketThreads + 1) * E, off, perm, pos_of,
                                       nullptr, tiles, tiles + max_tiles, tiles + 2 * max_tiles, tiles + 3 * max_tiles,
                                       (hipStream_t)stream);
    const hipError_t r2 = hipStreamSynchronize((hipStream_t)stream);
    (void)hipFree(scr);
    return r == hipSuccess && r2 == hipSuccess ? 0 : -1;
}

} // extern "C"

int mllm_moe_needs_gemv(const mllm_packed *tab_dev, int sem_g, int sem_u, int sem_d, int N, int M, int E)
{
    int *f = nullptr, h[3] = {0, 0, 0};
    if (hipMalloc(&f, sizeof h) != hipSuccess) return -1;
    hipError_t r = hipMemset(f, 0, sizeof h);
    if (r == hipSuccess && sem_g >= 0) r = mllm_launch_scale_scan(tab_dev, nullptr, E, sem_g, M, N, f, nullptr);
    if (r == hipSuccess && sem_u >= 0) r = mllm_launch_scale_scan(tab_dev + E, nullptr, E, sem_u, M, N, f + 1, nullptr);
    if (r == hipSuccess && sem_d >= 0)
        r = mllm_launch_scale_scan(tab_dev + 2 * E, nullptr, E, sem_d, N, M, f + 2, nullptr);
    if (r == hipSuccess) r = hipMemcpy(h, f, sizeof h, hipMemcpyDeviceToHost);
    (void)hipFree(f);
    if (r != hipSuccess) return -1;
    return (sem_g >= 0 && mllm_scales_need_gemv(sem_g, h[0])) || (sem_u >= 0 && mllm_scales_need_gemv(sem_u, h[1])) ||
           (sem_d >= 0 && mllm_scales_need_gemv(sem_d, h[2])) ? 1 : 0;
}

// moe_ffn's SiLU is unclamped (CE:649-652).
mllm_moe_layer *mllm_moe_layer_from_views(int sem_g, int sem_u, int sem_d, int N, int M, int E, int K,
                                          const mllm_packed *tab_dev, const float *router_p, int renorm, int clamp,
                                          int gemv_only)
{
    if (E <= 0 || E > 256 || K <= 0 || K > 16 || K > E || N <= 0 || M <= 0 || !tab_dev || !router_p) return nullptr;
    mllm_moe_layer *L = new mllm_moe_layer;
    L->N = N; L->M = M; L->E = E; L->K = K; L->renorm = renorm;
    L->clamp = clamp;
    L->owns_router = 0;
    L->owns_tab = 0;
    L->sem_g = sem_g; L->sem_u = sem_u; L->sem_d = sem_d;
    L->router_p = const_cast<float *>(router_p);
    L->tab = const_cast<mllm_packed *>(tab_dev);
    L->gemv_only = gemv_only;
    return L;
}

bool mllm_moe_batched_supported(int sem_g, int sem_u, int sem_d)
{
    return mllm_qgemm_supported(sem_g) && mllm_qgemm_supported(sem_u) && (sem_d < 0 || mllm_qgemm_supported(sem_d));
}
