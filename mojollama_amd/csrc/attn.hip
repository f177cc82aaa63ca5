// attn.hip — decode attention over a KV cache held contiguously or in
// pages, the KV append of a new token, RoPE, and the host-side page table.
//
// A decode step reads every cached K and V row once: at B = 1 the work is
// HBM-bound streaming of 2 * seq * n_kv_head * head_dim * 4 bytes.  The
// positions are split into 64-row chunks so a long context spreads over
// n_kv_head * ceil(seq / 64) workgroups; each workgroup stages its chunk's K
// (then V) rows in LDS once and serves all n_head / n_kv_head query heads
// that share them (GQA).  Both reference softmaxes need the maximum over all
// positions before any weight (gqa_attention.c's exp_ps_simd is not an
// exponential, so the online rescaling of flash decoding would not reproduce
// it), hence three launches:
//   k_attn_scores : scores and per-chunk maxima
//   k_attn_values : global maximum, weights, per-chunk weight sums and
//                   weighted V sums
//   k_attn_combine: out = (sum of chunk V sums) * 1 / (sum of weights [+ 1e-10])
#include <math.h>
#include <vector>
#include "decode.h"
#include "gemv.h"
#include "moe.h"

namespace {

constexpr int kChunk = 64;        // positions per workgroup (one per lane)
constexpr int kMaxHD = 256;
constexpr int kMaxRep = 16;       // query heads per KV head

struct attn_args {
    const float *q;               // [B][NH*HD]
    mllm_kv_view kv;
    const int *seq_lens;          // [B]
    int max_seq, n_chunks;        // n_chunks = ceil(max_seq / kChunk)
    int NH, NKH, HD, mode;
    float *scores;                // [B][NH][max_seq]
    float *pmax, *psum;           // [B][NH][n_chunks]
    float *pout;                  // [B][NH][n_chunks][HD]
    float *out;                   // [B][NH*HD]
};

// Row s of sequence b, KV head j (nullptr past a page table's reach: the
// row then reads as zeros).
__device__ __forceinline__ const float *kv_row(const float *base, const mllm_kv_view &kv, int b, int s, int NKH, int HD,
                                               int j)
{
    const long rs = (long)NKH * HD;
    if (!kv.block_tables) return base + b * kv.seq_stride + (long)s * rs + (long)j * HD;
    const int blk = s / kv.page_size;
    if (blk >= kv.max_blocks) return nullptr;
    const int page = kv.block_tables[(long)b * kv.max_blocks + blk];
    if (page < 0 || page >= kv.n_pages) return nullptr;
    return base + ((long)page * kv.page_size + s % kv.page_size) * rs + (long)j * HD;
}

// Offsets (floats from the pool base) of a chunk's rows for KV head j, -1
// past the sequence or on an unmapped page; the first wave computes them.
__device__ __forceinline__ void chunk_rows(long *ro, const mllm_kv_view &kv, int b, int s0, int rows, int NKH, int HD,
                                           int j)
{
    if (threadIdx.x < kChunk) {
        const int p = threadIdx.x;
        long off = -1;
        if (p < rows) {
            const float *r = kv_row(kv.k, kv, b, s0 + p, NKH, HD, j);
            if (r) off = r - kv.k;
        }
        ro[p] = off;
    }
}

// The chunk's rows [kChunk][HD] from base + ro[p] into LDS rows of ld floats,
// in 16-byte pieces (HD % 4 == 0, base 16-byte aligned); every load is issued
// unconditionally (a missing row reads row 0 and stores zeros), so a thread's
// pieces are all in flight at once.
__device__ __forceinline__ void stage_chunk(float *dst, int ld, const float *__restrict__ base, const long *ro, int HD)
{
    const int hd4 = HD >> 2, n = kChunk * hd4;
    float4 v[kMaxHD / 16];
    bool ok[kMaxHD / 16];
#pragma unroll
    for (int k = 0; k < kMaxHD / 16; k++) {
        const int i = threadIdx.x + 256 * k;
        const int p = min(i, n - 1) / hd4, d4 = min(i, n - 1) - p * hd4;
        const long off = ro[p];
        ok[k] = i < n && off >= 0;
        v[k] = *reinterpret_cast<const float4 *>(base + (off >= 0 ? off : 0) + 4 * d4);
    }
#pragma unroll
    for (int k = 0; k < kMaxHD / 16; k++) {
        const int i = threadIdx.x + 256 * k;
        if (i >= n) break;
        const int p = i / hd4, d4 = i - p * hd4;
        const float4 w = ok[k] ? v[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float *o = dst + p * ld + 4 * d4;
        o[0] = w.x; o[1] = w.y; o[2] = w.z; o[3] = w.w;
    }
}

__device__ __forceinline__ int seq_len_of(const attn_args &a, int b)
{
    const int n = a.seq_lens[b];
    return n < 0 ? 0 : n > a.max_seq ? a.max_seq : n;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { const float w = __shfl_xor(v, o, 64); v = v > w ? v : w; }
    return v;
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// exp_ps_simd (gqa_attention.c:32-48) on one lane, as the source writes it:
// t = x log2e, n = rne(t + 0.5), f = t - n, an FMA chain that starts from 1
// and adds the coefficients in ascending order, times 2^n from the clamped
// biased exponent.  (Not an exponential: it gives 0.0013 at 0 and negative
// values below; the reference's weights are these values.)
__device__ __forceinline__ float exp_ps_simd_lane(float x)
{
    const float t = x * 1.4426950408889634f;
    const float nf = rintf(t + 0.5f);
    const float f = t - nf;
    float p = 1.0f;
    p = fmaf(p, f, 0.6931471805599453f);
    p = fmaf(p, f, 0.2402265069591007f);
    p = fmaf(p, f, 0.0555041086648216f);
    p = fmaf(p, f, 0.0096181291076285f);
    p = fmaf(p, f, 0.0013333558146428f);
    int biased = (int)nf + 127;
    biased = biased < 0 ? 0 : biased > 255 ? 255 : biased;
    return p * __uint_as_float((uint32_t)biased << 23);
}

// scores[b][h][s] = (q_h . k_s) * (1 / sqrtf(HD)) for the chunk's positions,
// and the chunk's maximum per head.  grid (n_chunks, NKH, B), 256 threads:
// lane = position, wave w serves heads w, w + 4, ... of the group.
__global__ __launch_bounds__(256) void k_attn_scores(attn_args a)
{
    extern __shared__ float lds[];
    const int c = blockIdx.x, j = blockIdx.y, b = blockIdx.z;
    const int len = seq_len_of(a, b), s0 = c * kChunk;
    if (s0 >= len) return;
    const int HD = a.HD, G = a.NH / a.NKH, ld = HD + 1;
    long *ro = reinterpret_cast<long *>(lds);     // [kChunk] row offsets
    float *qs = lds + 2 * kChunk;                  // [G][HD]
    float *ks = qs + G * HD;                       // [kChunk][HD + 1]
    const float *qb = a.q + (long)b * a.NH * HD + (long)j * G * HD;
    const int rows = min(kChunk, len - s0);
    chunk_rows(ro, a.kv, b, s0, rows, a.NKH, HD, j);
    for (int i = threadIdx.x; i < G * HD; i += 256) qs[i] = qb[i];
    __syncthreads();
    stage_chunk(ks, ld, a.kv.k, ro, HD);
    __syncthreads();
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const float scale = 1.0f / sqrtf((float)HD);
    for (int g = w; g < G; g += 4) {
        const float *qg = qs + g * HD, *kr = ks + lane * ld;
        float dot = 0.0f;
        for (int d = 0; d < HD; d++) dot = fmaf(qg[d], kr[d], dot);
        const float sc = dot * scale;                         // CE:152 dot *= inv; sgemm's alpha
        const int h = j * G + g;
        if (lane < rows) a.scores[((long)b * a.NH + h) * a.max_seq + s0 + lane] = sc;
        const float m = wave_max(lane < rows ? sc : -INFINITY);
        if (lane == 0) a.pmax[((long)b * a.NH + h) * a.n_chunks + c] = m;
    }
}

// Weights of the chunk's positions from the maximum over all chunks, their
// sum, and the chunk's weighted V sum per head.
//   mode 0 (CE:141-158): w = expf(s - max)
//   mode 1 (gqa_attention.c:50-88): positions below floor(len/8)*8 take
//     exp_ps_simd(clamp(s - max, -80, 80)), the rest expf(s - max) capped at 1e38
// The maximum starts from -1e30 (CE:146, gqa_attention.c:53).
__global__ __launch_bounds__(256) void k_attn_values(attn_args a)
{
    extern __shared__ float lds[];
    const int c = blockIdx.x, j = blockIdx.y, b = blockIdx.z;
    const int len = seq_len_of(a, b), s0 = c * kChunk;
    if (s0 >= len) return;
    const int HD = a.HD, G = a.NH / a.NKH;
    long *ro = reinterpret_cast<long *>(lds);     // [kChunk] row offsets (V mirrors K's layout)
    float *wt = lds + 2 * kChunk;                  // [G][kChunk]
    float *vs = wt + G * kChunk;                   // [kChunk][HD]
    const int rows = min(kChunk, len - s0), nc = (len + kChunk - 1) / kChunk;
    chunk_rows(ro, a.kv, b, s0, rows, a.NKH, HD, j);
    __syncthreads();
    stage_chunk(vs, HD, a.kv.v, ro, HD);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int vec_end = a.mode == 1 ? len / 8 * 8 : 0;
    for (int g = w; g < G; g += 4) {
        const int h = j * G + g;
        const float *pm = a.pmax + ((long)b * a.NH + h) * a.n_chunks;
        float m = -1e30f;
        for (int i = lane; i < nc; i += 64) m = pm[i] > m ? pm[i] : m;
        m = wave_max(m);
        float e = 0.0f;
        if (lane < rows) {
            const int s = s0 + lane;
            const float sc = a.scores[((long)b * a.NH + h) * a.max_seq + s];
            if (s < vec_end) {
                float z = sc - m;
                z = z > -80.0f ? z : -80.0f;
                z = z < 80.0f ? z : 80.0f;
                e = exp_ps_simd_lane(z);
            } else {
                e = expf(sc - m);
                if (a.mode == 1 && e > 1e38f) e = 1e38f;
            }
        }
        wt[g * kChunk + lane] = e;
        const float sum = wave_sum(e);
        if (lane == 0) a.psum[((long)b * a.NH + h) * a.n_chunks + c] = sum;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < G * HD; i += 256) {
        const int g = i / HD, d = i - g * HD;
        const float *wg = wt + g * kChunk;
        float acc = 0.0f;
        for (int p = 0; p < rows; p++) acc = fmaf(wg[p], vs[p * HD + d], acc);
        const int h = j * G + g;
        a.pout[(((long)b * a.NH + h) * a.n_chunks + c) * HD + d] = acc;
    }
}

// out[b][h][d] = sum_c pout * 1 / (sum_c psum [+ 1e-10 in mode 1]); an empty
// sequence gives zeros (the reference's products over no positions).
// grid (NH, B), 256 threads: 256 / HD groups of HD lanes each take every
// ng-th chunk (four loads in flight per lane), then group 0 adds the groups.
__global__ __launch_bounds__(256) void k_attn_combine(attn_args a)
{
    __shared__ float part[256], spart[256];
    const int h = blockIdx.x, b = blockIdx.y, HD = a.HD, ng = 256 / HD;
    const int gi = threadIdx.x / HD, d = threadIdx.x - gi * HD;
    const int len = seq_len_of(a, b), nc = (len + kChunk - 1) / kChunk;
    const float *ps = a.psum + ((long)b * a.NH + h) * a.n_chunks;
    const float *po = a.pout + ((long)b * a.NH + h) * a.n_chunks * HD + d;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (gi < ng) {
        int c = gi;
        for (; c + 3 * ng < nc; c += 4 * ng) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                acc[u] += po[(long)(c + u * ng) * HD];
                sum[u] += ps[c + u * ng];
            }
        }
        for (; c < nc; c += ng) { acc[0] += po[(long)c * HD]; sum[0] += ps[c]; }
        part[threadIdx.x] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        spart[threadIdx.x] = (sum[0] + sum[1]) + (sum[2] + sum[3]);
    }
    __syncthreads();
    if (gi != 0) return;
    float o = 0.0f, s = 0.0f;
    for (int g = 0; g < ng; g++) { o += part[g * HD + d]; s += spart[g * HD + d]; }
    const float inv = a.mode == 1 ? 1.0f / (s + 1e-10f) : 1.0f / s;
    a.out[((long)b * a.NH + h) * HD + d] = len == 0 ? 0.0f : o * inv;
}

// New K/V rows: token b's k/v [NKH*HD] to row pos[b] of its cache (CE:1363-1381,
// GO:158-161).  A position whose page is unmapped or past the table is skipped.
__global__ void k_kv_append(mllm_kv_view kv, const int *pos, const float *k_new, const float *v_new, int NKH, int HD)
{
    const int b = blockIdx.y, n = NKH * HD;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int s = pos[b];
    if (s < 0) return;
    const int j = i / HD, d = i - j * HD;
    const float *kr = kv_row(kv.k, kv, b, s, NKH, HD, j);
    if (!kr) return;
    const long off = kr - kv.k;
    kv.k[off + d] = k_new[(long)b * n + i];
    kv.v[off + d] = v_new[(long)b * n + i];
}

// rope_apply (GO:37-51, CE's rope_apply): per head the pairs (j, j + r/2),
// r = rope_dim (head_dim when <= 0), rotated by cos/sin rows [pos][r/2].
// grid (T), threads over NH * r/2; buf [T][NH*HD], pos [T].
__global__ void k_rope(float *buf, int NH, int HD, const int *pos, const float *cos_t, const float *sin_t, int r)
{
    const int t = blockIdx.x, hd2 = r / 2;
    const long p = pos[t];
    for (int i = threadIdx.x; i < NH * hd2; i += blockDim.x) {
        const int h = i / hd2, jj = i - h * hd2;
        float *bh = buf + ((long)t * NH + h) * HD;
        const float a0 = bh[jj], a1 = bh[jj + hd2];
        const float cs = cos_t[p * hd2 + jj], sn = sin_t[p * hd2 + jj];
        bh[jj] = a0 * cs - a1 * sn;
        bh[jj + hd2] = a1 * cs + a0 * sn;
    }
}

long a256(long n) { return (n + 255) / 256 * 256; }

// Workspace carve-up of mllm_gqa_decode.
long attn_ws(int B, int NH, int HD, int max_seq, attn_args *a, uint8_t *base)
{
    const int nc = (max_seq + kChunk - 1) / kChunk;
    long o = 0;
    auto take = [&](long bytes) { long at = o; o += a256(bytes); return base ? (float *)(base + at) : nullptr; };
    float *scores = take((long)B * NH * max_seq * 4);
    float *pmax = take((long)B * NH * nc * 4);
    float *psum = take((long)B * NH * nc * 4);
    float *pout = take((long)B * NH * nc * HD * 4);
    if (a) { a->scores = scores; a->pmax = pmax; a->psum = psum; a->pout = pout; a->n_chunks = nc; }
    return o > 0 ? o : 256;
}

bool attn_shape_ok(int NH, int NKH, int HD)
{
    return NH > 0 && NKH > 0 && NH % NKH == 0 && NH / NKH <= kMaxRep && HD > 0 && HD <= kMaxHD && HD % 4 == 0;
}

} // namespace

extern "C" {

MLLM_API long mllm_gqa_workspace_size(int B, int NH, int HD, int max_seq)
{
    if (B <= 0 || NH <= 0 || HD <= 0 || max_seq <= 0) return 256;
    return attn_ws(B, NH, HD, max_seq, nullptr, nullptr);
}

MLLM_API int mllm_gqa_decode(int mode, const float *q, const mllm_kv_view *kv, const int *seq_lens, int max_seq, int B,
                             int NH, int NKH, int HD, float *out, void *workspace, long ws_bytes, void *stream)
{
    if ((mode != 0 && mode != 1) || !q || !kv || !kv->k || !kv->v || !seq_lens || !out || B <= 0 || max_seq < 0 ||
        !attn_shape_ok(NH, NKH, HD)) {
        mllm_set_error("mllm_gqa_decode: bad arguments (mode 0/1, NH % NKH == 0, NH/NKH <= 16, HD <= 256 and a "
                       "multiple of 4)");
        return -1;
    }
    if (((uintptr_t)kv->k | (uintptr_t)kv->v) & 15) {
        mllm_set_error("mllm_gqa_decode: K and V must be 16-byte aligned");
        return -1;
    }
    if (kv->block_tables && (kv->page_size <= 0 || kv->max_blocks <= 0 || kv->n_pages <= 0)) {
        mllm_set_error("mllm_gqa_decode: a paged view needs page_size, max_blocks and n_pages > 0");
        return -1;
    }
    // contiguous rows are read as float4 from b * seq_stride + s * NKH * HD: the
    // stride keeps that 16-byte aligned and, with several sequences, past the
    // max_seq rows of the previous one
    if (!kv->block_tables && (kv->seq_stride < 0 || kv->seq_stride % 4 ||
                              (B > 1 && kv->seq_stride < (long)max_seq * NKH * HD))) {
        mllm_set_error("mllm_gqa_decode: seq_stride must be a non-negative multiple of 4 floats and, for B > 1, at "
                       "least max_seq * NKH * HD");
        return -1;
    }
    hipStream_t st = (hipStream_t)stream;
    attn_args a{};
    a.q = q; a.kv = *kv; a.seq_lens = seq_lens; a.max_seq = max_seq > 0 ? max_seq : 1;
    a.NH = NH; a.NKH = NKH; a.HD = HD; a.mode = mode; a.out = out;
    if (ws_bytes < attn_ws(B, NH, HD, a.max_seq, nullptr, nullptr)) {
        mllm_set_error("mllm_gqa_decode: workspace below mllm_gqa_workspace_size");
        return -1;
    }
    attn_ws(B, NH, HD, a.max_seq, &a, (uint8_t *)workspace);
    const int G = NH / NKH;
    const dim3 grid(a.n_chunks, NKH, B);
    const size_t lds1 = (2 * (size_t)kChunk + (size_t)G * HD + (size_t)kChunk * (HD + 1)) * 4;
    const size_t lds2 = (2 * (size_t)kChunk + (size_t)G * kChunk + (size_t)kChunk * HD) * 4;
    hipLaunchKernelGGL(k_attn_scores, grid, dim3(256), lds1, st, a);
    hipLaunchKernelGGL(k_attn_values, grid, dim3(256), lds2, st, a);
    hipLaunchKernelGGL(k_attn_combine, dim3(NH, B), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

MLLM_API int mllm_kv_append(const mllm_kv_view *kv, const int *pos, const float *k_new, const float *v_new, int B,
                            int NKH, int HD, void *stream)
{
    if (!kv || !kv->k || !kv->v || !pos || !k_new || !v_new || B <= 0 || NKH <= 0 || HD <= 0 ||
        (kv->block_tables && (kv->page_size <= 0 || kv->max_blocks <= 0 || kv->n_pages <= 0))) {
        mllm_set_error("mllm_kv_append: bad arguments");
        return -1;
    }
    const int n = NKH * HD;
    if (!kv->block_tables && (kv->seq_stride < 0 || (B > 1 && kv->seq_stride < n))) {
        mllm_set_error("mllm_kv_append: seq_stride must be >= 0 and, for B > 1, at least NKH * HD");
        return -1;
    }
    hipLaunchKernelGGL(k_kv_append, dim3((n + 255) / 256, B), dim3(256), 0, (hipStream_t)stream, *kv, pos, k_new,
                       v_new, NKH, HD);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

MLLM_API int mllm_rope(float *buf, int T, int NH, int HD, const int *pos, const float *cos_t, const float *sin_t,
                       int rope_dim, void *stream)
{
    const int r = rope_dim <= 0 ? HD : rope_dim;
    if (!buf || !pos || !cos_t || !sin_t || T <= 0 || NH <= 0 || HD <= 0 || r > HD || (r & 1)) {
        mllm_set_error("mllm_rope: bad arguments (rope_dim even and <= head_dim)");
        return -1;
    }
    hipLaunchKernelGGL(k_rope, dim3(T), dim3(256), 0, (hipStream_t)stream, buf, NH, HD, pos, cos_t, sin_t, r);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ------------------------------------------------------------ page table
// CE:160-201: a free list initialised so that allocation hands out pages
// 0, 1, 2, ... in order, and a logical -> physical table of 1024 entries
// (MAX_BLOCKS, CE:23), -1 when unmapped.
struct mllm_page_table {
    int page_size, n_pages, free_count;
    std::vector<int> table, free_pages;
};

MLLM_API mllm_page_table *mllm_page_table_create(int max_pages, int page_size)
{
    if (max_pages <= 0 || page_size <= 0) return nullptr;
    mllm_page_table *pt = new mllm_page_table;
    pt->page_size = page_size;
    pt->n_pages = max_pages;
    pt->table.assign(MLLM_PAGE_TABLE_BLOCKS, -1);
    pt->free_pages.resize(max_pages);
    for (int i = 0; i < max_pages; i++) pt->free_pages[i] = max_pages - 1 - i;
    pt->free_count = max_pages;
    return pt;
}

MLLM_API void mllm_page_table_destroy(mllm_page_table *pt) { delete pt; }

MLLM_API int mllm_page_table_alloc(mllm_page_table *pt)
{
    if (!pt || pt->free_count <= 0) return -1;
    return pt->free_pages[--pt->free_count];
}

MLLM_API void mllm_page_table_free(mllm_page_table *pt, int page_id)
{
    if (pt && pt->free_count < pt->n_pages) pt->free_pages[pt->free_count++] = page_id;
}

MLLM_API void mllm_page_table_map(mllm_page_table *pt, int logical_page, int physical_page)
{
    if (pt && logical_page >= 0 && logical_page < MLLM_PAGE_TABLE_BLOCKS) pt->table[logical_page] = physical_page;
}

MLLM_API const int *mllm_page_table_entries(const mllm_page_table *pt) { return pt ? pt->table.data() : nullptr; }

MLLM_API int mllm_page_table_lookup(const mllm_page_table *pt, int logical_page)
{
    return pt && logical_page >= 0 && logical_page < MLLM_PAGE_TABLE_BLOCKS ? pt->table[logical_page] : -1;
}

} // extern "C"
