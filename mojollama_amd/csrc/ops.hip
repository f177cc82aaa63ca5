// ops.hip — the small kernels around the GEMVs: weight repack, Q8_0
// activation quantisation, MoE routing, SiLU-gate and the weighted combine.
#include <math.h>
#include "decode.h"
#include "gemv.h"

namespace {

// ------------------------------------------------------------------ repack
// Source byte offsets of each plane inside a raw GGUF block.
struct pack_src { int n; int off[4]; int len[4]; int plane[4]; };

__host__ __device__ pack_src pack_plan(int ly)
{
    switch (ly) {
    case LY_Q4_0: return {2, {2, 0}, {16, 2}, {0, 1}};
    case LY_Q4_1: return {2, {4, 0}, {16, 4}, {0, 1}};
    case LY_Q5_0: return {3, {6, 2, 0}, {16, 4, 2}, {0, 1, 2}};
    case LY_Q8_0: return {2, {2, 0}, {32, 2}, {0, 1}};
    // K-quant meta planes get d, dmin here; the scale pairs are re-laid below.
    case LY_Q4_K: return {2, {16, 0}, {128, 4}, {0, 1}};
    // block_q5_K (ggml, QK:211-246): d dmin scales[12] qh[32] qs[128]
    case LY_Q5_K_GGML: return {3, {48, 16, 0}, {128, 32, 4}, {0, 1, 2}};
    // the engine's block_q5_K (CE:46-52): d dmin qh[32] ql[128] scales[12]
    case LY_Q5_K_CE: return {3, {36, 4, 0}, {128, 32, 4}, {0, 1, 2}};
    // block_q6_K (CE:34-39): ql[128] qh[64] scales[16] d
    case LY_Q6_K: return {4, {0, 128, 192, 208}, {128, 64, 16, 2}, {0, 1, 2, 3}};
    case LY_MXFP4: return {2, {0, 16}, {16, 1}, {0, 1}};
    }
    return {0, {0}, {0}, {0}};
}

// 6-bit (scale, min) pair j of a K-quant scale array (get_scale_min_k4 QK:62-71).
__device__ void k4_pair(int j, const uint8_t *q, uint32_t &sc, uint32_t &m)
{
    if (j < 4) { sc = q[j] & 63; m = q[j + 4] & 63; }
    else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m  = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

__global__ void k_pack(int ly, const uint8_t *__restrict__ raw, uint8_t *__restrict__ packed, long nblk,
                       long off0, long off1, long off2, long off3)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    const mllm_layout_desc L = mllm_layout_info(ly);
    const pack_src ps = pack_plan(ly);
    const long offs[4] = {off0, off1, off2, off3};
    const uint8_t *src = raw + i * L.block_bytes;
    for (int s = 0; s < ps.n; s++) {
        const int p = ps.plane[s];
        uint8_t *dst = packed + offs[p] + i * L.plane_bytes[p];
        for (int j = 0; j < ps.len[s]; j++) dst[j] = src[ps.off[s] + j];
    }
    if (ly == LY_Q4_K || ly == LY_Q5_K_GGML || ly == LY_Q5_K_CE) {
        // meta = [d | dmin] [sc_0..7 as 6-bit fields, 48 bits] [m_0..7, 48 bits]
        const uint8_t *sc = src + (ly == LY_Q5_K_CE ? 164 : 4);
        uint64_t S = 0, M = 0;
        for (int j = 0; j < 8; j++) {
            uint32_t a, b;
            k4_pair(j, sc, a, b);
            S |= (uint64_t)a << (6 * j);
            M |= (uint64_t)b << (6 * j);
        }
        uint32_t *meta = reinterpret_cast<uint32_t *>(packed + offs[ly == LY_Q4_K ? 1 : 2] + i * 16);
        meta[1] = (uint32_t)S;
        meta[2] = (uint32_t)(S >> 32) | ((uint32_t)M << 16);
        meta[3] = (uint32_t)(M >> 16);
    }
}

// ---------------------------------------------------------------- quantise
// One thread per 32-element block.  Mirrors quantize_row_q8_0 (QK:1406-1455):
// amax (in the reference's vmaxps order, which decides whether a NaN reaches
// it), d = amax/127 (1 if 0), id = 1/d, q = RNE(clamp(x*id, +-127)) with a
// NaN product clamped to -127 (maxps returns its second operand), scale
// stored as fp16 RNE.
__global__ void k_quantize_q8_0(const float *__restrict__ x, int T, int n_cols, uint8_t *__restrict__ q8_raw,
                                int8_t *__restrict__ xq_q, float *__restrict__ xq_d, float *__restrict__ xq_s4,
                                int *__restrict__ xq_sq, const float *__restrict__ x_up)
{
    const int nb = n_cols / 32;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)T * nb) return;
    const long t = i / nb, j = i % nb;
    const float *s = x + t * (long)n_cols + 32 * j;
    float v[32];
    if (x_up) {
        const float *su = x_up + t * (long)n_cols + 32 * j;
#pragma unroll
        for (int k = 0; k < 32; k++) v[k] = mllm_silu_mul(s[k], su[k]);
    } else {
#pragma unroll
        for (int k = 0; k < 32; k++) v[k] = s[k];
    }
    const float amax = mllm_q8_amax_ref([&](int k) { return fabsf(v[k]); });
    float d = amax / 127.0f;
    if (d == 0.0f) d = 1.0f;
    const float id = 1.0f / d;
    const uint16_t dh = __builtin_bit_cast(uint16_t, (_Float16)d);  // RNE
    int q[32];
    int sq = 0, s4 = 0;
#pragma unroll
    for (int k = 0; k < 32; k++) {
        float p = v[k] * id;
        p = (p > -127.0f) ? p : -127.0f;
        p = (p < 127.0f) ? p : 127.0f;
        q[k] = (int)rintf(p);
        sq += q[k];
        if ((k & 16) == 0 ? k < 8 : k < 24) s4 += q[k];
    }
    if (q8_raw) {
        uint8_t *dst = q8_raw + i * 34;
        dst[0] = dh & 0xFF;
        dst[1] = dh >> 8;
#pragma unroll
        for (int k = 0; k < 32; k++) dst[2 + k] = (uint8_t)(int8_t)q[k];
    }
    if (xq_q) {
        uint32_t w[8];
#pragma unroll
        for (int k = 0; k < 8; k++)
            w[k] = (uint32_t)(q[4 * k] & 0xFF) | ((uint32_t)(q[4 * k + 1] & 0xFF) << 8) |
                   ((uint32_t)(q[4 * k + 2] & 0xFF) << 16) | ((uint32_t)(q[4 * k + 3] & 0xFF) << 24);
        uint4 *dq = reinterpret_cast<uint4 *>(xq_q + i * 32);
        dq[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dq[1] = make_uint4(w[4], w[5], w[6], w[7]);
        const float dd = h2f(dh);
        xq_d[i] = dd;
        xq_s4[i] = dd * (float)s4;
        xq_sq[i] = sq;
    }
}

// ------------------------------------------------------------------ routing
// exp rounded from double: within half an ulp of the exact value, as the
// host libm's expf is, so the probabilities (and every comparison on them)
// match the reference's except where the two roundings straddle a midpoint.
__device__ __forceinline__ float expf_cr(float v) { return (float)exp((double)v); }

// Softmax and insertion top-k (CE:620-638) of the logits of TW tokens held in
// LDS as p[tw * PS + e], PS = route_pitch(E): max by strict '>' from p[0],
// exp element-wise, sequential sum, x 1/(sum+1e-10), then the top-K of the
// strict-'>' insertion in index order, optionally renormalised by the
// sequential sum of the K weights.
//   * The strict-'>' scan from p[0] ends at p[0] when p[0] is NaN and at the
//     largest non-NaN value otherwise (a NaN never compares greater); of equal
//     +0/-0 it keeps the first, and x - (+0) and x - (-0) are equal for every
//     x but -0, where exp gives 1 either way.  So the maximum is taken as a
//     wave reduction with fmaxf (which drops NaNs) and p[0] checked for NaN.
//   * The sums stay sequential, one lane reading 16-byte groups.
//   * The insertion keeps a stable descending order (an element goes after
//     every earlier one that is >= it) and never takes a NaN, so element j
//     lands at slot rank(j) = #{j' : p[j'] > p[j]} + #{j' < j : p[j'] == p[j]}
//     when that is < K -- computed one thread per element.
// Slots no element reaches keep (-1, -1e30), as the reference's initial list
// does.  Needs route_finish_floats(TW, E) floats at p (16-byte aligned).
__host__ __device__ constexpr int route_pitch(int E) { return (E + 3) / 4 * 4 + 4; }
__host__ __device__ constexpr int route_finish_floats(int TW, int E) { return TW * route_pitch(E) + 2 * TW + 32 * TW; }

// Sequential sum of n floats at v (16-byte aligned).
__device__ __forceinline__ float seq_sum(const float *v, int n)
{
    const float4 *v4 = reinterpret_cast<const float4 *>(v);
    float s = 0.0f;
    int j = 0;
#pragma unroll 4
    for (; j + 4 <= n; j += 4) {
        const float4 q = v4[j >> 2];
        s += q.x; s += q.y; s += q.z; s += q.w;
    }
    for (; j < n; j++) s += v[j];
    return s;
}

__device__ __forceinline__ void route_finish(float *p, int TW, int t0, int T, int E, int K, int renorm,
                                             int *__restrict__ top_idx, float *__restrict__ top_w)
{
    const int PS = route_pitch(E);
    float *s_mx = p + TW * PS, *s_inv = s_mx + TW, *s_v = s_inv + TW;
    int *s_i = reinterpret_cast<int *>(s_v + 16 * TW);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    for (int q = tid; q < 16 * TW; q += blockDim.x) { s_v[q] = -1e30f; s_i[q] = -1; }
    for (int tw = wave; tw < TW; tw += nw) {
        const float *pt = p + tw * PS;
        float m = -INFINITY;
        for (int j = lane; j < E; j += 64) m = fmaxf(m, pt[j]);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        if (lane == 0) s_mx[tw] = pt[0] != pt[0] ? pt[0] : m;
    }
    __syncthreads();
    for (int q = tid; q < TW * E; q += blockDim.x) {
        const int tw = q / E, j = q - tw * E;
        p[tw * PS + j] = expf_cr(p[tw * PS + j] - s_mx[tw]);
    }
    __syncthreads();
    if (tid < TW) s_inv[tid] = 1.0f / (seq_sum(p + tid * PS, E) + 1e-10f);   // sequential, as CE:624
    __syncthreads();
    for (int q = tid; q < TW * E; q += blockDim.x) {
        const int tw = q / E, j = q - tw * E;
        p[tw * PS + j] *= s_inv[tw];
    }
    __syncthreads();
    for (int q = tid; q < TW * E; q += blockDim.x) {
        const int tw = q / E, j = q - tw * E;
        const float *pt = p + tw * PS;
        const float4 *pt4 = reinterpret_cast<const float4 *>(pt);
        const float v = pt[j];
        if (v != v) continue;                    // NaN: never inserted
        int r = 0, jj = 0;
        for (; jj + 4 <= E; jj += 4) {
            const float4 u = pt4[jj >> 2];
            r += (u.x > v) || (u.x == v && jj < j);
            r += (u.y > v) || (u.y == v && jj + 1 < j);
            r += (u.z > v) || (u.z == v && jj + 2 < j);
            r += (u.w > v) || (u.w == v && jj + 3 < j);
        }
        for (; jj < E; jj++) r += (pt[jj] > v) || (pt[jj] == v && jj < j);
        if (r < K) { s_v[tw * 16 + r] = v; s_i[tw * 16 + r] = j; }
    }
    __syncthreads();
    if (tid >= TW || t0 + tid >= T) return;
    const int t = t0 + tid;
    float r = 1.0f;
    if (renorm) {
        float sw = 0.0f;
        for (int k = 0; k < K; k++) sw += s_v[tid * 16 + k];
        r = 1.0f / (sw + 1e-10f);
    }
    for (int k = 0; k < K; k++) {
        top_idx[(long)t * K + k] = s_i[tid * 16 + k];
        top_w[(long)t * K + k] = renorm ? s_v[tid * 16 + k] * r : s_v[tid * 16 + k];
    }
}

// Router layout for routing: element (i, e) of the [E][N] router (row e =
// expert e's weights over the N inputs) sits at ((i/4)*E + e)*4 + i%4 --
// four consecutive inputs of one expert are 16 contiguous bytes, and a run
// of rows is one contiguous block.  Rows from N up to a multiple of 32 are 0.
constexpr int kRouteRowPad = 32;

__global__ void k_router_pack(const float *__restrict__ router, int N, int E, float *__restrict__ out)
{
    const long n4 = (long)((N + kRouteRowPad - 1) / kRouteRowPad) * (kRouteRowPad / 4) * E;
    const long q = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= n4) return;
    const int i4 = (int)(q / E), e = (int)(q - (long)i4 * E);
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int i = 4 * i4 + j;
        v[j] = i < N ? router[(long)e * N + i] : 0.0f;
    }
    reinterpret_cast<float4 *>(out)[q] = make_float4(v[0], v[1], v[2], v[3]);
}

// Routing logits: logit[t][e] is a sequential fp32 FMA chain over i = 0..N-1
// (CE:614-618 compiles to scalar vfmadd231ss).  Thread (g, e) of a workgroup,
// g < G token groups of TT tokens, runs the TT chains of expert e for its
// group's tokens side by side (independent chains overlap their latency).
// The workgroup streams KC-row chunks of the packed router (contiguous) and
// of its TW = G*TT tokens' x (as [token][KC+4]) through two LDS buffers,
// loading chunk c+1 into registers while chunk c is consumed.  Rows run to
// N rounded up to 32: the router's pad rows are zero and so is x there, and
// fma(0, 0, d) == d, so every chunk is whole 32-step batches.  A lane reads
// four steps of its chain with one ds_read_b128 (router lanes contiguous, x
// a broadcast), 16 steps per batch, two register sets so the next batch's
// reads are in flight during this batch's FMAs.  x slots use a power-of-two
// row pitch 2^lgq >= KC/4 so a slot's (token, column) is a shift and a mask.
// Needs N % 4 == 0, KC % 32 == 0, KC*E/4 <= 256*PF and TW << lgq <= 256*XS,
// and route_slack(E) floats of LDS past the two buffers.
__host__ __device__ constexpr int route_slack(int E) { return 16 * E + 16; }
template <int TT, int PF, int XS>
__global__ __launch_bounds__(256) void k_route(const float *__restrict__ router_p, const float *__restrict__ x,
                                               int T, int N, int E, int K, int renorm, int KC, int G, int lgq,
                                               int lgES, float *__restrict__ logits,
                                               int *__restrict__ top_idx, float *__restrict__ top_w)
{
    extern __shared__ float4 lds4[];
    float *lds = reinterpret_cast<float *>(lds4);
    // experts of this workgroup: all E, or (lgES >= 0) the slice of 2^lgES starting at
    // blockIdx.y * 2^lgES, whose raw logits go to logits[t][e] for k_route_finish
    const int ES = lgES >= 0 ? (1 << lgES) : E, e0 = lgES >= 0 ? blockIdx.y * ES : 0;
    const int TW = G * TT, KCR = KC + 4;
    const int per = KC * ES + TW * KCR;          // floats per buffer (multiple of 4)
    const int NP = (N + kRouteRowPad - 1) / kRouteRowPad * kRouteRowPad;
    const int t0 = blockIdx.x * TW;
    const int tid = threadIdx.x;
    const int g = tid / ES, e = tid - g * ES;
    const int nch = (NP + KC - 1) / KC;
    const int qmask = (1 << lgq) - 1;
    float4 pr[PF], px[XS];

    auto load_chunk = [&](int c) {
        const int i0 = c * KC, kq = min(KC, NP - i0) >> 2, kv = min(KC, N - i0) >> 2;
        const float4 *src = reinterpret_cast<const float4 *>(router_p + (long)i0 * E);
        const int nr4 = kq * ES;
#pragma unroll
        for (int s = 0; s < PF; s++) {
            const int j = tid + s * 256;
            // slice: row group j >> lgES, expert e0 + (j & (ES-1)) of E (16 bytes each)
            if (j < nr4) pr[s] = gld<float4>(lgES >= 0 ? src + (long)(j >> lgES) * E + e0 + (j & (ES - 1)) : src + j);
        }
#pragma unroll
        for (int s = 0; s < XS; s++) {
            const int q = tid + s * 256, tw = q >> lgq, ii = q & qmask;
            px[s] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (tw < TW && ii < kv && t0 + tw < T) px[s] = gld<float4>(x + (long)(t0 + tw) * N + i0 + 4 * ii);
        }
    };
    auto store_chunk = [&](int c) {
        float4 *rb = lds4 + (c & 1) * (per >> 2), *xb = rb + ((KC * ES) >> 2);
        const int kq = min(KC, NP - c * KC) >> 2;
        const int nr4 = kq * ES;
#pragma unroll
        for (int s = 0; s < PF; s++) {
            const int j = tid + s * 256;
            if (j < nr4) rb[j] = pr[s];
        }
#pragma unroll
        for (int s = 0; s < XS; s++) {
            const int q = tid + s * 256, tw = q >> lgq, ii = q & qmask;
            if (tw < TW && ii < kq) xb[tw * (KCR >> 2) + ii] = px[s];
        }
    };

    float dot[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++) dot[tt] = 0.0f;
    load_chunk(0);
    store_chunk(0);
    for (int c = 0; c < nch; c++) {
        if (c + 1 < nch) load_chunk(c + 1);
        __syncthreads();                         // chunk c stored by every thread
        const int kc = min(KC, NP - c * KC);     // multiple of 32
        if (g < G) {
            const float *rr = lds + (c & 1) * per + 4 * e;           // + (i/4)*4ES
            const float *xr = lds + (c & 1) * per + KC * ES + g * TT * KCR;
            auto ldb = [&](int i0, float4(&r)[4], float4(&xx)[TT][4]) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    r[q] = *reinterpret_cast<const float4 *>(rr + (i0 + 4 * q) * ES);
#pragma unroll
                    for (int tt = 0; tt < TT; tt++) xx[tt][q] = *reinterpret_cast<const float4 *>(xr + tt * KCR + i0 + 4 * q);
                }
            };
            auto fmb = [&](const float4(&r)[4], const float4(&xx)[TT][4]) {
#pragma unroll
                for (int q = 0; q < 4; q++)
#pragma unroll
                    for (int tt = 0; tt < TT; tt++) {
                        dot[tt] = fmaf(xx[tt][q].x, r[q].x, dot[tt]);
                        dot[tt] = fmaf(xx[tt][q].y, r[q].y, dot[tt]);
                        dot[tt] = fmaf(xx[tt][q].z, r[q].z, dot[tt]);
                        dot[tt] = fmaf(xx[tt][q].w, r[q].w, dot[tt]);
                    }
            };
            // The read of batch i0 + 32 after the last batch is not used; it stays
            // inside the allocation (route_slack(E) floats past the two buffers).
            float4 ra[4], rb2[4], xa[TT][4], xb2[TT][4];
            ldb(0, ra, xa);
            // Scheduling barriers keep each batch's reads issued ahead of the
            // previous batch's FMAs (the scheduler would sink them to their uses).
            for (int i0 = 0; i0 < kc; i0 += 32) {
                ldb(i0 + 16, rb2, xb2);
                __builtin_amdgcn_sched_barrier(0);
                fmb(ra, xa);
                __builtin_amdgcn_sched_barrier(0);
                ldb(i0 + 32, ra, xa);
                __builtin_amdgcn_sched_barrier(0);
                fmb(rb2, xb2);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // buffer (c+1)&1 was last read in iteration c-1, before this iteration's barrier
        if (c + 1 < nch) store_chunk(c + 1);
    }
    if (logits) {
        if (g < G)
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
                if (t0 + g * TT + tt < T) logits[(long)(t0 + g * TT + tt) * E + e0 + e] = dot[tt];
        return;
    }
    __syncthreads();                             // every chain done: LDS reused for the logits
    float *p = lds;
    if (g < G)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) p[(g * TT + tt) * route_pitch(E) + e] = dot[tt];
    __syncthreads();
    route_finish(p, TW, t0, T, E, K, renorm, top_idx, top_w);
}

// Routing logits for a few tokens (decode), spread over many CUs: a
// workgroup takes an ES-expert slice of the router (ES small, so the slice of
// all N rows fits in registers and LDS at once) and one token, lane e of
// wave 0 running the chain of expert e0 + e (the other waves help load; a
// second chain wave per workgroup would share the LDS issue slots the chain
// is bound by); raw logits go to `logits` for k_route_finish.  Every load of
// the slice and of the token's x is issued at the start, in NCH chunks of KC
// steps; chunk c is stored to LDS and its chains advanced while the later
// chunks are still in flight.  LDS holds each expert's router values as one
// contiguous row of float4 (stride RS, RS % 16 == 1 so the lanes' 16-byte
// reads fall on distinct banks) and x after them; steps from N up to NCH*KC
// are zero in both, and fma(0, 0, d) == d (up to the sign of a zero, which
// neither the softmax nor the comparisons of the selection can see).
//
// The chain itself (chain72) is scheduled by hand: its operands come from
// LDS in groups of 24 steps (12 ds_read_b128: 6 of router, 6 of x) with two
// groups in flight, and lgkmcnt can only count 15 outstanding reads, so a
// compiler-scheduled loop waits for every read (lgkmcnt(0)) each group and
// runs about twice as slow as the FMA latency allows.  The loop reads up to
// 48 steps past its last group (rows carry that much slack).
__device__ __forceinline__ float chain72(float dot, unsigned r_lds, unsigned x_lds, int iters)
{
    // dot = fma(x[i], r[i], dot) for i = 0 .. 72*iters-1 in order; r and x
    // are float4 runs at LDS byte addresses r_lds and x_lds.
    asm volatile(
        "s_waitcnt lgkmcnt(0)\n"
        "ds_read_b128 v[64:67], %1 offset:0\n"
        "ds_read_b128 v[68:71], %1 offset:16\n"
        "ds_read_b128 v[72:75], %1 offset:32\n"
        "ds_read_b128 v[76:79], %1 offset:48\n"
        "ds_read_b128 v[80:83], %1 offset:64\n"
        "ds_read_b128 v[84:87], %1 offset:80\n"
        "ds_read_b128 v[88:91], %2 offset:0\n"
        "ds_read_b128 v[92:95], %2 offset:16\n"
        "ds_read_b128 v[96:99], %2 offset:32\n"
        "ds_read_b128 v[100:103], %2 offset:48\n"
        "ds_read_b128 v[104:107], %2 offset:64\n"
        "ds_read_b128 v[108:111], %2 offset:80\n"
        "ds_read_b128 v[112:115], %1 offset:96\n"
        "ds_read_b128 v[116:119], %1 offset:112\n"
        "ds_read_b128 v[120:123], %1 offset:128\n"
        "ds_read_b128 v[124:127], %1 offset:144\n"
        "ds_read_b128 v[128:131], %1 offset:160\n"
        "ds_read_b128 v[132:135], %1 offset:176\n"
        "ds_read_b128 v[136:139], %2 offset:96\n"
        "ds_read_b128 v[140:143], %2 offset:112\n"
        "ds_read_b128 v[144:147], %2 offset:128\n"
        "ds_read_b128 v[148:151], %2 offset:144\n"
        "ds_read_b128 v[152:155], %2 offset:160\n"
        "ds_read_b128 v[156:159], %2 offset:176\n"
        "1:\n"
        "ds_read_b128 v[160:163], %1 offset:192\n"
        "ds_read_b128 v[164:167], %1 offset:208\n"
        "ds_read_b128 v[168:171], %1 offset:224\n"
        "ds_read_b128 v[172:175], %1 offset:240\n"
        "ds_read_b128 v[176:179], %1 offset:256\n"
        "ds_read_b128 v[180:183], %1 offset:272\n"
        "ds_read_b128 v[184:187], %2 offset:192\n"
        "ds_read_b128 v[188:191], %2 offset:208\n"
        "ds_read_b128 v[192:195], %2 offset:224\n"
        "ds_read_b128 v[196:199], %2 offset:240\n"
        "ds_read_b128 v[200:203], %2 offset:256\n"
        "ds_read_b128 v[204:207], %2 offset:272\n"
        "s_waitcnt lgkmcnt(12)\n"
        "v_fmac_f32 %0, v88, v64\n"
        "v_fmac_f32 %0, v89, v65\n"
        "v_fmac_f32 %0, v90, v66\n"
        "v_fmac_f32 %0, v91, v67\n"
        "v_fmac_f32 %0, v92, v68\n"
        "v_fmac_f32 %0, v93, v69\n"
        "v_fmac_f32 %0, v94, v70\n"
        "v_fmac_f32 %0, v95, v71\n"
        "v_fmac_f32 %0, v96, v72\n"
        "v_fmac_f32 %0, v97, v73\n"
        "v_fmac_f32 %0, v98, v74\n"
        "v_fmac_f32 %0, v99, v75\n"
        "v_fmac_f32 %0, v100, v76\n"
        "v_fmac_f32 %0, v101, v77\n"
        "v_fmac_f32 %0, v102, v78\n"
        "v_fmac_f32 %0, v103, v79\n"
        "v_fmac_f32 %0, v104, v80\n"
        "v_fmac_f32 %0, v105, v81\n"
        "v_fmac_f32 %0, v106, v82\n"
        "v_fmac_f32 %0, v107, v83\n"
        "v_fmac_f32 %0, v108, v84\n"
        "v_fmac_f32 %0, v109, v85\n"
        "v_fmac_f32 %0, v110, v86\n"
        "v_fmac_f32 %0, v111, v87\n"
        "ds_read_b128 v[64:67], %1 offset:288\n"
        "ds_read_b128 v[68:71], %1 offset:304\n"
        "ds_read_b128 v[72:75], %1 offset:320\n"
        "ds_read_b128 v[76:79], %1 offset:336\n"
        "ds_read_b128 v[80:83], %1 offset:352\n"
        "ds_read_b128 v[84:87], %1 offset:368\n"
        "ds_read_b128 v[88:91], %2 offset:288\n"
        "ds_read_b128 v[92:95], %2 offset:304\n"
        "ds_read_b128 v[96:99], %2 offset:320\n"
        "ds_read_b128 v[100:103], %2 offset:336\n"
        "ds_read_b128 v[104:107], %2 offset:352\n"
        "ds_read_b128 v[108:111], %2 offset:368\n"
        "s_waitcnt lgkmcnt(12)\n"
        "v_fmac_f32 %0, v136, v112\n"
        "v_fmac_f32 %0, v137, v113\n"
        "v_fmac_f32 %0, v138, v114\n"
        "v_fmac_f32 %0, v139, v115\n"
        "v_fmac_f32 %0, v140, v116\n"
        "v_fmac_f32 %0, v141, v117\n"
        "v_fmac_f32 %0, v142, v118\n"
        "v_fmac_f32 %0, v143, v119\n"
        "v_fmac_f32 %0, v144, v120\n"
        "v_fmac_f32 %0, v145, v121\n"
        "v_fmac_f32 %0, v146, v122\n"
        "v_fmac_f32 %0, v147, v123\n"
        "v_fmac_f32 %0, v148, v124\n"
        "v_fmac_f32 %0, v149, v125\n"
        "v_fmac_f32 %0, v150, v126\n"
        "v_fmac_f32 %0, v151, v127\n"
        "v_fmac_f32 %0, v152, v128\n"
        "v_fmac_f32 %0, v153, v129\n"
        "v_fmac_f32 %0, v154, v130\n"
        "v_fmac_f32 %0, v155, v131\n"
        "v_fmac_f32 %0, v156, v132\n"
        "v_fmac_f32 %0, v157, v133\n"
        "v_fmac_f32 %0, v158, v134\n"
        "v_fmac_f32 %0, v159, v135\n"
        "ds_read_b128 v[112:115], %1 offset:384\n"
        "ds_read_b128 v[116:119], %1 offset:400\n"
        "ds_read_b128 v[120:123], %1 offset:416\n"
        "ds_read_b128 v[124:127], %1 offset:432\n"
        "ds_read_b128 v[128:131], %1 offset:448\n"
        "ds_read_b128 v[132:135], %1 offset:464\n"
        "ds_read_b128 v[136:139], %2 offset:384\n"
        "ds_read_b128 v[140:143], %2 offset:400\n"
        "ds_read_b128 v[144:147], %2 offset:416\n"
        "ds_read_b128 v[148:151], %2 offset:432\n"
        "ds_read_b128 v[152:155], %2 offset:448\n"
        "ds_read_b128 v[156:159], %2 offset:464\n"
        "s_waitcnt lgkmcnt(12)\n"
        "v_fmac_f32 %0, v184, v160\n"
        "v_fmac_f32 %0, v185, v161\n"
        "v_fmac_f32 %0, v186, v162\n"
        "v_fmac_f32 %0, v187, v163\n"
        "v_fmac_f32 %0, v188, v164\n"
        "v_fmac_f32 %0, v189, v165\n"
        "v_fmac_f32 %0, v190, v166\n"
        "v_fmac_f32 %0, v191, v167\n"
        "v_fmac_f32 %0, v192, v168\n"
        "v_fmac_f32 %0, v193, v169\n"
        "v_fmac_f32 %0, v194, v170\n"
        "v_fmac_f32 %0, v195, v171\n"
        "v_fmac_f32 %0, v196, v172\n"
        "v_fmac_f32 %0, v197, v173\n"
        "v_fmac_f32 %0, v198, v174\n"
        "v_fmac_f32 %0, v199, v175\n"
        "v_fmac_f32 %0, v200, v176\n"
        "v_fmac_f32 %0, v201, v177\n"
        "v_fmac_f32 %0, v202, v178\n"
        "v_fmac_f32 %0, v203, v179\n"
        "v_fmac_f32 %0, v204, v180\n"
        "v_fmac_f32 %0, v205, v181\n"
        "v_fmac_f32 %0, v206, v182\n"
        "v_fmac_f32 %0, v207, v183\n"
        "v_add_u32 %1, 288, %1\n"
        "v_add_u32 %2, 288, %2\n"
        "s_sub_i32 %3, %3, 1\n"
        "s_cmp_lg_u32 %3, 0\n"
        "s_cbranch_scc1 1b\n"
        "s_waitcnt lgkmcnt(0)\n"
        : "+v"(dot), "+v"(r_lds), "+v"(x_lds), "+s"(iters)
        :
        : "v64", "v65", "v66", "v67", "v68", "v69", "v70", "v71", "v72", "v73", "v74", "v75",
          "v76", "v77", "v78", "v79", "v80", "v81", "v82", "v83", "v84", "v85", "v86", "v87",
          "v88", "v89", "v90", "v91", "v92", "v93", "v94", "v95", "v96", "v97", "v98", "v99",
          "v100", "v101", "v102", "v103", "v104", "v105", "v106", "v107", "v108", "v109", "v110", "v111",
          "v112", "v113", "v114", "v115", "v116", "v117", "v118", "v119", "v120", "v121", "v122", "v123",
          "v124", "v125", "v126", "v127", "v128", "v129", "v130", "v131", "v132", "v133", "v134", "v135",
          "v136", "v137", "v138", "v139", "v140", "v141", "v142", "v143", "v144", "v145", "v146", "v147",
          "v148", "v149", "v150", "v151", "v152", "v153", "v154", "v155", "v156", "v157", "v158", "v159",
          "v160", "v161", "v162", "v163", "v164", "v165", "v166", "v167", "v168", "v169", "v170", "v171",
          "v172", "v173", "v174", "v175", "v176", "v177", "v178", "v179", "v180", "v181", "v182", "v183",
          "v184", "v185", "v186", "v187", "v188", "v189", "v190", "v191", "v192", "v193", "v194", "v195",
          "v196", "v197", "v198", "v199", "v200", "v201", "v202", "v203", "v204", "v205", "v206", "v207",
          "scc", "memory");
    return dot;
}

constexpr int kChainIter = 72, kChainSlack = 48;

template <int NCH, int SPC, int XPC>
__global__ __launch_bounds__(256) void k_route_slice(const float *__restrict__ router_p, const float *__restrict__ x,
                                                     int T, int N, int E, int KC, int ES, int RS, int XS,
                                                     float *__restrict__ logits)
{
    extern __shared__ float4 lds4[];
    const int e0 = blockIdx.x * ES, t = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int KC4 = KC >> 2, N4 = N >> 2;
    float4 *rl = lds4;                                        // [ES][RS]
    float4 *xl = lds4 + (long)ES * RS;                        // [XS]
    const float4 *r4 = reinterpret_cast<const float4 *>(router_p) + e0;
    float4 pr[NCH][SPC], px[NCH][XPC];
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int q0 = c * KC4;
#pragma unroll
        for (int s = 0; s < SPC; s++) {
            const int j = tid + s * 256, r = j / ES;
            pr[c][s] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (r < KC4 && q0 + r < N4) pr[c][s] = gld<float4>(r4 + (long)(q0 + r) * E + (j - r * ES));
        }
#pragma unroll
        for (int s = 0; s < XPC; s++) {
            const int q = tid + s * 256;
            px[c][s] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (q < KC4 && q0 + q < N4) px[c][s] = gld<float4>(x + (long)t * N + 4 * (q0 + q));
        }
    }
    float dot = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int q0 = c * KC4;
#pragma unroll
        for (int s = 0; s < SPC; s++) {
            const int j = tid + s * 256, r = j / ES;
            if (r < KC4) rl[(j - r * ES) * RS + q0 + r] = pr[c][s];
        }
#pragma unroll
        for (int s = 0; s < XPC; s++) {
            const int q = tid + s * 256;
            if (q < KC4) xl[q0 + q] = px[c][s];
        }
        __syncthreads();
        if (wave == 0 && lane < ES)
            dot = chain72(dot, (unsigned)(uintptr_t)(rl + lane * RS + q0), (unsigned)(uintptr_t)(xl + q0), KC / kChainIter);
    }
    if (wave == 0 && lane < ES) logits[(long)t * E + e0 + lane] = dot;
}

// Routing logits for many tokens with each token's x broadcast across a DPP
// row.  A workgroup takes RB_E = 16 experts and 16 tokens: lane column
// c = lane & 15 is expert e0 + c and each 16-lane row (4 per wave) one token,
// so every lane runs one chain.  Per 16-step group a lane holds x[t][k + c]
// of its row's token in a register, and step i of the group takes x[t][k + i]
// from lane i of the row as the DPP source of its FMA (row_newbcast:i): x
// costs no LDS traffic, only the lane's router values do (a float4 per four
// steps).  Router chunks of 16 * G steps are staged in LDS ([quad][expert],
// two buffers), loaded into registers one chunk ahead like the x values of
// the next chunk; steps from N up to the padded length are zero in both
// operands (x through the range check of its buffer loads), and
// fma(0, 0, d) == d as in chain72.  The chunk count is even so the loop
// alternates two register sets for x, which only buffer loads write (a DPP
// source written by a VALU instruction needs two wait states; every group's
// FMAs start with them anyway).  Measured against two or four chains per
// lane (more router reuse per LDS read, fewer waves): one chain is fastest
// at both benchmark shapes, whose time is the chains' FMA latency.
constexpr int RB_E = 16;
#define RB1(i, r) "v_fmac_f32_dpp %0, %1, %" #r " row_newbcast:" #i " row_mask:0xf bank_mask:0xf\n"

// acc = fma(x[k + i], r[i], acc) for i = 0..15 in order, x[k + i] from lane i
// of the row of xv.
__device__ __forceinline__ float rb_group(float acc, float xv, const float4 (&r)[4])
{
    asm("s_nop 1\n" RB1(0, 2) RB1(1, 3) RB1(2, 4) RB1(3, 5) RB1(4, 6) RB1(5, 7) RB1(6, 8) RB1(7, 9) RB1(8, 10)
            RB1(9, 11) RB1(10, 12) RB1(11, 13) RB1(12, 14) RB1(13, 15) RB1(14, 16) RB1(15, 17)
        : "+v"(acc)
        : "v"(xv), "v"(r[0].x), "v"(r[0].y), "v"(r[0].z), "v"(r[0].w), "v"(r[1].x), "v"(r[1].y), "v"(r[1].z),
          "v"(r[1].w), "v"(r[2].x), "v"(r[2].y), "v"(r[2].z), "v"(r[2].w), "v"(r[3].x), "v"(r[3].y), "v"(r[3].z),
          "v"(r[3].w));
    return acc;
}
#undef RB1

template <int G>
__global__ __launch_bounds__(256) void k_route_bc(const float *__restrict__ router_p, const float *__restrict__ x,
                                                  int T, int N, int E, int nch, float *__restrict__ logits)
{
    constexpr int KQ = 4 * G, KC = 16 * G;       // quads and steps per chunk
    constexpr int SL = KQ * RB_E / 256;          // staged router float4 per thread and chunk
    static_assert(SL * 256 == KQ * RB_E, "whole staging slots");
    __shared__ float4 rl[2][KQ * RB_E];
    const int tid = threadIdx.x, c = tid & 15;
    const int e0 = blockIdx.y * RB_E, t = blockIdx.x * 16 + (tid >> 4);
    const int N4 = N >> 2;
    const float4 *r4 = reinterpret_cast<const float4 *>(router_p);
    // x through buffer loads: lanes past the tokens or past N read zeros (offset
    // 2^31 >= the buffer's T*N*4 bytes)
    const __amdgpu_buffer_rsrc_t xs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(x), (short)0, T * N * 4, 0x00020000);
    constexpr uint32_t kOut = 0x80000000u;
    const uint32_t xo = t < T ? (uint32_t)(t * N + c) * 4u : kOut;
    float4 st[SL];
    auto stage_load = [&](int ch) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < SL; s++) {
            const int i = tid + 256 * s, q = ch * KQ + (i >> 4), e = e0 + (i & 15);
            st[s] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (q < N4 && e < E) st[s] = gld<float4>(r4 + (long)q * E + e);
        }
    };
    auto stage_store = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < SL; s++) rl[buf][tid + 256 * s] = st[s];
    };
    auto load_x = [&](int ch, float (&xv)[G]) __attribute__((always_inline)) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            const int k = ch * KC + 16 * g;
            // sign bit set where c >= N - k (past the row's end): arithmetic, not a
            // select, which the compiler would turn into branches around the loads
            const uint32_t oob = (uint32_t)(N - 1 - k - c) & kOut;
            xv[g] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xs, xo | oob, 4 * k, 0));
        }
    };
    float acc = 0.0f;
    auto chains = [&](int buf, const float (&xv)[G]) __attribute__((always_inline)) {
        const float4 *b = rl[buf] + c;
        float4 rc[4], rn[4];
#pragma unroll
        for (int u = 0; u < 4; u++) rc[u] = b[u * RB_E];
#pragma unroll
        for (int g = 0; g < G; g++) {
            if (g + 1 < G) {
#pragma unroll
                for (int u = 0; u < 4; u++) rn[u] = b[(4 * (g + 1) + u) * RB_E];
            }
            acc = rb_group(acc, xv[g], rc);
            if (g + 1 < G) {
#pragma unroll
                for (int u = 0; u < 4; u++) rc[u] = rn[u];
            }
        }
    };
    float xa[G], xb[G];
    stage_load(0);
    stage_store(0);
    load_x(0, xa);
    // chunk ch: load chunk ch + 1 (the last one again at the end: harmless),
    // barrier (chunk ch stored), chains over chunk ch, store chunk ch + 1 into
    // the buffer chunk ch - 1's chains finished reading before the barrier
    for (int ch = 0; ch < nch; ch += 2) {
        stage_load(min(ch + 1, nch - 1));
        load_x(min(ch + 1, nch - 1), xb);
        __syncthreads();
        chains(0, xa);
        stage_store(1);
        stage_load(min(ch + 2, nch - 1));
        load_x(min(ch + 2, nch - 1), xa);
        __syncthreads();
        chains(1, xb);
        stage_store(0);
    }
    if (t < T && e0 + c < E) logits[(long)t * E + e0 + c] = acc;
}

// Softmax and top-K of logits[t][0..E) written by the expert slices of k_route.
__global__ __launch_bounds__(256) void k_route_finish(const float *__restrict__ logits, int T, int E, int K, int renorm,
                                                      int *__restrict__ top_idx, float *__restrict__ top_w)
{
    __shared__ __align__(16) float p[route_finish_floats(1, 256)];
    const int t = blockIdx.x;
    if (threadIdx.x < E) p[threadIdx.x] = logits[(long)t * E + threadIdx.x];
    __syncthreads();
    route_finish(p, 1, t, T, E, K, renorm, top_idx, top_w);
}

// Any N: one workgroup per token reading the packed router straight from
// global memory, same chain order.
__global__ __launch_bounds__(256) void k_route_any(const float *__restrict__ router_p, const float *__restrict__ x,
                                                   int T, int N, int E, int K, int renorm,
                                                   int *__restrict__ top_idx, float *__restrict__ top_w)
{
    __shared__ __align__(16) float p[route_finish_floats(1, 256)];
    const int t = blockIdx.x, e = threadIdx.x;
    if (e < E) {
        const float *xt = x + (long)t * N;
        float dot = 0.0f;
        for (int i = 0; i < N; i++) dot = fmaf(xt[i], router_p[((long)(i >> 2) * E + e) * 4 + (i & 3)], dot);
        p[e] = dot;
    }
    __syncthreads();
    route_finish(p, 1, t, T, E, K, renorm, top_idx, top_w);
}

// ---------------------------------------------------------------- MoE glue
__global__ void k_silu_mul(const float *__restrict__ g, const float *__restrict__ u, float *__restrict__ h, long n,
                           int clamp)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float gv = g[i];
    h[i] = clamp ? mllm_silu_mul(gv, u[i]) : (gv / (1.0f + expf(-gv))) * u[i];
}

// The activation of a fused GEMV formed on its own, for launches the fused
// prologue does not take (see mllm_gemv_args): one workgroup per token b,
// v = x + x_res, res_out = v, RMS norm with rms_w, or silu(x) * x_up.
__global__ __launch_bounds__(256) void k_act_prologue(const float *__restrict__ x, const float *__restrict__ x_res,
                                                      float *__restrict__ res_out, const float *__restrict__ rms_w,
                                                      float eps, int div, const float *__restrict__ x_up, int clamp,
                                                      int n, int ldx, float *__restrict__ out)
{
    __shared__ float red[4];
    const long xo = (long)blockIdx.x * ldx, o = (long)blockIdx.x * n;
    const int tid = threadIdx.x;
    float ss = 0.0f;
    for (int i = tid; i < n; i += 256) {
        float v = x[xo + i];
        if (x_up) v = mllm_silu_mul(v, x_up[xo + i], clamp != 0);
        if (x_res) v += x_res[xo + i];
        if (res_out) res_out[xo + i] = v;
        ss = fmaf(v, v, ss);
        out[o + i] = v;
    }
    if (!rms_w) return;
    for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d, 64);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float r = sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)n + eps);
    const float sc = div ? r : 1.0f / r;
    for (int i = tid; i < n; i += 256) {
        const float v = out[o + i];       // written by this same thread above
        out[o + i] = (div ? v / sc : v * sc) * rms_w[i];
    }
}

// out[b][r] = silu(y[b][r]) * y[b][n + r] (+ add[b][r]) for the stacked
// gate/up rows of a paired GEMV that ran unfused (y: [B][2n]).
__global__ void k_silu_pair(const float *__restrict__ y, int B, int n, int clamp, float *__restrict__ out,
                            const float *__restrict__ add)
{
    const int r = blockIdx.x * blockDim.x + threadIdx.x, b = blockIdx.y;
    if (r >= n || b >= B) return;
    const float *yb = y + (long)b * 2 * n;
    const float v = mllm_silu_mul(yb[r], yb[n + r], clamp != 0);
    const long o = (long)b * n + r;
    out[o] = add ? add[o] + v : v;
}


// The reference caller's lm_head requantisation (TE:620-666) of fp32 rows:
// per 32 elements amax = max(max|x|, 1e-10f), d = amax / 127,
// q = rint(x / d) clamped to +-127 (IEEE division, round half to even, as
// numpy's float32 ops), written as raw Q8_0 blocks: fp16(d), then 32 quants.
__global__ void k_requant_q8_0(const float *__restrict__ w, int n_rows, int n_cols, uint8_t *__restrict__ out)
{
    const int nb = n_cols / 32;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)n_rows * nb) return;
    const long r = i / nb, b = i - r * nb;
    const float *x = w + r * n_cols + 32 * b;
    float v[32];
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; k++) {
        v[k] = x[k];
        const float a = fabsf(v[k]);
        amax = a > amax ? a : amax;
    }
    amax = amax < 1e-10f ? 1e-10f : amax;
    const float d = __fdiv_rn(amax, 127.0f);
    const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)d);
    uint8_t *dst = out + i * 34;
    dst[0] = (uint8_t)(h & 0xFF);
    dst[1] = (uint8_t)(h >> 8);
#pragma unroll
    for (int k = 0; k < 32; k++) {
        float q = rintf(__fdiv_rn(v[k], d));
        q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
        dst[2 + k] = (uint8_t)(int8_t)(int)q;
    }
}

// TE:643-645's F16 conversion, raw_u16.astype(np.float32).view(np.float32): each
// 16-bit pattern becomes its integer value (exact in fp32), not its fp16 value.
__global__ void k_u16_value_f32(const uint16_t *__restrict__ u, long n, float *__restrict__ out)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = (float)u[i];
}

__global__ void k_fill_f32(float *__restrict__ p, long n, float v)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// Scale scan of n_mats packed matrices (tab, or the one view) of layout ly,
// nblk blocks each: *flags |= 1 when a block scale is not finite (fp16
// exponent 31, or an E8M0 byte of 255), |= 2 when an E8M0 byte is >= 178:
// there 2^(E-127) times the largest fp16 Q8_0 scale (65504) can exceed 1e20,
// where mxfp4_row_dot_q8 clamps the combined scale (QK:648-650), and from
// E = 194 on mxfp4_batch_matmul's scale clamp to 1e20 (CE:454-456) gives
// weights no longer exact in bf16.
__global__ void k_scale_scan(const mllm_packed *__restrict__ tab, mllm_packed one, int ly, long nblk,
                             int *__restrict__ flags)
{
    const mllm_packed v = tab ? tab[blockIdx.y] : one;
    int f = 0;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < nblk; i += (long)gridDim.x * blockDim.x) {
        auto h = [&](int plane, int stride, int off) {
            const uint8_t *q = v.p[plane] + i * stride + off;
            return ((q[0] | (q[1] << 8)) & 0x7C00) == 0x7C00;
        };
        switch (ly) {
        case LY_Q4_0: case LY_Q8_0: f |= h(1, 2, 0); break;
        case LY_Q4_1: f |= h(1, 4, 0) | h(1, 4, 2); break;
        case LY_Q5_0: f |= h(2, 2, 0); break;
        case LY_Q4_K: f |= h(1, 16, 0) | h(1, 16, 2); break;
        case LY_Q5_K_GGML: case LY_Q5_K_CE: f |= h(2, 16, 0) | h(2, 16, 2); break;
        case LY_Q6_K: f |= h(3, 2, 0); break;
        case LY_MXFP4: {
            const uint8_t e = v.p[1][i];
            f |= (e == 255 ? 1 : 0) | (e >= 178 ? 2 : 0);
            break;
        }
        default: break;
        }
    }
    if (f) atomicOr(flags, f);
}

// out[i] += add[i], i < n (the residual epilogue of launches that cannot fuse it).
__global__ void k_add(float *__restrict__ out, const float *__restrict__ add, long n)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] += add[i];
}

__global__ void k_combine(const float *__restrict__ d, const float *__restrict__ w, const int *__restrict__ idx,
                          int K, int N, float *__restrict__ out, int fused)
{
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    float acc = 0.0f;
    for (int k = 0; k < K; k++) {
        // a slot the routing left empty (expert -1: a token whose logits hold
        // an inf or NaN never inserts an expert) adds nothing, as the
        // reference skips e < 0 (CE:640-641)
        if (idx && idx[(long)t * K + k] < 0) continue;
        const float wk = w[(long)t * K + k], dv = d ? d[((long)t * K + k) * N + i] : 0.0f;
        acc = fused ? fmaf(wk, dv, acc) : acc + wk * dv;
    }
    out[(long)t * N + i] = acc;
}

} // namespace

mllm_packed mllm_packed_view(int ly, const uint8_t *packed, int n_rows, int n_cols)
{
    long offs[MLLM_MAX_PLANES] = {0, 0, 0, 0};
    mllm_packed_bytes(ly, n_rows, n_cols, offs);
    mllm_packed v;
    const mllm_layout_desc L = mllm_layout_info(ly);
    for (int i = 0; i < MLLM_MAX_PLANES; i++) v.p[i] = i < L.n_planes ? packed + offs[i] : nullptr;
    if (ly == LY_F32) v.p[0] = packed;
    return v;
}

hipError_t mllm_launch_pack(int ly, const uint8_t *raw, uint8_t *packed, int n_rows, int n_cols, hipStream_t st)
{
    if (ly == LY_F32)
        return hipMemcpyAsync(packed, raw, (size_t)n_rows * n_cols * 4, hipMemcpyDeviceToDevice, st);
    long offs[MLLM_MAX_PLANES] = {0, 0, 0, 0};
    mllm_packed_bytes(ly, n_rows, n_cols, offs);
    const mllm_layout_desc L = mllm_layout_info(ly);
    const long nblk = (long)n_rows * (n_cols / L.block_elems);
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL(k_pack, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, st, ly, raw, packed, nblk,
                       offs[0], offs[1], offs[2], offs[3]);
    return hipGetLastError();
}

hipError_t mllm_launch_quantize_q8_0(const float *x, int T, int n_cols, uint8_t *q8_raw, int8_t *xq_q, float *xq_d,
                                     float *xq_s4, int *xq_sq, hipStream_t st, const float *x_up)
{
    const long n = (long)T * (n_cols / 32);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_quantize_q8_0, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, st, x, T, n_cols, q8_raw,
                       xq_q, xq_d, xq_s4, xq_sq, x_up);
    return hipGetLastError();
}

long mllm_router_packed_floats(int N, int E)
{
    return (long)((N + kRouteRowPad - 1) / kRouteRowPad) * kRouteRowPad * E;
}

hipError_t mllm_launch_router_pack(const float *router, int N, int E, float *out, hipStream_t st)
{
    if (N <= 0 || E <= 0) return hipErrorInvalidValue;
    const long n4 = mllm_router_packed_floats(N, E) / 4;
    hipLaunchKernelGGL(k_router_pack, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, router, N, E, out);
    return hipGetLastError();
}

long mllm_route_workspace_floats(int T, int E) { return (long)T * E; }

// Workgroups the T > 8 routing launch aims for.
constexpr int kRouteMinGroups = 128;

// Decode routing shape: row chunks, and router / x float4 loads per thread and chunk.
constexpr int kRouteSliceChunks = 2, kRouteSliceSlots = 8, kRouteSliceXSlots = 2;

hipError_t mllm_launch_route_finish(const float *logits, int T, int E, int K, int renorm, int *top_idx, float *top_w,
                                    hipStream_t st)
{
    if (E <= 0 || E > 256 || K <= 0 || K > 16 || K > E || T <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_route_finish, dim3(T), dim3(256), 0, st, logits, T, E, K, renorm, top_idx, top_w);
    return hipGetLastError();
}

hipError_t mllm_launch_route(const float *router_p, const float *x, int T, int N, int E, int K, int renorm,
                             int *top_idx, float *top_w, float *logits_ws, hipStream_t st)
{
    if (E <= 0 || E > 256 || K <= 0 || K > 16 || K > E || T <= 0 || N <= 0) return hipErrorInvalidValue;
    const bool vec = (N % 4) == 0 && ((uintptr_t)router_p % 16) == 0 && ((uintptr_t)x % 16) == 0;
    if (!vec) {
        hipLaunchKernelGGL(k_route_any, dim3(T), dim3(256), 0, st, router_p, x, T, N, E, K, renorm, top_idx, top_w);
        return hipGetLastError();
    }
    // T <= 8, N % 4 == 0 and a logits workspace: k_route_slice over the
    // widest power-of-two expert slices whose rows fit its registers, then
    // k_route_finish.
    if (T <= 8 && logits_ws) {
        constexpr int NCH = kRouteSliceChunks, SPC = kRouteSliceSlots, XPC = kRouteSliceXSlots;
        const int KC = (N + NCH * kChainIter - 1) / (NCH * kChainIter) * kChainIter;   // steps per chunk
        int ES = 16;
        while (ES > 1 && ((KC / 4) * ES > 256 * SPC || E % ES != 0)) ES >>= 1;
        if ((KC / 4) * ES <= 256 * SPC && KC / 4 <= 256 * XPC && E % ES == 0) {
            // row strides in float4: NCH*KC/4 steps + slack, rounded to 1 mod 16
            const int rows = NCH * KC / 4 + kChainSlack / 4;
            const int RS = (rows + 15) / 16 * 16 + 1, XS = RS;
            const size_t lds = ((size_t)ES * RS + (size_t)XS) * sizeof(float4);
            hipLaunchKernelGGL((k_route_slice<NCH, SPC, XPC>), dim3(E / ES, T), dim3(256), lds, st, router_p,
                               x, T, N, E, KC, ES, RS, XS, logits_ws);
            hipLaunchKernelGGL(k_route_finish, dim3(T), dim3(256), 0, st, logits_ws, T, E, K, renorm, top_idx, top_w);
            return hipGetLastError();
        }
    }
    // More tokens with a logits workspace: k_route_bc, then k_route_finish,
    // over token ranges that keep each launch's x below 2^31 bytes (the range
    // check of its buffer loads).
    if (T > 8 && logits_ws) {
        constexpr int G = 16, KC = 16 * G;
        const int nch = ((N + KC - 1) / KC + 1) & ~1;   // even: the loop runs chunk pairs
        const long lim = ((1l << 31) - 1) / ((long)N * 4) / 16 * 16;
        if (lim < 16) return hipErrorInvalidValue;
        for (int t0 = 0; t0 < T; t0 += (int)lim) {
            const int Tc = (int)(T - t0 < lim ? T - t0 : lim);
            hipLaunchKernelGGL((k_route_bc<G>), dim3((Tc + 15) / 16, (E + RB_E - 1) / RB_E), dim3(256), 0, st,
                               router_p, x + (long)t0 * N, Tc, N, E, nch, logits_ws + (long)t0 * E);
        }
        hipLaunchKernelGGL(k_route_finish, dim3(T), dim3(256), 0, st, logits_ws, T, E, K, renorm, top_idx, top_w);
        return hipGetLastError();
    }
    // Other T <= 8: a workgroup per token, and with a logits workspace and E
    // a multiple of 16 (>= 32), one per 32- or 16-expert slice of it (each
    // streams its slice of the router; k_route_finish then takes the softmax
    // and top-K).  More tokens: token groups over the idle lanes and four
    // tokens per thread.
    auto go = [&](auto tt_c, auto pf_c, auto xs_c, int G, int ES, int lgES) {
        constexpr int TT = decltype(tt_c)::value, PF = decltype(pf_c)::value, XS = decltype(xs_c)::value;
        const int TW = G * TT;
        const int NP = (N + kRouteRowPad - 1) / kRouteRowPad * kRouteRowPad;
        int KC = 4 * 256 * PF / ES / 32 * 32;         // router slots fit
        KC = KC < NP ? KC : NP;
        int lgq = 0;
        for (;;) {                                     // x slots fit
            lgq = 0;
            while ((1 << lgq) < KC / 4) lgq++;
            if ((TW << lgq) <= 256 * XS || KC <= 32) break;
            KC -= 32;
        }
        if (KC < 32 || (TW << lgq) > 256 * XS) return hipErrorInvalidValue;
        const size_t fl = 2 * ((size_t)KC * ES + (size_t)TW * (KC + 4)) + route_slack(ES);
        const size_t fin = (size_t)route_finish_floats(TW, E);
        const size_t lds = (fl > fin ? fl : fin) * sizeof(float);
        hipLaunchKernelGGL((k_route<TT, PF, XS>), dim3((T + TW - 1) / TW, E / ES), dim3(256), lds, st, router_p, x,
                           T, N, E, K, renorm, KC, G, lgq, lgES, lgES >= 0 ? logits_ws : nullptr, top_idx, top_w);
        return hipGetLastError();
    };
    using I = std::integral_constant<int, 1>;
    if (T <= 8) {
        if (logits_ws && E % 16 == 0 && E >= 32) {
            const bool s32 = E % 32 == 0 && E >= 64;   // 32-expert slices, or 16 for E = 32, 48, ...
            hipError_t r = go(I{}, std::integral_constant<int, 16>{}, I{}, 1, s32 ? 32 : 16, s32 ? 5 : 4);
            if (r != hipSuccess) return r;
            hipLaunchKernelGGL(k_route_finish, dim3(T), dim3(256), 0, st, logits_ws, T, E, K, renorm, top_idx, top_w);
            return hipGetLastError();
        }
        return go(I{}, std::integral_constant<int, 16>{}, I{}, 1, E, -1);
    }
    // token groups per workgroup: as many as the 256 threads hold, but few
    // enough that the launch has about one workgroup per CU (each
    // workgroup's time is its chains' latency, whatever its token count)
    int G = 256 / E;
    G = G > 8 ? 8 : G;
    while (G > 1 && (T + 4 * G - 1) / (4 * G) < kRouteMinGroups) G >>= 1;
    return go(std::integral_constant<int, 4>{}, std::integral_constant<int, 8>{}, std::integral_constant<int, 4>{}, G,
              E, -1);
}

hipError_t mllm_launch_act_prologue(const float *x, const float *x_res, float *res_out, const float *rms_w, float eps,
                                    int div, const float *x_up, int clamp, int T, int n, int ldx, float *out,
                                    hipStream_t st)
{
    if (T <= 0 || n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_act_prologue, dim3(T), dim3(256), 0, st, x, x_res, res_out, rms_w, eps, div, x_up, clamp, n,
                       ldx, out);
    return hipGetLastError();
}

// Plain streaming read: two 16-byte loads in flight per lane, each word once.
__global__ __launch_bounds__(256) void k_read_probe(const uint4 *__restrict__ p, long n16, uint4 *__restrict__ sink)
{
    const long G = (long)gridDim.x * 256;
    uint32_t acc = 0;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n16; i += 2 * G) {
        const uint4 a = p[i];
        const uint4 b = i + G < n16 ? p[i + G] : make_uint4(0, 0, 0, 0);
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w;
    }
    if (acc == 0x9E3779B9u) sink[0] = make_uint4(acc, acc, acc, acc);
}

hipError_t mllm_launch_read_probe(const void *p, long bytes, void *sink, hipStream_t st)
{
    const long n16 = bytes / 16;
    if (n16 <= 0) return hipSuccess;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 256;
    long g = std::min<long>(4L * cus, (n16 + 511) / 512);
    hipLaunchKernelGGL(k_read_probe, dim3((unsigned)std::max<long>(1, g)), dim3(256), 0, st, (const uint4 *)p, n16,
                       (uint4 *)sink);
    return hipGetLastError();
}

hipError_t mllm_launch_silu_pair(const float *y, int B, int n, int clamp, float *out, const float *add, hipStream_t st)
{
    if (B <= 0 || n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_silu_pair, dim3((n + 255) / 256, B), dim3(256), 0, st, y, B, n, clamp, out, add);
    return hipGetLastError();
}

hipError_t mllm_launch_requant_q8_0(const float *w, int n_rows, int n_cols, uint8_t *out, hipStream_t st)
{
    const long n = (long)n_rows * (n_cols / 32);
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_requant_q8_0, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, n_rows, n_cols, out);
    return hipGetLastError();
}

hipError_t mllm_launch_u16_value_f32(const uint16_t *u, long n, float *out, hipStream_t st)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_u16_value_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, u, n, out);
    return hipGetLastError();
}

hipError_t mllm_launch_fill(float *p, long n, float v, hipStream_t st)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p, n, v);
    return hipGetLastError();
}

hipError_t mllm_launch_scale_scan(const mllm_packed *tab_dev, const mllm_packed *one, int n_mats, int sem, int n_rows,
                                  int n_cols, int *flags, hipStream_t st)
{
    const int ly = mllm_sem_layout(sem);
    const long nblk = (long)n_rows * (n_cols / mllm_layout_info(ly).block_elems);
    if (n_mats <= 0 || nblk <= 0 || ly == LY_F32 || (!tab_dev && !one)) return hipSuccess;
    const unsigned gx = (unsigned)std::min<long>((nblk + 255) / 256, 64);
    hipLaunchKernelGGL(k_scale_scan, dim3(gx, tab_dev ? (unsigned)n_mats : 1u), dim3(256), 0, st, tab_dev,
                       tab_dev ? mllm_packed{} : *one, ly, nblk, flags);
    return hipGetLastError();
}

bool mllm_scales_need_gemv(int sem, int flags)
{
    return (flags & 1) || ((sem == SEM_MXFP4_Q8 || sem == SEM_MXFP4_CLAMP) && (flags & 2));
}

hipError_t mllm_launch_add(float *out, const float *add, long n, hipStream_t st)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_add, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, add, n);
    return hipGetLastError();
}

hipError_t mllm_launch_silu_mul(const float *g, const float *u, float *h, long n, int clamp, hipStream_t st)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, h, n, clamp);
    return hipGetLastError();
}

hipError_t mllm_launch_combine(const float *d, const float *w, const int *idx, int T, int K, int N, float *out,
                               int fused, hipStream_t st)
{
    if (T <= 0 || N <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_combine, dim3((N + 255) / 256, T), dim3(256), 0, st, d, w, idx, K, N, out, fused);
    return hipGetLastError();
}
