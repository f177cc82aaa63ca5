// gemv_mf.h — decode GEMV at batch 2..8 on the matrix cores (Q4_K ggml, Q6_K
// sequential, Q8_0, Q4_0, MXFP4 with and without the scale clamp).
//
// The batch-1 kernel (gemv_impl.h) dots every weight code with three int8
// digit planes of each token on the VALU; at B tokens that is 3·B v_dot4 per
// four codes, and B = 8 runs VALU-bound at a few % of HBM bandwidth.  Here the
// same exact integer products run on v_mfma_i32_32x32x16_i8:
//
//   D[32 x 32] += A[32 x 16] · B[16 x 32]
//   A row m = token t (m / 4) x digit plane p (m % 4; plane 3 is zero),
//   B column n = one weight row, k = 16 consecutive elements of one scale
//   group (a "run"; the codes are the format's unsigned codes u, as the
//   batch-1 kernel uses them, or Q8_0's signed quants).
//
// Lane l of the result holds column n = l % 32 and rows 8j + 4(l / 32) + i,
// i.e. the three planes of token t = 2j + l / 32 in consecutive registers, so
// I = (I0·2^7 + I1)·2^7 + I2 is formed in-lane and the run's fp32 epilogue
// is   acc_t += (s·P'_t)·I + o'·sum_t   (P'_t = P_t·2^-14, o' = o - s·bias).
// |I| < 2^31 for the unsigned-code forms: codes <= 15 (Q4_K, Q4_0, MXFP4)
// over 32 elements and Q6_K codes <= 63 over 16 elements, digits |d| <= 64
// (Q8_0 combines its planes in fp32).
//
// Activation digits are those of the batch-1 kernel (x = P·(d0 + d1/2^7 +
// d2/2^14), P a power of two with max|x| / P in [32, 64)), with one P per
// 32 elements for Q4_K (a sub-block: its two MFMAs accumulate into one
// integer before the epilogue) and per 16 for Q6_K (its scale group).
//
// Weights: lane (n, h = l / 32) loads 16 bytes of row n -- chunk 2q + h of a
// chunk pair -- so the two lanes of a row read 32 contiguous bytes, and one
// v_permlane32_swap per pair of words moves each half of every run to the
// lane half whose k-slots it fills.  A wave owns a 32-row tile (16 gate + 16
// up rows for paired gate/up) over a quarter of the workgroup's K range; the
// four waves' partials meet in LDS.  A workgroup stages the activations of
// its K range only, so short matrices split K over S workgroups (grid.y) and
// a second kernel adds the S partials in order (mf_part, host-provided).
//
// Non-finite values: a group holding inf / NaN is staged as the batch-1
// kernel's rare path does (P = +inf with digits +-64 / 0, or P = NaN); any
// non-finite partial makes its wave recompute that (row, token) element by
// element from the codes and digits, in the reference's product-then-sum
// form, so inf / NaN come out where the reference's do.
#pragma once
#include "gemv_impl.h"

namespace mllm_gemv {

typedef int mf_v16i __attribute__((ext_vector_type(16)));

template <int SEM> struct mf_traits {
    static constexpr bool kKQ = SEM == SEM_Q4_K_GGML || SEM == SEM_Q6_K_SEQ;
    static constexpr bool kOk = kKQ || SEM == SEM_Q8_0 || SEM == SEM_Q4_0 || SEM == SEM_MXFP4 ||
                                SEM == SEM_MXFP4_CLAMP;
    static constexpr int kG = SEM == SEM_Q6_K_SEQ ? 16 : 32;   // elements per activation scale P
    static constexpr int kBE = kKQ ? 256 : 32;                 // elements per quant block
    // elements per unit, the step of one lane pair of a row: a K-quant chunk
    // pair (64), one 32-element block of the others
    static constexpr int kUE = kKQ ? 64 : 32;
};

constexpr int kMfMaxSplits = 8;
constexpr int kMfLdsCap = 80 * 1024;   // per workgroup: two per CU
constexpr int kMfWaves = 8;            // waves per workgroup, splitting the K range's chunk pairs
constexpr int kMfThreads = 64 * kMfWaves;
static_assert(kMfWaves >= 8, "wave b computes token b's RMS scale");

// LDS of one workgroup staging kn elements of BM tokens.
struct mf_geom {
    int gs;     // bytes per 16-element digit group: [half][token * 3 + plane] x 8 bytes
    int rec;    // records [P-group][token & 1][token >> 1] float2 (P * 2^-14, group sum)
    int ssq;    // prologue sum-of-squares pieces, one per 8 elements and token
    int red;    // cross-wave partials [wave][j][lane]
    int scl;    // per-token RMS scale
    int zero;   // 16 zero bytes (A rows of plane 3 and of absent tokens)
    int total;
};

__host__ __device__ inline mf_geom mf_geom_for(int BM, int G, int kn, bool pro)
{
    mf_geom g;
    g.gs = 48 * BM;
    int o = (kn / 16) * g.gs;
    g.rec = o;
    o += (kn / G) * 64;
    g.ssq = o;
    if (pro) o += BM * (kn / 8) * 4;
    g.red = o;
    o += kMfWaves * 64 * (BM / 2) * 4;
    g.scl = o;
    o += 32;
    g.zero = o;
    o += 16;
    g.total = o;
    return g;
}

// One unit's loads for lane (n, h) of row n.  K-quants: 16 bytes of chunk
// 2q + h and the pair's side data (Q4_K: the block's d, dmin and scales;
// Q6_K: the qh bytes of both chunks, their four scales, the block's d).
// Q8_0: bytes 8h .. 8h+7 of each 16-element run (a.xy, a.zw) and d (m.x);
// Q4_0: bytes 8h .. 8h+7 of the 16 code bytes (a.xy) and d; MXFP4: the 16
// code bytes and the E8M0 byte.
template <int SEM> struct mf_pair {
    uint4 a;
    uint4 m;
};
template <> struct mf_pair<SEM_Q6_K_SEQ> {
    uint4 a;
    uint4 qh;
    uint32_t sc, d;
};

// bi: block index (row * blocks per row + block); q: chunk pair of a K-quant block.
template <int SEM>
MLLM_DEV void mf_fetch(const mllm_packed &P, long bi, int q, int h, mf_pair<SEM> &r)
{
    if constexpr (SEM == SEM_Q4_K_GGML) {
        r.a = ld16(P.p[0] + bi * 128 + 16 * (2 * q + h));
        r.m = ld16c(P.p[1] + bi * 16);
    } else if constexpr (SEM == SEM_Q6_K_SEQ) {
        r.a = ld16(P.p[0] + bi * 128 + 16 * (2 * q + h));
        r.qh = ld16c(P.p[1] + bi * 64 + 16 * q);
        r.sc = gld<uint32_t>(P.p[2] + bi * 16 + 4 * q);
        r.d = gld<uint16_t>(P.p[3] + bi * 2);
    } else if constexpr (SEM == SEM_Q8_0) {
        const uint2 lo = gld<uint2>(P.p[0] + bi * 32 + 8 * h), hi = gld<uint2>(P.p[0] + bi * 32 + 16 + 8 * h);
        r.a = make_uint4(lo.x, lo.y, hi.x, hi.y);
        r.m.x = gld<uint16_t>(P.p[1] + bi * 2);
    } else if constexpr (SEM == SEM_Q4_0) {
        const uint2 v = gld<uint2>(P.p[0] + bi * 16 + 8 * h);
        r.a = make_uint4(v.x, v.y, 0u, 0u);
        r.m.x = gld<uint16_t>(P.p[1] + bi * 2);
    } else {
        r.a = ld16(P.p[0] + bi * 16);
        r.m.x = gld<uint8_t>(P.p[1] + bi);
    }
}

MLLM_DEV void mf_swap(uint32_t &lo_half_keep, uint32_t &hi_half_keep)
{
    // lanes 32..63 of the first word trade with lanes 0..31 of the second
    const auto r = __builtin_amdgcn_permlane32_swap(lo_half_keep, hi_half_keep, false, false);
    lo_half_keep = r[0];
    hi_half_keep = r[1];
}

MLLM_DEV long mf_pack(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }

// Q6_K sequential codes of one ql word (8 elements, ILV order) and its 16 qh
// bits: the even-element word and the odd-element word (decode.h's
// SEM_Q6_K_SEQ, per word).
MLLM_DEV long mf_q6_codes(uint32_t A, uint32_t h16)
{
    uint32_t nb = __builtin_amdgcn_perm(h16, h16, 0x01010000u);
    nb = (nb & 0x000F000Fu) | ((nb >> 4) & 0x0F000F00u);
    const uint32_t L4 = 0x0F0F0F0Fu;
    return mf_pack((A & L4) | ((nb & 0x03030303u) << 4), ((A >> 4) & L4) | ((nb & 0x0C0C0C0Cu) << 2));
}

template <int JT>
MLLM_DEV void mf_epilogue(const mf_v16i &C, float s, float o, const float *rec, float (&acc)[JT])
{
#pragma unroll
    for (int j = 0; j < JT; j++) {
        const int I = (((C[4 * j] << 7) + C[4 * j + 1]) << 7) + C[4 * j + 2];   // two v_lshl_add
        acc[j] = fmaf((float)I, s * rec[2 * j], acc[j]);
        acc[j] = fmaf(o, rec[2 * j + 1], acc[j]);
    }
}

// Q8_0's signed codes reach -128 and 32 elements: a plane's integer stays
// below 2^18 but the shifted combination would pass 2^31, so the planes
// combine in fp32 (as the batch-1 kernel's three accumulators do); no offset.
template <int JT>
MLLM_DEV void mf_epilogue_f(const mf_v16i &C, float s, const float *rec, float (&acc)[JT])
{
#pragma unroll
    for (int j = 0; j < JT; j++) {
        const float t = fmaf((float)C[4 * j], 16384.0f, fmaf((float)C[4 * j + 1], 128.0f, (float)C[4 * j + 2]));
        acc[j] = fmaf(t, s * rec[2 * j], acc[j]);
    }
}

// Records of the lane's tokens (2j + h, j < JT) for P-group gp.
template <int JT>
MLLM_DEV void mf_rec(const uint8_t *lds, const mf_geom &g, int gp, int h, float (&r)[2 * JT])
{
    const float *p = reinterpret_cast<const float *>(lds + g.rec + gp * 64 + h * 32);
    if constexpr (JT >= 2) {
#pragma unroll
        for (int i = 0; i < JT / 2; i++) {
            const float4 v = reinterpret_cast<const float4 *>(p)[i];
            r[4 * i] = v.x; r[4 * i + 1] = v.y; r[4 * i + 2] = v.z; r[4 * i + 3] = v.w;
        }
    } else {
        const float2 v = *reinterpret_cast<const float2 *>(p);
        r[0] = v.x; r[1] = v.y;
    }
}

// The activation loads of staging pass `pass` (stage_load / pro_load's
// indices): every slot of every lane is loaded, indices clamped to the last
// half-group and the residual / RMS-weight loads taken from x when absent,
// so the number of loads in flight never depends on a branch and the wait
// before the digits covers these loads only, not the weight loads behind
// them.  x rows are 16-byte aligned (the launcher checks).
template <bool PRO>
MLLM_DEV void mf_stage_load(x_stage<false> &st, pro_regs &pr, const mllm_gemv_args &a, int k0, int kn, int pass)
{
    const int nh = kn >> 3, n = a.B * nh;
#pragma unroll
    for (int q = 0; q < kStageSlots; q++) {
        const int idx = min(kMfThreads * (q + pass * kStageSlots) + (int)threadIdx.x, n - 1);
        const int b = idx / nh, hh = idx - b * nh;
        const long o = (long)b * a.ldx + k0 + 8 * hh;
        st.v[q][0] = gld<float4>(a.x + o);
        st.v[q][1] = gld<float4>(a.x + o + 4);
        if constexpr (PRO) {
            const float *r = a.x_res ? a.x_res + o : a.x + o;
            const float *w = a.rms_w ? a.rms_w + k0 + 8 * hh : a.x + k0 + 8 * hh;
            pr.r[q][0] = gld<float4>(r);
            pr.r[q][1] = gld<float4>(r + 4);
            pr.w[q][0] = gld<float4>(w);
            pr.w[q][1] = gld<float4>(w + 4);
        }
    }
}

// Stage pass `pass` of the half-groups (8 elements, one thread each) of
// tokens b < B, elements [k0, k0 + kn): digits into the MFMA layout, records,
// and with the prologue the residual / RMS-weight work of gemv_impl.h.
template <int SEM, int BM, bool PRO>
MLLM_DEV void mf_stage_store(const x_stage<false> &st, const pro_regs &pr, uint8_t *lds, const mf_geom &g,
                             const mllm_gemv_args &a, int k0, int kn, int pass, bool writer)
{
    constexpr int G = mf_traits<SEM>::kG;
    constexpr float M = 12582912.0f;   // 1.5 * 2^23: rne(y) in the low mantissa bits of y + M
    const int nh = kn >> 3, B = a.B;
    float *ssq = reinterpret_cast<float *>(lds + g.ssq);
#pragma unroll
    for (int q = 0; q < kStageSlots; q++) {
        const int idx = threadIdx.x + kMfThreads * (q + pass * kStageSlots);
        // nh is a multiple of 4: the half-groups of a 32-element group sit in
        // one aligned quad of lanes and take this branch together
        if (idx >= B * nh) continue;
        const int b = idx / nh, hh = idx - b * nh, g16 = hh >> 1, half = hh & 1;
        float v[8] = {st.v[q][0].x, st.v[q][0].y, st.v[q][0].z, st.v[q][0].w,
                      st.v[q][1].x, st.v[q][1].y, st.v[q][1].z, st.v[q][1].w};
        if constexpr (PRO) prologue8(v, pr.r[q], pr.w[q], a, b, k0 + 8 * hh, writer, ssq + idx);
        float m = 0.0f, sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) { m = fmaxf(m, fabsf(v[e])); sum += v[e]; }
        m = fmaxf(m, lane_pair(m));
        sum += lane_pair(sum);             // the 16-element group's sum
        float gsum = sum;
        if constexpr (G == 32) {
            m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x4E, 0xF, 0xF, false)));
            gsum += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(gsum), 0x4E, 0xF, 0xF, false));
        }
        const bool bad = !isfinite(gsum);
        const int E = (int)((__float_as_uint(m) >> 23) & 0xFF) - 132;
        uint32_t t[3][8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float y = ldexpf(v[e], -E);
            const float t0 = y + M, r0 = y - (t0 - M);
            const float t1 = fmaf(r0, 128.0f, M), r1 = fmaf(r0, 128.0f, M - t1);
            t[0][e] = __float_as_uint(t0); t[1][e] = __float_as_uint(t1);
            t[2][e] = __float_as_uint(fmaf(r1, 128.0f, M));
        }
        float P = ldexpf(1.0f, E - 14);
        if (__builtin_expect(__any(bad), 0)) {
            // the rare path: class of the group (1 per infinite element, 256 per NaN)
            asm volatile("");
            float nf = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) nf += v[e] != v[e] ? 256.0f : isinf(v[e]) ? 1.0f : 0.0f;
            nf += lane_pair(nf);
            if constexpr (G == 32)
                nf += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(nf), 0x4E, 0xF, 0xF, false));
            if (bad && nf != 0.0f) {
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    t[0][e] = __float_as_uint(M + (isinf(v[e]) ? copysignf(64.0f, v[e]) : 0.0f));
                    t[1][e] = t[2][e] = __float_as_uint(M);
                }
                P = nf < 256.0f ? __builtin_inff() : __int_as_float(0x7FC00000);
                gsum = 0.0f;
            }
        }
        uint8_t *dst = lds + g16 * g.gs + half * (3 * BM * 8) + b * 24;
#pragma unroll
        for (int p = 0; p < 3; p++) {
            uint32_t w[2];
#pragma unroll
            for (int jj = 0; jj < 2; jj++)
                w[jj] = pack_b0(t[p][code_pos<SEM>(jj, 0)], t[p][code_pos<SEM>(jj, 1)], t[p][code_pos<SEM>(jj, 2)],
                                t[p][code_pos<SEM>(jj, 3)]);
            *reinterpret_cast<uint2 *>(dst + 8 * p) = make_uint2(w[0], w[1]);
        }
        if ((hh & (G / 8 - 1)) == 0) {
            const int gp = hh / (G / 8);
            *reinterpret_cast<float2 *>(lds + g.rec + gp * 64 + (b & 1) * 32 + (b >> 1) * 8) = make_float2(P, gsum);
        }
    }
}

// The element-by-element value of one (row, token) over the wave's chunks:
// w = s * (u - bias) + o, x = P * (d0 + d1/2^7 + d2/2^14), t += w * x in
// chunk order (decode.h codes, the batch-1 kernel's rare path).
template <int SEM, int BM>
MLLM_DEV float mf_slow(const mllm_packed &W, int nb, int row, int n_units, int wave, int tok, const uint8_t *lds,
                       const mf_geom &g, int k0)
{
    constexpr int G = mf_traits<SEM>::kG, CU = mf_traits<SEM>::kUE / 32;   // 32-element chunks per unit
    constexpr float bias = (float)digit_bias<SEM>();
    float t = 0.0f;
    for (int p = wave; p < n_units; p += kMfWaves) {
        for (int i = 0; i < CU; i++) {
            const int c = k0 / 32 + p * CU + i;   // decode.h's chunk index (a K-quant pair is chunks 2q, 2q+1)
            raw_chunk raw;
            fetch<SEM>(W, nb, row, c, raw);
            chunk_codes k;
            codes<SEM, true>(raw, c, k);
            const int e0 = k.x0 - k0, e1 = k.x1 - k0;
            const float *r0 = reinterpret_cast<const float *>(lds + g.rec + (e0 / G) * 64 + (tok & 1) * 32 + (tok >> 1) * 8);
            const float *r1 = reinterpret_cast<const float *>(lds + g.rec + (e1 / G) * 64 + (tok & 1) * 32 + (tok >> 1) * 8);
            float P0 = r0[0] * 16384.0f, P1 = r1[0] * 16384.0f;
            P0 = P0 > 0x1p127f ? 0x1p127f : P0;
            P1 = P1 > 0x1p127f ? 0x1p127f : P1;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint8_t *d0 = lds + (e0 >> 4) * g.gs + (j >> 1) * (3 * BM * 8) + tok * 24 + (j & 1) * 4;
                const uint8_t *d1 = lds + (e1 >> 4) * g.gs + (j >> 1) * (3 * BM * 8) + tok * 24 + (j & 1) * 4;
#pragma unroll
                for (int qb = 0; qb < 4; qb++) {
                    const float w0 = fmaf(k.s0, code_f<SEM>(k.U[j], qb) - bias, k.o0);
                    const float w1 = fmaf(k.s1, code_f<SEM>(k.U[4 + j], qb) - bias, k.o1);
                    const float x0 = fmaf((float)(int8_t)d0[16 + qb], 0x1p-14f,
                                          fmaf((float)(int8_t)d0[8 + qb], 0x1p-7f, (float)(int8_t)d0[qb]));
                    const float x1 = fmaf((float)(int8_t)d1[16 + qb], 0x1p-14f,
                                          fmaf((float)(int8_t)d1[8 + qb], 0x1p-7f, (float)(int8_t)d1[qb]));
                    t = fmaf(w0, P0 * x0, t);
                    t = fmaf(w1, P1 * x1, t);
                }
            }
        }
    }
    return t;
}

// grid (tiles, S): workgroup (x, s) stages K-range s (whole quant blocks) and
// walks row tiles x, x + gridDim.x, ...; wave w takes the range's chunk
// pairs w, w + 8, ... of each tile.
template <int SEM, int BM, bool PRO, bool PAIR>
__global__ __launch_bounds__(kMfThreads) void k_gemv_mf(mllm_gemv_args a)
{
    static_assert(mf_traits<SEM>::kOk, "no MFMA decode form for this semantic");
    constexpr int JT = BM / 2;
    constexpr int G = mf_traits<SEM>::kG, BE = mf_traits<SEM>::kBE, UE = mf_traits<SEM>::kUE;
    constexpr int NW = kMfWaves;
    extern __shared__ __align__(16) uint8_t lds[];
    const mllm_packed W = a.W;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nl = lane & 31, h = lane >> 5;
    const int nb = a.n_cols / BE;
    const int S = gridDim.y, s = blockIdx.y;
    const int kb0 = (int)((long)nb * s / S), nbk = (int)((long)nb * (s + 1) / S) - kb0;
    const int k0 = kb0 * BE, kn = nbk * BE;
    const mf_geom g = mf_geom_for(BM, G, kn, PRO);
    const int n_rows = a.n_rows;
    const int n_tiles = PAIR ? (n_rows + 15) / 16 : (n_rows + 31) / 32;
    // this wave's units of the K range: wave, wave + NW, ...
    const int npr = kn / UE;
    const int nw = wave < npr ? (npr - wave + NW - 1) / NW : 0;

    auto row_of = [&](int T, int n) __attribute__((always_inline)) {
        if constexpr (PAIR) {
            const int r = min(T * 16 + (n & 15), n_rows - 1);
            return n >= 16 ? r + n_rows : r;
        } else {
            return min(T * 32 + n, n_rows - 1);
        }
    };
    // every fetch is issued, clamped to a valid tile and pair, so the loads in
    // flight are the same on every path and each wait covers only the older buffers
    auto fetch_pair = [&](int T, int i, mf_pair<SEM> &r) __attribute__((always_inline)) {
        const int p = max(min(wave + NW * min(i, nw - 1), npr - 1), 0);
        const long rb = (long)row_of(min(T, n_tiles - 1), nl) * nb + kb0;
        if constexpr (mf_traits<SEM>::kKQ) mf_fetch<SEM>(W, rb + p / 4, p & 3, h, r);
        else mf_fetch<SEM>(W, rb + p, 0, h, r);
    };
    auto adv = [&](int &T, int &i) __attribute__((always_inline)) {
        if (++i >= nw) { i = 0; T += gridDim.x; }
    };

    // A operand: lane (m = nl, h) reads the digits of token m / 4, plane m % 4
    const int tA = nl >> 2, pA = nl & 3;
    const bool aval = pA < 3 && tA < a.B;
    const int abase = aval ? h * (3 * BM * 8) + (tA * 3 + pA) * 8 : g.zero;
    const int astr = aval ? g.gs : 0;
    auto opA = [&](int g16) __attribute__((always_inline)) {
        return *reinterpret_cast<const long *>(lds + abase + g16 * astr);
    };

    float acc[JT];
    auto run_pair = [&](int i, const mf_pair<SEM> &r) __attribute__((always_inline)) {
        const int p = wave + NW * i;
        const int gq = p * (UE / 16);   // first 16-element group of the unit
        const uint32_t L4 = 0x0F0F0F0Fu;
        const mf_v16i z = {};
        uint32_t w0 = r.a.x, w1 = r.a.y, w2 = r.a.z, w3 = r.a.w;
        float rec[2 * JT];
        if constexpr (SEM == SEM_Q8_0) {
            // lane half h: bytes 8h .. 8h+7 of run 0 (w0, w1) and of run 1 (w2, w3), signed codes
            mf_v16i c = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq), mf_pack(w0, w1), z, 0, 0, 0);
            c = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq + 1), mf_pack(w2, w3), c, 0, 0, 0);
            mf_rec<JT>(lds, g, p, h, rec);
            mf_epilogue_f<JT>(c, h2f(r.m.x), rec, acc);
        } else if constexpr (SEM == SEM_Q4_0) {
            // lane half h: bytes 8h .. 8h+7; low nibbles run 0, high nibbles run 1
            mf_v16i c = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq), mf_pack(w0 & L4, w1 & L4), z, 0, 0, 0);
            c = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq + 1), mf_pack((w0 >> 4) & L4, (w1 >> 4) & L4), c,
                                                      0, 0, 0);
            const float d = h2f(r.m.x);
            mf_rec<JT>(lds, g, p, h, rec);
            mf_epilogue<JT>(c, d, -8.0f * d, rec, acc);
        } else if constexpr (SEM == SEM_MXFP4 || SEM == SEM_MXFP4_CLAMP) {
            // word m holds elements 8m .. 8m+7 (even ones in the low nibbles): lane half
            // h takes word h (run 0) and word 2 + h (run 1); u = n ^ 8 = v + 8
            const uint32_t u0 = (h ? w1 : w0) ^ 0x88888888u, u1 = (h ? w3 : w2) ^ 0x88888888u;
            mf_v16i c = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq), mf_pack(u0 & L4, (u0 >> 4) & L4), z, 0, 0, 0);
            c = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq + 1), mf_pack(u1 & L4, (u1 >> 4) & L4), c, 0, 0, 0);
            float sc = e8m0f(r.m.x);
            if constexpr (SEM == SEM_MXFP4_CLAMP) sc = fminf(sc, 1e20f);
            mf_rec<JT>(lds, g, p, h, rec);
            mf_epilogue<JT>(c, sc, -8.0f * sc, rec, acc);
        } else if constexpr (SEM == SEM_Q4_K_GGML) {
            // lane half h: words 2h, 2h+1 of chunk 2q (w0, w1) and of chunk 2q+1 (w2, w3)
            mf_swap(w0, w2);
            mf_swap(w1, w3);
            mf_v16i clo = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq), mf_pack(w0 & L4, w1 & L4), z, 0, 0, 0);
            mf_v16i chi = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq + 2), mf_pack((w0 >> 4) & L4, (w1 >> 4) & L4),
                                                                z, 0, 0, 0);
            clo = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq + 1), mf_pack(w2 & L4, w3 & L4), clo, 0, 0, 0);
            chi = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq + 3), mf_pack((w2 >> 4) & L4, (w3 >> 4) & L4), chi,
                                                        0, 0, 0);
            int s1, m1, s2, m2;
            kq_pairs(r.m, 2 * (p & 3), s1, m1, s2, m2);
            const float d = h2f(r.m.x & 0xFFFF), dmin = h2f(r.m.x >> 16);
            mf_rec<JT>(lds, g, gq >> 1, h, rec);
            mf_epilogue<JT>(clo, d * (float)s1, -(dmin * (float)m1), rec, acc);
            mf_rec<JT>(lds, g, (gq >> 1) + 1, h, rec);
            mf_epilogue<JT>(chi, d * (float)s2, -(dmin * (float)m2), rec, acc);
        } else {
            // lane half h: word h of chunk 2q (w0) and of 2q+1 (w1), word 2+h of each (w2, w3)
            mf_swap(w0, w1);
            mf_swap(w2, w3);
            const uint32_t sh = 16 * h;
            const float d = h2f(r.d);
            const mf_v16i c0 = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq), mf_q6_codes(w0, r.qh.x >> sh), z, 0, 0, 0);
            const mf_v16i c1 = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq + 1), mf_q6_codes(w2, r.qh.y >> sh), z, 0, 0, 0);
            float sc = d * (float)(int8_t)(r.sc & 0xFF);
            mf_rec<JT>(lds, g, gq, h, rec);
            mf_epilogue<JT>(c0, sc, -32.0f * sc, rec, acc);
            sc = d * (float)(int8_t)((r.sc >> 8) & 0xFF);
            mf_rec<JT>(lds, g, gq + 1, h, rec);
            mf_epilogue<JT>(c1, sc, -32.0f * sc, rec, acc);
            const mf_v16i c2 = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq + 2), mf_q6_codes(w1, r.qh.z >> sh), z, 0, 0, 0);
            const mf_v16i c3 = __builtin_amdgcn_mfma_i32_32x32x16_i8(opA(gq + 3), mf_q6_codes(w3, r.qh.w >> sh), z, 0, 0, 0);
            sc = d * (float)(int8_t)((r.sc >> 16) & 0xFF);
            mf_rec<JT>(lds, g, gq + 2, h, rec);
            mf_epilogue<JT>(c2, sc, -32.0f * sc, rec, acc);
            sc = d * (float)(int8_t)(r.sc >> 24);
            mf_rec<JT>(lds, g, gq + 3, h, rec);
            mf_epilogue<JT>(c3, sc, -32.0f * sc, rec, acc);
        }
    };

    float *red = reinterpret_cast<float *>(lds + g.red);
    float *scl = reinterpret_cast<float *>(lds + g.scl);
    // end of tile T: element-by-element recomputation of non-finite partials,
    // the waves' sum, the epilogue (or the split's partial)
    auto finish_tile = [&](int T) __attribute__((always_inline)) {
        bool nonfinite = false;
#pragma unroll
        for (int j = 0; j < JT; j++) nonfinite |= !isfinite(acc[j]);
        if (__builtin_expect(__any(nonfinite), 0)) {
            asm volatile("");
            const int row = row_of(T, nl);
#pragma unroll
            for (int j = 0; j < JT; j++)
                if (!isfinite(acc[j]))
                    acc[j] = mf_slow<SEM, BM>(W, nb, row, npr, wave, 2 * j + h, lds, g, k0);
        }
#pragma unroll
        for (int j = 0; j < JT; j++) red[(wave * JT + j) * 64 + lane] = acc[j];
        __syncthreads();
        if (threadIdx.x < 64 * JT) {
            const int L = threadIdx.x & 63, j = threadIdx.x >> 6;
            float v = red[j * 64 + L];
#pragma unroll
            for (int w = 1; w < NW; w++) v += red[((w * JT) + j) * 64 + L];
            const int n = L & 31, tok = 2 * j + (L >> 5);
            const int nre = PAIR ? 2 * n_rows : n_rows;
            if (S > 1) {
                const int r = PAIR ? T * 16 + (n & 15) : T * 32 + n;
                if (tok < a.B && r < n_rows)
                    a.mf_part[((long)s * a.B + tok) * nre + (PAIR && n >= 16 ? r + n_rows : r)] = v;
            } else {
                if constexpr (PRO) {
                    if (a.rms_w && tok < a.B) v = a.rms_div ? v / scl[tok] : v * scl[tok];
                }
                int r = T * 32 + n;
                bool writes = tok < a.B;
                if constexpr (PAIR) {
                    const float u = __shfl_xor(v, 16, 64);   // the up row's value
                    v = mllm_silu_mul(v, u, !a.silu_noclamp);
                    r = T * 16 + n;
                    writes = writes && n < 16;
                }
                if (writes && r < n_rows) {
                    const long oi = (long)tok * a.ldo + r;
                    a.out[oi] = a.out_add ? a.out_add[oi] + v : v;
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < JT; j++) acc[j] = 0.0f;
    };

    int T = blockIdx.x;
    if (T >= n_tiles) return;
    // The activation loads, the first two chunk pairs' loads, the digits of
    // the first pass, then the next two pairs' loads.  Pass 0 stays out of the
    // pass loop: there the wait before the digits covers the activation loads
    // only (at a loop head it would cover every load in flight), and loads
    // complete in order, so a later pass's activation loads, issued behind
    // the weights, wait for them.
    int Tf = T, iff = 0;   // the next position to fetch
    mf_pair<SEM> b0, b1, b2, b3;
    {
        x_stage<false> xst;
        pro_regs pr;
        const bool writer = PRO && a.res_out && blockIdx.x == 0;
        mf_stage_load<PRO>(xst, pr, a, k0, kn, 0);
        __builtin_amdgcn_sched_barrier(0);
        fetch_pair(Tf, iff, b0);
        adv(Tf, iff);
        fetch_pair(Tf, iff, b1);
        adv(Tf, iff);
        if (threadIdx.x < 4) reinterpret_cast<uint32_t *>(lds + g.zero)[threadIdx.x] = 0u;
        // records of absent tokens (b >= B) hold P = 0: their rows are zero and stay finite
        for (int e = threadIdx.x; e < (kn / G) * 8; e += kMfThreads) {
            const int b = 2 * (e & 3) + ((e >> 2) & 1);   // entry e of a group: [token & 1][token >> 1]
            if (b >= a.B) reinterpret_cast<float2 *>(lds + g.rec)[e] = make_float2(0.0f, 0.0f);
        }
        mf_stage_store<SEM, BM, PRO>(xst, pr, lds, g, a, k0, kn, 0, writer);
        const int passes = (a.B * (kn >> 3) + kMfThreads * kStageSlots - 1) / (kMfThreads * kStageSlots);
        for (int pass = 1; pass < passes; pass++) {
            mf_stage_load<PRO>(xst, pr, a, k0, kn, pass);
            mf_stage_store<SEM, BM, PRO>(xst, pr, lds, g, a, k0, kn, pass, writer);
        }
        fetch_pair(Tf, iff, b2);
        adv(Tf, iff);
        fetch_pair(Tf, iff, b3);
        adv(Tf, iff);
    }
    __syncthreads();
    if constexpr (PRO) {
        // wave b sums token b's squares of the staged pieces in one fixed order;
        // the scale is read after the barrier of the first tile's end, so the
        // other waves go on meanwhile
        if (a.rms_w && wave < a.B) {
            const int nh = kn >> 3, b = wave;
            const float *ssq = reinterpret_cast<const float *>(lds + g.ssq);
            float t = 0.0f;
            for (int e = lane; e < nh; e += 64) t += ssq[b * nh + e];
            t = group_sum<64>(t);
            if (S == 1) {
                const float r = sqrtf(t / (float)a.n_cols + a.rms_eps);
                if (lane == 0) scl[b] = a.rms_div ? r : 1.0f / r;
            } else if (blockIdx.x == 0 && lane == 0) {
                // the split's share, summed by the reduction kernel
                const int nre = PAIR ? 2 * n_rows : n_rows;
                a.mf_part[(long)S * a.B * nre + s * a.B + b] = t;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < JT; j++) acc[j] = 0.0f;
    if (nw == 0) {
        // a wave without pairs in this K range still takes part in every tile's sum
        for (; T < n_tiles; T += gridDim.x) finish_tile(T);
        return;
    }
    // four chunk pairs in flight: each buffer is refilled with the position
    // four ahead as soon as it is consumed
    int i = 0;
    auto step = [&](mf_pair<SEM> &buf) __attribute__((always_inline)) {
        run_pair(i, buf);
        fetch_pair(Tf, iff, buf);
        adv(Tf, iff);
        const bool last = i == nw - 1;
        if (last) finish_tile(T);
        adv(T, i);
        return last && T >= n_tiles;
    };
    for (;;) {
        if (step(b0)) break;
        if (step(b1)) break;
        if (step(b2)) break;
        if (step(b3)) break;
    }
}

// Sum of the S split partials in split order, then the fused epilogue.
template <bool PAIR>
__global__ __launch_bounds__(256) void k_mf_reduce(mllm_gemv_args a, int S)
{
    const int n_rows = a.n_rows, nre = PAIR ? 2 * n_rows : n_rows;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)a.B * n_rows) return;
    const int tok = (int)(i / n_rows), r = (int)(i - (long)tok * n_rows);
    float v = 0.0f, u = 0.0f;
    for (int s = 0; s < S; s++) {
        v += a.mf_part[((long)s * a.B + tok) * nre + r];
        if (PAIR) u += a.mf_part[((long)s * a.B + tok) * nre + n_rows + r];
    }
    if (a.rms_w) {
        float t = 0.0f;
        for (int s = 0; s < S; s++) t += a.mf_part[(long)S * a.B * nre + s * a.B + tok];
        const float rr = sqrtf(t / (float)a.n_cols + a.rms_eps);
        if (a.rms_div) { v = v / rr; u = u / rr; }
        else { const float sc = 1.0f / rr; v *= sc; u *= sc; }
    }
    if (PAIR) v = mllm_silu_mul(v, u, !a.silu_noclamp);
    const long oi = (long)tok * a.ldo + r;
    a.out[oi] = a.out_add ? a.out_add[oi] + v : v;
}

} // namespace mllm_gemv
