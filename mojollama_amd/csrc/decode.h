// decode.h — device-side block decoders for every semantic, on the packed
// plane layout of mllm_common.h.
//
// Unit of work: a "chunk" of 32 weights of one row, split into two runs of
// 16 that each have one scale s and offset o (w = s*q + o, q integer-valued),
// and whose activations sit at 16 consecutive element offsets x0.. / x1...
// A lane loads one chunk with one or two 16-byte loads from the bulk plane
// plus its scales, and decodes it in registers.
#pragma once
#include <hip/hip_runtime.h>
#include "mllm_common.h"

#define MLLM_DEV __device__ __forceinline__

MLLM_DEV float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// E8M0 byte -> float with bits (E << 23)  (QK:542, CE:449): 0 -> 0.0, 255 -> +inf.
MLLM_DEV float e8m0f(uint32_t e) { return __uint_as_float(e << 23); }

// 6-bit (scale, min) pair j of a K-quant scale array (get_scale_min_k4 QK:62-71).
MLLM_DEV void k4_pair(int j, const uint8_t *q, int &sc, int &m)
{
    if (j < 4) { sc = q[j] & 63; m = q[j + 4] & 63; }
    else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m  = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

MLLM_DEV uint4 ld16(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }

struct mllm_chunk {
    float q[32];
    float s0, s1, o0, o1;
    int x0, x1;
};

template <int SEM> struct sem_traits {
    static constexpr int kBlockElems = (SEM == SEM_Q4_K_GGML || SEM == SEM_Q4_K_Q8 || SEM == SEM_Q5_K_GGML ||
                                        SEM == SEM_Q5_K_CE || SEM == SEM_Q6_K_GGML || SEM == SEM_Q6_K_LOWNIB ||
                                        SEM == SEM_Q6_K_SEQ) ? 256 : 32;
    static constexpr int kChunksPerBlock = kBlockElems / 32;
    static constexpr bool kHasOffset = (SEM == SEM_Q4_1 || SEM == SEM_Q4_K_GGML || SEM == SEM_Q5_K_GGML ||
                                        SEM == SEM_Q5_K_CE);
};

MLLM_DEV void bytes16(uint4 v, uint8_t b[16])
{
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 16; i++) b[i] = (w[i >> 2] >> (8 * (i & 3))) & 0xFF;
}

// Decode chunk c (0 <= c < chunks per row) of row `row`; nb = blocks per row.
template <int SEM>
MLLM_DEV void load_chunk(const mllm_packed &P, int nb, int row, int c, mllm_chunk &k)
{
    constexpr int CPB = sem_traits<SEM>::kChunksPerBlock;
    const int blk = c / CPB, cc = c % CPB;
    const long bi = (long)row * nb + blk;
    k.o0 = k.o1 = 0.0f;
    uint8_t b[16];
    if constexpr (SEM == SEM_Q8_0) {
        // CE:216-253 / QK:376-416: w = d * q
        const uint8_t *qs = P.p[0] + bi * 32;
        uint8_t b2[16];
        bytes16(ld16(qs), b);
        bytes16(ld16(qs + 16), b2);
        float d = h2f(*reinterpret_cast<const uint16_t *>(P.p[1] + bi * 2));
#pragma unroll
        for (int i = 0; i < 16; i++) { k.q[i] = (float)(int8_t)b[i]; k.q[16 + i] = (float)(int8_t)b2[i]; }
        k.s0 = k.s1 = d;
        k.x0 = 32 * blk; k.x1 = k.x0 + 16;
    } else if constexpr (SEM == SEM_Q4_0 || SEM == SEM_Q4_1) {
        // QK:77-117: low nibble -> element k, high -> 16+k; Q4_0 w = (n-8)d, Q4_1 w = n d + m
        bytes16(ld16(P.p[0] + bi * 16), b);
        const int bias = (SEM == SEM_Q4_0) ? 8 : 0;
#pragma unroll
        for (int i = 0; i < 16; i++) { k.q[i] = (float)((b[i] & 15) - bias); k.q[16 + i] = (float)((b[i] >> 4) - bias); }
        if constexpr (SEM == SEM_Q4_0) {
            k.s0 = k.s1 = h2f(*reinterpret_cast<const uint16_t *>(P.p[1] + bi * 2));
        } else {
            uint32_t dm = *reinterpret_cast<const uint32_t *>(P.p[1] + bi * 4);
            k.s0 = k.s1 = h2f(dm & 0xFFFF);
            k.o0 = k.o1 = h2f(dm >> 16);
        }
        k.x0 = 32 * blk; k.x1 = k.x0 + 16;
    } else if constexpr (SEM == SEM_Q5_0_F32) {
        // QK:1245-1266: element e = nibble (e&1) of ql[e/2] | bit e of qh << 4, minus 16
        bytes16(ld16(P.p[0] + bi * 16), b);
        uint32_t qh = *reinterpret_cast<const uint32_t *>(P.p[1] + bi * 4);
#pragma unroll
        for (int e = 0; e < 32; e++) {
            int v = ((b[e >> 1] >> ((e & 1) * 4)) & 15) | (((qh >> e) & 1) << 4);
            k.q[e] = (float)(v - 16);
        }
        k.s0 = k.s1 = h2f(*reinterpret_cast<const uint16_t *>(P.p[2] + bi * 2));
        k.x0 = 32 * blk; k.x1 = k.x0 + 16;
    } else if constexpr (SEM == SEM_MXFP4 || SEM == SEM_MXFP4_CLAMP) {
        // QK:485-627, CE:427-534: element e = sext4(nibble (e&1) of q[e/2]); w = v * 2^(E-127)
        bytes16(ld16(P.p[0] + bi * 16), b);
        float s = e8m0f(P.p[1][bi]);
        if constexpr (SEM == SEM_MXFP4_CLAMP) s = fminf(s, 1e20f);
#pragma unroll
        for (int e = 0; e < 32; e++) {
            int n = (b[e >> 1] >> ((e & 1) * 4)) & 15;
            k.q[e] = (float)(n >= 8 ? n - 16 : n);
        }
        k.s0 = k.s1 = s;
        k.x0 = 32 * blk; k.x1 = k.x0 + 16;
    } else if constexpr (SEM == SEM_Q4_K_GGML || SEM == SEM_Q5_K_GGML) {
        // CE:255-313 / QK:830-866: chunk cc = qs[16cc..16cc+16) of group g = cc/2, half h = cc&1:
        // low nibbles -> elements 64g+16h+i (pair 2g), high -> 64g+32+16h+i (pair 2g+1).
        const int g = cc >> 1, h = cc & 1;
        bytes16(ld16(P.p[0] + bi * 128 + 16 * cc), b);
        const uint8_t *meta = P.p[SEM == SEM_Q4_K_GGML ? 1 : 2] + bi * 16;
        uint4 mv = ld16(meta);
        uint8_t mb[16];
        bytes16(mv, mb);
        float d = h2f(mv.x & 0xFFFF), dmin = h2f(mv.x >> 16);
        int s1, m1, s2, m2;
        k4_pair(2 * g, mb + 4, s1, m1);
        k4_pair(2 * g + 1, mb + 4, s2, m2);
        if constexpr (SEM == SEM_Q4_K_GGML) {
#pragma unroll
            for (int i = 0; i < 16; i++) { k.q[i] = (float)(b[i] & 15); k.q[16 + i] = (float)(b[i] >> 4); }
        } else {
            uint8_t qh[16];
            bytes16(ld16(P.p[1] + bi * 32 + 16 * h), qh);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                k.q[i] = (float)((b[i] & 15) + (((qh[i] >> (2 * g)) & 1) << 4));
                k.q[16 + i] = (float)((b[i] >> 4) + (((qh[i] >> (2 * g + 1)) & 1) << 4));
            }
        }
        k.s0 = d * (float)s1; k.o0 = -(dmin * (float)m1);
        k.s1 = d * (float)s2; k.o1 = -(dmin * (float)m2);
        k.x0 = 256 * blk + 64 * g + 16 * h;
        k.x1 = k.x0 + 32;
    } else if constexpr (SEM == SEM_Q5_K_CE) {
        // CE:380-425: sequential; element e = nibble (e&1) of ql[e/2] | bit (e&7) of qh[e/8] << 4, pair e/32.
        bytes16(ld16(P.p[0] + bi * 128 + 16 * cc), b);
        uint32_t qh = *reinterpret_cast<const uint32_t *>(P.p[1] + bi * 32 + 4 * cc);
        uint4 mv = ld16(P.p[2] + bi * 16);
        uint8_t mb[16];
        bytes16(mv, mb);
        float d = h2f(mv.x & 0xFFFF), dmin = h2f(mv.x >> 16);
        int s, m;
        k4_pair(cc, mb + 4, s, m);
#pragma unroll
        for (int e = 0; e < 32; e++)
            k.q[e] = (float)(((b[e >> 1] >> ((e & 1) * 4)) & 15) | (((qh >> e) & 1) << 4));
        k.s0 = k.s1 = d * (float)s;
        k.o0 = k.o1 = -(dmin * (float)m);
        k.x0 = 256 * blk + 32 * cc; k.x1 = k.x0 + 16;
    } else if constexpr (SEM == SEM_Q6_K_GGML || SEM == SEM_Q6_K_LOWNIB) {
        // QK:762-800 (ggml) and QK:1778-1812 (low nibble for quadrants 2,3):
        // chunk cc = ql[16cc..), half h = cc/4, quadrant pair q1 = (cc/2)&1, l-half lh = cc&1.
        const int h = cc >> 2, q1 = (cc >> 1) & 1, lh = cc & 1;
        bytes16(ld16(P.p[0] + bi * 128 + 16 * cc), b);
        uint8_t qh[16];
        bytes16(ld16(P.p[1] + bi * 64 + 32 * h + 16 * lh), qh);
        const int8_t *sc = reinterpret_cast<const int8_t *>(P.p[2] + bi * 16);
        float d = h2f(*reinterpret_cast<const uint16_t *>(P.p[3] + bi * 2));
#pragma unroll
        for (int i = 0; i < 16; i++) {
            int lo = b[i] & 15;
            int hi = (SEM == SEM_Q6_K_LOWNIB) ? lo : (b[i] >> 4);
            k.q[i] = (float)((lo | (((qh[i] >> (2 * q1)) & 3) << 4)) - 32);
            k.q[16 + i] = (float)((hi | (((qh[i] >> (2 * q1 + 4)) & 3) << 4)) - 32);
        }
        k.s0 = d * (float)sc[8 * h + lh + 2 * q1];
        k.s1 = d * (float)sc[8 * h + lh + 2 * q1 + 4];
        k.x0 = 256 * blk + 128 * h + 32 * q1 + 16 * lh;
        k.x1 = k.x0 + 64;
    } else if constexpr (SEM == SEM_Q6_K_SEQ) {
        // CE:315-378: element e = nibble (e&1) of ql[e/2] | ((qh[e/4] >> 2(e&3)) & 3) << 4, minus 32; scale sc[e/16].
        bytes16(ld16(P.p[0] + bi * 128 + 16 * cc), b);
        uint2 qv = *reinterpret_cast<const uint2 *>(P.p[1] + bi * 64 + 8 * cc);
        const int8_t *sc = reinterpret_cast<const int8_t *>(P.p[2] + bi * 16);
        float d = h2f(*reinterpret_cast<const uint16_t *>(P.p[3] + bi * 2));
#pragma unroll
        for (int e = 0; e < 32; e++) {
            uint32_t qw = (e < 16) ? qv.x : qv.y;
            int up = (qw >> (2 * (e & 15))) & 3;
            k.q[e] = (float)((((b[e >> 1] >> ((e & 1) * 4)) & 15) | (up << 4)) - 32);
        }
        k.s0 = d * (float)sc[2 * cc];
        k.s1 = d * (float)sc[2 * cc + 1];
        k.x0 = 256 * blk + 32 * cc; k.x1 = k.x0 + 16;
    }
}

// ---------------------------------------------------------------- Q8_0-activation semantics
//
// Chunks: Q4_K_Q8 -> 4 per super-block (group g: qs[32g..32g+16), sub-blocks 2g, 2g+1, k < 16);
//         MXFP4_Q8 / Q5_0_Q8 -> one per 32-element block.
template <int SEM> struct q8_traits {
    static constexpr int kChunksPerBlock = (SEM == SEM_Q4_K_Q8) ? 4 : 1;
    static constexpr int kBlockElems = (SEM == SEM_Q4_K_Q8) ? 256 : 32;
};

MLLM_DEV int dot4_i8(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

// Value of chunk c of `row` against token b's Q8_0 activation (xq offset already applied).
template <int SEM>
MLLM_DEV float q8_chunk_dot(const mllm_packed &P, int nb, int row, int c, const mllm_xq &xq, long tok_q, long tok_b)
{
    if constexpr (SEM == SEM_Q4_K_Q8) {
        // dot_q4_k_q8_0 QK:1647-1735: integer term over k < 16 of each sub-block, no Q8 scale;
        // min term dmin * sum_j d8_j (sum q8[0..8) + sum q8[16..24)).
        const int sb = c >> 2, g = c & 3;
        const long bi = (long)row * nb + sb;
        uint4 w = ld16(P.p[0] + bi * 128 + 32 * g);
        uint4 mv = ld16(P.p[1] + bi * 16);
        uint8_t mb[16];
        bytes16(mv, mb);
        float d = h2f(mv.x & 0xFFFF), dmin = h2f(mv.x >> 16);
        int s1, m1, s2, m2;
        k4_pair(2 * g, mb + 4, s1, m1);
        k4_pair(2 * g + 1, mb + 4, s2, m2);
        const int jlo = 8 * sb + 2 * g, jhi = jlo + 1;
        uint4 qlo = *reinterpret_cast<const uint4 *>(xq.q + tok_q + 32L * jlo);
        uint4 qhi = *reinterpret_cast<const uint4 *>(xq.q + tok_q + 32L * jhi);
        const uint32_t M = 0x0F0F0F0Fu;
        int dlo = 0, dhi = 0;
        dlo = dot4_i8(w.x & M, qlo.x, dlo); dlo = dot4_i8(w.y & M, qlo.y, dlo);
        dlo = dot4_i8(w.z & M, qlo.z, dlo); dlo = dot4_i8(w.w & M, qlo.w, dlo);
        dhi = dot4_i8((w.x >> 4) & M, qhi.x, dhi); dhi = dot4_i8((w.y >> 4) & M, qhi.y, dhi);
        dhi = dot4_i8((w.z >> 4) & M, qhi.z, dhi); dhi = dot4_i8((w.w >> 4) & M, qhi.w, dhi);
        float mins = xq.s4[tok_b + jlo] + xq.s4[tok_b + jhi];
        return d * (float)(s1 * dlo + s2 * dhi) - dmin * mins;
    } else if constexpr (SEM == SEM_MXFP4_Q8) {
        // mxfp4_row_dot_q8 QK:629-678: cs = clamp(2^(E-127) * d8, +-1e20); cs * sum v*q8.
        const long bi = (long)row * nb + c;
        uint4 w = ld16(P.p[0] + bi * 16);
        float cs = e8m0f(P.p[1][bi]) * xq.d[tok_b + c];
        cs = fminf(fmaxf(cs, -1e20f), 1e20f);
        const int8_t *q = xq.q + tok_q + 32L * c;
        uint4 qa = *reinterpret_cast<const uint4 *>(q), qb = *reinterpret_cast<const uint4 *>(q + 16);
        uint32_t wv[4] = {w.x, w.y, w.z, w.w};
        uint32_t qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        int acc = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // bytes 4i..4i+3 hold elements 8i..8i+7 (low nibble even, high nibble odd).
            // Nibble n scaled by 16 is a valid int8 (16*sext4(n)) when placed in the high half of a byte.
            uint32_t lo16 = (wv[i] << 4) & 0xF0F0F0F0u;   // 16 * even elements
            uint32_t hi16 = wv[i] & 0xF0F0F0F0u;          // 16 * odd elements
            uint32_t qe = __builtin_amdgcn_perm(qv[2 * i + 1], qv[2 * i], 0x06040200u); // even q8 bytes
            uint32_t qo = __builtin_amdgcn_perm(qv[2 * i + 1], qv[2 * i], 0x07050301u); // odd q8 bytes
            acc = dot4_i8(lo16, qe, acc);
            acc = dot4_i8(hi16, qo, acc);
        }
        return cs * (float)(acc >> 4);
    } else {
        // dot_q5_0_q8_0 QK:1268-1320: d5 * d8 * sum v * q8
        const long bi = (long)row * nb + c;
        uint8_t b[16];
        bytes16(ld16(P.p[0] + bi * 16), b);
        uint32_t qh = *reinterpret_cast<const uint32_t *>(P.p[1] + bi * 4);
        float d5 = h2f(*reinterpret_cast<const uint16_t *>(P.p[2] + bi * 2));
        const int8_t *q = xq.q + tok_q + 32L * c;
        int acc = 0;
#pragma unroll
        for (int e = 0; e < 32; e++) {
            int v = (((b[e >> 1] >> ((e & 1) * 4)) & 15) | (((qh >> e) & 1) << 4)) - 16;
            acc += v * (int)q[e];
        }
        return d5 * xq.d[tok_b + c] * (float)acc;
    }
}
