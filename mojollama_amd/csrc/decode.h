// decode.h — device-side block decoders for every semantic, on the packed
// plane layout of mllm_common.h.
//
// Unit of work: a "chunk" of 32 weights of one row.  A chunk is two runs of
// 16 weights; run r has one scale s_r, one offset o_r and an integer bias
// b, and its activations sit at 16 consecutive element offsets starting at
// x_r.  The weights are w = s_r * (u - b) + o_r, where the unsigned codes u
// (0..255) arrive packed four to a dword (U[0..3] run 0, U[4..7] run 1) so
// that one v_cvt_f32_ubyteN converts each, and a dot product needs
//     sum_i w_i x_i = s_r * sum_i u_i x_i + (o_r - s_r * b) * sum_i x_i.
// Byte t of U[j] holds element code_pos<SEM>(j, t) of its run: in order for
// formats that keep a run's elements in one nibble half ("SEQ": Q8_0, Q4_0,
// Q4_1, Q4_K, Q5_K ggml, Q6_K ggml), interleaved for formats that put
// elements 2i and 2i+1 in the two nibbles of byte i ("ILV": MXFP4, Q5_0,
// the engine's Q5_K, Q6_K sequential).
//
// fetch<SEM>() issues the global loads of one chunk (one or two 16-byte
// loads from the bulk plane plus the block scales), codes<SEM>() decodes them
// in registers; callers fetch several rows before decoding any so the loads
// are in flight together.
#pragma once
#include <hip/hip_runtime.h>
#include <type_traits>
#include "mllm_common.h"

#define MLLM_DEV __device__ __forceinline__

MLLM_DEV float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// E8M0 byte -> float with bits (E << 23)  (QK:542, CE:449): 0 -> 0.0, 255 -> +inf.
MLLM_DEV float e8m0f(uint32_t e) { return __uint_as_float(e << 23); }

// Loads through the global address space: generic (flat) loads would share
// the LDS wait counter and serialise the weight stream behind LDS reads.
#define MLLM_GLOBAL __attribute__((address_space(1)))
typedef unsigned int mllm_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int mllm_u32x2 __attribute__((ext_vector_type(2)));
typedef float mllm_f32x4 __attribute__((ext_vector_type(4)));
template <class T> struct gld_impl {
    static MLLM_DEV T load(const void *p) { return *(const MLLM_GLOBAL T *)p; }
};
template <> struct gld_impl<uint4> {
    static MLLM_DEV uint4 load(const void *p)
    {
        const mllm_u32x4 v = *(const MLLM_GLOBAL mllm_u32x4 *)p;
        return make_uint4(v.x, v.y, v.z, v.w);
    }
};
typedef unsigned int mllm_u32x3 __attribute__((ext_vector_type(3)));
template <> struct gld_impl<uint3> {
    static MLLM_DEV uint3 load(const void *p)
    {
        const mllm_u32x3 v = *(const MLLM_GLOBAL mllm_u32x3 *)p;
        return make_uint3(v.x, v.y, v.z);
    }
};
template <> struct gld_impl<uint2> {
    static MLLM_DEV uint2 load(const void *p)
    {
        const mllm_u32x2 v = *(const MLLM_GLOBAL mllm_u32x2 *)p;
        return make_uint2(v.x, v.y);
    }
};
template <> struct gld_impl<float4> {
    static MLLM_DEV float4 load(const void *p)
    {
        const mllm_f32x4 v = *(const MLLM_GLOBAL mllm_f32x4 *)p;
        return make_float4(v.x, v.y, v.z, v.w);
    }
};
template <class T> MLLM_DEV T gld(const void *p) { return gld_impl<T>::load(p); }

// Streamed weight bytes: read once per pass, so loaded non-temporally.
MLLM_DEV uint4 ld16(const uint8_t *p)
{
    const mllm_u32x4 v = __builtin_nontemporal_load((const MLLM_GLOBAL mllm_u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
MLLM_DEV uint4 ld16c(const uint8_t *p) { return gld<uint4>(p); }

template <int SEM> struct sem_traits {
    static constexpr bool kKQuant = (SEM == SEM_Q4_K_GGML || SEM == SEM_Q4_K_Q8 || SEM == SEM_Q5_K_GGML ||
                                     SEM == SEM_Q5_K_CE || SEM == SEM_Q6_K_GGML || SEM == SEM_Q6_K_LOWNIB ||
                                     SEM == SEM_Q6_K_SEQ);
    static constexpr int kBlockElems = kKQuant ? 256 : 32;
    static constexpr int kChunksPerBlock = kBlockElems / 32;
    // element order of the codes: interleaved nibbles
    static constexpr bool kIlv = (SEM == SEM_MXFP4 || SEM == SEM_MXFP4_CLAMP || SEM == SEM_Q5_0_F32 ||
                                  SEM == SEM_Q5_K_CE || SEM == SEM_Q6_K_SEQ);
    static constexpr int kBias = (SEM == SEM_Q8_0) ? 128 : (SEM == SEM_Q4_0 || SEM == SEM_MXFP4 ||
                                  SEM == SEM_MXFP4_CLAMP) ? 8 : (SEM == SEM_Q5_0_F32) ? 16 :
                                 (SEM == SEM_Q6_K_GGML || SEM == SEM_Q6_K_LOWNIB || SEM == SEM_Q6_K_SEQ) ? 32 : 0;
    // weights carry an offset term o (Q4_1 min, K-quant mins) besides the bias
    static constexpr bool kOffset = (SEM == SEM_Q4_1 || SEM == SEM_Q4_K_GGML || SEM == SEM_Q5_K_GGML ||
                                     SEM == SEM_Q5_K_CE);
    // raw GGUF bytes per 32 weights (rounded), for launch-shape choices
    static constexpr int kBytesPer32 = (SEM == SEM_Q8_0) ? 34 : (SEM == SEM_Q4_1) ? 20 :
                                       (SEM == SEM_Q5_0_F32 || SEM == SEM_Q5_0_Q8 || SEM == SEM_Q5_K_GGML ||
                                        SEM == SEM_Q5_K_CE) ? 22 :
                                       (SEM == SEM_Q6_K_GGML || SEM == SEM_Q6_K_LOWNIB || SEM == SEM_Q6_K_SEQ) ? 26 :
                                       (SEM == SEM_MXFP4 || SEM == SEM_MXFP4_CLAMP || SEM == SEM_MXFP4_Q8) ? 17 : 18;
};

// Element offset (0..15) within its run of byte t of code word U[j].
template <int SEM>
__host__ __device__ constexpr int code_pos(int j, int t)
{
    return sem_traits<SEM>::kIlv ? 8 * ((j & 3) >> 1) + 2 * t + (j & 1) : 4 * (j & 3) + t;
}

struct raw_chunk {
    uint4 a;      // bulk quant bytes of the chunk
    uint4 b;      // second bulk piece (Q8_0 upper half, qh bytes)
    uint4 m;      // block metadata (K-quant scales)
    uint32_t d;   // scalar scale bits / scale bytes
};

struct chunk_codes {
    uint32_t U[8];
    float s0, s1, o0, o1;   // w = s*(u - bias) + o
    int x0, x1;
};

// K-quant metadata as packed by k_pack: [d:16 | dmin:16] [sc6 x 8 : 48 bits] [m6 x 8 : 48 bits]
// (the 6-bit pairs of get_scale_min_k4, QK:62-71, laid out for shift extraction).
// 32 bits of the 64-bit value hi:lo starting at bit sh (0 <= sh < 32): v_alignbit_b32.
MLLM_DEV uint32_t funnel(uint32_t hi, uint32_t lo, uint32_t sh) { return __builtin_amdgcn_alignbit(hi, lo, sh); }

MLLM_DEV void kq_pairs(const uint4 &m, int j0, int &s_a, int &m_a, int &s_b, int &m_b)
{
    // S occupies bits [0, 48) of m.y:m.z, M bits [48, 96) of m.y:m.z:m.w.
    // 32-bit funnel shifts only: 64-bit shifts would need register pairs.
    // The word pair is selected, not branched on (j0 differs between the lanes
    // of a wave): a funnel from m.w:m.z past bit 32 keeps the low 12 bits of
    // m.z >> (so - 32) since so + 12 <= 64, and 0:m.w gives m.w >> (mo - 64).
    const int so = 6 * j0, mo = 48 + 6 * j0;              // so < 48, 48 <= mo < 96
    const bool s_lo = so < 32, m_lo = mo < 64;
    const uint32_t sv = funnel(s_lo ? m.z : m.w, s_lo ? m.y : m.z, (uint32_t)so & 31);
    const uint32_t mv = funnel(m_lo ? m.w : 0u, m_lo ? m.z : m.w, (uint32_t)mo & 31);
    s_a = sv & 63; s_b = (sv >> 6) & 63;
    m_a = mv & 63; m_b = (mv >> 6) & 63;
}

template <int SEM>
MLLM_DEV void fetch(const mllm_packed &P, int nb, int row, int c, raw_chunk &r)
{
    constexpr int CPB = sem_traits<SEM>::kChunksPerBlock;
    const int blk = (int)((unsigned)c / CPB), cc = (int)((unsigned)c % CPB);   // c >= 0
    const long bi = (long)row * nb + blk;
    if constexpr (SEM == SEM_Q8_0) {
        r.a = ld16(P.p[0] + bi * 32);
        r.b = ld16(P.p[0] + bi * 32 + 16);
        r.d = gld<uint16_t>(P.p[1] + bi * 2);
    } else if constexpr (SEM == SEM_Q4_0) {
        r.a = ld16(P.p[0] + bi * 16);
        r.d = gld<uint16_t>(P.p[1] + bi * 2);
    } else if constexpr (SEM == SEM_Q4_1) {
        r.a = ld16(P.p[0] + bi * 16);
        r.d = gld<uint32_t>(P.p[1] + bi * 4);
    } else if constexpr (SEM == SEM_Q5_0_F32) {
        r.a = ld16(P.p[0] + bi * 16);
        r.b.x = gld<uint32_t>(P.p[1] + bi * 4);
        r.d = gld<uint16_t>(P.p[2] + bi * 2);
    } else if constexpr (SEM == SEM_MXFP4 || SEM == SEM_MXFP4_CLAMP) {
        r.a = ld16(P.p[0] + bi * 16);
        r.d = gld<uint8_t>(P.p[1] + bi);
    } else if constexpr (SEM == SEM_Q4_K_GGML) {
        r.a = ld16(P.p[0] + bi * 128 + 16 * cc);
        r.m = ld16c(P.p[1] + bi * 16);
    } else if constexpr (SEM == SEM_Q5_K_GGML) {
        r.a = ld16(P.p[0] + bi * 128 + 16 * cc);
        r.b = ld16c(P.p[1] + bi * 32 + 16 * (cc & 1));
        r.m = ld16c(P.p[2] + bi * 16);
    } else if constexpr (SEM == SEM_Q5_K_CE) {
        r.a = ld16(P.p[0] + bi * 128 + 16 * cc);
        r.b.x = gld<uint32_t>(P.p[1] + bi * 32 + 4 * cc);
        r.m = ld16c(P.p[2] + bi * 16);
    } else if constexpr (SEM == SEM_Q6_K_GGML || SEM == SEM_Q6_K_LOWNIB) {
        const int h = cc >> 2, q1 = (cc >> 1) & 1, lh = cc & 1;
        r.a = ld16(P.p[0] + bi * 128 + 16 * cc);
        r.b = ld16c(P.p[1] + bi * 64 + 32 * h + 16 * lh);
        const uint8_t *sc = P.p[2] + bi * 16 + 8 * h + lh + 2 * q1;
        r.m.x = gld<uint8_t>(sc);
        r.m.y = gld<uint8_t>(sc + 4);
        r.d = gld<uint16_t>(P.p[3] + bi * 2);
    } else if constexpr (SEM == SEM_Q6_K_SEQ) {
        r.a = ld16(P.p[0] + bi * 128 + 16 * cc);
        const uint2 q = gld<uint2>(P.p[1] + bi * 64 + 8 * cc);
        r.b.x = q.x; r.b.y = q.y;
        r.m.x = gld<uint16_t>(P.p[2] + bi * 16 + 2 * cc);
        r.d = gld<uint16_t>(P.p[3] + bi * 2);
    }
}

// fetch<SEM> for the chunks c = 64 it + l of one row whose 64 lanes l take a step together:
// the step's first block is uniform (ublk = row * nb + it * 64 / CPB), so each plane is
// read through a buffer resource with the step's offset in an SGPR and a lane-constant
// offset in a VGPR, without per-step 64-bit address arithmetic.  Lanes past the row's last
// chunk read the next row's bytes, or zeros past the plane's end (the resource's range
// check): their values are discarded, like the clamped chunk of fetch.  Each plane of the
// matrix must be below 4 GiB (the launcher keeps larger matrices off this path).
template <int SEM>
constexpr bool kFetchLin = SEM == SEM_Q4_K_GGML || SEM == SEM_MXFP4 || SEM == SEM_Q8_0 || SEM == SEM_Q6_K_SEQ;

struct lin_planes {
    __amdgpu_buffer_rsrc_t r[4];
};

template <int SEM>
MLLM_DEV lin_planes lin_make(const mllm_packed &P, uint32_t nblk)   // nblk: the matrix's blocks
{
    lin_planes L{};
    auto mk = [&](int i, uint32_t per) {
        L.r[i] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(P.p[i]), (short)0, (int)(nblk * per),
                                                   0x00020000);
    };
    if constexpr (SEM == SEM_Q4_K_GGML) { mk(0, 128); mk(1, 16); }
    else if constexpr (SEM == SEM_MXFP4) { mk(0, 16); mk(1, 1); }
    else if constexpr (SEM == SEM_Q8_0) { mk(0, 32); mk(1, 2); }
    else { mk(0, 128); mk(1, 64); mk(2, 16); mk(3, 2); }
    return L;
}

template <int SEM>
MLLM_DEV void fetch_lin(const lin_planes &L, uint32_t ublk, int l, raw_chunk &r)
{
    static_assert(kFetchLin<SEM>, "formats with a linear chunk layout");
    // codes: cache policy non-temporal (they stream once, as ld16); metadata: default
    auto b128 = [&](int i, int vo, uint32_t so, auto nt_c) {
        const mllm_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(L.r[i], vo, (int)so, decltype(nt_c)::value ? 2 : 0);
        return make_uint4(v.x, v.y, v.z, v.w);
    };
    using NT = std::true_type;
    using TC = std::false_type;
    if constexpr (SEM == SEM_Q4_K_GGML) {
        r.a = b128(0, 16 * l, ublk * 128u, NT{});
        r.m = b128(1, 16 * (l >> 3), ublk * 16u, TC{});
    } else if constexpr (SEM == SEM_MXFP4) {
        r.a = b128(0, 16 * l, ublk * 16u, NT{});
        r.d = __builtin_amdgcn_raw_buffer_load_b8(L.r[1], l, (int)ublk, 0);
    } else if constexpr (SEM == SEM_Q8_0) {
        r.a = b128(0, 32 * l, ublk * 32u, NT{});
        r.b = b128(0, 32 * l + 16, ublk * 32u, NT{});
        r.d = __builtin_amdgcn_raw_buffer_load_b16(L.r[1], 2 * l, (int)(ublk * 2u), 0);
    } else {   // SEM_Q6_K_SEQ
        r.a = b128(0, 16 * l, ublk * 128u, NT{});
        const auto q = __builtin_amdgcn_raw_buffer_load_b64(L.r[1], 8 * l, (int)(ublk * 64u), 0);
        r.b.x = q[0];
        r.b.y = q[1];
        r.m.x = __builtin_amdgcn_raw_buffer_load_b16(L.r[2], 2 * l, (int)(ublk * 16u), 0);
        r.d = __builtin_amdgcn_raw_buffer_load_b16(L.r[3], 2 * (l >> 3), (int)(ublk * 2u), 0);
    }
}

// Spread bit k of each of four elements (positions e0, e0+2, e0+4, e0+6 of
// `bits`) into bit 4 of the four bytes of a dword (ILV element order).
MLLM_DEV uint32_t ilv_bit4(uint32_t bits, int e0)
{
    const uint32_t v = bits >> e0;
    return ((v & 1u) << 4) | ((v & 4u) << 10) | ((v & 16u) << 16) | ((v & 64u) << 22);
}

// SIGNED_Q8: Q8_0 codes are left as the signed quant bytes (bias 0) instead of
// q + 128, for the integer-dot GEMV.
// Chunk cc of block blk of a row (chunk index c = blk * CPB + cc).
template <int SEM, bool SIGNED_Q8 = false>
MLLM_DEV void codes_at(const raw_chunk &r, int blk, int cc, chunk_codes &k)
{
    const uint32_t A[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
    const uint32_t L4 = 0x0F0F0F0Fu;
    k.o0 = k.o1 = 0.0f;
    if constexpr (SEM == SEM_Q8_0) {
        // CE:216-253 / QK:376-416: w = d*q; u = q + 128
        const uint32_t Bv[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        const uint32_t flip = SIGNED_Q8 ? 0u : 0x80808080u;
#pragma unroll
        for (int j = 0; j < 4; j++) { k.U[j] = A[j] ^ flip; k.U[4 + j] = Bv[j] ^ flip; }
        k.s0 = k.s1 = h2f(r.d);
        k.x0 = 32 * blk; k.x1 = k.x0 + 16;
    } else if constexpr (SEM == SEM_Q4_0 || SEM == SEM_Q4_1) {
        // QK:77-117: low nibble -> element k, high nibble -> 16+k; Q4_0 w = (n-8)d, Q4_1 w = n d + m
#pragma unroll
        for (int j = 0; j < 4; j++) { k.U[j] = A[j] & L4; k.U[4 + j] = (A[j] >> 4) & L4; }
        k.s0 = k.s1 = h2f(r.d & 0xFFFF);
        if constexpr (SEM == SEM_Q4_1) k.o0 = k.o1 = h2f(r.d >> 16);
        k.x0 = 32 * blk; k.x1 = k.x0 + 16;
    } else if constexpr (SEM == SEM_Q5_0_F32) {
        // QK:1245-1266: element e = nibble (e&1) of ql[e/2] | bit e of qh << 4, minus 16
        const uint32_t qh = r.b.x;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            k.U[2 * m] = (A[m] & L4) | ilv_bit4(qh, 8 * m);
            k.U[2 * m + 1] = ((A[m] >> 4) & L4) | ilv_bit4(qh, 8 * m + 1);
        }
        k.s0 = k.s1 = h2f(r.d);
        k.x0 = 32 * blk; k.x1 = k.x0 + 16;
    } else if constexpr (SEM == SEM_MXFP4 || SEM == SEM_MXFP4_CLAMP) {
        // QK:485-627, CE:427-534: element e = sext4(nibble (e&1) of q[e/2]); w = v * 2^(E-127);
        // u = n ^ 8 = v + 8.
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const uint32_t w = A[m] ^ 0x88888888u;
            k.U[2 * m] = w & L4;
            k.U[2 * m + 1] = (w >> 4) & L4;
        }
        float s = e8m0f(r.d);
        if constexpr (SEM == SEM_MXFP4_CLAMP) s = fminf(s, 1e20f);
        k.s0 = k.s1 = s;
        k.x0 = 32 * blk; k.x1 = k.x0 + 16;
    } else if constexpr (SEM == SEM_Q4_K_GGML || SEM == SEM_Q5_K_GGML) {
        // CE:255-313 / QK:830-866: chunk cc = qs[16cc..16cc+16) of group g = cc/2, half h = cc&1:
        // low nibbles -> elements 64g+16h+i (pair 2g), high -> 64g+32+16h+i (pair 2g+1).
        const int g = cc >> 1, h = cc & 1;
#pragma unroll
        for (int j = 0; j < 4; j++) { k.U[j] = A[j] & L4; k.U[4 + j] = (A[j] >> 4) & L4; }
        if constexpr (SEM == SEM_Q5_K_GGML) {
            const uint32_t Q[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                k.U[j] |= ((Q[j] >> (2 * g)) & 0x01010101u) << 4;
                k.U[4 + j] |= ((Q[j] >> (2 * g + 1)) & 0x01010101u) << 4;
            }
        }
        int s1, m1, s2, m2;
        kq_pairs(r.m, 2 * g, s1, m1, s2, m2);
        const float d = h2f(r.m.x & 0xFFFF), dmin = h2f(r.m.x >> 16);
        k.s0 = d * (float)s1; k.o0 = -(dmin * (float)m1);
        k.s1 = d * (float)s2; k.o1 = -(dmin * (float)m2);
        k.x0 = 256 * blk + 64 * g + 16 * h;
        k.x1 = k.x0 + 32;
    } else if constexpr (SEM == SEM_Q5_K_CE) {
        // CE:380-425: sequential; element e = nibble (e&1) of ql[e/2] | bit (e&7) of qh[e/8] << 4, pair e/32.
        const uint32_t qh = r.b.x;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            k.U[2 * m] = (A[m] & L4) | ilv_bit4(qh, 8 * m);
            k.U[2 * m + 1] = ((A[m] >> 4) & L4) | ilv_bit4(qh, 8 * m + 1);
        }
        int s1, m1, s2, m2;
        kq_pairs(r.m, cc, s1, m1, s2, m2);
        const float d = h2f(r.m.x & 0xFFFF), dmin = h2f(r.m.x >> 16);
        k.s0 = k.s1 = d * (float)s1;
        k.o0 = k.o1 = -(dmin * (float)m1);
        k.x0 = 256 * blk + 32 * cc; k.x1 = k.x0 + 16;
    } else if constexpr (SEM == SEM_Q6_K_GGML || SEM == SEM_Q6_K_LOWNIB) {
        // QK:762-800 (ggml) and QK:1778-1812 (low nibble for quadrants 2,3):
        // chunk cc = ql[16cc..), half h = cc/4, quadrant pair q1 = (cc/2)&1, l-half lh = cc&1.
        const int h = cc >> 2, q1 = (cc >> 1) & 1, lh = cc & 1;
        const uint32_t Q[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t lo = A[j] & L4;
            const uint32_t hi = (SEM == SEM_Q6_K_LOWNIB) ? lo : ((A[j] >> 4) & L4);
            k.U[j] = lo | (((Q[j] >> (2 * q1)) & 0x03030303u) << 4);
            k.U[4 + j] = hi | (((Q[j] >> (2 * q1 + 4)) & 0x03030303u) << 4);
        }
        const float d = h2f(r.d);
        k.s0 = d * (float)(int8_t)r.m.x;
        k.s1 = d * (float)(int8_t)r.m.y;
        k.x0 = 256 * blk + 128 * h + 32 * q1 + 16 * lh;
        k.x1 = k.x0 + 64;
    } else if constexpr (SEM == SEM_Q6_K_SEQ) {
        // CE:315-378: element e = nibble (e&1) of ql[e/2] | ((qh[e/4] >> 2(e&3)) & 3) << 4, minus 32; scale sc[e/16].
        // Word m covers elements 8m' .. 8m'+7 of its qh word (m' = m & 1): their 16 qh bits h hold, in
        // nibble t, element 2t's two bits below element 2t+1's.  Nibble t goes to byte t (one byte
        // permute, one masked shift), then each half lands at bits 4-5 of its code byte.
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const uint32_t qw = (m < 2) ? r.b.x : r.b.y;
            const uint32_t h = qw >> (16 * (m & 1));
            uint32_t nb = __builtin_amdgcn_perm(h, h, 0x01010000u);     // bytes h0, h0, h1, h1
            nb = (nb & 0x000F000Fu) | ((nb >> 4) & 0x0F000F00u);         // byte t = nibble t of h
            k.U[2 * m] = (A[m] & L4) | ((nb & 0x03030303u) << 4);
            k.U[2 * m + 1] = ((A[m] >> 4) & L4) | ((nb & 0x0C0C0C0Cu) << 2);
        }
        const float d = h2f(r.d);
        k.s0 = d * (float)(int8_t)(r.m.x & 0xFF);
        k.s1 = d * (float)(int8_t)(r.m.x >> 8);
        k.x0 = 256 * blk + 32 * cc; k.x1 = k.x0 + 16;
    }
}

template <int SEM, bool SIGNED_Q8 = false>
MLLM_DEV void codes(const raw_chunk &r, int c, chunk_codes &k)
{
    constexpr int CPB = sem_traits<SEM>::kChunksPerBlock;
    codes_at<SEM, SIGNED_Q8>(r, (int)((unsigned)c / CPB), (int)((unsigned)c % CPB), k);   // c >= 0
}

// Byte t of w as a float: one v_cvt_f32_ubyte{t} (the compiler's own
// lowering of the shift-and-mask takes a v_bfe_u32 plus a conversion).
MLLM_DEV float ubyte_f(uint32_t w, int t)
{
    float r;
    switch (t) {
    case 0: asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(w)); break;
    case 1: asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(w)); break;
    case 2: asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(w)); break;
    default: asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(w)); break;
    }
    return r;
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

template <int SEM>
MLLM_DEV void q8_fetch(const mllm_packed &P, int nb, int row, int c, raw_chunk &r)
{
    if constexpr (SEM == SEM_Q4_K_Q8) {
        const int sb = c >> 2, g = c & 3;
        const long bi = (long)row * nb + sb;
        r.a = ld16(P.p[0] + bi * 128 + 32 * g);
        r.m = ld16c(P.p[1] + bi * 16);
    } else if constexpr (SEM == SEM_MXFP4_Q8) {
        const long bi = (long)row * nb + c;
        r.a = ld16(P.p[0] + bi * 16);
        r.d = gld<uint8_t>(P.p[1] + bi);
    } else {
        const long bi = (long)row * nb + c;
        r.a = ld16(P.p[0] + bi * 16);
        r.b.x = gld<uint32_t>(P.p[1] + bi * 4);
        r.d = gld<uint16_t>(P.p[2] + bi * 2);
    }
}

// Value of one chunk against a token's Q8_0 activation: q = its 32 (Q4_K: the
// two 16-byte halves at the chunk's sub-blocks) int8 quants, d8 its scale(s),
// s4 the Q4_K min-term sums.
//   Q4_K_Q8  (dot_q4_k_q8_0 QK:1647-1735): d * sum_j sc_j sum_{k<16} nib q8 - dmin * (s4_lo + s4_hi)
//   MXFP4_Q8 (mxfp4_row_dot_q8 QK:629-678): clamp(2^(E-127) d8, +-1e20) * sum v q8
//   Q5_0_Q8  (dot_q5_0_q8_0 QK:1268-1320): d5 * d8 * sum v q8
template <int SEM>
MLLM_DEV float q8_dot(const raw_chunk &r, int c, const uint4 &qa, const uint4 &qb, float d8, float s4sum)
{
    if constexpr (SEM == SEM_Q4_K_Q8) {
        const int g = c & 3;
        const uint32_t M = 0x0F0F0F0Fu;
        int dlo = 0, dhi = 0;
        dlo = dot4_i8(r.a.x & M, qa.x, dlo); dlo = dot4_i8(r.a.y & M, qa.y, dlo);
        dlo = dot4_i8(r.a.z & M, qa.z, dlo); dlo = dot4_i8(r.a.w & M, qa.w, dlo);
        dhi = dot4_i8((r.a.x >> 4) & M, qb.x, dhi); dhi = dot4_i8((r.a.y >> 4) & M, qb.y, dhi);
        dhi = dot4_i8((r.a.z >> 4) & M, qb.z, dhi); dhi = dot4_i8((r.a.w >> 4) & M, qb.w, dhi);
        int s1, m1, s2, m2;
        kq_pairs(r.m, 2 * g, s1, m1, s2, m2);
        const float d = h2f(r.m.x & 0xFFFF), dmin = h2f(r.m.x >> 16);
        return d * (float)(s1 * dlo + s2 * dhi) - dmin * s4sum;
    } else if constexpr (SEM == SEM_MXFP4_Q8) {
        float cs = e8m0f(r.d) * d8;
        cs = cs > 1e20f ? 1e20f : cs;      // comparisons, as QK:648-649: a NaN scale stays NaN
        cs = cs < -1e20f ? -1e20f : cs;
        const uint32_t wv[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        const uint32_t qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        int acc = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // bytes 4i..4i+3 hold elements 8i..8i+7 (low nibble even, high nibble odd); a nibble
            // placed in the high half of a byte is the int8 16*sext4(n).
            const uint32_t lo16 = (wv[i] << 4) & 0xF0F0F0F0u;
            const uint32_t hi16 = wv[i] & 0xF0F0F0F0u;
            const uint32_t qe = __builtin_amdgcn_perm(qv[2 * i + 1], qv[2 * i], 0x06040200u);  // even q8 bytes
            const uint32_t qo = __builtin_amdgcn_perm(qv[2 * i + 1], qv[2 * i], 0x07050301u);  // odd q8 bytes
            acc = dot4_i8(lo16, qe, acc);
            acc = dot4_i8(hi16, qo, acc);
        }
        return cs * (float)(acc >> 4);
    } else {
        const uint32_t qh = r.b.x;
        const uint32_t wv[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        const uint32_t qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        int acc = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // elements 8i..8i+7: v = (nibble | qh bit << 4) - 16; as bytes u = v + 16 in [0,31]
            const uint32_t ue = (wv[i] & 0x0F0F0F0Fu) | ilv_bit4(qh, 8 * i);
            const uint32_t uo = ((wv[i] >> 4) & 0x0F0F0F0Fu) | ilv_bit4(qh, 8 * i + 1);
            const uint32_t qe = __builtin_amdgcn_perm(qv[2 * i + 1], qv[2 * i], 0x06040200u);
            const uint32_t qo = __builtin_amdgcn_perm(qv[2 * i + 1], qv[2 * i], 0x07050301u);
            acc = dot4_i8(ue, qe, acc);
            acc = dot4_i8(uo, qo, acc);
            acc -= 16 * (dot4_i8(0x01010101u, qe, 0) + dot4_i8(0x01010101u, qo, 0));
        }
        return h2f(r.d) * d8 * (float)acc;
    }
}
