// gemm16.hip — the K-quant GEMM on one exact fp16 weight plane (see gemm16.h).
//
// Workgroup = 4 wave64s.  A tile is 128 weight rows (DUAL: 128 gate rows and
// the same 128 up rows) x TM = 32 * EB entries; wave w owns rows 32w .. 32w+31
// (and their up rows) against all TM entries, so no two waves decode the same
// weights.  K advances in 64-position steps (a quarter of a super-block; half
// for Q4_K x Q8_0, whose dot reads 16 of every 32 elements).  Per step a lane
// (row lane % 32, K half lane / 32) loads its row's bytes for the step (one
// 16-byte load of nibbles, plus Q6_K's 2-bit planes and scales), turns them
// into four 8-element fp16 MFMA operands with the 0x6400 exponent trick (a
// 4-bit code n in the mantissa of 1024 + n) and one v_pk_fma_f16 by the
// sub-block scale (sc * n - 1024 sc: an integer <= 1024, exact), and
// multiplies them on v_mfma_f32_32x32x16_f16 against the step's activation
// tile, which the workgroup double-buffers in LDS.  The activation rows are
// laid out in exactly the K order each lane's codes arrive in (act16), so the
// weights never pass through LDS.  Each super-block's products accumulate
// apart (T) and join the result as acc += d * T, d exchanged per row through
// a few bytes of LDS into the MFMA output layout (lane l holds entry l % 32,
// rows 8 g + 4 (l / 32) + r).  Q4_K's min terms run after the loop as a small
// MFMA product of per-row hi/lo fp16 weights (-dmin m) and fp16 hi/lo sums.
#include <algorithm>
#include <cmath>
#include <type_traits>
#include "decode.h"
#include "gemm16.h"
#include "gemv.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

template <int SEM> struct q16_traits {
    static constexpr bool A4 = SEM == SEM_Q4_K_Q8;
    static constexpr bool GGML = SEM == SEM_Q4_K_GGML;
    static constexpr bool Q6 = SEM == SEM_Q6_K_SEQ || SEM == SEM_Q6_K_LOWNIB;
    // MXFP4: the scale rides in the weights, so a "super-block" is one step (two 32-blocks)
    static constexpr bool MX = SEM == SEM_MXFP4 || SEM == SEM_MXFP4_Q8;
    static constexpr bool Q8IN = SEM == SEM_MXFP4_Q8;   // activations from the Q8_0 pack
    static constexpr int PPS = MX ? 64 : A4 ? 128 : 256;   // activation positions per super-block
    static constexpr int EPS = MX ? 64 : 256;              // elements per super-block
    static constexpr int SPB = PPS / 64;                   // steps per super-block
    static constexpr int NPL = A4 ? 1 : 2;                 // activation planes
};

// Waves per workgroup (each owns 32 weight rows).  Single-matrix launches over the MoE
// layer's 64-entry expert tiles (the MXFP4 and Q6_K down projections) take 256 rows, so
// each activation tile staged in LDS serves twice the rows (the activation loads bound
// these GEMMs; Qwen3's short-K Q6_K down gained 4%, bit-identical); gate + up, whose
// two matrices already share each tile, and the 128-entry dense tiles keep 128.
template <int SEM, bool DUAL, int EB> constexpr int q16_wpg()
{
    return (q16_traits<SEM>::MX || (q16_traits<SEM>::Q6 && EB == 2)) && !DUAL ? 8 : 4;
}

// Bits 3 and 4 ... of a step position p: i = p >> 4 (MFMA of the step), kh = (p >> 3) & 1
// (lane half), j = p & 7 (slot).  sw(j): slot -> byte order of the nibble pairs (j bits 0,1 swapped).
__host__ __device__ constexpr int sw3(int j) { return (j & 4) | ((j & 1) << 1) | ((j >> 1) & 1); }
// MXFP4 slot order: slots 0,1 / 2,3 come from the low nibbles of bytes 0,2 / 1,3 of a word,
// slots 4,5 / 6,7 from their high nibbles, i.e. elements 0,4,2,6,1,5,3,7 (bits reversed).
__host__ __device__ constexpr int rev3(int j) { return ((j & 1) << 2) | (j & 2) | ((j >> 2) & 1); }

// Element (within its super-block) of activation position P (within the super-block's PPS).
template <int SEM>
__host__ __device__ constexpr int q16_elem(int P)
{
    const int st = P >> 6, p = P & 63, i = p >> 4, kh = (p >> 3) & 1, j = p & 7;
    if (SEM == SEM_Q4_K_GGML) return 64 * st + 32 * (i >> 1) + 16 * kh + 8 * (i & 1) + sw3(j);
    if (SEM == SEM_Q4_K_Q8) return 32 * (2 * (2 * st + kh) + (i >> 1)) + 8 * (i & 1) + sw3(j);
    if (SEM == SEM_Q6_K_SEQ) return 64 * st + 32 * kh + 8 * i + 4 * (j & 1) + (j >> 1);
    // MXFP4 (one step = two 32-blocks): lane half kh takes block kh, MFMA i its word i
    if (SEM == SEM_MXFP4 || SEM == SEM_MXFP4_Q8) return 32 * kh + 8 * i + rev3(j);
    // SEM_Q6_K_LOWNIB: step = (half h, l-half lh); quad q = kh + 2 (i >> 1)
    return 128 * (st >> 1) + 32 * (kh + 2 * (i >> 1)) + 16 * (st & 1) + 8 * (i & 1) + sw3(j);
}

MLLM_DEV uint32_t mk(uint32_t x, int sh) { return ((x >> sh) & 0x000F000Fu) | 0x64006400u; }

// 0x6400 in both halves: fp16 1024, whose ulp is 1 (a code in mantissa bits 0..9 adds to it).
constexpr uint32_t kMagic = 0x64006400u;

// (x & m) | c in one VOP3 instruction (m from an SGPR, c from a VGPR: gfx9 VOP3 takes no literal).
MLLM_DEV uint32_t and_or(uint32_t x, uint32_t m, uint32_t c)
{
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(c));
    return r;
}

MLLM_DEV uint32_t scl(uint32_t w, h2 s, h2 c)
{
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2, w), s, c));
}

MLLM_DEV h2 hh(float v) { return h2{(_Float16)v, (_Float16)v}; }

// Raw bytes of one row for one step.
struct q16_raw {
    u32x4 a;       // nibble bytes
    u32x4 b;       // Q6_K: qh bytes (SEQ: .x, .y)
    uint4 m;       // Q6_K: .x = scales (2 bytes), .y = d
};

// A super-block's metadata as the loop holds it: Q4_K the 16-byte record (kq_pairs layout);
// Q6_K from the step-major copy, its 16 sub-block scales and d.
struct q16_meta {
    uint4 m;
    uint32_t d;
};

// Component i (compile-time) of a uint4.
template <int I> MLLM_DEV uint32_t u4at(const uint4 &v) { return I == 0 ? v.x : I == 1 ? v.y : I == 2 ? v.z : v.w; }

// The step's four MFMA operands (8 fp16 each, as 4 words) and the super-block's d.
// SM: Q6_K's scales and d come from the step-major metadata (meta), not the step's loads.
template <int SEM, bool SM, int ST>
MLLM_DEV void q16_decode(const q16_raw &r, const q16_meta &mt, int kh, u32x4 (&o)[4], float &d)
{
    constexpr int st = ST;
    const uint4 &meta = mt.m;
    if constexpr (SEM == SEM_Q4_K_GGML || SEM == SEM_Q4_K_Q8) {
        // group g's sub-blocks 2g (low nibbles) and 2g+1 (high nibbles), QK:62-71 pairs
        const int g = SEM == SEM_Q4_K_GGML ? st : 2 * st + kh;
        int s1, m1, s2, m2;
        kq_pairs(meta, 2 * g, s1, m1, s2, m2);
        d = h2f(meta.x & 0xFFFF);
        // low nibbles (bits 0-3 of each half) give 1024 + n: sa n = (1024 + n) sa - 1024 sa;
        // high nibbles stay in bits 4-7 and give 1024 + 16 n: sb n = (1024 + 16 n) (sb / 16) - 64 sb
        const h2 sa = hh((float)s1), ca = hh(-1024.0f * (float)s1);
        const h2 sb = hh((float)s2 * 0.0625f), cb = hh(-64.0f * (float)s2);
        const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t y = w[q] >> 8;
            lo[2 * q] = scl(and_or(w[q], 0x000F000Fu, kMagic), sa, ca);
            lo[2 * q + 1] = scl(and_or(y, 0x000F000Fu, kMagic), sa, ca);
            hi[2 * q] = scl(and_or(w[q], 0x00F000F0u, kMagic), sb, cb);
            hi[2 * q + 1] = scl(and_or(y, 0x00F000F0u, kMagic), sb, cb);
        }
        o[0] = u32x4{lo[0], lo[1], lo[2], lo[3]};
        o[1] = u32x4{lo[4], lo[5], lo[6], lo[7]};
        o[2] = u32x4{hi[0], hi[1], hi[2], hi[3]};
        o[3] = u32x4{hi[4], hi[5], hi[6], hi[7]};
    } else if constexpr (SEM == SEM_Q6_K_SEQ) {
        // CE:315-378: element e = nibble (e&1) of ql[e/2] | 2 bits (e&3) of qh[e/4], minus 32, scale sc[e/16]
        // (scales 4 st + 2 kh and + 1)
        const uint32_t sp = SM ? __builtin_amdgcn_ubfe(u4at<ST>(meta), 16 * kh, 16) : r.m.x;
        d = h2f(SM ? mt.d : r.m.y);
        const float s0 = (float)(int8_t)(sp & 0xFF), s1 = (float)(int8_t)(sp >> 8);
        const h2 sa = hh(s0), ca = hh(-1056.0f * s0), sb = hh(s1), cb = hh(-1056.0f * s1);
        const uint32_t L[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t hv = ((i < 2 ? r.b.x : r.b.y) >> (16 * (i & 1))) & 0xFFFFu;
            const uint32_t hs = (hv & 0xFFu) | ((hv & 0xFF00u) << 8);
            const h2 s = i < 2 ? sa : sb, c = i < 2 ? ca : cb;
            o[i] = u32x4{scl(mk(L[i], 0) | ((hs << 4) & 0x00300030u), s, c),
                         scl(mk(L[i], 4) | ((hs << 2) & 0x00300030u), s, c),
                         scl(mk(L[i], 8) | (hs & 0x00300030u), s, c),
                         scl(mk(L[i], 12) | ((hs >> 2) & 0x00300030u), s, c)};
        }
    } else {
        // QK:1778-1812 (low nibble in all four quadrants): quad q = kh + 2 (i >> 1) takes qh bits 2q
        // (scales 8 h + lh + 2 kh and + 4 of half h = st / 2, l-half lh = st % 2)
        d = h2f(SM ? mt.d : r.m.y);
        float s0, s1;
        if constexpr (SM) {
            s0 = (float)(int8_t)__builtin_amdgcn_ubfe(u4at<2 * (ST >> 1)>(meta), 8 * ((ST & 1) + 2 * kh), 8);
            s1 = (float)(int8_t)__builtin_amdgcn_ubfe(u4at<2 * (ST >> 1) + 1>(meta), 8 * ((ST & 1) + 2 * kh), 8);
        } else {
            s0 = (float)(int8_t)(r.m.x & 0xFF);
            s1 = (float)(int8_t)(r.m.x >> 8);
        }
        const h2 sa = hh(s0), ca = hh(-1056.0f * s0), sb = hh(s1), cb = hh(-1056.0f * s1);
        const uint32_t L[4] = {r.a.x, r.a.y, r.a.z, r.a.w}, Q[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = kh + 2 * (i >> 1), w0 = 2 * (i & 1);
            const uint32_t t0 = Q[w0] >> (2 * q), t1 = Q[w0 + 1] >> (2 * q);
            const h2 s = i < 2 ? sa : sb, c = i < 2 ? ca : cb;
            o[i] = u32x4{scl(mk(L[w0], 0) | ((t0 << 4) & 0x00300030u), s, c),
                         scl(mk(L[w0], 8) | ((t0 >> 4) & 0x00300030u), s, c),
                         scl(mk(L[w0 + 1], 0) | ((t1 << 4) & 0x00300030u), s, c),
                         scl(mk(L[w0 + 1], 8) | ((t1 >> 4) & 0x00300030u), s, c)};
        }
    }
}

// MXFP4 (QK:683-720, 629-678): element e of a 32-block is v = sext4(nibble e & 1 of byte
// e / 2) times 2^(E - 127).  With the nibbles flipped by 8 (n ^ 8 = v + 8) the low nibble
// of a byte gives the fp16 1032 + v and the high nibble, left in place, 1152 + 16 v; with
// s = 2^(E + eoff) (E + eoff in [-20, 5]: every value below exact in fp16)
//     v s = (1032 + v) s - 1032 s = (1152 + 16 v) (s / 16) - 72 s,
// one v_pk_fma_f16 per pair.  E = 0 gives s = 0 (the reference's zero scale).
MLLM_DEV void q16_decode_mx(const q16_raw &r, int kh, int eoff, u32x4 (&o)[4])
{
    // E of the lane's block (byte kh of the pair); min(E, 1) 2^(E + eoff): no compare,
    // whose flag the compiler would form (and wait for) where E is loaded, not used
    const uint32_t E = __builtin_amdgcn_ubfe(r.m.x, 8 * kh, 8);
    const float s = __builtin_ldexpf(fminf((float)E, 1.0f), (int)E + eoff);
    const h2 sa = hh(s), ca = hh(-1032.0f * s), sb = hh(0.0625f * s), cb = hh(-72.0f * s);
    const uint32_t w[4] = {r.a.x ^ 0x88888888u, r.a.y ^ 0x88888888u, r.a.z ^ 0x88888888u, r.a.w ^ 0x88888888u};
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint32_t y = w[q] >> 8;
        o[q] = u32x4{scl(and_or(w[q], 0x000F000Fu, kMagic), sa, ca), scl(and_or(y, 0x000F000Fu, kMagic), sa, ca),
                     scl(and_or(w[q], 0x00F000F0u, kMagic), sb, cb), scl(and_or(y, 0x00F000F0u, kMagic), sb, cb)};
    }
}

// v and its fp16 remainder: v = hi + lo (lo the fp16 rounding of v - hi).
MLLM_DEV void split16(float v, _Float16 &hi, _Float16 &lo)
{
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// Q4_K min-term weights of one row for one k16 slice of the min product: 8 values at once.
// GGML: -dmin_b * m_j for the 8 sub-blocks of super-block b (hi/lo fp16); A4: -dmin_b for
// super-blocks b0 .. b0+7 (exact in fp16).  Loaded (q16_min_ld) one slice ahead of their
// use (q16_min_mk), so the min product's loads overlap the previous slice's MFMAs.
struct q16_min_raw {
    uint4 m;          // GGML: super-block b's metadata; A4: .x .. .w and m2 hold dmin words
    uint4 m2;
};
template <int SEM>
MLLM_DEV void q16_min_ld(const mllm_packed &W, int nb, int row, int u0, q16_min_raw &r, const uint8_t *sm, int n_rows)
{
    if (sm) {   // step-major metadata: record (b, row) at (b * n_rows + row) * 16
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(sm), (short)0, -1,
                                                                            0x00020000);
        if constexpr (SEM == SEM_Q4_K_GGML) {
            const int b = min(u0 / 8, nb - 1);
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * row, 16 * b * n_rows, 0);
            r.m = make_uint4(v.x, v.y, v.z, v.w);
        } else {
            uint32_t v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, 16 * row, 16 * min(u0 + j, nb - 1) * n_rows, 0);
            r.m = make_uint4(v[0], v[1], v[2], v[3]);
            r.m2 = make_uint4(v[4], v[5], v[6], v[7]);
        }
        return;
    }
    if constexpr (SEM == SEM_Q4_K_GGML) {
        const int b = min(u0 / 8, nb - 1);   // the 8 sub-blocks of super-block u0 / 8 (past nb: zeros, below)
        r.m = gld<uint4>(W.p[1] + ((long)row * nb + b) * 16);
    } else {
        uint32_t v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = gld<uint32_t>(W.p[1] + ((long)row * nb + min(u0 + j, nb - 1)) * 16);
        r.m = make_uint4(v[0], v[1], v[2], v[3]);
        r.m2 = make_uint4(v[4], v[5], v[6], v[7]);
    }
}
template <int SEM>
MLLM_DEV void q16_min_mk(const q16_min_raw &r, int nb, int u0, f16x8 &hi, f16x8 &lo)
{
    if constexpr (SEM == SEM_Q4_K_GGML) {
        const bool live = u0 / 8 < nb;
        const float dmin = h2f(r.m.x >> 16);
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            int s1, m1, s2, m2;
            kq_pairs(r.m, j, s1, m1, s2, m2);
            v[j] = live ? -(dmin * (float)m1) : 0.0f;
            v[j + 1] = live ? -(dmin * (float)m2) : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            _Float16 a, c;
            split16(v[j], a, c);
            hi[j] = a;
            lo[j] = c;
        }
    } else {
        const uint32_t w[8] = {r.m.x, r.m.y, r.m.z, r.m.w, r.m2.x, r.m2.y, r.m2.z, r.m2.w};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            hi[j] = (_Float16)(u0 + j < nb ? -h2f(w[j] >> 16) : 0.0f);
            lo[j] = (_Float16)0.0f;
        }
    }
}

// ---------------------------------------------------------------- the GEMM
// Raw buffer resource over p: byte offsets from p, no range limit below 2^32 - 1.
MLLM_DEV __amdgpu_buffer_rsrc_t mk_rsrc(const void *p)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, -1, 0x00020000);
}

// silu(g) = g / (1 + e^-g) with e^-g = 2^t (1 + r ln 2), t = -g log2(e) rounded and r its
// rounding error (an fma), on v_exp_f32 and v_rcp_f32 (each within 1 ulp): a few ulp from
// the correctly rounded quotient, in a third of the instructions of expf and the IEEE
// division.  Where the correction is not a number (2^t = inf, or g = +-inf and r NaN) 2^t
// stands: inf (silu = -0), 0 (g = +inf: silu = inf), inf (g = -inf: NaN), as the quotient.
MLLM_DEV float silu16(float g)
{
    constexpr float L = 1.44269502f, Llo = 1.92596299e-8f;   // log2(e) = L + Llo
    const float t = -g * L;
    const float r = fmaf(-g, L, -t) - g * Llo;
    const float e0 = __builtin_amdgcn_exp2f(t);
    const float e1 = fmaf(e0 * r, 0.693147181f, e0);
    const float e = e1 == e1 ? e1 : e0;
    return g * __builtin_amdgcn_rcpf(1.0f + e);
}
// Byte offset loads from a wave-uniform base: the address is base (SGPRs) +
// a 32-bit per-lane offset, so the loop issues no 64-bit address arithmetic.
template <class T> MLLM_DEV T gldo(const void *base, uint32_t off) { return gld<T>((const uint8_t *)base + off); }

// SM: the matrices' super-block metadata (MXFP4: exponents) read from the step-major copy
// (a.sm, mllm_launch_q16_smeta) instead of the packed planes.
template <int SEM, bool DUAL, int EB, bool SM>
__global__ __launch_bounds__((64 * q16_wpg<SEM, DUAL, EB>()), (8 / q16_wpg<SEM, DUAL, EB>())) void k_q16(q16_args a)
{
    using Q = q16_traits<SEM>;
    constexpr int WPG = q16_wpg<SEM, DUAL, EB>(), RB = DUAL ? 2 : 1, TM = 32 * EB, TN = 32 * WPG, SPB = Q::SPB, NPL = Q::NPL;
    constexpr bool MX = Q::MX;
    static_assert(SPB == 2 || SPB == 4 || MX, "steps run in units of four");
    static_assert(SM || !MX, "MXFP4 reads its exponents step-major");
    __shared__ __attribute__((aligned(16))) float sD[WPG][RB * 32];
    __shared__ int s_row[TM];

    // ---- work tile (XCD-contiguous ranges of the live tiles; entry tile fastest, so
    // the workgroups an XCD runs at once share weight rows, or with rows_fast row block
    // fastest, so they share activation tiles)
    int bx, by;
    {
        const int nx = gridDim.x, ny = a.tile_expert ? *a.n_tiles : (int)gridDim.y, total = nx * ny;
        const int L = blockIdx.x + nx * blockIdx.y;
        if (L >= total) return;
        const int xcd = L & 7;
        const int w = xcd * (total >> 3) + min(xcd, total & 7) + (L >> 3);
        if (a.rows_fast) {
            bx = w % nx;
            by = w / nx;
        } else {
            by = w % ny;
            bx = w / ny;
        }
    }
    int p0, p1;
    mllm_packed W, W2;
    const uint8_t *sm0 = nullptr, *sm1 = nullptr;   // this tile's matrices' step-major metadata
    if (a.tile_expert) {
        const int e = a.tile_expert[by];
        p0 = a.tile_begin[by];
        p1 = a.tile_end[by];
        W = a.table[e];
        if constexpr (DUAL) W2 = a.table2[e];
        if constexpr (SM) {
            sm0 = a.sm + (long)e * a.sm_stride;
            if constexpr (DUAL) sm1 = a.sm2 + (long)e * a.sm_stride;
        }
    } else {
        p0 = by * TM;
        p1 = min(p0 + TM, a.n_entries);
        W = a.W;
        if constexpr (DUAL) W2 = a.W2;
        if constexpr (SM) { sm0 = a.sm; sm1 = a.sm2; }
    }
    const int n_ent = __builtin_amdgcn_readfirstlane(p1 - p0);
    if (n_ent <= 0) return;
    const int n0 = bx * TN;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 31, kh = lane >> 5;
    int lo_any = 0;
    if (tid < TM) {
        const int row = tid < n_ent ? (a.row_of ? a.row_of[p0 + tid] : p0 + tid) : (a.row_of ? a.row_of[p0] : p0);
        s_row[tid] = row;
        if (NPL > 1) lo_any = tid < n_ent && a.x.lo_nz[row] != 0;
    }
    lo_any = __syncthreads_or(lo_any);
    const int npl = __builtin_amdgcn_readfirstlane(NPL > 1 && lo_any ? 2 : 1);

    const int nb = a.n_cols / Q::EPS;
    // super-blocks of this workgroup: all, or split z of a.ksplit (whole super-blocks: d joins per block)
    int b_beg = 0, b_end = nb;
    if (a.ksplit > 1) {
        const int bpp = (nb + a.ksplit - 1) / a.ksplit;
        b_beg = min(nb, (int)blockIdx.z * bpp);
        b_end = min(nb, b_beg + bpp);
    }
    const int wrow = min(n0 + 32 * wave + lr, a.n_rows - 1);   // the row this lane decodes

    // ---- activation tiles: direct global -> LDS loads (global_load_lds_dwordx4, 16 bytes a
    // lane).  One load instruction of a wave fills 1 KB of a buffer = 8 entry rows of 128
    // bytes (the step's 64 positions); lane i writes row i / 8, slot i % 8, and fetches
    // chunk slot ^ f(row) of its entry row, f(r) = (r ^ r >> 3) & 7 over r mod 32, so the
    // MFMA reads of 16 lanes (rows r .. r+15, one chunk each) fall in distinct banks.
    // Buffers, each its own LDS object: the compiler then tracks which outstanding loads
    // write which buffer.  One plane: buffer = step % 4, loads run three steps ahead; two
    // planes, MXFP4: buffer = 2 (step % 4) + plane, three steps ahead (eight buffers); two
    // planes, K-quants: buffer = 2 (step % 2) + plane, one step ahead.
    // load instructions per wave, plane and step (four waves: EB; MXFP4's eight: one, for
    // waves whose rows the tile's entry blocks reach)
    constexpr int NCH = TM * 8 / (64 * WPG);
    constexpr bool B8 = MX;   // K-quant tiles keep four buffers (their LDS then admits a third workgroup per CU)
    constexpr int D2 = B8 ? 3 : 1;      // two-plane prefetch distance (steps)
    __shared__ __attribute__((aligned(16))) _Float16 sB0[TM * 64], sB1[TM * 64], sB2[TM * 64], sB3[TM * 64];
    __shared__ __attribute__((aligned(16))) _Float16 sB4[B8 ? TM * 64 : 8], sB5[B8 ? TM * 64 : 8],
        sB6[B8 ? TM * 64 : 8], sB7[B8 ? TM * 64 : 8];
    auto sbuf = [&](auto i_c) __attribute__((always_inline)) -> _Float16 * {
        constexpr int i = decltype(i_c)::value;
        if constexpr (i == 0) return sB0;
        else if constexpr (i == 1) return sB1;
        else if constexpr (i == 2) return sB2;
        else if constexpr (i == 3) return sB3;
        else if constexpr (i == 4) return sB4;
        else if constexpr (i == 5) return sB5;
        else if constexpr (i == 6) return sB6;
        else return sB7;
    };
    // buffer of unit step u (0..3), plane p of a two-plane tile
    auto bidx2 = [](int u, int p) constexpr { return D2 == 3 ? 2 * u + p : 2 * (u & 1) + p; };
    auto fsw = [](int r) { return (r ^ (r >> 3)) & 7; };
    // boff: a lane's byte offsets in the first plane; boff1 in the second (from its base,
    // set by the two-plane path): rows whose second plane is zero read the zero row after it
    uint32_t boff[NCH], boff1[NCH];
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int ch = 64 * WPG * c + 64 * wave + lane, r = ch >> 3;
        boff[c] = (uint32_t)s_row[r] * (uint32_t)(a.x.ldh * 2) + 16u * (uint32_t)((ch & 7) ^ fsw(r & 31));
        boff1[c] = boff[c];
    }
    auto set_boff1 = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const int ch = 64 * WPG * c + 64 * wave + lane, r = ch >> 3;
            if (!a.x.lo_nz[s_row[r]])
                boff1[c] = (uint32_t)(a.x.zero - (a.x.h + a.x.hplane)) * 2u + 16u * (uint32_t)((ch & 7) ^ fsw(r & 31));
        }
    };
    uint32_t raddr[4];   // byte offset of the lane's MFMA operand i in a 32-row block
    {
        const int fl = fsw(lr);
#pragma unroll
        for (int i = 0; i < 4; i++) raddr[i] = 128u * lr + 16u * (uint32_t)((2 * i + kh) ^ fl);
    }
    // MXFP4 reads through buffer resources (base in SGPRs, a 32-bit lane offset, the step's
    // offset in an SGPR): no per-load 64-bit address arithmetic in the loop
    const __amdgpu_buffer_rsrc_t xrs = mk_rsrc(a.x.h);
    auto dma = [&](auto nb_c, int s, int p, _Float16 *dst) __attribute__((always_inline)) {
        constexpr int NEB = decltype(nb_c)::value;   // chunk c holds entry block c
        if constexpr (MX) {
            const int so = 2 * (p * (int)a.x.hplane + 64 * s);
            if constexpr (WPG == 8) {
                // one instruction of each of the eight waves covers two entry blocks (64 rows);
                // a one-block tile is loaded by waves 0..3
                static_assert(NCH == 1 && NEB <= 2, "eight-wave MXFP4 tiles: 64 entries");
                if (NEB == 2 || wave < 4)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *)(dst + 512 * wave),
                                                             16, (int)(p ? boff1[0] : boff[0]), so, 0, 0);
            } else {
#pragma unroll
                for (int c = 0; c < NEB; c++)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        xrs, (__attribute__((address_space(3))) void *)(dst + (256 * c + 64 * wave) * 8), 16,
                        (int)(p ? boff1[c] : boff[c]), so, 0, 0);
            }
        } else {
            const uint8_t *src = (const uint8_t *)(a.x.h + p * a.x.hplane + 64 * (long)s);
            if constexpr (WPG == 8) {
                static_assert(NCH == 1 && NEB <= 2, "eight-wave tiles: 64 entries");
                if (NEB == 2 || wave < 4)
                    __builtin_amdgcn_global_load_lds((const void *)(src + (p ? boff1[0] : boff[0])),
                                                     (void *)(dst + 512 * wave), 16, 0, 0);
            } else {
#pragma unroll
                for (int c = 0; c < NEB; c++)
                    __builtin_amdgcn_global_load_lds((const void *)(src + (p ? boff1[c] : boff[c])),
                                                     (void *)(dst + (256 * c + 64 * wave) * 8), 16, 0, 0);
            }
        }
    };
    // this wave's loads older than the newest n are done, then the workgroup meets: every
    // wave's older loads have landed and every wave has finished the previous step
    // (the builtins, not asm: the compiler's own wait tracking then knows of the wait)
    auto sync_loads = [&](auto n_c) __attribute__((always_inline)) {
        constexpr int n = decltype(n_c)::value;
        static_assert(n < 64, "vmcnt is six bits");
        __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | 0x0F70);   // vmcnt(n), expcnt/lgkmcnt: no wait
        __builtin_amdgcn_s_barrier();
    };

    // weight rows: bulk plane bytes per super-block (Q4_K / Q6_K ql: 128) and per-row offsets
    const uint32_t rq = (uint32_t)wrow * (uint32_t)(MX ? 2 * nb : nb);   // row's first super-block (MX: 32-block)
    auto fetch_w = [&](const mllm_packed &M, const uint8_t *smp, int b, int st, q16_raw &r) __attribute__((always_inline)) {
        const uint32_t bi = rq + (uint32_t)b;
        if constexpr (SEM == SEM_Q4_K_GGML) {
            r.a = gldo<u32x4>(M.p[0] + 32 * st, bi * 128u + 16u * kh);
        } else if constexpr (SEM == SEM_Q4_K_Q8) {
            r.a = gldo<u32x4>(M.p[0] + 64 * st, bi * 128u + 32u * kh);
        } else if constexpr (MX) {
            // step b: blocks 2b (lane half 0) and 2b + 1 (half 1), 16 nibble bytes and E each
            r.a = __builtin_amdgcn_raw_buffer_load_b128(mk_rsrc(M.p[0]), (int)(rq * 16u + 16u * kh), 32 * b, 0);
            // both blocks' E from the step-major copy: the wave's 32 rows read 64 contiguous
            // bytes, where the row-major plane spreads them over ~23 lines
            r.m.x = __builtin_amdgcn_raw_buffer_load_b16(mk_rsrc(smp), (int)(2u * (uint32_t)wrow), 2 * b * a.n_rows, 0);
        } else if constexpr (SEM == SEM_Q6_K_SEQ) {
            r.a = gldo<u32x4>(M.p[0] + 32 * st, bi * 128u + 16u * kh);
            const uint2 q = gldo<uint2>(M.p[1] + 16 * st, bi * 64u + 8u * kh);
            r.b.x = q.x; r.b.y = q.y;
            if constexpr (!SM) {
                r.m.x = gldo<uint16_t>(M.p[2] + 4 * st, bi * 16u + 2u * kh);
                r.m.y = gldo<uint16_t>(M.p[3], bi * 2u);
            }
        } else {   // SEM_Q6_K_LOWNIB
            const int h = st >> 1, lh = st & 1;
            r.a = gldo<u32x4>(M.p[0] + 64 * h + 16 * lh, bi * 128u + 32u * kh);
            r.b = gldo<u32x4>(M.p[1] + 32 * h + 16 * lh, bi * 64u);
            if constexpr (!SM) {
                const uint32_t so = bi * 16u + 2u * kh;
                r.m.x = gldo<uint8_t>(M.p[2] + 8 * h + lh, so) | ((uint32_t)gldo<uint8_t>(M.p[2] + 8 * h + lh + 4, so) << 8);
                r.m.y = gldo<uint16_t>(M.p[3], bi * 2u);
            }
        }
    };

    f32x16 acc[RB][EB], T[RB][EB];
#pragma unroll
    for (int r = 0; r < RB; r++)
#pragma unroll
        for (int e = 0; e < EB; e++)
#pragma unroll
            for (int v = 0; v < 16; v++) { acc[r][e][v] = 0.0f; T[r][e][v] = 0.0f; }

    // step st of a super-block: decode, then the MFMAs into T (fresh at st == 0) against
    // the step's buffers.  Entry blocks past the tile's entries run on copies of its first
    // row; the epilogue drops them.
    auto mfmas = [&](auto np_c, auto nb_c, auto st_c, auto u_c, const q16_raw (&r)[RB], const q16_meta (&meta)[RB])
                     __attribute__((always_inline)) {
        constexpr int NP = decltype(np_c)::value, NEB = decltype(nb_c)::value;
        constexpr int st = decltype(st_c)::value, u = decltype(u_c)::value;
        u32x4 A[RB][4];
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            if constexpr (MX) {
                q16_decode_mx(r[rb], kh, a.eoff, A[rb]);
            } else {
                float d;
                q16_decode<SEM, SM, st>(r[rb], meta[rb], kh, A[rb], d);
                if (st == 0 && kh == 0) sD[wave][rb * 32 + lr] = d;
            }
        }
        const uint8_t *bp[NP];
        bp[0] = (const uint8_t *)sbuf(std::integral_constant<int, NP == 1 ? u : bidx2(u, 0)>{});
        if constexpr (NP > 1) bp[1] = (const uint8_t *)sbuf(std::integral_constant<int, bidx2(u, 1)>{});
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int e = 0; e < NEB; e++) {
#pragma unroll
                for (int p = 0; p < NP; p++) {
                    const f16x8 bv = *reinterpret_cast<const f16x8 *>(bp[p] + 4096 * e + raddr[i]);
#pragma unroll
                    for (int rb = 0; rb < RB; rb++) {
                        const f16x8 av = __builtin_bit_cast(f16x8, A[rb][i]);
                        if constexpr (MX) {   // scaled weights: straight into the result
                            acc[rb][e] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc[rb][e], 0, 0, 0);
                        } else {
                            const f32x16 c = (st == 0 && i == 0 && p == 0) ? f32x16{} : T[rb][e];
                            T[rb][e] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, c, 0, 0, 0);
                        }
                    }
                }
            }
    };
    auto d_apply = [&](auto nb_c) __attribute__((always_inline)) {
        constexpr int NEB = decltype(nb_c)::value;
        // the super-block's d, per output row (rows 8 g + 4 kh + r of the lane's 16)
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            float dv[16];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 q = *reinterpret_cast<const float4 *>(&sD[wave][rb * 32 + 8 * g + 4 * kh]);
                dv[4 * g] = q.x; dv[4 * g + 1] = q.y; dv[4 * g + 2] = q.z; dv[4 * g + 3] = q.w;
            }
#pragma unroll
            for (int e = 0; e < NEB; e++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[rb][e][v] = fmaf(dv[v], T[rb][e][v], acc[rb][e][v]);
        }
        __builtin_amdgcn_wave_barrier();
    };

    // Steps run in units of four (one super-block, or two for Q4_K x Q8_0's two-step
    // super-blocks); weights are fetched three steps ahead into a ring of four.
    // NEB: the entry blocks the tile's entries occupy (a bucketing tile of at most 32
    // entries runs one: half the MFMAs and activation loads)
    auto main_loop = [&](auto np_c, auto nb_c) __attribute__((always_inline)) {
        constexpr int NP = decltype(np_c)::value, NEB = decltype(nb_c)::value, D = NP == 1 ? 3 : D2;
        // weight load instructions every step issues at least (16-byte loads, and MXFP4's
        // exponent pair: none the compiler could merge)
        constexpr int NW = RB * (MX || Q::Q6 ? 2 : 1);
        // ORD: loads issued in order (a step's activations, then its weights), so the wait
        // below counts the weights issued after them (measured: MXFP4; Q6_K down 134 -> 132
        // us at Qwen3 T = 1280).  Not Q4_K (its fused gate + up there: 92 -> 99 us, the
        // fence costs more than the wait) nor gate and up in Q6_K (their registers would
        // spill): those wait for every older load instead
        constexpr bool ORD = MX || (Q::Q6 && !DUAL);
        // activation load instructions per wave and step (eight waves: a wave whose rows the
        // tile reaches issues one per plane; the others none, and for them the count only
        // overstates what may stay in flight, which their own loads never need)
        constexpr int NDMA = WPG == 8 ? NP : NEB * NP;
        const int s_beg = b_beg * SPB, s_last = b_end * SPB - 1;
        q16_raw rw[4][RB];
        // super-block metadata (Q4_K: kq_pairs layout; Q6_K step-major: scales and d): mA
        // for the unit's first super-block, mB for its second (SPB == 2) or the next unit's
        // (SPB == 4), one unit half ahead
        q16_meta mA[RB], mB[RB];
        auto fw = [&](int s, q16_raw (&r)[RB]) __attribute__((always_inline)) {
            const int sc = min(s, s_last);
            fetch_w(W, sm0, sc / SPB, sc % SPB, r[0]);
            if constexpr (DUAL) fetch_w(W2, sm1, sc / SPB, sc % SPB, r[1]);
        };
        auto fm = [&](int b, q16_meta (&m)[RB]) __attribute__((always_inline)) {
            const int bc = min(b, b_end - 1);
            if constexpr (SM && (Q::GGML || Q::A4 || Q::Q6)) {
                // the step-major record (bc, wrow): the wave's 32 rows are contiguous
#pragma unroll
                for (int rb = 0; rb < RB; rb++) {
                    const __amdgpu_buffer_rsrc_t rs = mk_rsrc(rb == 0 ? sm0 : sm1);
                    const int so = 16 * bc * a.n_rows;
                    if constexpr (Q::Q6) {
                        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * wrow, so, 0);
                        m[rb].m = make_uint4(v.x, v.y, v.z, v.w);
                        m[rb].d = __builtin_amdgcn_raw_buffer_load_b16(rs, 2 * wrow, (int)a.sm_doff + 2 * bc * a.n_rows, 0);
                    } else {
                        const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(rs, 16 * wrow, so, 0);
                        m[rb].m = make_uint4(v.x, v.y, v.z, 0u);
                    }
                }
            } else if constexpr (Q::GGML || Q::A4) {
                // d, dmin and the six-bit scales (the mins enter through the min-term product)
                const uint32_t bi = rq + (uint32_t)bc;
                const uint3 q0 = gldo<uint3>(W.p[1], bi * 16u);
                m[0].m = make_uint4(q0.x, q0.y, q0.z, 0u);
                if constexpr (DUAL) {
                    const uint3 q1 = gldo<uint3>(W2.p[1], bi * 16u);
                    m[1].m = make_uint4(q1.x, q1.y, q1.z, 0u);
                }
            }
        };
        // the loads of step s (unit position u = (s - s_beg) % 4)
        auto load_b = [&](int s, auto u_c) __attribute__((always_inline)) {
            constexpr int u = decltype(u_c)::value;
            const int sc = min(s, s_last);
            if constexpr (NP == 1) {
                dma(nb_c, sc, 0, sbuf(std::integral_constant<int, u>{}));
            } else {
                dma(nb_c, sc, 0, sbuf(std::integral_constant<int, bidx2(u, 0)>{}));
                dma(nb_c, sc, 1, sbuf(std::integral_constant<int, bidx2(u, 1)>{}));
            }
        };
        // the prologue issues its loads in the loop's order (per step its activations, then
        // its weights), so the loads in flight at the loop head are counted alike on entry and
        // on the back edge (else the compiler waits for all of them there)
        fm(b_beg, mA);
        if constexpr (!ORD) {
            load_b(s_beg, std::integral_constant<int, 0>{});
            if constexpr (D >= 3) {
                load_b(s_beg + 1, std::integral_constant<int, 1>{});
                load_b(s_beg + 2, std::integral_constant<int, 2>{});
            }
            fw(s_beg, rw[0]);
            fw(s_beg + 1, rw[1]);
            fw(s_beg + 2, rw[2]);
        } else if constexpr (D == 3) {
            load_b(s_beg, std::integral_constant<int, 0>{});
            fw(s_beg, rw[0]);
            __builtin_amdgcn_sched_barrier(0);
            load_b(s_beg + 1, std::integral_constant<int, 1>{});
            fw(s_beg + 1, rw[1]);
            __builtin_amdgcn_sched_barrier(0);
            load_b(s_beg + 2, std::integral_constant<int, 2>{});
            fw(s_beg + 2, rw[2]);
            __builtin_amdgcn_sched_barrier(0);
        } else {   // D == 1: step s issues the activations of s + 1 and the weights of s + 3
            fw(s_beg, rw[0]);
            __builtin_amdgcn_sched_barrier(0);
            fw(s_beg + 1, rw[1]);
            __builtin_amdgcn_sched_barrier(0);
            load_b(s_beg, std::integral_constant<int, 0>{});
            __builtin_amdgcn_sched_barrier(0);
            fw(s_beg + 2, rw[2]);
            __builtin_amdgcn_sched_barrier(0);
        }
        // unit of four steps from s0.  MXFP4: a short unit (the last, when the step count is
        // not a multiple of four) runs its first s_last - s0 + 1 steps, after the loop: inside
        // it, the skipped steps would hide the count of loads in flight at the loop head from
        // the compiler, which then waits for all of them
        auto unit = [&](int s0, auto full_c) __attribute__((always_inline)) {
            constexpr bool full = decltype(full_c)::value;
            const int b0 = s0 / SPB;
            // unit step u (= step s0 + u): wait for its activation loads, start those of
            // step + D into the buffer the previous step read, and the weights of step + 3
            auto one = [&](auto u_c) __attribute__((always_inline)) {
                constexpr int u = decltype(u_c)::value;
                const int s = s0 + u;
                // the loads that surely follow step s's activation loads: each step issues its
                // activation loads, then (after a scheduling fence) at least NW weight loads,
                // so the weights issued with them and those of steps s + 1 .. s + D - 1
                sync_loads(std::integral_constant<int, ORD ? NW + (D - 1) * (NDMA + NW) : (D - 1) * NDMA>{});
                // MXFP4: keep each step's decode in its step (hoisted into an earlier one, it
                // would wait there for weight loads just issued)
                if constexpr (MX) __builtin_amdgcn_sched_barrier(0);
                load_b(s + D, std::integral_constant<int, (u + D) & 3>{});
                if constexpr (ORD) __builtin_amdgcn_sched_barrier(0);
                fw(s + 3, rw[(u + 3) & 3]);
                if constexpr (u == 0) fm(b0 + 1, mB);
                if constexpr (SPB == 2 && u == 2) fm(b0 + 2, mA);
                mfmas(np_c, nb_c, std::integral_constant<int, u % SPB>{}, u_c, rw[u], (SPB == 2 && u >= 2) ? mB : mA);
                if constexpr (!MX && u % SPB == SPB - 1) d_apply(nb_c);
            };
            one(std::integral_constant<int, 0>{});
            if constexpr (MX) {
                if (full || s0 + 1 <= s_last) one(std::integral_constant<int, 1>{});
                if (full || s0 + 2 <= s_last) one(std::integral_constant<int, 2>{});
                if (full || s0 + 3 <= s_last) one(std::integral_constant<int, 3>{});
            } else if constexpr (SPB == 4) {
                one(std::integral_constant<int, 1>{});
                one(std::integral_constant<int, 2>{});
                one(std::integral_constant<int, 3>{});
#pragma unroll
                for (int rb = 0; rb < RB; rb++) mA[rb] = mB[rb];
            } else {   // two-step super-blocks: a unit holds one or two
                one(std::integral_constant<int, 1>{});
                if (s0 + 2 <= s_last) {
                    one(std::integral_constant<int, 2>{});
                    one(std::integral_constant<int, 3>{});
                }
            }
        };
        if constexpr (MX) {
            int s0 = s_beg;
            for (; s0 + 3 <= s_last; s0 += 4) unit(s0, std::true_type{});
            if (s0 <= s_last) unit(s0, std::false_type{});
        } else {
            for (int s0 = s_beg; s0 <= s_last; s0 += 4) unit(s0, std::true_type{});
        }
        // no load may still be writing the buffers when the workgroup's LDS is released
        __builtin_amdgcn_s_waitcnt(0x0F70);
    };
    const int neb = __builtin_amdgcn_readfirstlane(min(EB, (n_ent + 31) / 32));
    // the epilogue's per-entry values, loaded now (their latency hides under the main loop)
    float inv_s[EB], inv_m[EB];
    long orow_e[EB];
#pragma unroll
    for (int e = 0; e < EB; e++) {
        const int ent = 32 * e + lr, row = s_row[ent];
        inv_s[e] = a.x.inv_s[row];
        inv_m[e] = Q::A4 ? a.x.inv_m[row] : 1.0f;
        orow_e[e] = a.out_row ? (long)a.out_row[p0 + min(ent, n_ent - 1)] : (long)(p0 + ent);
    }
    auto by_blocks = [&](auto np_c) __attribute__((always_inline)) {
        if constexpr (EB == 2) {
            if (neb == 1) main_loop(np_c, std::integral_constant<int, 1>{});
            else main_loop(np_c, std::integral_constant<int, 2>{});
        } else {
            main_loop(np_c, std::integral_constant<int, EB>{});
        }
    };
    if (b_beg < b_end) {
        if (NPL > 1 && npl > 1) {
            set_boff1();
            by_blocks(std::integral_constant<int, NPL>{});
        } else {
            by_blocks(std::integral_constant<int, 1>{});
        }
    }

    // ---- Q4_K min terms (split 0 only): acc += sum over units of (-dmin m) (x) sums, in
    // slices of 16 units, each slice's loads issued while the previous slice multiplies
    if constexpr (Q::GGML || Q::A4) {
        if (blockIdx.z == 0) {
            const int nu = Q::GGML ? nb * 8 : nb;                 // sub-blocks / super-blocks
            struct slice_ld {
                q16_min_raw w[RB];
                u32x4 s0[EB], s1[EB];
            };
            auto ld = [&](int u0, slice_ld &L) __attribute__((always_inline)) {
#pragma unroll
                for (int rb = 0; rb < RB; rb++)
                    q16_min_ld<SEM>(rb == 0 ? W : W2, nb, wrow, u0 + 8 * kh, L.w[rb], rb == 0 ? sm0 : sm1, a.n_rows);
#pragma unroll
                for (int e = 0; e < EB; e++) {
                    const _Float16 *mp = a.x.m + (long)s_row[32 * e + lr] * a.x.ldm + u0 + 8 * kh;
                    L.s0[e] = gld<u32x4>(mp);
                    L.s1[e] = gld<u32x4>(mp + a.x.mplane);
                }
            };
            slice_ld cur, nxt;
            ld(0, cur);
            for (int u0 = 0; u0 < nu; u0 += 16) {
                if (u0 + 16 < nu) ld(u0 + 16, nxt);
#pragma unroll
                for (int rb = 0; rb < RB; rb++) {
                    f16x8 whi, wlo;
                    q16_min_mk<SEM>(cur.w[rb], nb, u0 + 8 * kh, whi, wlo);
#pragma unroll
                    for (int e = 0; e < EB; e++) {
                        if (e >= neb) continue;
                        const f16x8 s0 = __builtin_bit_cast(f16x8, cur.s0[e]);
                        const f16x8 s1 = __builtin_bit_cast(f16x8, cur.s1[e]);
                        f32x16 t = u0 == 0 ? f32x16{} : T[rb][e];
                        t = __builtin_amdgcn_mfma_f32_32x32x16_f16(whi, s0, t, 0, 0, 0);
                        t = __builtin_amdgcn_mfma_f32_32x32x16_f16(whi, s1, t, 0, 0, 0);
                        if constexpr (Q::GGML) t = __builtin_amdgcn_mfma_f32_32x32x16_f16(wlo, s0, t, 0, 0, 0);
                        T[rb][e] = t;
                    }
                }
                cur = nxt;
            }
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
#pragma unroll
                for (int e = 0; e < EB; e++) {
                    const float im = Q::A4 ? inv_m[e] : 1.0f;
#pragma unroll
                    for (int v = 0; v < 16; v++) acc[rb][e][v] = fmaf(im, T[rb][e][v], acc[rb][e][v]);
                }
        }
    }

    // ---- epilogue
    float *out = a.out;
    long ldo = a.ldo;
    if (a.ksplit > 1) { out = a.part + (long)blockIdx.z * a.n_entries * a.n_rows; ldo = a.n_rows; }
#pragma unroll
    for (int e = 0; e < EB; e++) {
        const int ent = 32 * e + lr;
        if (ent >= n_ent) continue;
        const float is = inv_s[e];
        const float ws = MX ? a.wscale : 1.0f;   // the weights' scale, after the row's (exact powers of two)
        const long orow = orow_e[e];
        float *o = out + orow * ldo;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int n = n0 + 32 * wave + 8 * g + 4 * kh;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float x0 = acc[0][e][4 * g + r] * is;
                if constexpr (MX) x0 *= ws;
                if constexpr (DUAL) {
                    // moe_forward_omp SiLU (QK:2157-2164): clamp to +-80, then silu(g) * u
                    if (a.clamp_silu) x0 = fminf(fmaxf(x0, -80.0f), 80.0f);
                    float x1 = acc[DUAL ? 1 : 0][e][4 * g + r] * is;
                    if constexpr (MX) x1 *= ws;
                    x0 = silu16(x0) * x1;
                }
                v[r] = x0;
            }
            if (n + 3 < a.n_rows && (ldo & 3) == 0) {
                *reinterpret_cast<float4 *>(o + n) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (n + r < a.n_rows) o[n + r] = v[r];
            }
        }
    }
}

// out[e][n] = sum over z < ks of part[z][e][n], in order.
__global__ void k_q16_ksum(const float *__restrict__ part, int ks, long plane, int n_rows, float *__restrict__ out,
                           int ldo)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= plane) return;
    float v = part[i];
    for (int z = 1; z < ks; z++) v += part[z * plane + i];
    const long e = i / n_rows, n = i - e * n_rows;
    out[e * ldo + n] = v;
}

// ---------------------------------------------------------------- activations
// fp32 row -> scaled fp16 planes in the semantic's K order, the row's inverse
// scale, lo_nz, and (Q4_K ggml) the fp16 hi/lo sums of each 32-element
// sub-block.  One workgroup per row.  MXFP4 x Q8_0 first quantises the row to
// Q8_0 and takes quant times block scale (int8 times an fp16 value: exact in
// fp32), the activation mxfp4_row_dot_q8 (QK:629-678) multiplies.
template <int SEM, int TPR>
__global__ __launch_bounds__(256) void k_act16(const float *__restrict__ x, int ldx, int K, int rows, act16 a)
{
    using Q = q16_traits<SEM>;
    // TPR threads per row: the workgroup (256), or a wave (64) for short rows (at most
    // kHeld * 512 positions), four rows per workgroup and no barrier
    static_assert(TPR == 256 || TPR == 64, "a workgroup or a wave per row");
    constexpr int STR = 8 * TPR;   // positions per iteration
    __shared__ float red[4];
    const int tid = threadIdx.x, lt = tid % TPR;
    const int row = blockIdx.x * (256 / TPR) + tid / TPR;
    if (blockIdx.x == gridDim.x - 1) {   // the last workgroup: the zero row
        for (int P = 8 * tid; P < a.ldh; P += 2048) *reinterpret_cast<f16x8 *>(a.zero + P) = f16x8{};
        return;
    }
    if (TPR < 256 && row >= rows) return;
    const float *xr = x + (long)row * ldx;
    const bool vec = ((uintptr_t)xr & 15) == 0;
    const int nb = K / Q::EPS;
    // eight consecutive elements from k (a multiple of 8)
    auto ld8 = [&](int k, float (&v)[8]) __attribute__((always_inline)) {
        if (vec) {
            const float4 p = *reinterpret_cast<const float4 *>(xr + k), q = *reinterpret_cast<const float4 *>(xr + k + 4);
            v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w; v[4] = q.x; v[5] = q.y; v[6] = q.z; v[7] = q.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = xr[k + j];
        }
        if constexpr (Q::Q8IN) {
            // the row's Q8_0 quantisation (k_quantize_q8_0, QK:1406-1455), block k / 32 held by
            // the four threads whose tid differs in bits 1 and 2 (quarters 8 i .. 8 i + 7):
            // amax (without a NaN the plain maximum; with one the reference's vector order,
            // from the block's 32 values), d = amax / 127 (1 if 0), q = rint(clamp(v / d)),
            // and the value the dot multiplies, q * fp16(d) (exact in fp32)
            float m = 0.0f;
            bool nan = false;
#pragma unroll
            for (int j = 0; j < 8; j++) { m = fmaxf(m, fabsf(v[j])); nan |= v[j] != v[j]; }
            m = fmaxf(m, __shfl_xor(m, 2, 64));
            m = fmaxf(m, __shfl_xor(m, 4, 64));
            nan |= __shfl_xor((int)nan, 2, 64) != 0;
            nan |= __shfl_xor((int)nan, 4, 64) != 0;
            if (nan) {
                const float *bp = xr + (k & ~31);
                m = mllm_q8_amax_ref([&](int i) { return fabsf(bp[i]); });
            }
            float d = m / 127.0f;
            if (d == 0.0f) d = 1.0f;
            const float id = 1.0f / d;
            const float d8 = (float)(_Float16)d;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                float p = v[j] * id;
                p = (p > -127.0f) ? p : -127.0f;
                p = (p < 127.0f) ? p : 127.0f;
                v[j] = (float)(int)rintf(p) * d8;
            }
        }
    };
    // thread t of the row takes positions P = 8 t + STR it (it < nit): eight positions
    // hold one aligned group of 8 elements, in the order q16_elem gives
    // (base + q16_elem(j)).  The first kHeld groups stay in registers between the passes.
    constexpr int kHeld = 4;
    const int npos = nb * Q::PPS;   // positions in use (the row stride ldh is padded past them)
    const int nit = (npos - 8 * lt + STR - 1) / STR;
    auto gbase = [&](int P) __attribute__((always_inline)) { return (P / Q::PPS) * Q::EPS + q16_elem<SEM>(P % Q::PPS); };
    float g[kHeld][8];
    // largest finite |x| (a NaN fails the comparison and is skipped)
    float m = 0.0f;
    auto mx = [&](const float (&v)[8]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (fabsf(v[j]) < INFINITY) m = fmaxf(m, fabsf(v[j]));
    };
#pragma unroll
    for (int it = 0; it < kHeld; it++)
        if (it < nit) {
            ld8(gbase(8 * lt + STR * it), g[it]);
            mx(g[it]);
        }
    for (int it = kHeld; it < nit; it++) {
        float v[8];
        ld8(gbase(8 * lt + STR * it), v);
        mx(v);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if constexpr (TPR == 256) {
        if ((tid & 63) == 0) red[tid >> 6] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    }
    // s = 2^(9 - e) puts the largest element in [2^8, 2^9) (m = f 2^e, f in [0.5, 1))
    int e = 0;
    if (m > 0.0f) (void)frexpf(m, &e);
    e = max(e, -117);
    const float s = m > 0.0f ? ldexpf(1.0f, 9 - e) : 1.0f;
    const float inv = m > 0.0f ? ldexpf(1.0f, e - 9) : 1.0f;
    int nz = 0;
    _Float16 *h0 = a.h + (long)row * a.ldh, *h1 = h0 + a.hplane;
    // rows that fit the held groups store their second plane only when it holds a
    // non-zero element (the GEMM reads the zero row for the others); longer rows store it
    const bool whole = npos <= kHeld * STR;
    f16x8 held1[kHeld];
    auto emit = [&](int P, const float (&gv)[8], f16x8 &v1) __attribute__((always_inline)) {
        const int sb = P / Q::PPS, pw = P % Q::PPS;
        f16x8 v0;
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float v = gv[q16_elem<SEM>(j)] * s;
            _Float16 hi, lo;
            split16(v, hi, lo);
            v0[j] = hi;
            v1[j] = lo;
            nz |= (float)lo != 0.0f;
            if constexpr (Q::GGML) part += gv[j] * s;
        }
        *reinterpret_cast<f16x8 *>(h0 + P) = v0;
        if (!whole) *reinterpret_cast<f16x8 *>(h1 + P) = v1;
        if constexpr (Q::GGML) {
            // sub-block 8 sb + 2 (pw / 64) + (pw / 32) % 2: the four groups of threads 4q .. 4q+3
            part += __shfl_xor(part, 1, 64);
            part += __shfl_xor(part, 2, 64);
            if ((tid & 3) == 0) {
                const int j = 8 * sb + pw / 32;
                _Float16 hi, lo;
                split16(part, hi, lo);
                a.m[(long)row * a.ldm + j] = hi;
                a.m[a.mplane + (long)row * a.ldm + j] = lo;
            }
        }
    };
#pragma unroll
    for (int it = 0; it < kHeld; it++)
        if (it < nit) emit(8 * lt + STR * it, g[it], held1[it]);
    for (int it = kHeld; it < nit; it++) {
        float v[8];
        f16x8 v1;
        ld8(gbase(8 * lt + STR * it), v);
        emit(8 * lt + STR * it, v, v1);
    }
    if constexpr (Q::GGML) {
        for (int j = nb * 8 + lt; j < a.ldm; j += TPR) {
            a.m[(long)row * a.ldm + j] = (_Float16)0.0f;
            a.m[a.mplane + (long)row * a.ldm + j] = (_Float16)0.0f;
        }
    }
    if constexpr (TPR == 256) nz = __syncthreads_or(nz);
    else nz = __any(nz);
    if (whole && nz) {
#pragma unroll
        for (int it = 0; it < kHeld; it++)
            if (it < nit) *reinterpret_cast<f16x8 *>(h1 + 8 * lt + STR * it) = held1[it];
    }
    if (lt == 0) {
        a.lo_nz[row] = nz;
        a.inv_s[row] = inv;
    }
}

// Q4_K x Q8_0 (dot_q4_k_q8_0): the Q8_0 quants of elements 32 j + k, k < 16,
// as fp16 in the K order; u_b = sum over the 8 sub-blocks of super-block b of
// the Q8_0 min-term sums (QK:1714-1732) as scaled fp16 hi/lo.
__global__ __launch_bounds__(256) void k_act16_q8(mllm_xq xq, int K, act16 a)
{
    __shared__ float red[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const int nb = K / 256, nbk = K / 32;
    const int8_t *q = xq.q + (long)row * nbk * 32;
    _Float16 *h0 = a.h + (long)row * a.ldh;
    for (int P = 8 * tid; P < nb * 128; P += 2048) {
        f16x8 v0;
        const int sb = P / 128, pw = P % 128;
        const uint2 w = *reinterpret_cast<const uint2 *>(q + sb * 256 + q16_elem<SEM_Q4_K_Q8>(pw));
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int t = q16_elem<SEM_Q4_K_Q8>(j);
            v0[j] = (_Float16)(float)(int8_t)(((t < 4 ? w.x : w.y) >> (8 * (t & 3))) & 0xFF);
        }
        *reinterpret_cast<f16x8 *>(h0 + P) = v0;
    }
    // super-block sums and their scale: largest |u| into [2^10, 2^11)
    float u = 0.0f;
    if (tid < nb) {
        const float *s4 = xq.s4 + (long)row * nbk + 8 * tid;
#pragma unroll
        for (int j = 0; j < 8; j++) u += s4[j];
    }
    float m = tid < nb && fabsf(u) < INFINITY ? fabsf(u) : 0.0f;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (m > 0.0f) (void)frexpf(m, &e);
    e = max(e, -115);
    const float s = m > 0.0f ? ldexpf(1.0f, 11 - e) : 1.0f;
    _Float16 *m0 = a.m + (long)row * a.ldm, *m1 = m0 + a.mplane;
    for (int j = tid; j < a.ldm; j += 256) {
        _Float16 hi = (_Float16)0.0f, lo = (_Float16)0.0f;
        if (j < nb) split16((j == tid ? u : 0.0f) * s, hi, lo);
        m0[j] = hi;
        m1[j] = lo;
    }
    if (tid == 0) {
        a.lo_nz[row] = 0;
        a.inv_s[row] = 1.0f;
        a.inv_m[row] = m > 0.0f ? ldexpf(1.0f, e - 11) : 1.0f;
    }
}

size_t al256(size_t n) { return (n + 255) / 256 * 256; }

// Step-major copy of one metadata plane: for matrix m = blockIdx.y, the record of R bytes
// at src = tab[m].p[plane] + (row * nb + b) * R goes to dst + m * stride + off + (b * n_rows + row) * R.
template <int R>
__global__ void k_smeta(const mllm_packed *__restrict__ tab, int plane, int n_rows, int nb, uint8_t *__restrict__ dst,
                        long stride, long off)
{
    const uint8_t *src = tab[blockIdx.y].p[plane];
    uint8_t *d = dst + (long)blockIdx.y * stride + off;
    const long n = (long)n_rows * nb;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
        const long b = i / n_rows, row = i - b * n_rows;
        if constexpr (R == 16) *reinterpret_cast<uint4 *>(d + i * 16) = *reinterpret_cast<const uint4 *>(src + (row * nb + b) * 16);
        else *reinterpret_cast<uint16_t *>(d + i * 2) = *reinterpret_cast<const uint16_t *>(src + (row * nb + b) * 2);
    }
}

// range[0] = min over non-zero E, range[1] = max E of the matrices' E8M0 bytes.
__global__ void k_mx_erange(const mllm_packed *__restrict__ tab, long nblk, int *__restrict__ range)
{
    const uint8_t *e = tab[blockIdx.y].p[1];
    int lo = 255, hi = 0;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < nblk; i += (long)gridDim.x * blockDim.x) {
        const int v = e[i];
        if (v) lo = min(lo, v);
        hi = max(hi, v);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        lo = min(lo, __shfl_xor(lo, o, 64));
        hi = max(hi, __shfl_xor(hi, o, 64));
    }
    if ((threadIdx.x & 63) == 0) {
        if (lo < 255) atomicMin(range, lo);
        if (hi > 0) atomicMax(range + 1, hi);
    }
}

// Grouped launches whose activation planes hold at least this many bytes are walked row
// block fastest: an XCD's L2 (4 MB) then keeps the few activation tiles its workgroups
// read at once, where entry tile fastest would read every tile once per row block.
// Measured on the MoE down projections: GPT-OSS T = 1280 (62 MB) 256 -> 234 us, Qwen3
// T = 1280 (37 MB) 158 -> 146 us; GPT-OSS T = 256 (12 MB) 93 -> 104 us, so smaller
// planes keep entry tile fastest.
constexpr long kRowsFastBytes = 24l << 20;

template <int SEM, bool DUAL, int EB, bool SM>
hipError_t launch16(const q16_args &a, int max_tiles, hipStream_t st)
{
    constexpr int TM = 32 * EB;
    const int ks = (a.ksplit > 1 && !DUAL && !a.tile_expert && !a.out_row) ? a.ksplit : 1;
    constexpr int TN = 32 * q16_wpg<SEM, DUAL, EB>();
    dim3 grid((a.n_rows + TN - 1) / TN, a.tile_expert ? max_tiles : (a.n_entries + TM - 1) / TM, ks);
    if (grid.y == 0) return hipSuccess;
    q16_args b = a;
    b.ksplit = ks;
    b.rows_fast = a.tile_expert && (long)a.n_entries * a.x.ldh * 2 * q16_traits<SEM>::NPL >= kRowsFastBytes;
    hipLaunchKernelGGL((k_q16<SEM, DUAL, EB, SM>), grid, dim3(2 * TN), 0, st, b);
    if (ks > 1) {
        const long plane = (long)a.n_entries * a.n_rows;
        hipLaunchKernelGGL(k_q16_ksum, dim3((unsigned)((plane + 255) / 256)), dim3(256), 0, st, a.part, ks, plane,
                           a.n_rows, a.out, a.ldo);
    }
    return hipGetLastError();
}

} // namespace

bool mllm_q16_supported(int sem)
{
    return sem == SEM_Q4_K_GGML || sem == SEM_Q4_K_Q8 || sem == SEM_Q6_K_SEQ || sem == SEM_Q6_K_LOWNIB;
}

bool mllm_q16_mx(int sem) { return sem == SEM_MXFP4 || sem == SEM_MXFP4_Q8; }

hipError_t mllm_launch_mx_erange(const mllm_packed *tab_dev, int n_mats, int n_rows, int n_cols, int *range,
                                 hipStream_t st)
{
    const long nblk = (long)n_rows * (n_cols / 32);
    if (n_mats <= 0 || nblk <= 0) return hipSuccess;
    const unsigned gx = (unsigned)std::min<long>((nblk + 255) / 256, 64);
    hipLaunchKernelGGL(k_mx_erange, dim3(gx, (unsigned)n_mats), dim3(256), 0, st, tab_dev, nblk, range);
    return hipGetLastError();
}

long mllm_q16_smeta_bytes(int sem, int n_rows, int n_cols, long *doff)
{
    long a = 0, d = 0;
    if (mllm_q16_mx(sem)) {
        a = (long)n_rows * (n_cols / 64) * 2;
    } else if (mllm_q16_supported(sem)) {
        a = (long)n_rows * (n_cols / 256) * 16;
        if (sem == SEM_Q6_K_SEQ || sem == SEM_Q6_K_LOWNIB) d = (long)n_rows * (n_cols / 256) * 2;
    }
    const long ao = (long)al256((size_t)a);
    if (doff) *doff = ao;
    return ao + (long)al256((size_t)d);
}

hipError_t mllm_launch_q16_smeta(int sem, const mllm_packed *tab_dev, int n_mats, int n_rows, int n_cols, uint8_t *dst,
                                 long stride, hipStream_t st)
{
    long doff = 0;
    if (n_mats <= 0 || mllm_q16_smeta_bytes(sem, n_rows, n_cols, &doff) <= 0) return hipErrorInvalidValue;
    const bool mx = mllm_q16_mx(sem);
    const int nb = mx ? n_cols / 64 : n_cols / 256;
    const unsigned gx = (unsigned)std::min<long>(((long)n_rows * nb + 255) / 256, 256);
    const dim3 g(gx, (unsigned)n_mats);
    if (mx) {
        hipLaunchKernelGGL(k_smeta<2>, g, dim3(256), 0, st, tab_dev, 1, n_rows, nb, dst, stride, 0l);
    } else if (sem == SEM_Q6_K_SEQ || sem == SEM_Q6_K_LOWNIB) {
        hipLaunchKernelGGL(k_smeta<16>, g, dim3(256), 0, st, tab_dev, 2, n_rows, nb, dst, stride, 0l);
        hipLaunchKernelGGL(k_smeta<2>, g, dim3(256), 0, st, tab_dev, 3, n_rows, nb, dst, stride, doff);
    } else {
        hipLaunchKernelGGL(k_smeta<16>, g, dim3(256), 0, st, tab_dev, 1, n_rows, nb, dst, stride, 0l);
    }
    return hipGetLastError();
}

// Largest exponent to E' = 5 (then 1032 s <= 33024 and 8 s <= 256 fit fp16), smallest
// non-zero to E' >= -20 (then s / 16 >= 2^-24, the least fp16 subnormal); emax <= 177
// (2^50 scales: the Q8_0 form's scale clamp never binds, as in the scale scan) and
// emax >= 6 (wscale a normal float).  No non-zero exponent: all weights zero.
bool mllm_q16_mx_shift(int emin, int emax, int *eoff, float *wscale)
{
    if (emax <= 0) { *eoff = 0; *wscale = 1.0f; return true; }
    if (emax - emin > 25 || emax < 6 || emax > 177) return false;
    *eoff = 5 - emax;
    *wscale = std::ldexp(1.0f, -127 - *eoff);
    return true;
}

// Activation layout: h [planes][rows][ldh] | m [2][rows][ldm] | inv_s | inv_m | lo_nz.
static void act16_dims(int sem, int K, int &nplanes, int &ldh, int &ldm)
{
    const int nb = K / 256;
    const bool a4 = sem == SEM_Q4_K_Q8;
    nplanes = a4 ? 1 : 2;
    // the row stride is padded by 256 bytes: a power-of-two stride would put the same
    // 128-byte column of every row on one L2 channel
    ldh = (mllm_q16_mx(sem) ? K : nb * (a4 ? 128 : 256)) + 128;
    ldm = sem == SEM_Q4_K_GGML ? (nb * 8 + 15) / 16 * 16 : a4 ? (nb + 15) / 16 * 16 : 0;
}

size_t mllm_act16_bytes(int sem, long rows, int K)
{
    int np, ldh, ldm;
    act16_dims(sem, K, np, ldh, ldm);
    return al256((size_t)(np * rows + 1) * ldh * 2) + al256((size_t)2 * rows * ldm * 2) + 3 * al256((size_t)rows * 4);
}

act16 mllm_act16_carve(int sem, void *ws, long rows, int K)
{
    int np, ldh, ldm;
    act16_dims(sem, K, np, ldh, ldm);
    uint8_t *p = (uint8_t *)ws;
    act16 a{};
    a.h = (_Float16 *)p;
    a.hplane = (long)rows * ldh;
    a.ldh = ldh;
    a.zero = a.h + (long)np * rows * ldh;
    p += al256((size_t)(np * rows + 1) * ldh * 2);
    a.m = ldm ? (_Float16 *)p : nullptr;
    a.mplane = (long)rows * ldm;
    a.ldm = ldm;
    p += al256((size_t)2 * rows * ldm * 2);
    a.inv_s = (float *)p;
    p += al256((size_t)rows * 4);
    a.inv_m = (float *)p;
    p += al256((size_t)rows * 4);
    a.lo_nz = (int *)p;
    return a;
}

hipError_t mllm_launch_act16(int sem, const float *x, int ldx, const mllm_xq *xq, int rows, int K, const act16 &act,
                             hipStream_t st)
{
    if (rows <= 0) return hipSuccess;
    const int unit = mllm_q16_mx(sem) ? 64 : 256;
    if (K < unit || K % unit || ((uintptr_t)act.h & 15)) return hipErrorInvalidValue;
    // a wave per row for short rows (Qwen3's 768-element h: 19.4 -> 15.3 us at 10240 rows;
    // at 2048 the workgroup per row is faster, 7.8 against 8.5 us at 1280 rows)
    const bool wave = K <= 1024;
    auto go = [&](auto sem_c) {
        constexpr int S = decltype(sem_c)::value;
        if (wave)
            hipLaunchKernelGGL((k_act16<S, 64>), dim3((rows + 3) / 4 + 1), dim3(256), 0, st, x, ldx, K, rows, act);
        else
            hipLaunchKernelGGL((k_act16<S, 256>), dim3(rows + 1), dim3(256), 0, st, x, ldx, K, rows, act);
    };
    switch (sem) {
    case SEM_Q4_K_GGML: go(std::integral_constant<int, SEM_Q4_K_GGML>{}); break;
    case SEM_Q6_K_SEQ: go(std::integral_constant<int, SEM_Q6_K_SEQ>{}); break;
    case SEM_Q6_K_LOWNIB: go(std::integral_constant<int, SEM_Q6_K_LOWNIB>{}); break;
    case SEM_MXFP4: go(std::integral_constant<int, SEM_MXFP4>{}); break;
    case SEM_MXFP4_Q8: go(std::integral_constant<int, SEM_MXFP4_Q8>{}); break;
    case SEM_Q4_K_Q8:
        if (!xq || K / 256 > 256) return hipErrorInvalidValue;
        hipLaunchKernelGGL(k_act16_q8, dim3(rows), dim3(256), 0, st, *xq, K, act);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Dense launches take 128-entry tiles once there are 256 entries, else 64;
// grouped launches the bucketing's 64-entry tiles.
int mllm_q16_tile_entries(bool grouped, int n_entries) { return !grouped && n_entries >= 256 ? 128 : 64; }

// Split along K (whole super-blocks) while a dense launch has fewer than two
// tiles per CU (512), each split keeping at least 4 super-blocks.
int mllm_q16_ksplit(int sem, int n_rows, int n_cols, int n_entries)
{
    if (!mllm_q16_supported(sem) || n_entries <= 0) return 1;   // MXFP4: grouped launches, no split
    const int tm = mllm_q16_tile_entries(false, n_entries);
    const long tiles = (long)((n_rows + 127) / 128) * ((n_entries + tm - 1) / tm);
    if (tiles >= 384) return 1;
    const int nb = n_cols / 256;
    int ks = (int)(512 / tiles);
    ks = std::min(ks, std::max(1, nb / 4));
    return std::max(1, std::min(ks, 8));
}

hipError_t mllm_launch_q16(int sem, bool dual, const q16_args &a, int max_tiles, hipStream_t st)
{
    const int unit = mllm_q16_mx(sem) ? 64 : 256;
    if (a.n_cols < unit || a.n_cols % unit) return hipErrorInvalidValue;
    if (mllm_q16_mx(sem) && a.ksplit > 1) return hipErrorInvalidValue;
    const bool grouped = a.tile_expert != nullptr;
    const int tm = mllm_q16_tile_entries(grouped, a.n_entries);
    // grouped launches with step-major metadata take the SM forms (not gate and up in Q6_K,
    // whose registers the SM form would spill)
#define Q16(S)                                                                                   \
    if (sem == S) {                                                                              \
        constexpr bool q6 = S == SEM_Q6_K_SEQ || S == SEM_Q6_K_LOWNIB;                           \
        if (grouped && a.sm && !dual) return launch16<S, false, 2, true>(a, max_tiles, st);      \
        if constexpr (!q6) if (grouped && a.sm) return launch16<S, true, 2, true>(a, max_tiles, st); \
        if (dual) return launch16<S, true, 2, false>(a, max_tiles, st);                          \
        return tm == 128 ? launch16<S, false, 4, false>(a, max_tiles, st) : launch16<S, false, 2, false>(a, max_tiles, st); \
    }
    Q16(SEM_Q4_K_GGML)
    Q16(SEM_Q4_K_Q8)
    Q16(SEM_Q6_K_SEQ)
    Q16(SEM_Q6_K_LOWNIB)
#undef Q16
    // MXFP4: the grouped expert GEMMs (gate + up fused against fp32 x, down against Q8_0 h)
    if (sem == SEM_MXFP4 && dual && grouped && a.sm) return launch16<SEM_MXFP4, true, 2, true>(a, max_tiles, st);
    if (sem == SEM_MXFP4_Q8 && !dual && grouped && a.sm) return launch16<SEM_MXFP4_Q8, false, 2, true>(a, max_tiles, st);
    return hipErrorInvalidValue;
}
