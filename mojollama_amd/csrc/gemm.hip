// gemm.hip — quantised-weight GEMM on CDNA4 MFMA: prefill matmuls and the
// grouped expert GEMMs of the batched MoE layer.
//
// out[e][n] = sum_k w[n][k] * b[e][k] for a tile of "entries" e (tokens, or
// token-expert pairs of one expert bucket) against the tile's weight rows n.
//
// Precision.  Each weight tile is dequantised once into LDS and split into
// NA bf16 planes (w = w0 + w1 + w2, each plane the bf16 rounding of what the
// previous ones leave; three planes carry all 24 bits of a float); the
// activations into NB planes.  v_mfma_f32_16x16x32_bf16 accumulates the
// products wi*bj in fp32.  Operands exact in one bf16 use one plane: MXFP4
// weights (int4 times a power of two) and Q8_0 quants; their partners then
// get three, which makes those products exact to fp32.  Everything else uses
// two planes each and the three leading products (normalised error ~5e-6).
// Q4_K against Q8_0 quants runs on v_mfma_f32_16x16x32_f16 instead: the
// sub-block scale times the nibble and the quants are small integers, exact
// in fp16, so each MFMA returns the step's integer dot exactly and the
// super-block scale d is applied to it per row.
//
// Tiling.  Workgroup = 4 wave64s, tile TN (128, or 64 when gate and up share
// it) rows x 64 entries, K staged KE columns at a time; a wave owns 32 rows
// x (64 or 32) entries = 2 x JT MFMA 16x16 outputs.  LDS rows are padded by
// 16 bytes so the 16 lanes reading one k-slice hit distinct banks.  Global
// loads run two K-steps ahead of the MFMAs (register double buffer).
#include <algorithm>
#include "decode.h"
#include <type_traits>
#include "gemm.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int SEM, int XM> struct gemm_cfg {
    // Q4_K against Q8_0 quants (dot_q4_k_q8_0): the integer part sc * nibble
    // (<= 945) and the quants are exact in fp16, so one fp16 MFMA per tile
    // gives the sub-blocks' integer dot exactly; d is applied per step.
    static constexpr bool A4 = (SEM == SEM_Q4_K_Q8);
    static constexpr bool WEXACT = (SEM == SEM_MXFP4 || SEM == SEM_MXFP4_CLAMP || SEM == SEM_MXFP4_Q8);
    static constexpr int NA = (WEXACT || A4) ? 1 : 2;
    // Q8_0 quants are exact in one bf16 plane; XM_Q8D applies their block scale
    // after each 32-column MFMA (one Q8_0 block per k-slice).
    static constexpr int NB = (XM == XM_Q8 || XM == XM_Q8D) ? 1 : (XM == XM_PLANES && !WEXACT) ? 2 : 3;
    // K columns per step: A4 keeps only the 32 columns its dot reads of each 64
    static constexpr int KS = 64;
    static constexpr int KE = A4 ? 32 : 64;
    // LDS rows: 64-column bf16 tiles unpadded and swizzled (tile_off), except the
    // exact-weight planes (their tiles already fit three workgroups per CU and the
    // swizzle's addressing would spill there); others padded
    static constexpr bool SWZ = (KE == 64) && !WEXACT;
    static constexpr int LDA = SWZ ? 64 : KE + 8;
    // products w_i * b_j taken: i + j <= MAXT.  Two planes each: the three leading
    // terms (the dropped w1*b1 is ~2^-16 of the product, below the two-plane
    // truncation itself).  One exact plane against three, or three against
    // exact quants: all three (one exact plane against exact quants: the one).
    static constexpr int MAXT = (NA == 2 && NB == 2) ? 1 : 2;
};

// Wide tiles: dense-weight tiles, and fused tiles whose weights take one plane
// (measured on the MoE layers at T = 1280: GPT-OSS MXFP4 gate+up 1272 -> 1217
// us per layer decoded, 1098 -> 964 us over bf16 copies; Qwen3's Q4_K x Q8_0
// unchanged).
// Tile kinds: 0 the default; 1 wide (above); 2 narrow: 64 rows of two-plane
// weights against 64-entry tiles (the grouped expert GEMMs), 2 x 2 waves
// (Qwen3's Q6_K down at T = 1280: 745 -> 664 us per layer; the 128-entry
// dense prefill tiles keep 128 rows, measured faster there).
template <int SEM, int XM, bool DUAL, bool DW, int TM> constexpr int tile_kind()
{
    if (!DUAL && TM == 64 && gemm_cfg<SEM, XM>::NA == 2) return 2;
    return (DW || (DUAL && gemm_cfg<SEM, XM>::NA == 1)) ? 1 : 0;
}

// Tile of TN weight rows x TM_ entries; 4 waves in a WR x WE grid, each owning
// IT x JT MFMA 16x16 outputs.
// WIDE: 128 weight rows also for the fused gate+up tiles (each matrix's tile
// one bf16 plane: its LDS still admits two workgroups per CU), waves 2 x 2.
template <bool DUAL, int TM_, int KIND> struct tile_cfg {
    static constexpr int TN = (KIND == 2 || (DUAL && KIND == 0)) ? 64 : 128;
    static constexpr int WR = (TN == 128 && TM_ == 64 && KIND == 0) ? 4 : 2;
    static constexpr int WE = 4 / WR;
    static constexpr int IT = TN / WR / 16;
    static constexpr int JT = TM_ / WE / 16;
};

// Element offset of (row, col) in an LDS tile; col is a multiple of 8 (every
// access moves 16-byte pieces).  Taking the LDS to serve a 16-byte access 16
// lanes at a time over 64 banks (256 bytes) -- the model that fits the bank
// conflict counters of padded rows -- SWZ tiles keep 128-byte rows and store
// piece p of row r at piece p ^ ((r >> 1) & 7): the MFMA operand reads (16 rows,
// one piece each), the weight stores (8 rows x two 32-column halves) and the
// activation stores (2 rows x 8 pieces) each touch 16 distinct 16-byte bank
// groups, and the unpadded tile is small enough for a third workgroup per CU.
template <bool SWZ, int LDA>
MLLM_DEV int tile_off(int row, int col)
{
    if constexpr (SWZ) return row * 64 + ((((col >> 3) ^ (row >> 1)) & 7) << 3);
    else return row * LDA + col;
}

// 16 values exact in fp16 (integers below 2048) as fp16, in bf16-typed storage.
MLLM_DEV void put16_f16(__bf16 *dst, const float (&v)[16])
{
    f16x8 a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) { a[i] = (_Float16)v[i]; b[i] = (_Float16)v[8 + i]; }
    *reinterpret_cast<f16x8 *>(dst) = a;
    *reinterpret_cast<f16x8 *>(dst + 8) = b;
}

// 16 values as bf16 at columns col .. col+15 of row `row`.
template <bool SWZ, int LDA>
MLLM_DEV void put16(__bf16 *base, int row, int col, const float (&v)[16])
{
    bf16x8 a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) { a[i] = (__bf16)v[i]; b[i] = (__bf16)v[8 + i]; }
    *reinterpret_cast<bf16x8 *>(base + tile_off<SWZ, LDA>(row, col)) = a;
    *reinterpret_cast<bf16x8 *>(base + tile_off<SWZ, LDA>(row, col + 8)) = b;
}

// Store 16 values as NP bf16 planes (plane p at base + p*pstride), row `row`, columns col ..
template <int NP, bool SWZ, int LDA>
MLLM_DEV void put16_planes(__bf16 *base, int pstride, int row, int col, const float (&v)[16])
{
    float r[16];
#pragma unroll
    for (int i = 0; i < 16; i++) r[i] = v[i];
#pragma unroll
    for (int p = 0; p < NP; p++) {
        float t[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            t[i] = (float)(__bf16)r[i];
            r[i] -= t[i];
        }
        put16<SWZ, LDA>(base + p * pstride, row, col, t);
    }
}

MLLM_DEV void zero16(float (&v)[16])
{
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = 0.0f;
}

// Dequantise one 32-weight chunk (fp32-weight semantics) into its two runs of 16.
template <int SEM>
MLLM_DEV void chunk_weights(const raw_chunk &raw, int c, float (&w0)[16], float (&w1)[16], int &x0, int &x1)
{
    chunk_codes k;
    codes<SEM>(raw, c, k);
    constexpr float bias = (float)sem_traits<SEM>::kBias;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
            w0[code_pos<SEM>(j, t)] = fmaf(k.s0, ubyte_f(k.U[j], t) - bias, k.o0);
            w1[code_pos<SEM>(j, t)] = fmaf(k.s1, ubyte_f(k.U[4 + j], t) - bias, k.o1);
        }
    x0 = k.x0;
    x1 = k.x1;
}

// ---------------------------------------------------------------- staging
//
// A K-step's operands are fetched from global memory into registers two
// steps ahead of their use (fetch_*), then decoded, split into bf16 planes and
// stored to LDS (put_*).  Every fetch is issued unconditionally -- indices past
// the matrix are clamped to valid ones and put_* writes zeros for them -- so
// the number of loads in flight is the same on every path and the compiler's
// waits cover only the older step.

// Weight tasks per row and step: Q4_K_Q8 the two 16-weight halves of one chunk; MXFP4_Q8 two 32-blocks;
// otherwise the two chunks covering the 64 columns, or four for the ggml
// Q6_K orders whose chunks put their two runs 64 columns apart.
template <int SEM, int XM> struct wtask {
    static constexpr bool SPLIT = (SEM == SEM_Q6_K_GGML || SEM == SEM_Q6_K_LOWNIB);
    static constexpr int NT = gemm_cfg<SEM, XM>::A4 ? 2 : (SEM == SEM_MXFP4_Q8) ? 2 : SPLIT ? 4 : 2;
};

template <int SEM, int XM, int TN_> struct wraw {
    static constexpr int WT = (TN_ * wtask<SEM, XM>::NT + 255) / 256;
    raw_chunk r[WT];
};

// Row, chunk index and validity of task t (t may exceed the task count: clamped, invalid).
template <int SEM, int XM, int TN_>
MLLM_DEV void wtask_at(int t, int n_rows, int nb, int n0, int k0, int &rr, int &sub, int &row, int &c, bool &valid)
{
    using C = gemm_cfg<SEM, XM>;
    constexpr int NT = wtask<SEM, XM>::NT, NTOT = TN_ * NT;
    valid = t < NTOT;
    t = min(t, NTOT - 1);
    rr = t / NT;
    sub = t % NT;
    row = min(n0 + rr, n_rows - 1);
    if constexpr (C::A4) {
        c = k0 / 64;
    } else if constexpr (SEM == SEM_MXFP4_Q8) {
        c = k0 / 32 + sub;
        if (c >= nb) { valid = false; c = nb - 1; }
    } else {
        constexpr int CPB = sem_traits<SEM>::kChunksPerBlock, BE = sem_traits<SEM>::kBlockElems;
        const int q = (k0 % 256) / 64;
        if constexpr (BE == 256) {
            c = (k0 / 256) * CPB + (wtask<SEM, XM>::SPLIT ? 4 * (q >> 1) + sub : 2 * q + sub);
        } else {
            c = k0 / 32 + sub;
            if (c >= nb) { valid = false; c = nb - 1; }   // past the last block of an odd block count
        }
    }
}

// Task numbering starts at thread `rot` (mod 256): the two matrices of a fused
// gate+up tile start half a workgroup apart, so their decode lands on
// different waves when each has at most 128 tasks.
template <int SEM, int XM, int TN_>
MLLM_DEV void fetch_w(const mllm_packed &W, int n_rows, int nb, int n0, int k0, wraw<SEM, XM, TN_> &wr, int rot)
{
    const int tt = (threadIdx.x + rot) & 255;
#pragma unroll
    for (int i = 0; i < wraw<SEM, XM, TN_>::WT; i++) {
        int rr, sub, row, c;
        bool valid;
        wtask_at<SEM, XM, TN_>(tt + 256 * i, n_rows, nb, n0, k0, rr, sub, row, c, valid);
        if constexpr (mllm_sem_uses_q8(SEM)) q8_fetch<SEM>(W, nb, row, c, wr.r[i]);
        else fetch<SEM>(W, nb, row, c, wr.r[i]);
    }
}

// Decode the fetched weight tasks into LDS planes (plane p at A + p*TN_*LDA);
// for Q4_K_Q8 also each row's dmin.
template <int SEM, int XM, int TN_>
MLLM_DEV void put_w(const wraw<SEM, XM, TN_> &wr, int n_rows, int nb, int n0, int k0, __bf16 *A, float *dmin_l,
                    int rot)
{
    using C = gemm_cfg<SEM, XM>;
    constexpr int LDA = C::LDA, NA = C::NA, PS = TN_ * C::LDA;
    const int tt = (threadIdx.x + rot) & 255;
#pragma unroll
    for (int i = 0; i < wraw<SEM, XM, TN_>::WT; i++) {
        int rr, sub, row, c;
        bool valid;
        wtask_at<SEM, XM, TN_>(tt + 256 * i, n_rows, nb, n0, k0, rr, sub, row, c, valid);
        if (tt + 256 * i >= TN_ * wtask<SEM, XM>::NT) continue;   // clamped duplicate
        const raw_chunk &r = wr.r[i];
        if constexpr (C::A4) {
            // dot_q4_k_q8_0 (QK:1647-1735): the integer term reads k < 16 of each 32-element
            // sub-block; group g of a super-block holds sub-blocks 2g (low nibbles) and 2g+1
            // (high nibbles).  Step columns: 0..15 = sub-block 2g, 16..31 = 2g+1, w = d*sc_j*nib.
            // this task: half sub = 0 (sub-block 2g, low nibbles) or 1 (2g+1, high nibbles);
            // stored: sc_j * nibble (fp16, exact); per row dmin at dmin_l[rr], d at dmin_l[TN_ + rr]
            const int g = c & 3;
            int s1, m1, s2, m2;
            kq_pairs(r.m, 2 * g, s1, m1, s2, m2);
            const float sc = (float)(sub ? s2 : s1);
            const uint32_t Aw[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
            float v[16];
#pragma unroll
            for (int e = 0; e < 16; e++) v[e] = sc * (float)((Aw[e >> 2] >> (8 * (e & 3) + 4 * sub)) & 15);
            put16_f16(A + rr * LDA + 16 * sub, v);
            if (dmin_l && sub == 0) {
                dmin_l[rr] = h2f(r.m.x >> 16);
                dmin_l[TN_ + rr] = h2f(r.m.x & 0xFFFF);
            }
        } else if constexpr (SEM == SEM_MXFP4_Q8) {
            // mxfp4_row_dot_q8 (QK:629-678) with the token's Q8 scale moved to the activation
            // side: w = sext4(n) * 2^(E-127), exact in bf16.
            float v0[16], v1[16];
            if (valid) {
                const float sc = e8m0f(r.d);
                const uint32_t Aw[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
                for (int e = 0; e < 32; e++) {
                    const int n = (Aw[e >> 3] >> (4 * (e & 7))) & 15;
                    const float w = (float)(n >= 8 ? n - 16 : n) * sc;
                    if (e < 16) v0[e] = w; else v1[e - 16] = w;
                }
            } else {
                zero16(v0); zero16(v1);
            }
            put16_planes<NA, C::SWZ, LDA>(A, PS, rr, 32 * sub, v0);
            put16_planes<NA, C::SWZ, LDA>(A, PS, rr, 32 * sub + 16, v1);
        } else {
            constexpr bool SPLIT = wtask<SEM, XM>::SPLIT;
            if (!valid) {   // past the last block of an odd block count: zero columns
                float z[16];
                zero16(z);
                put16_planes<NA, C::SWZ, LDA>(A, PS, rr, 32 * sub, z);
                put16_planes<NA, C::SWZ, LDA>(A, PS, rr, 32 * sub + 16, z);
                continue;
            }
            const int q = (k0 % 256) / 64;
            float w0[16], w1[16];
            int x0, x1;
            chunk_weights<SEM>(r, c, w0, w1, x0, x1);
            if (!SPLIT || (q & 1) == 0) put16_planes<NA, C::SWZ, LDA>(A, PS, rr, x0 - k0, w0);
            if (!SPLIT || (q & 1) == 1) put16_planes<NA, C::SWZ, LDA>(A, PS, rr, x1 - k0, w1);
        }
    }
}

// Dense bf16 weights (dense_ld > 0): a step is TN_ rows x 64 columns, eight
// 16-byte pieces per row, copied into the tile as they are (rows past the
// matrix clamped to its last row, whose outputs are never stored).
template <int TN_, int NA> struct wdense {
    static constexpr int NP = TN_ * 8 / 256;
    uint4 p[NA][NP];
};

// Plane p of the copy starts p * plane elements after W.p[0].
template <int TN_, int NA>
MLLM_DEV void fetch_wd(const mllm_packed &W, int n_rows, int ldw, long plane, int n0, int k0, wdense<TN_, NA> &wd)
{
    const __bf16 *base = reinterpret_cast<const __bf16 *>(W.p[0]);
#pragma unroll
    for (int i = 0; i < wdense<TN_, NA>::NP; i++) {
        const int q = threadIdx.x + 256 * i, row = min(n0 + (q >> 3), n_rows - 1);
#pragma unroll
        for (int p = 0; p < NA; p++) wd.p[p][i] = gld<uint4>(base + p * plane + (long)row * ldw + k0 + 8 * (q & 7));
    }
}

template <int TN_, int NA, bool SWZ, int LDA>
MLLM_DEV void put_wd(const wdense<TN_, NA> &wd, __bf16 *A)
{
#pragma unroll
    for (int i = 0; i < wdense<TN_, NA>::NP; i++) {
        const int q = threadIdx.x + 256 * i;
#pragma unroll
        for (int p = 0; p < NA; p++)
            *reinterpret_cast<uint4 *>(A + p * TN_ * LDA + tile_off<SWZ, LDA>(q >> 3, 8 * (q & 7))) = wd.p[p][i];
    }
}

// The weights of a packed matrix exactly as the tiles hold them (put_w's
// chunk_weights and plane split): NA bf16 planes [NA][n_rows][ldw], plane p
// the bf16 rounding of what planes < p leave; columns past the last block are
// left as they are (the caller clears the buffer).  One thread per chunk.
template <int SEM>
__global__ __launch_bounds__(256) void k_dense_planes(mllm_packed W, int n_rows, int n_cols, int ldw, __bf16 *out)
{
    constexpr int NA = gemm_cfg<SEM, XM_PLANES>::NA;
    constexpr int CPB = sem_traits<SEM>::kChunksPerBlock;
    const int nb = n_cols / sem_traits<SEM>::kBlockElems, nch = nb * CPB;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)n_rows * nch) return;
    const int row = (int)(i / nch), c = (int)(i % nch);
    raw_chunk raw;
    fetch<SEM>(W, nb, row, c, raw);
    float w[2][16];
    int x[2];
    chunk_weights<SEM>(raw, c, w[0], w[1], x[0], x[1]);
    const long plane = (long)n_rows * ldw;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        __bf16 *o = out + (long)row * ldw + x[h];
#pragma unroll
        for (int e = 0; e < 16; e++) {
            float r = w[h][e];
#pragma unroll
            for (int p = 0; p < NA; p++) {
                const float t = (float)(__bf16)r;
                r -= t;
                o[p * plane + e] = (__bf16)t;
            }
        }
    }
}

// Activation task of thread tid.  XM_PLANES: TM_/32 16-byte pieces per plane
// (entry q/8, columns 8*(q%8) .. +8 of the step, q = tid + 256*i), planes
// p < npl only (the lower plane of a tile whose activations are all exact in
// bf16 is zero and neither loaded, stored nor read); Q4_K_Q8:
// entry tid/2, part tid&1 (16 quants of one sub-block, k < 16); other Q8
// forms: entry tid/4, 16 columns at (tid&3)*16.
template <int TM_, int NB> struct araw {
    static constexpr int NP = TM_ / 32;
    uint4 p[NB][NP];
    uint4 q;
    float s0, s1;
};

template <int SEM, int XM, int TM_>
MLLM_DEV void fetch_a(const qgemm_args &a, const int *ent_row, int n_ent, int k0, int kused,
                      araw<TM_, gemm_cfg<SEM, XM>::NB> &ar, int npl)
{
    using C = gemm_cfg<SEM, XM>;
    const int tid = threadIdx.x;
    const long nbk = a.n_cols / 32;
    if constexpr (XM == XM_PLANES) {
        // rows past n_ent read row ent_row[] = 0; their columns are never stored
#pragma unroll
        for (int i = 0; i < araw<TM_, C::NB>::NP; i++) {
            const int q = tid + 256 * i, er = q >> 3, c8 = q & 7;
            const __bf16 *src = a.xp.base + (long)ent_row[er] * a.xp.ldp + k0 + 8 * c8;
#pragma unroll
            for (int p = 0; p < C::NB; p++)
                if (p < npl) ar.p[p][i] = gld<uint4>(reinterpret_cast<const uint4 *>(src + p * a.xp.plane));
        }
    } else if constexpr (C::A4) {
        const int er = min(tid >> 1, TM_ - 1), part = tid & 1;
        const long row = ent_row[min(er, n_ent - 1)];
        ar.q = gld<uint4>(a.xq.q + row * (nbk * 32) + k0 + 32 * part);
        ar.s0 = gld<float>(a.xq.s4 + row * nbk + k0 / 32);
        ar.s1 = gld<float>(a.xq.s4 + row * nbk + k0 / 32 + 1);
    } else {
        const int er = min(tid >> 2, TM_ - 1), seg = min((tid & 3) * 16, kused - k0 - 16);
        const long row = ent_row[min(er, n_ent - 1)];
        ar.q = gld<uint4>(a.xq.q + row * (nbk * 32) + k0 + seg);
        if constexpr (XM == XM_Q8D) ar.s0 = gld<float>(a.xq.d + row * nbk + (k0 + seg) / 32);
    }
}

// Store the step's activation planes (plane p at Bp + p*TM_*LDA); Q8 columns past
// kused and entries past n_ent are zero.
template <int SEM, int XM, int TM_>
MLLM_DEV void put_a(const araw<TM_, gemm_cfg<SEM, XM>::NB> &ar, int n_ent, int k0, int kused, __bf16 *Bp,
                    float *tsum_l, int npl)
{
    using C = gemm_cfg<SEM, XM>;
    constexpr int LDA = C::LDA, NB = C::NB, PS = TM_ * C::LDA;
    const int tid = threadIdx.x;
    float v[16];
    if constexpr (XM == XM_PLANES) {
#pragma unroll
        for (int i = 0; i < araw<TM_, NB>::NP; i++) {
            const int q = tid + 256 * i, er = q >> 3, c8 = q & 7;
#pragma unroll
            for (int p = 0; p < NB; p++)
                if (p < npl) *reinterpret_cast<uint4 *>(Bp + p * PS + tile_off<C::SWZ, LDA>(er, 8 * c8)) = ar.p[p][i];
        }
    } else if constexpr (C::A4) {
        if (tid < 2 * TM_) {
            const int er = tid >> 1, part = tid & 1;
            if (er < n_ent) {
                const uint32_t Q[4] = {ar.q.x, ar.q.y, ar.q.z, ar.q.w};
#pragma unroll
                for (int i = 0; i < 16; i++) v[i] = (float)(int8_t)((Q[i >> 2] >> (8 * (i & 3))) & 0xFF);
                if (part == 0 && tsum_l) tsum_l[er] = ar.s0 + ar.s1;   // Q4_K min term of the step's two sub-blocks
            } else {
                zero16(v);
                if (part == 0 && tsum_l) tsum_l[er] = 0.0f;
            }
            put16_f16(Bp + er * LDA + 16 * part, v);
        }
    } else {
        if (tid < 4 * TM_) {
            const int er = tid >> 2, seg = (tid & 3) * 16;
            const bool live = er < n_ent && k0 + seg < kused;
            if (live) {
                const uint32_t Q[4] = {ar.q.x, ar.q.y, ar.q.z, ar.q.w};
#pragma unroll
                for (int i = 0; i < 16; i++) v[i] = (float)(int8_t)((Q[i >> 2] >> (8 * (i & 3))) & 0xFF);
            } else {
                zero16(v);
            }
            put16_planes<NB, C::SWZ, LDA>(Bp, PS, er, seg, v);
            // Q8D: block scale of the entry's 32 columns at seg (one writer per block)
            if (XM == XM_Q8D && tsum_l && (seg & 16) == 0) tsum_l[2 * er + (seg >> 5)] = live ? ar.s0 : 0.0f;
        }
    }
}

// Workgroups per CU the tile's LDS allows (160 KB per CU), at most 3 (2 for
// the Q8D form, whose registers do not fit a third); the compiler then
// budgets registers for that many.
template <int SEM, int XM, bool DUAL, int TM, bool DW = false> constexpr int qgemm_wgs_per_cu()
{
    using C = gemm_cfg<SEM, XM>;
    constexpr int TN = tile_cfg<DUAL, TM, tile_kind<SEM, XM, DUAL, DW, TM>()>::TN;
    // fused gate+up tiles are sized with padded rows (KE + 8 columns): their
    // unpadded tiles would admit a third workgroup whose register budget spills
    constexpr int RW = DUAL ? C::KE + 8 : C::LDA;
    constexpr int lds = 2 * (C::NA * TN * RW * (DUAL ? 2 : 1) + C::NB * TM * RW) + 4 * TM + 4 * 3 * TN + 8 * TM + 64;
    constexpr int cap = XM == XM_Q8D ? 2 : 3;
    constexpr int n = 163840 / lds;
    return n < 1 ? 1 : n > cap ? cap : n;
}

template <int SEM, int XM, bool DUAL, int TM, bool DW>
__global__ __launch_bounds__(256, (qgemm_wgs_per_cu<SEM, XM, DUAL, TM, DW>())) void k_qgemm(qgemm_args a)
{
    using C = gemm_cfg<SEM, XM>;
    using G = tile_cfg<DUAL, TM, tile_kind<SEM, XM, DUAL, DW, TM>()>;
    constexpr int NA = C::NA, NB = C::NB, LDA = C::LDA, KE = C::KE, KS = C::KS, MAXT = C::MAXT;
    // 128 weight rows per tile; 64 when gate and up share a tile of two-plane weights (LDS budget)
    constexpr int TN = G::TN, IT = G::IT, JT = G::JT;
    __shared__ __attribute__((aligned(16))) __bf16 s_a[NA * TN * LDA];
    __shared__ __attribute__((aligned(16))) __bf16 s_u[DUAL ? NA * TN * LDA : 8];
    __shared__ __attribute__((aligned(16))) __bf16 s_b[NB * TM * LDA];
    __shared__ int s_row[TM];
    // s_tsum: Q4_K_Q8 min-term sums per entry, or Q8D block scales per entry and 32-column half
    __shared__ __attribute__((aligned(16))) float s_dmin[C::A4 ? 2 * TN : 1], s_dmin2[C::A4 && DUAL ? 2 * TN : 1],
        s_tsum[C::A4 ? TM : (XM == XM_Q8D ? 2 * TM : 1)];
    constexpr int BE = mllm_sem_uses_q8(SEM) ? q8_traits<SEM>::kBlockElems : sem_traits<SEM>::kBlockElems;

    // ---- work tile.  Workgroups reach the 8 XCDs round-robin by linear id and
    // each XCD has its own L2.  The live (weight tile, entry tile) pairs -- an
    // expert launch sizes its grid for the most tiles the bucketing can make,
    // of which *n_tiles are real -- are remapped so that each XCD takes an
    // equal contiguous range of them, entry tile fastest: the entry tiles that
    // share a weight tile run on one XCD, close together in time.
    int bx, by;
    {
        const int nx = gridDim.x, ny = a.tile_expert ? *a.n_tiles : (int)gridDim.y, total = nx * ny;
        const int L = blockIdx.x + nx * blockIdx.y;
        if (L >= total) return;
        const int xcd = L & 7;
        const int w = xcd * (total >> 3) + min(xcd, total & 7) + (L >> 3);
        by = w % ny;
        bx = w / ny;
    }
    int p0, p1;
    mllm_packed W, W2;
    if (a.tile_expert) {
        const int ti = by;
        const int e = a.tile_expert[ti];
        p0 = a.tile_begin[ti];
        p1 = a.tile_end[ti];
        W = a.table[e];
        if constexpr (DUAL) W2 = a.table2[e];
    } else {
        p0 = by * TM;
        p1 = min(p0 + TM, a.n_entries);
        W = a.W;
        if constexpr (DUAL) W2 = a.W2;
    }
    const int n_ent = p1 - p0;
    if (n_ent <= 0) return;
    const int n0 = bx * TN;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int lo_any = 0;   // some entry's activation is not bf16-exact: the lo plane takes part
    if (tid < TM) {
        const int row = tid < n_ent ? (a.row_of ? a.row_of[p0 + tid] : p0 + tid) : 0;
        s_row[tid] = row;
        if constexpr (XM == XM_PLANES) lo_any = tid < n_ent && a.xp.lo_nz[row] != 0;
    }
    lo_any = __syncthreads_or(lo_any);

    const int nb = a.n_cols / BE;
    const int kused = nb * BE;
    const int nsteps = (kused + KS - 1) / KS;
    // K steps of this workgroup: all, or split z of a.ksplit
    int s_beg = 0, s_end = nsteps;
    if (a.ksplit > 1) {
        const int spp = (nsteps + a.ksplit - 1) / a.ksplit;
        s_beg = min(nsteps, (int)blockIdx.z * spp);
        s_end = min(nsteps, s_beg + spp);
    }
    const int wr0 = (wave % G::WR) * 16 * IT, we0 = (wave / G::WR) * 16 * JT;
    f32x4 acc[IT][JT], acc2[DUAL ? IT : 1][DUAL ? JT : 1];
#pragma unroll
    for (int i = 0; i < IT; i++)
#pragma unroll
        for (int j = 0; j < JT; j++) acc[i][j] = f32x4{0, 0, 0, 0};
    if constexpr (DUAL) {
#pragma unroll
        for (int i = 0; i < IT; i++)
#pragma unroll
            for (int j = 0; j < JT; j++) acc2[i][j] = f32x4{0, 0, 0, 0};
    }
    // activation planes past the first all zero: their products are skipped (uniform per workgroup)
    const int pb_end = (XM == XM_PLANES && !lo_any) ? 1 : NB;
    const int li = lane & 15, lk = (lane >> 4) * 8;
    // MFMA operand offset of row base + li (base a multiple of 16), columns ks + lk:
    // on swizzled tiles (row >> 1) & 7 = li >> 1, and ks (0 or 32) flips piece bit 2
    const int rsw = ((lane >> 4) ^ (li >> 1)) << 3;
    auto roff = [&](int base, int ks) __attribute__((always_inline)) {
        if constexpr (C::SWZ) return (base + li) * 64 + (rsw ^ ks);
        else return (base + li) * LDA + ks + lk;
    };

    static_assert(!DW || (!C::A4 && KS == 64), "dense bf16 weights: plane-split forms, 64-column steps");
    using WB = typename std::conditional<DW, wdense<TN, NA>, wraw<SEM, XM, TN>>::type;
    struct stepbuf {
        WB w, u;
        araw<TM, NB> x;
    };
    auto fetch_step = [&](int s, stepbuf &b) __attribute__((always_inline)) {
        const int k0 = min(s, s_end - 1) * KS;   // past the end: refetch the last step (unused)
        if constexpr (DW) {
            fetch_wd<TN, NA>(W, a.n_rows, a.dense_ld, (long)a.n_rows * a.dense_ld, n0, k0, b.w);
            if constexpr (DUAL) fetch_wd<TN, NA>(W2, a.n_rows, a.dense_ld, (long)a.n_rows * a.dense_ld, n0, k0, b.u);
        } else {
            fetch_w<SEM, XM, TN>(W, a.n_rows, nb, n0, k0, b.w, 0);
            if constexpr (DUAL) fetch_w<SEM, XM, TN>(W2, a.n_rows, nb, n0, k0, b.u, 128);
        }
        fetch_a<SEM, XM, TM>(a, s_row, n_ent, k0, kused, b.x, pb_end);
    };
    auto put_step = [&](int s, const stepbuf &b) __attribute__((always_inline)) {
        const int k0 = s * KS;
        if constexpr (DW) {
            put_wd<TN, NA, C::SWZ, LDA>(b.w, s_a);
            if constexpr (DUAL) put_wd<TN, NA, C::SWZ, LDA>(b.u, s_u);
        } else {
            put_w<SEM, XM, TN>(b.w, a.n_rows, nb, n0, k0, s_a, C::A4 ? s_dmin : nullptr, 0);
            if constexpr (DUAL) put_w<SEM, XM, TN>(b.u, a.n_rows, nb, n0, k0, s_u, C::A4 ? s_dmin2 : nullptr, 128);
        }
        put_a<SEM, XM, TM>(b.x, n_ent, k0, kused, s_b, (C::A4 || XM == XM_Q8D) ? s_tsum : nullptr, pb_end);
    };
    auto mfma_step = [&]() __attribute__((always_inline)) {
        // MFMA 16x16x32: lane l supplies row/entry (l % 16), k = 8*(l/16) .. +8 of a 32-wide slice
#pragma unroll
        for (int ks = 0; ks < KE; ks += 32) {
            bf16x8 bv[NB][JT];
#pragma unroll
            for (int p = 0; p < NB; p++)
#pragma unroll
                for (int j = 0; j < JT; j++)
                    if (p < pb_end) bv[p][j] = *reinterpret_cast<const bf16x8 *>(s_b + p * TM * LDA + roff(we0 + 16 * j, ks));
#pragma unroll
            for (int i = 0; i < IT; i++) {
                const int ar_ = roff(wr0 + 16 * i, ks);
                bf16x8 av[NA];
#pragma unroll
                for (int p = 0; p < NA; p++) av[p] = *reinterpret_cast<const bf16x8 *>(s_a + p * TN * LDA + ar_);
                if constexpr (XM == XM_Q8D) {
                    // exact block product (MXFP4 weight x Q8_0 quant), then its activation scale
#pragma unroll
                    for (int j = 0; j < JT; j++) {
                        const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[0], bv[0][j], f32x4{0, 0, 0, 0}, 0, 0, 0);
                        const float sc = s_tsum[2 * (we0 + 16 * j + li) + (ks >> 5)];
#pragma unroll
                        for (int v = 0; v < 4; v++) acc[i][j][v] = fmaf(sc, d[v], acc[i][j][v]);
                    }
                } else if constexpr (C::A4) {
                    // exact integer dot of the step's two 16-column sub-block halves, then d per row
                    const f32x4 dr = *reinterpret_cast<const f32x4 *>(s_dmin + TN + wr0 + 16 * i + 4 * (lane >> 4));
#pragma unroll
                    for (int j = 0; j < JT; j++) {
                        const f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av[0]),
                                                                             __builtin_bit_cast(f16x8, bv[0][j]),
                                                                             f32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; v++) acc[i][j][v] = fmaf(dr[v], t[v], acc[i][j][v]);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < JT; j++)
#pragma unroll
                        for (int pa = 0; pa < NA; pa++)
#pragma unroll
                            for (int pb = 0; pb < NB; pb++)
                                if (pa + pb <= MAXT && pb < pb_end)
                                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[pa], bv[pb][j], acc[i][j], 0, 0, 0);
                }
                if constexpr (DUAL) {
#pragma unroll
                    for (int p = 0; p < NA; p++) av[p] = *reinterpret_cast<const bf16x8 *>(s_u + p * TN * LDA + ar_);
                    if constexpr (XM == XM_Q8D) {
#pragma unroll
                        for (int j = 0; j < JT; j++) {
                            const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[0], bv[0][j], f32x4{0, 0, 0, 0}, 0, 0, 0);
                            const float sc = s_tsum[2 * (we0 + 16 * j + li) + (ks >> 5)];
#pragma unroll
                            for (int v = 0; v < 4; v++) acc2[i][j][v] = fmaf(sc, d[v], acc2[i][j][v]);
                        }
                    } else if constexpr (C::A4) {
                        const f32x4 dr = *reinterpret_cast<const f32x4 *>(s_dmin2 + TN + wr0 + 16 * i + 4 * (lane >> 4));
#pragma unroll
                        for (int j = 0; j < JT; j++) {
                            const f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av[0]),
                                                                                 __builtin_bit_cast(f16x8, bv[0][j]),
                                                                                 f32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                            for (int v = 0; v < 4; v++) acc2[i][j][v] = fmaf(dr[v], t[v], acc2[i][j][v]);
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < JT; j++)
#pragma unroll
                            for (int pa = 0; pa < NA; pa++)
#pragma unroll
                                for (int pb = 0; pb < NB; pb++)
                                    if (pa + pb <= MAXT && pb < pb_end)
                                        acc2[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[pa], bv[pb][j], acc2[i][j], 0, 0, 0);
                    }
                }
            }
        }
        if constexpr (C::A4) {
            // min term: acc[row][ent] -= dmin[row] * (d8-weighted q8 sums of the step's two sub-blocks).
            // D layout of a 16x16 output: lane l holds entry (l % 16), rows 4*(l/16) .. +3.
#pragma unroll
            for (int i = 0; i < IT; i++)
#pragma unroll
                for (int j = 0; j < JT; j++) {
                    const float ts = s_tsum[we0 + 16 * j + li];
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const int rr = wr0 + 16 * i + 4 * (lane >> 4) + v;
                        acc[i][j][v] = fmaf(-s_dmin[rr], ts, acc[i][j][v]);
                        if constexpr (DUAL) acc2[i][j][v] = fmaf(-s_dmin2[rr], ts, acc2[i][j][v]);
                    }
                }
        }
    };

    // two steps in flight: buffer A holds steps s_beg, s_beg+2, ..., B the others.
    // A wave whose entries all lie past the tile's last one (a part-filled
    // expert tile) skips its MFMAs; the branch also keeps the step's global
    // loads in a block of their own, ahead of the MFMA sequence, which the
    // dense launches measured ~25% faster with.
    if (s_beg < s_end) {
        stepbuf bA, bB;
        fetch_step(s_beg, bA);
        fetch_step(s_beg + 1, bB);
        put_step(s_beg, bA);
        __syncthreads();
        for (int s = s_beg;; s += 2) {
            fetch_step(s + 2, bA);
            if (we0 < n_ent) mfma_step();
            __syncthreads();
            if (s + 1 >= s_end) break;
            put_step(s + 1, bB);
            __syncthreads();
            fetch_step(s + 3, bB);
            if (we0 < n_ent) mfma_step();
            __syncthreads();
            if (s + 2 >= s_end) break;
            put_step(s + 2, bA);
            __syncthreads();
        }
    }

    // ---- epilogue
    float *out = a.out;
    long ldo = a.ldo;
    if (a.ksplit > 1) { out = a.part + (long)blockIdx.z * a.n_entries * a.n_rows; ldo = a.n_rows; }
#pragma unroll
    for (int i = 0; i < IT; i++)
#pragma unroll
        for (int j = 0; j < JT; j++) {
            const int ent = we0 + 16 * j + li;
            if (ent >= n_ent) continue;
            const long orow = a.out_row ? a.out_row[p0 + ent] : (long)(p0 + ent);
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int n = n0 + wr0 + 16 * i + 4 * (lane >> 4) + v;
                if (n >= a.n_rows) continue;
                float r = acc[i][j][v];
                if constexpr (DUAL) {
                    // moe_forward_omp SiLU (QK:2157-2164): clamp to +-80, then silu(g) * u
                    float g = r;
                    if (a.clamp_silu) { g = g < -80.0f ? -80.0f : g; g = g > 80.0f ? 80.0f : g; }
                    r = (g / (1.0f + expf(-g))) * acc2[i][j][v];
                }
                out[orow * ldo + n] = r;
            }
        }
}

// out[e][n] = sum over z < ks of part[z][e][n], in order.
__global__ void k_ksum(const float *__restrict__ part, int ks, long plane, int n_rows, float *__restrict__ out, int ldo)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= plane) return;
    float v = part[i];
    for (int z = 1; z < ks; z++) v += part[z * plane + i];
    const long e = i / n_rows, n = i - e * n_rows;
    out[e * ldo + n] = v;
}

template <int SEM, int XM, bool DUAL, int TM, bool DW = false>
hipError_t launch(const qgemm_args &a, int max_tiles, hipStream_t st)
{
    constexpr int TN = tile_cfg<DUAL, TM, tile_kind<SEM, XM, DUAL, DW, TM>()>::TN;
    const int ks = (a.ksplit > 1 && !DUAL && !a.tile_expert && !a.out_row) ? a.ksplit : 1;
    dim3 grid((a.n_rows + TN - 1) / TN, a.tile_expert ? max_tiles : (a.n_entries + TM - 1) / TM, ks);
    if (grid.y == 0) return hipSuccess;
    qgemm_args b = a;
    b.ksplit = ks;
    hipLaunchKernelGGL((k_qgemm<SEM, XM, DUAL, TM, DW>), grid, dim3(256), 0, st, b);
    if (ks > 1) {
        const long plane = (long)a.n_entries * a.n_rows;
        hipLaunchKernelGGL(k_ksum, dim3((unsigned)((plane + 255) / 256)), dim3(256), 0, st, a.part, ks, plane,
                           a.n_rows, a.out, a.ldo);
    }
    return hipGetLastError();
}

} // namespace

// Grouped (expert-tile) launches use the 64-entry tiles the bucketing makes;
// dense split-plane launches take 128-entry tiles once there are enough
// entries to fill them.
hipError_t mllm_launch_qgemm(int sem, int xmode, bool dual, const qgemm_args &a, int max_tiles, hipStream_t st)
{
    if (a.dense_ld > 0) {
        // dense bf16 plane copies (mllm_launch_dense_planes) of the MoE layer's
        // semantics, 64-entry tiles
        if (a.dense_ld % 64 || a.dense_ld < a.n_cols || mllm_dense_planes(sem) == 0) return hipErrorInvalidValue;
#define QGD(S, X)                                                                           \
    if (sem == S && xmode == X) return dual ? launch<S, X, true, 64, true>(a, max_tiles, st) \
                                            : launch<S, X, false, 64, true>(a, max_tiles, st);
        QGD(SEM_MXFP4, XM_PLANES)
        QGD(SEM_MXFP4_Q8, XM_Q8D)
#undef QGD
        return hipErrorInvalidValue;
    }
    const bool wide = !dual && !a.tile_expert && a.n_entries >= 512;
#define QGP(S)                                                                        \
    if (sem == S && xmode == XM_PLANES) {                                             \
        if (dual) return launch<S, XM_PLANES, true, 64>(a, max_tiles, st);            \
        return wide ? launch<S, XM_PLANES, false, 128>(a, max_tiles, st)              \
                    : launch<S, XM_PLANES, false, 64>(a, max_tiles, st);              \
    }
#define QGQ(S, X)                                                                     \
    if (sem == S && xmode == X) return dual ? launch<S, X, true, 64>(a, max_tiles, st) \
                                            : launch<S, X, false, 64>(a, max_tiles, st);
    QGP(SEM_Q4_0)
    QGP(SEM_Q4_1)
    QGP(SEM_Q5_0_F32)
    QGP(SEM_Q8_0)
    QGP(SEM_Q4_K_GGML)
    QGP(SEM_Q5_K_GGML)
    QGP(SEM_Q5_K_CE)
    QGP(SEM_Q6_K_GGML)
    QGP(SEM_Q6_K_LOWNIB)
    QGP(SEM_Q6_K_SEQ)
    QGP(SEM_MXFP4)
    QGP(SEM_MXFP4_CLAMP)
    QGQ(SEM_Q4_K_Q8, XM_Q8)
    QGQ(SEM_MXFP4_Q8, XM_Q8D)
#undef QGP
#undef QGQ
    return hipErrorInvalidValue;
}

bool mllm_qgemm_supported(int sem)
{
    return sem != SEM_F32 && sem != SEM_Q5_0_Q8;
}

// A dense launch with fewer output tiles than CUs is split along K into at
// most 512 workgroups (two per CU: a launch past that runs a second, partial
// round of workgroups), each split keeping at least 4 K steps of 64 columns,
// and into at most 8 splits (the partial sums cost an extra pass over ksplit x
// entries x rows floats, which does not pay on a launch that already fills the
// GPU; 16 splits of the 2048-row down projection at M = 128 measured slower
// than 8).
int mllm_qgemm_ksplit(int sem, int n_rows, int n_cols, int n_entries)
{
    if (!mllm_qgemm_supported(sem) || n_entries <= 0) return 1;
    const int tm = (n_entries >= 512 && sem != SEM_Q4_K_Q8 && sem != SEM_MXFP4_Q8) ? 128 : 64;
    const long tiles = (long)((n_rows + 127) / 128) * ((n_entries + tm - 1) / tm);
    if (tiles >= 256) return 1;
    const int steps = (n_cols + 63) / 64;
    int ks = (int)(512 / tiles);
    ks = std::min(ks, std::max(1, steps / 4));
    return std::max(1, std::min(ks, 8));
}

// fp32 rows -> NP bf16 planes (one workgroup per row, 8 columns per thread and
// pass), zero padded to act_planes_ld(K); lo_nz[row] = a plane past the first
// has a non-zero element.
template <int NP>
__global__ __launch_bounds__(256) void k_act_split(const float *__restrict__ x, int ldx, int K,
                                                   __bf16 *__restrict__ base, long plane, int ldp, int *lo_nz)
{
    const int row = blockIdx.x;
    const float *xr = x + (long)row * ldx;
    __bf16 *pr = base + (long)row * ldp;
    const bool vec = (ldx & 3) == 0 && (K & 7) == 0;
    int nz = 0;
    for (int k = 8 * threadIdx.x; k < ldp; k += 8 * blockDim.x) {
        float v[8];
        if (vec && k + 8 <= K) {
            const float4 f0 = gld<float4>(xr + k), f1 = gld<float4>(xr + k + 4);
            v[0] = f0.x; v[1] = f0.y; v[2] = f0.z; v[3] = f0.w; v[4] = f1.x; v[5] = f1.y; v[6] = f1.z; v[7] = f1.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = k + e < K ? xr[k + e] : 0.0f;
        }
#pragma unroll
        for (int p = 0; p < NP; p++) {
            bf16x8 h;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                h[e] = (__bf16)v[e];
                v[e] -= (float)h[e];
                if (p) nz |= (float)h[e] != 0.0f;
            }
            *reinterpret_cast<bf16x8 *>(pr + p * plane + k) = h;
        }
    }
    nz = __syncthreads_or(nz);
    if (threadIdx.x == 0) lo_nz[row] = nz;
}

hipError_t mllm_launch_act_split(const float *x, int ldx, int rows, int K, int nplanes, __bf16 *base, long plane,
                                 int *lo_nz, hipStream_t st)
{
    if (rows <= 0) return hipSuccess;
    if (K <= 0 || ((uintptr_t)base & 15) || (plane & 7) || (nplanes != 2 && nplanes != 3)) return hipErrorInvalidValue;
    if (nplanes == 2)
        hipLaunchKernelGGL(k_act_split<2>, dim3(rows), dim3(256), 0, st, x, ldx, K, base, plane, act_planes_ld(K), lo_nz);
    else
        hipLaunchKernelGGL(k_act_split<3>, dim3(rows), dim3(256), 0, st, x, ldx, K, base, plane, act_planes_ld(K), lo_nz);
    return hipGetLastError();
}

// bf16 planes of a packed matrix for the GEMM's dense-weight tiles; 0: not
// offered for this semantic.  Offered for the MXFP4 forms (one exact plane).
// Two-plane copies (the Q6_K / Q4_0 expert forms) ran no faster than the
// decoding narrow tiles: Qwen3's Q6_K down layer 677 us over them, 664 us
// decoded.
int mllm_dense_planes(int sem)
{
    return (sem == SEM_MXFP4 || sem == SEM_MXFP4_Q8) ? gemm_cfg<SEM_MXFP4, XM_PLANES>::NA : 0;
}

hipError_t mllm_launch_dense_planes(int sem, const mllm_packed &W, int n_rows, int n_cols, int ldw, __bf16 *out,
                                    hipStream_t st)
{
    const long nch = (long)n_rows * (n_cols / 32);   // chunks of 32 weights
    if (nch == 0) return hipSuccess;
    const dim3 g((unsigned)((nch + 255) / 256));
    if (mllm_dense_planes(sem) == 0) return hipErrorInvalidValue;
    // MXFP4 and MXFP4_Q8: one layout and the same weights, sext4(n) * 2^(E-127)
    hipLaunchKernelGGL(k_dense_planes<SEM_MXFP4>, g, dim3(256), 0, st, W, n_rows, n_cols, ldw, out);
    return hipGetLastError();
}
