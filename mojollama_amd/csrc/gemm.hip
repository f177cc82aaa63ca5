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
// products wi*bj with i + j <= 2 in fp32, i.e. every term down to 2^-16 of
// the leading one.  Operands exact in one bf16 use one plane: MXFP4 weights
// (int4 times a power of two) and Q8_0 quants; their partners then get
// three, which makes those products exact to fp32.  Everything else uses
// two planes each (normalised error ~1e-5).
//
// Tiling.  Workgroup = 4 wave64s, tile TN (128, or 64 when gate and up share
// it) rows x 64 entries, K staged KE columns at a time; a wave owns 32 rows
// x (64 or 32) entries = 2 x JT MFMA 16x16 outputs.  LDS rows are padded by
// 16 bytes so the 16 lanes reading one k-slice hit distinct banks.
#include "decode.h"
#include "gemm.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int TM = 64;   // entries per tile

template <int SEM, int XM> struct gemm_cfg {
    static constexpr bool A4 = (SEM == SEM_Q4_K_Q8);
    static constexpr bool WEXACT = (SEM == SEM_MXFP4 || SEM == SEM_MXFP4_CLAMP || SEM == SEM_MXFP4_Q8);
    static constexpr int NA = WEXACT ? 1 : (A4 ? 3 : 2);
    static constexpr int NB = (XM == XM_Q8) ? 1 : (NA == 1 ? 3 : 2);
    // K columns per step: A4 keeps only the 32 columns its dot reads of each 64
    static constexpr int KS = 64;
    static constexpr int KE = A4 ? 32 : 64;
    static constexpr int LDA = KE + 8;
};

MLLM_DEV void put16(__bf16 *dst, const float (&v)[16])
{
    bf16x8 a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) { a[i] = (__bf16)v[i]; b[i] = (__bf16)v[8 + i]; }
    *reinterpret_cast<bf16x8 *>(dst) = a;
    *reinterpret_cast<bf16x8 *>(dst + 8) = b;
}

// Store 16 values as NP bf16 planes (plane p at base + p*pstride, element offset off).
template <int NP>
MLLM_DEV void put16_planes(__bf16 *base, int pstride, int off, const float (&v)[16])
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
        put16(base + p * pstride + off, t);
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

// Stage weight rows [n0, n0+TN_) x the step's columns into LDS planes
// (plane p at A + p*TN_*LDA).  For Q4_K_Q8 also each row's dmin.
template <int SEM, int XM, int TN_>
MLLM_DEV void stage_weights(const mllm_packed &W, int n_rows, int nb, int n0, int k0, __bf16 *A, float *dmin_l)
{
    using C = gemm_cfg<SEM, XM>;
    constexpr int LDA = C::LDA, NA = C::NA, PS = TN_ * C::LDA;
    const int tid = threadIdx.x;
    if constexpr (C::A4) {
        // dot_q4_k_q8_0 (QK:1647-1735): the integer term reads k < 16 of each 32-element sub-block;
        // group g of a super-block holds sub-blocks 2g (low nibbles) and 2g+1 (high nibbles).
        // Step columns: 0..15 = sub-block 2g, 16..31 = sub-block 2g+1, weight d*sc_j*nib.
        if (tid < TN_) {
            const int row = min(n0 + tid, n_rows - 1);
            const int c = k0 / 64;
            raw_chunk r;
            q8_fetch<SEM>(W, nb, row, c, r);
            const int g = c & 3;
            int s1, m1, s2, m2;
            kq_pairs(r.m, 2 * g, s1, m1, s2, m2);
            const float d = h2f(r.m.x & 0xFFFF);
            const float ds1 = d * (float)s1, ds2 = d * (float)s2;
            const uint32_t Aw[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
            float lo[16], hi[16];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                lo[i] = ds1 * (float)((Aw[i >> 2] >> (8 * (i & 3))) & 15);
                hi[i] = ds2 * (float)((Aw[i >> 2] >> (8 * (i & 3) + 4)) & 15);
            }
            put16_planes<NA>(A, PS, tid * LDA, lo);
            put16_planes<NA>(A, PS, tid * LDA + 16, hi);
            if (dmin_l) dmin_l[tid] = h2f(r.m.x >> 16);
        }
    } else if constexpr (SEM == SEM_MXFP4_Q8) {
        // mxfp4_row_dot_q8 (QK:629-678) with the token's Q8 scale moved to the activation side:
        // w = sext4(n) * 2^(E-127), exact in bf16.
        for (int t = tid; t < TN_ * 2; t += blockDim.x) {
            const int rr = t >> 1, cc = t & 1;
            const int row = min(n0 + rr, n_rows - 1);
            const int c = k0 / 32 + cc;
            float v0[16], v1[16];
            if (c < nb) {
                raw_chunk r;
                q8_fetch<SEM>(W, nb, row, c, r);
                const float s = e8m0f(r.d);
                const uint32_t Aw[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
                for (int e = 0; e < 32; e++) {
                    const int n = (Aw[e >> 3] >> (4 * (e & 7))) & 15;
                    const float w = (float)(n >= 8 ? n - 16 : n) * s;
                    if (e < 16) v0[e] = w; else v1[e - 16] = w;
                }
            } else {   // past the last block of an odd block count
                zero16(v0); zero16(v1);
            }
            put16_planes<NA>(A, PS, rr * LDA + 32 * cc, v0);
            put16_planes<NA>(A, PS, rr * LDA + 32 * cc + 16, v1);
        }
    } else {
        constexpr int CPB = sem_traits<SEM>::kChunksPerBlock, BE = sem_traits<SEM>::kBlockElems;
        // Chunks touching columns [k0, k0+64): 32-element blocks -> two whole chunks; K-quants ->
        // chunks 2q, 2q+1 of the super-block's quarter q, except the ggml Q6_K orders, whose chunks
        // put their two runs 64 columns apart: four chunks, one run each.
        constexpr bool SPLIT = (SEM == SEM_Q6_K_GGML || SEM == SEM_Q6_K_LOWNIB);
        constexpr int NT = SPLIT ? 4 : 2;
        const int q = (k0 % 256) / 64;
        for (int t = tid; t < TN_ * NT; t += blockDim.x) {
            const int rr = t / NT, sub = t % NT;
            const int row = min(n0 + rr, n_rows - 1);
            int c;
            if constexpr (BE == 256) c = (k0 / 256) * CPB + (SPLIT ? 4 * (q >> 1) + sub : 2 * q + sub);
            else c = k0 / 32 + sub;
            if (BE == 32 && c >= nb) {   // past the last block of an odd block count: zero columns
                float z[16];
                zero16(z);
                put16_planes<NA>(A, PS, rr * LDA + 32 * sub, z);
                put16_planes<NA>(A, PS, rr * LDA + 32 * sub + 16, z);
                continue;
            }
            raw_chunk r;
            fetch<SEM>(W, nb, row, c, r);
            float w0[16], w1[16];
            int x0, x1;
            chunk_weights<SEM>(r, c, w0, w1, x0, x1);
            if (!SPLIT || (q & 1) == 0) put16_planes<NA>(A, PS, rr * LDA + (x0 - k0), w0);
            if (!SPLIT || (q & 1) == 1) put16_planes<NA>(A, PS, rr * LDA + (x1 - k0), w1);
        }
    }
}

// Stage the activations of the tile's entries for the step into LDS planes
// (plane p at Bp + p*TM*LDA).  Columns past kused stay zero.
template <int SEM, int XM>
MLLM_DEV void stage_acts(const qgemm_args &a, const int *ent_row, int n_ent, int k0, int kused, __bf16 *Bp,
                         float *tsum_l)
{
    using C = gemm_cfg<SEM, XM>;
    constexpr int LDA = C::LDA, NB = C::NB, PS = TM * C::LDA;
    const int tid = threadIdx.x;
    const long nbk = a.n_cols / 32;
    float v[16];
    if constexpr (C::A4) {
        // columns 0..15: q8 of sub-block k0/32, k < 16; 16..31: sub-block k0/32 + 1, k < 16
        if (tid < 2 * TM) {
            const int er = tid >> 1, part = tid & 1;
            if (er < n_ent) {
                const long row = ent_row[er];
                const uint4 q = gld<uint4>(a.xq.q + row * (nbk * 32) + k0 + 32 * part);
                const uint32_t Q[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int i = 0; i < 16; i++) v[i] = (float)(int8_t)((Q[i >> 2] >> (8 * (i & 3))) & 0xFF);
                if (part == 0 && tsum_l)   // Q4_K min term of the step's two sub-blocks
                    tsum_l[er] = gld<float>(a.xq.s4 + row * nbk + k0 / 32) + gld<float>(a.xq.s4 + row * nbk + k0 / 32 + 1);
            } else {
                zero16(v);
                if (part == 0 && tsum_l) tsum_l[er] = 0.0f;
            }
            put16_planes<NB>(Bp, PS, er * LDA + 16 * part, v);
        }
    } else {
        // 4 threads per entry row, 16 columns each
        const int er = tid >> 2, seg = (tid & 3) * 16;
        if (er < n_ent && k0 + seg < kused) {
            const long row = ent_row[er];
            if constexpr (XM == XM_F32) {
                const float *src = a.x + row * a.ldx + k0 + seg;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 f = gld<float4>(src + 4 * q);
                    v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
                }
            } else {
                const uint4 q = gld<uint4>(a.xq.q + row * (nbk * 32) + k0 + seg);
                const uint32_t Q[4] = {q.x, q.y, q.z, q.w};
                float d8 = 1.0f;
                if constexpr (XM == XM_Q8D) d8 = gld<float>(a.xq.d + row * nbk + (k0 + seg) / 32);
#pragma unroll
                for (int i = 0; i < 16; i++) v[i] = (float)(int8_t)((Q[i >> 2] >> (8 * (i & 3))) & 0xFF) * d8;
            }
        } else {
            zero16(v);
        }
        put16_planes<NB>(Bp, PS, er * LDA + seg, v);
    }
}

template <int SEM, int XM, bool DUAL>
__global__ __launch_bounds__(256) void k_qgemm(qgemm_args a)
{
    using C = gemm_cfg<SEM, XM>;
    constexpr int NA = C::NA, NB = C::NB, LDA = C::LDA, KE = C::KE, KS = C::KS;
    // 128 weight rows per tile, 64 when gate and up share the tile (LDS budget)
    constexpr int TN = DUAL ? 64 : 128;
    constexpr int RG = TN / 32;              // 32-row groups per tile
    constexpr int EG = 4 / RG;               // entry groups
    constexpr int JT = TM / 16 / EG;         // 16-entry MFMA tiles per wave
    __shared__ __attribute__((aligned(16))) __bf16 s_a[NA * TN * LDA];
    __shared__ __attribute__((aligned(16))) __bf16 s_u[DUAL ? NA * TN * LDA : 8];
    __shared__ __attribute__((aligned(16))) __bf16 s_b[NB * TM * LDA];
    __shared__ int s_row[TM];
    __shared__ float s_dmin[C::A4 ? TN : 1], s_dmin2[C::A4 && DUAL ? TN : 1], s_tsum[C::A4 ? TM : 1];
    constexpr int BE = mllm_sem_uses_q8(SEM) ? q8_traits<SEM>::kBlockElems : sem_traits<SEM>::kBlockElems;

    // ---- work tile
    int p0, p1;
    mllm_packed W, W2;
    if (a.tile_expert) {
        const int ti = blockIdx.y;
        if (ti >= *a.n_tiles) return;
        const int e = a.tile_expert[ti];
        p0 = a.tile_begin[ti];
        p1 = a.tile_end[ti];
        W = a.table[e];
        if constexpr (DUAL) W2 = a.table2[e];
    } else {
        p0 = blockIdx.y * TM;
        p1 = min(p0 + TM, a.n_entries);
        W = a.W;
        if constexpr (DUAL) W2 = a.W2;
    }
    const int n_ent = p1 - p0;
    const int n0 = blockIdx.x * TN;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (tid < TM) s_row[tid] = tid < n_ent ? (a.row_of ? a.row_of[p0 + tid] : p0 + tid) : 0;
    __syncthreads();

    const int nb = a.n_cols / BE;
    const int kused = nb * BE;
    const int wr0 = (wave % RG) * 32, we0 = (wave / RG) * 16 * JT;
    f32x4 acc[2][JT], acc2[DUAL ? 2 : 1][DUAL ? JT : 1];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < JT; j++) acc[i][j] = f32x4{0, 0, 0, 0};
    if constexpr (DUAL) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < JT; j++) acc2[i][j] = f32x4{0, 0, 0, 0};
    }
    const int li = lane & 15, lk = (lane >> 4) * 8;

    for (int k0 = 0; k0 < kused; k0 += KS) {
        stage_weights<SEM, XM, TN>(W, a.n_rows, nb, n0, k0, s_a, C::A4 ? s_dmin : nullptr);
        if constexpr (DUAL) stage_weights<SEM, XM, TN>(W2, a.n_rows, nb, n0, k0, s_u, C::A4 ? s_dmin2 : nullptr);
        stage_acts<SEM, XM>(a, s_row, n_ent, k0, kused, s_b, C::A4 ? s_tsum : nullptr);
        __syncthreads();
        // MFMA 16x16x32: lane l supplies row/entry (l % 16), k = 8*(l/16) .. +8 of a 32-wide slice
#pragma unroll
        for (int ks = 0; ks < KE; ks += 32) {
            bf16x8 bv[NB][JT];
#pragma unroll
            for (int p = 0; p < NB; p++)
#pragma unroll
                for (int j = 0; j < JT; j++)
                    bv[p][j] = *reinterpret_cast<const bf16x8 *>(s_b + p * TM * LDA + (we0 + 16 * j + li) * LDA + ks + lk);
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int ar = (wr0 + 16 * i + li) * LDA + ks + lk;
                bf16x8 av[NA];
#pragma unroll
                for (int p = 0; p < NA; p++) av[p] = *reinterpret_cast<const bf16x8 *>(s_a + p * TN * LDA + ar);
#pragma unroll
                for (int j = 0; j < JT; j++)
#pragma unroll
                    for (int pa = 0; pa < NA; pa++)
#pragma unroll
                        for (int pb = 0; pb < NB; pb++)
                            if (pa + pb <= 2)
                                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[pa], bv[pb][j], acc[i][j], 0, 0, 0);
                if constexpr (DUAL) {
#pragma unroll
                    for (int p = 0; p < NA; p++) av[p] = *reinterpret_cast<const bf16x8 *>(s_u + p * TN * LDA + ar);
#pragma unroll
                    for (int j = 0; j < JT; j++)
#pragma unroll
                        for (int pa = 0; pa < NA; pa++)
#pragma unroll
                            for (int pb = 0; pb < NB; pb++)
                                if (pa + pb <= 2)
                                    acc2[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[pa], bv[pb][j], acc2[i][j], 0, 0, 0);
                }
            }
        }
        if constexpr (C::A4) {
            // min term: acc[row][ent] -= dmin[row] * (d8-weighted q8 sums of the step's two sub-blocks).
            // D layout of a 16x16 output: lane l holds entry (l % 16), rows 4*(l/16) .. +3.
#pragma unroll
            for (int i = 0; i < 2; i++)
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
        __syncthreads();
    }

    // ---- epilogue
#pragma unroll
    for (int i = 0; i < 2; i++)
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
                a.out[orow * a.ldo + n] = r;
            }
        }
}

template <int SEM, int XM, bool DUAL>
hipError_t launch(const qgemm_args &a, int max_tiles, hipStream_t st)
{
    constexpr int TN = DUAL ? 64 : 128;
    dim3 grid((a.n_rows + TN - 1) / TN, a.tile_expert ? max_tiles : (a.n_entries + TM - 1) / TM);
    if (grid.y == 0) return hipSuccess;
    hipLaunchKernelGGL((k_qgemm<SEM, XM, DUAL>), grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

} // namespace

hipError_t mllm_launch_qgemm(int sem, int xmode, bool dual, const qgemm_args &a, int max_tiles, hipStream_t st)
{
#define QG(S, X)                                                                      \
    if (sem == S && xmode == X) return dual ? launch<S, X, true>(a, max_tiles, st)    \
                                            : launch<S, X, false>(a, max_tiles, st);
    QG(SEM_Q4_0, XM_F32)
    QG(SEM_Q4_1, XM_F32)
    QG(SEM_Q5_0_F32, XM_F32)
    QG(SEM_Q8_0, XM_F32)
    QG(SEM_Q4_K_GGML, XM_F32)
    QG(SEM_Q5_K_GGML, XM_F32)
    QG(SEM_Q5_K_CE, XM_F32)
    QG(SEM_Q6_K_GGML, XM_F32)
    QG(SEM_Q6_K_LOWNIB, XM_F32)
    QG(SEM_Q6_K_SEQ, XM_F32)
    QG(SEM_MXFP4, XM_F32)
    QG(SEM_MXFP4_CLAMP, XM_F32)
    QG(SEM_Q4_K_Q8, XM_Q8)
    QG(SEM_MXFP4_Q8, XM_Q8D)
#undef QG
    return hipErrorInvalidValue;
}

bool mllm_qgemm_supported(int sem)
{
    return sem != SEM_F32 && sem != SEM_Q5_0_Q8;
}
