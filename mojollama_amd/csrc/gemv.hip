// gemv.hip — decode GEMV for batch 1..8 on gfx950.
//
// out[b][row] = sum_k w[row][k] * x[b][k] for one weight matrix, or for a list
// of "jobs" (expert matrices picked through a device-side index array, as the
// MoE layer needs).  The path is HBM-bound: each lane streams 16-byte chunks
// of the packed quant plane, decodes them in registers and accumulates in
// fp32; the lanes of a row group reduce across the wavefront with DPP.
//
// Mapping: a workgroup is 4 wave64s; a wave owns R rows per lane group of LPR
// lanes (64/LPR groups per wave).  Lanes of a group stride over the row's
// chunks, so consecutive lanes read consecutive 16-byte pieces of the row.
// x is read through L1/L2 (it is at most a few hundred KB) and each x chunk
// is reused for the R rows a lane holds.
#include "decode.h"
#include "gemv.h"

namespace {

template <int W>
MLLM_DEV float group_sum(float v)
{
    // Sum over aligned groups of W lanes; every lane of the group ends with the total.
    if constexpr (W >= 2)  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false)); // quad_perm 1,0,3,2
    if constexpr (W >= 4)  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false)); // quad_perm 2,3,0,1
    if constexpr (W >= 8)  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false)); // row_half_mirror
    if constexpr (W >= 16) v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false)); // row_mirror
    if constexpr (W >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (W >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

MLLM_DEV void resolve_job(const mllm_gemv_args &a, int job, mllm_packed &W)
{
    if (a.table) {
        int e = a.idx ? a.idx[job] : job;
        W = a.table[e < 0 ? 0 : e];
    } else {
        W = a.W;
    }
}

// fp32-activation semantics
template <int SEM, int BM, int R, int LPR>
__global__ __launch_bounds__(256) void k_gemv(mllm_gemv_args a)
{
    constexpr int CPB = sem_traits<SEM>::kChunksPerBlock;
    constexpr bool OFF = sem_traits<SEM>::kHasOffset;
    const int job = blockIdx.y;
    mllm_packed W;
    resolve_job(a, job, W);
    const float *__restrict__ x = a.x + job * a.x_job_stride;
    float *__restrict__ out = a.out + job * a.out_job_stride;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = lane / LPR, sl = lane % LPR;
    const int row0 = ((blockIdx.x * 4 + wave) * (64 / LPR) + grp) * R;
    const int nb = a.n_cols / sem_traits<SEM>::kBlockElems;
    const int nch = nb * CPB;
    const int B = a.B;

    float acc[R][BM];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < BM; b++) acc[r][b] = 0.0f;

    for (int c = sl; c < nch; c += LPR) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(row0 + r, a.n_rows - 1);
            mllm_chunk k;
            load_chunk<SEM>(W, nb, row, c, k);
#pragma unroll
            for (int b = 0; b < BM; b++) {
                if (b < B) {
                    const float *xb = x + (long)b * a.ldx;
                    const float4 *p0 = reinterpret_cast<const float4 *>(xb + k.x0);
                    const float4 *p1 = reinterpret_cast<const float4 *>(xb + k.x1);
                    float d0 = 0.f, d1 = 0.f, s0 = 0.f, s1 = 0.f;
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        float4 xa = p0[v], xc = p1[v];
                        d0 = fmaf(k.q[4 * v + 0], xa.x, d0); d0 = fmaf(k.q[4 * v + 1], xa.y, d0);
                        d0 = fmaf(k.q[4 * v + 2], xa.z, d0); d0 = fmaf(k.q[4 * v + 3], xa.w, d0);
                        d1 = fmaf(k.q[16 + 4 * v + 0], xc.x, d1); d1 = fmaf(k.q[16 + 4 * v + 1], xc.y, d1);
                        d1 = fmaf(k.q[16 + 4 * v + 2], xc.z, d1); d1 = fmaf(k.q[16 + 4 * v + 3], xc.w, d1);
                        if constexpr (OFF) { s0 += (xa.x + xa.y) + (xa.z + xa.w); s1 += (xc.x + xc.y) + (xc.z + xc.w); }
                    }
                    float t = fmaf(k.s0, d0, k.s1 * d1);
                    if constexpr (OFF) t = fmaf(k.o0, s0, fmaf(k.o1, s1, t));
                    acc[r][b] += t;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int b = 0; b < BM; b++) {
            float v = group_sum<LPR>(acc[r][b]);
            const int row = row0 + r;
            if (sl == 0 && row < a.n_rows && b < B) out[(long)b * a.ldo + row] = v;
        }
    }
}

// Q8_0-activation semantics
template <int SEM, int BM, int R, int LPR>
__global__ __launch_bounds__(256) void k_gemv_q8(mllm_gemv_args a)
{
    constexpr int CPB = q8_traits<SEM>::kChunksPerBlock;
    const int job = blockIdx.y;
    mllm_packed W;
    resolve_job(a, job, W);
    float *__restrict__ out = a.out + job * a.out_job_stride;
    mllm_xq xq = a.xq;
    const long q_job = job * a.x_job_stride;          // elements
    const long b_job = job * (a.x_job_stride / 32);   // 32-blocks

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = lane / LPR, sl = lane % LPR;
    const int row0 = ((blockIdx.x * 4 + wave) * (64 / LPR) + grp) * R;
    const int nb = a.n_cols / q8_traits<SEM>::kBlockElems;
    const int nch = nb * CPB;
    const int B = a.B;

    float acc[R][BM];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < BM; b++) acc[r][b] = 0.0f;

    for (int c = sl; c < nch; c += LPR) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(row0 + r, a.n_rows - 1);
#pragma unroll
            for (int b = 0; b < BM; b++) {
                if (b < B) {
                    const long tq = q_job + (long)b * a.ldx;
                    const long tb = b_job + (long)b * (a.ldx / 32);
                    acc[r][b] += q8_chunk_dot<SEM>(W, nb, row, c, xq, tq, tb);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int b = 0; b < BM; b++) {
            float v = group_sum<LPR>(acc[r][b]);
            const int row = row0 + r;
            if (sl == 0 && row < a.n_rows && b < B) out[(long)b * a.ldo + row] = v;
        }
    }
}

// f32_matmul_omp (QK:884-913): plain fp32 rows, any n_cols.
template <int BM>
__global__ __launch_bounds__(256) void k_gemv_f32(mllm_gemv_args a)
{
    const int job = blockIdx.y;
    const float *Wf = reinterpret_cast<const float *>(a.table ? a.table[a.idx ? a.idx[job] : job].p[0] : a.W.p[0]);
    const float *x = a.x + job * a.x_job_stride;
    float *out = a.out + job * a.out_job_stride;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = blockIdx.x * 4 + wave;
    if (row >= a.n_rows) return;
    const float *w = Wf + (long)row * a.n_cols;
    float acc[BM];
#pragma unroll
    for (int b = 0; b < BM; b++) acc[b] = 0.f;
    for (int i = lane; i < a.n_cols; i += 64) {
        float wv = w[i];
#pragma unroll
        for (int b = 0; b < BM; b++)
            if (b < a.B) acc[b] = fmaf(wv, x[(long)b * a.ldx + i], acc[b]);
    }
#pragma unroll
    for (int b = 0; b < BM; b++) {
        float v = group_sum<64>(acc[b]);
        if (lane == 0 && b < a.B) out[(long)b * a.ldo + row] = v;
    }
}

template <int SEM, int BM>
void launch_sem(const mllm_gemv_args &a, int n_jobs, hipStream_t st)
{
    // Lanes per row: enough chunks per lane to keep every lane busy on short rows.
    const int nch = (mllm_sem_uses_q8(SEM) ? (a.n_cols / q8_traits<SEM>::kBlockElems) * q8_traits<SEM>::kChunksPerBlock
                                           : (a.n_cols / sem_traits<SEM>::kBlockElems) * sem_traits<SEM>::kChunksPerBlock);
    constexpr int R = (BM <= 2) ? 4 : 2;
    auto waste = [&](int lpr) { int it = (nch + lpr - 1) / lpr; return (double)(it * lpr - nch) / (it * lpr); };
    int lpr = 64;
    if (nch < 64 || waste(64) > waste(32) + 0.05) lpr = 32;
    if (nch < 32 || (lpr == 32 && waste(32) > waste(16) + 0.05)) lpr = 16;
    const int rows_per_wg = 4 * (64 / lpr) * R;
    dim3 grid((a.n_rows + rows_per_wg - 1) / rows_per_wg, n_jobs);
    if constexpr (mllm_sem_uses_q8(SEM)) {
        if (lpr == 64) hipLaunchKernelGGL((k_gemv_q8<SEM, BM, R, 64>), grid, dim3(256), 0, st, a);
        else if (lpr == 32) hipLaunchKernelGGL((k_gemv_q8<SEM, BM, R, 32>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((k_gemv_q8<SEM, BM, R, 16>), grid, dim3(256), 0, st, a);
    } else {
        if (lpr == 64) hipLaunchKernelGGL((k_gemv<SEM, BM, R, 64>), grid, dim3(256), 0, st, a);
        else if (lpr == 32) hipLaunchKernelGGL((k_gemv<SEM, BM, R, 32>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((k_gemv<SEM, BM, R, 16>), grid, dim3(256), 0, st, a);
    }
}

template <int BM>
void launch_bm(int sem, const mllm_gemv_args &a, int n_jobs, hipStream_t st)
{
    switch (sem) {
    case SEM_F32: {
        dim3 grid((a.n_rows + 3) / 4, n_jobs);
        hipLaunchKernelGGL((k_gemv_f32<BM>), grid, dim3(256), 0, st, a);
        break;
    }
    case SEM_Q4_0: launch_sem<SEM_Q4_0, BM>(a, n_jobs, st); break;
    case SEM_Q4_1: launch_sem<SEM_Q4_1, BM>(a, n_jobs, st); break;
    case SEM_Q5_0_F32: launch_sem<SEM_Q5_0_F32, BM>(a, n_jobs, st); break;
    case SEM_Q5_0_Q8: launch_sem<SEM_Q5_0_Q8, BM>(a, n_jobs, st); break;
    case SEM_Q8_0: launch_sem<SEM_Q8_0, BM>(a, n_jobs, st); break;
    case SEM_Q4_K_GGML: launch_sem<SEM_Q4_K_GGML, BM>(a, n_jobs, st); break;
    case SEM_Q4_K_Q8: launch_sem<SEM_Q4_K_Q8, BM>(a, n_jobs, st); break;
    case SEM_Q5_K_GGML: launch_sem<SEM_Q5_K_GGML, BM>(a, n_jobs, st); break;
    case SEM_Q5_K_CE: launch_sem<SEM_Q5_K_CE, BM>(a, n_jobs, st); break;
    case SEM_Q6_K_GGML: launch_sem<SEM_Q6_K_GGML, BM>(a, n_jobs, st); break;
    case SEM_Q6_K_LOWNIB: launch_sem<SEM_Q6_K_LOWNIB, BM>(a, n_jobs, st); break;
    case SEM_Q6_K_SEQ: launch_sem<SEM_Q6_K_SEQ, BM>(a, n_jobs, st); break;
    case SEM_MXFP4: launch_sem<SEM_MXFP4, BM>(a, n_jobs, st); break;
    case SEM_MXFP4_CLAMP: launch_sem<SEM_MXFP4_CLAMP, BM>(a, n_jobs, st); break;
    case SEM_MXFP4_Q8: launch_sem<SEM_MXFP4_Q8, BM>(a, n_jobs, st); break;
    default: break;
    }
}

// Dequantise rows to fp32 the way the reference's *_dequantize_row functions
// round: w = fl(s*q) + o, two roundings (QK:762-878).
template <int SEM>
__global__ __launch_bounds__(256) void k_dequant(mllm_packed W, int n_rows, int n_cols, float *__restrict__ out)
{
    constexpr int CPB = sem_traits<SEM>::kChunksPerBlock;
    const int nb = n_cols / sem_traits<SEM>::kBlockElems, nch = nb * CPB;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)n_rows * nch) return;
    const int row = (int)(i / nch), c = (int)(i % nch);
    mllm_chunk k;
    load_chunk<SEM>(W, nb, row, c, k);
    float *o = out + (long)row * n_cols;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        o[k.x0 + j] = __fadd_rn(__fmul_rn(k.s0, k.q[j]), k.o0);
        o[k.x1 + j] = __fadd_rn(__fmul_rn(k.s1, k.q[16 + j]), k.o1);
    }
}

template <int SEM>
hipError_t launch_dequant(const mllm_packed &W, int n_rows, int n_cols, float *out, hipStream_t st)
{
    const long n = (long)n_rows * (n_cols / sem_traits<SEM>::kBlockElems) * sem_traits<SEM>::kChunksPerBlock;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_dequant<SEM>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, W, n_rows, n_cols, out);
    return hipGetLastError();
}

} // namespace

int mllm_launch_dequant(int sem, const mllm_packed &W, int n_rows, int n_cols, float *out, hipStream_t st)
{
    hipError_t r;
    switch (sem) {
    case SEM_Q4_0: r = launch_dequant<SEM_Q4_0>(W, n_rows, n_cols, out, st); break;
    case SEM_Q4_1: r = launch_dequant<SEM_Q4_1>(W, n_rows, n_cols, out, st); break;
    case SEM_Q5_0_F32: r = launch_dequant<SEM_Q5_0_F32>(W, n_rows, n_cols, out, st); break;
    case SEM_Q8_0: r = launch_dequant<SEM_Q8_0>(W, n_rows, n_cols, out, st); break;
    case SEM_Q4_K_GGML: r = launch_dequant<SEM_Q4_K_GGML>(W, n_rows, n_cols, out, st); break;
    case SEM_Q5_K_GGML: r = launch_dequant<SEM_Q5_K_GGML>(W, n_rows, n_cols, out, st); break;
    case SEM_Q5_K_CE: r = launch_dequant<SEM_Q5_K_CE>(W, n_rows, n_cols, out, st); break;
    case SEM_Q6_K_GGML: r = launch_dequant<SEM_Q6_K_GGML>(W, n_rows, n_cols, out, st); break;
    case SEM_Q6_K_LOWNIB: r = launch_dequant<SEM_Q6_K_LOWNIB>(W, n_rows, n_cols, out, st); break;
    case SEM_Q6_K_SEQ: r = launch_dequant<SEM_Q6_K_SEQ>(W, n_rows, n_cols, out, st); break;
    case SEM_MXFP4: r = launch_dequant<SEM_MXFP4>(W, n_rows, n_cols, out, st); break;
    case SEM_MXFP4_CLAMP: r = launch_dequant<SEM_MXFP4_CLAMP>(W, n_rows, n_cols, out, st); break;
    default: return -1;   // F32 and the Q8_0-activation semantics have no fp32 weight form
    }
    return r == hipSuccess ? 0 : -1;
}

// B in 1..8; larger batches are split by the caller.
hipError_t mllm_launch_gemv(int sem, const mllm_gemv_args &a, int n_jobs, hipStream_t st)
{
    if (a.B <= 0 || a.n_rows <= 0 || n_jobs <= 0) return hipSuccess;
    if (a.B == 1) launch_bm<1>(sem, a, n_jobs, st);
    else if (a.B == 2) launch_bm<2>(sem, a, n_jobs, st);
    else if (a.B <= 4) launch_bm<4>(sem, a, n_jobs, st);
    else if (a.B <= 8) launch_bm<8>(sem, a, n_jobs, st);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}
