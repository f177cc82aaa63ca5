// gemv.hip — dispatch of the decode GEMV (kernels in gemv_impl.h, instantiated
// per semantic in gemv_*.hip) and of the fp32-row dequantiser.
#include "gemv_impl.h"

using namespace mllm_gemv;

namespace {

void launch_f32(const mllm_gemv_args &a, int n_jobs, hipStream_t st)
{
    dim3 grid((a.n_rows + 3) / 4, n_jobs);
    if (a.B == 1) hipLaunchKernelGGL(k_gemv_f32<1>, grid, dim3(256), 0, st, a);
    else if (a.B == 2) hipLaunchKernelGGL(k_gemv_f32<2>, grid, dim3(256), 0, st, a);
    else if (a.B <= 4) hipLaunchKernelGGL(k_gemv_f32<4>, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(k_gemv_f32<8>, grid, dim3(256), 0, st, a);
}

// Rows of a matrix with fewer columns than one quant block: the reference's
// dot products run over n_cols / block = 0 blocks and give 0, so every output
// row of every job and token is written 0 (no weight or activation is read).
__global__ void k_gemv_zero(mllm_gemv_args a)
{
    const int job = blockIdx.y;
    const bool second = a.job_split > 0 && job >= a.job_split;
    float *out = (second ? a.out2 : a.out) + (long)(second ? job - a.job_split : job) * a.out_job_stride;
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= a.n_rows) return;
    for (int b = 0; b < a.B; b++) out[(long)b * a.ldo + r] = a.out_add ? a.out_add[(long)b * a.ldo + r] : 0.0f;
}

} // namespace

bool mllm_gemv_fused_fits(int sem, int n_cols, int B, bool prologue)
{
    if (sem == SEM_F32 || B < 1 || B > 8 || n_cols < mllm_sem_block_elems(sem)) return false;
    // the prologue's norm covers the staged elements: whole blocks only
    if (prologue && n_cols % mllm_sem_block_elems(sem)) return false;
    const bool q8 = mllm_sem_uses_q8(sem);
    const int be = mllm_layout_info(mllm_sem_layout(sem)).block_elems;
    const int BM = B == 1 ? 1 : B == 2 ? 2 : B <= 4 ? 4 : 8;
    return persistent_lds(q8, be, n_cols, BM, prologue) <= kPersistentLds;
}

bool mllm_gemv_prologue_fits(int sem, int n_cols, int B) { return mllm_gemv_fused_fits(sem, n_cols, B, true); }

int mllm_sem_block_elems(int sem)
{
    if (sem == SEM_F32) return 1;
    return mllm_layout_info(mllm_sem_layout(sem)).block_elems;
}

int mllm_launch_dequant(int sem, const mllm_packed &W, int n_rows, int n_cols, float *out, hipStream_t st)
{
    hipError_t r;
    switch (sem) {
    case SEM_Q4_0: r = dequant_sem<SEM_Q4_0>(W, n_rows, n_cols, out, st); break;
    case SEM_Q4_1: r = dequant_sem<SEM_Q4_1>(W, n_rows, n_cols, out, st); break;
    case SEM_Q5_0_F32: r = dequant_sem<SEM_Q5_0_F32>(W, n_rows, n_cols, out, st); break;
    case SEM_Q8_0: r = dequant_sem<SEM_Q8_0>(W, n_rows, n_cols, out, st); break;
    case SEM_Q4_K_GGML: r = dequant_sem<SEM_Q4_K_GGML>(W, n_rows, n_cols, out, st); break;
    case SEM_Q5_K_GGML: r = dequant_sem<SEM_Q5_K_GGML>(W, n_rows, n_cols, out, st); break;
    case SEM_Q5_K_CE: r = dequant_sem<SEM_Q5_K_CE>(W, n_rows, n_cols, out, st); break;
    case SEM_Q6_K_GGML: r = dequant_sem<SEM_Q6_K_GGML>(W, n_rows, n_cols, out, st); break;
    case SEM_Q6_K_LOWNIB: r = dequant_sem<SEM_Q6_K_LOWNIB>(W, n_rows, n_cols, out, st); break;
    case SEM_Q6_K_SEQ: r = dequant_sem<SEM_Q6_K_SEQ>(W, n_rows, n_cols, out, st); break;
    case SEM_MXFP4: r = dequant_sem<SEM_MXFP4>(W, n_rows, n_cols, out, st); break;
    case SEM_MXFP4_CLAMP: r = dequant_sem<SEM_MXFP4_CLAMP>(W, n_rows, n_cols, out, st); break;
    default: return -1;   // F32 and the Q8_0-activation semantics have no fp32 weight form
    }
    return r == hipSuccess ? 0 : -1;
}

// B in 1..8; larger batches are split by the caller.
hipError_t mllm_launch_gemv(int sem, const mllm_gemv_args &a, int n_jobs, hipStream_t st)
{
    if (a.B <= 0 || a.n_rows <= 0 || n_jobs <= 0) return hipSuccess;
    if (a.B > 8) return hipErrorInvalidValue;
    // x_up: the SiLU product, formed in the digit staging (fp32-activation
    // semantics, B == 1) or in the in-kernel Q8_0 quantisation (Q8 semantics
    // with no precomputed pack).
    if (a.x_up && (sem == SEM_F32 || (mllm_sem_uses_q8(sem) ? a.xq.q != nullptr : a.B != 1)))
        return hipErrorInvalidValue;
    if (a.job_split > 0 && (a.job_split >= n_jobs || !a.out2 || (a.table && !a.table2))) return hipErrorInvalidValue;
    // batch 2..8 of one matrix: the MFMA form where the semantic has one
    if (a.B >= 2 && n_jobs == 1 && a.n_cols >= mllm_sem_block_elems(sem)) {
        const hipError_t r = mllm_launch_gemv_mf(sem, a, st);
        if (r != hipErrorNotSupported) return r;
    }
    // the fused forms run in the persistent kernel only: the prologue on one
    // matrix with a fp32 activation (or one the kernel quantises itself),
    // paired rows at batch 1
    const bool pro = mllm_has_prologue(a), pair = a.silu_pair != 0;
    if (pro && (a.table || n_jobs != 1 || a.x_up || a.xq.q)) return hipErrorInvalidValue;
    if (pair && (a.B != 1 || a.x_up || a.xq.q || (a.table && !a.table2) || a.job_split > 0)) return hipErrorInvalidValue;
    if ((pro || pair) && !mllm_gemv_fused_fits(sem, a.n_cols, a.B, pro)) return hipErrorInvalidValue;
    if (a.out_add && (a.table || n_jobs != 1)) return hipErrorInvalidValue;
    if (a.n_cols < mllm_sem_block_elems(sem)) {
        hipLaunchKernelGGL(k_gemv_zero, dim3((a.n_rows + 255) / 256, n_jobs), dim3(256), 0, st, a);
        return hipGetLastError();
    }
    if (pro || pair) {
        switch (sem) {
        case SEM_Q4_0: return gemv_fused_sem<SEM_Q4_0>(a, n_jobs, st);
        case SEM_Q4_1: return gemv_fused_sem<SEM_Q4_1>(a, n_jobs, st);
        case SEM_Q5_0_F32: return gemv_fused_sem<SEM_Q5_0_F32>(a, n_jobs, st);
        case SEM_Q5_0_Q8: return gemv_fused_sem<SEM_Q5_0_Q8>(a, n_jobs, st);
        case SEM_Q8_0: return gemv_fused_sem<SEM_Q8_0>(a, n_jobs, st);
        case SEM_Q4_K_GGML: return gemv_fused_sem<SEM_Q4_K_GGML>(a, n_jobs, st);
        case SEM_Q4_K_Q8: return gemv_fused_sem<SEM_Q4_K_Q8>(a, n_jobs, st);
        case SEM_Q5_K_GGML: return gemv_fused_sem<SEM_Q5_K_GGML>(a, n_jobs, st);
        case SEM_Q5_K_CE: return gemv_fused_sem<SEM_Q5_K_CE>(a, n_jobs, st);
        case SEM_Q6_K_GGML: return gemv_fused_sem<SEM_Q6_K_GGML>(a, n_jobs, st);
        case SEM_Q6_K_LOWNIB: return gemv_fused_sem<SEM_Q6_K_LOWNIB>(a, n_jobs, st);
        case SEM_Q6_K_SEQ: return gemv_fused_sem<SEM_Q6_K_SEQ>(a, n_jobs, st);
        case SEM_MXFP4: return gemv_fused_sem<SEM_MXFP4>(a, n_jobs, st);
        case SEM_MXFP4_CLAMP: return gemv_fused_sem<SEM_MXFP4_CLAMP>(a, n_jobs, st);
        case SEM_MXFP4_Q8: return gemv_fused_sem<SEM_MXFP4_Q8>(a, n_jobs, st);
        default: return hipErrorInvalidValue;
        }
    }
    switch (sem) {
    case SEM_F32: launch_f32(a, n_jobs, st); break;
    case SEM_Q4_0: gemv_sem<SEM_Q4_0>(a, n_jobs, st); break;
    case SEM_Q4_1: gemv_sem<SEM_Q4_1>(a, n_jobs, st); break;
    case SEM_Q5_0_F32: gemv_sem<SEM_Q5_0_F32>(a, n_jobs, st); break;
    case SEM_Q5_0_Q8: gemv_sem<SEM_Q5_0_Q8>(a, n_jobs, st); break;
    case SEM_Q8_0: gemv_sem<SEM_Q8_0>(a, n_jobs, st); break;
    case SEM_Q4_K_GGML: gemv_sem<SEM_Q4_K_GGML>(a, n_jobs, st); break;
    case SEM_Q4_K_Q8: gemv_sem<SEM_Q4_K_Q8>(a, n_jobs, st); break;
    case SEM_Q5_K_GGML: gemv_sem<SEM_Q5_K_GGML>(a, n_jobs, st); break;
    case SEM_Q5_K_CE: gemv_sem<SEM_Q5_K_CE>(a, n_jobs, st); break;
    case SEM_Q6_K_GGML: gemv_sem<SEM_Q6_K_GGML>(a, n_jobs, st); break;
    case SEM_Q6_K_LOWNIB: gemv_sem<SEM_Q6_K_LOWNIB>(a, n_jobs, st); break;
    case SEM_Q6_K_SEQ: gemv_sem<SEM_Q6_K_SEQ>(a, n_jobs, st); break;
    case SEM_MXFP4: gemv_sem<SEM_MXFP4>(a, n_jobs, st); break;
    case SEM_MXFP4_CLAMP: gemv_sem<SEM_MXFP4_CLAMP>(a, n_jobs, st); break;
    case SEM_MXFP4_Q8: gemv_sem<SEM_MXFP4_Q8>(a, n_jobs, st); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
