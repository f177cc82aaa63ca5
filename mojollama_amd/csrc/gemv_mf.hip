// gemv_mf.hip — launch plan and dispatch of the batch 2..8 MFMA decode GEMV
// (kernels in gemv_mf.h, instantiated per semantic in gemv_mf_*.hip).
#include "gemv_mf.h"

using namespace mllm_gemv;

namespace mllm_gemv {
template <int SEM> hipError_t gemv_mf_sem(const mllm_gemv_args &a, int BM, int n_tiles, int S, size_t lds, hipStream_t st);
}

namespace {

struct mf_plan {
    bool ok;
    int BM, S, n_tiles;
    size_t lds;
};

bool mf_sem_ok(int sem)
{
    return sem == SEM_Q4_K_GGML || sem == SEM_Q6_K_SEQ || sem == SEM_Q8_0 || sem == SEM_Q4_0 || sem == SEM_MXFP4 ||
           sem == SEM_MXFP4_CLAMP;
}
int mf_group(int sem) { return sem == SEM_Q6_K_SEQ ? 16 : 32; }

// Batch from which the MFMA form beats the VALU kernel on its own (measured on
// MI355X over TinyLlama / GPT-OSS shapes: the MFMA kernel's time hardly grows
// with B, the VALU kernel's grows per token).  Paired gate/up rows at B > 1
// exist only here.
int mf_min_batch(int sem, int n_rows)
{
    if (sem == SEM_Q6_K_SEQ && n_rows <= 4096) return 3;   // the down projection; not the 32000-row lm_head
    return sem == SEM_Q8_0 ? 7 : 5;
}
int mf_block(int sem) { return (sem == SEM_Q4_K_GGML || sem == SEM_Q6_K_SEQ) ? 256 : 32; }

// S: the fewest K splits whose range fits the LDS budget, raised (up to 8
// and one 256-element block per split) until rows x splits give a tile per
// CU; without a partials buffer only S = 1.
mf_plan mf_plan_for(int sem, int n_rows, int n_cols, int B, bool pro, bool pair, bool have_part)
{
    mf_plan p{};
    if (!mf_sem_ok(sem) || B < 2 || B > 8 || n_rows <= 0 || (!pair && B < mf_min_batch(sem, n_rows))) return p;
    const int BE = mf_block(sem), nb = n_cols / BE;
    if (nb < 1) return p;
    p.BM = B <= 2 ? 2 : B <= 4 ? 4 : 8;
    p.n_tiles = pair ? (n_rows + 15) / 16 : (n_rows + 31) / 32;
    const int cus = device_cus();
    auto lds_for = [&](int S) {
        const int kn = (nb + S - 1) / S * BE;
        return (size_t)mf_geom_for(p.BM, mf_group(sem), kn, pro).total;
    };
    int S = 1;
    const int smax = std::min(nb, kMfMaxSplits);
    while (S < smax && lds_for(S) > (size_t)kMfLdsCap) S++;
    if (lds_for(S) > (size_t)kMfLdsCap) return p;
    while (S < smax && (long)p.n_tiles * S < cus) S++;
    if (!have_part) {
        if (lds_for(1) > (size_t)kMfLdsCap) return p;
        S = 1;
    }
    p.S = S;
    p.lds = lds_for(S);
    p.ok = true;
    return p;
}

} // namespace

bool mllm_gemv_mf_fits(int sem, int n_rows, int n_cols, int B, bool pro, bool pair, bool have_part)
{
    return mf_plan_for(sem, n_rows, n_cols, B, pro, pair, have_part).ok;
}

long mllm_gemv_mf_part_floats(int sem, int n_rows, int n_cols, int B, bool pro, bool pair)
{
    const mf_plan p = mf_plan_for(sem, n_rows, n_cols, B, pro, pair, true);
    if (!p.ok || p.S == 1) return 0;
    const long nre = pair ? 2L * n_rows : n_rows;
    return (long)p.S * B * nre + (long)p.S * B;
}

hipError_t mllm_launch_gemv_mf(int sem, const mllm_gemv_args &a, hipStream_t st)
{
    const bool pro = mllm_has_prologue(a), pair = a.silu_pair != 0;
    if (a.table || a.x_up || a.xq.q || a.job_split > 0) return hipErrorNotSupported;
    // the prologue's norm covers whole blocks
    if (!mf_sem_ok(sem) || (pro && a.n_cols % mf_block(sem))) return hipErrorNotSupported;
    if ((a.ldx & 3) || ((uintptr_t)a.x & 15)) return hipErrorNotSupported;
    const mf_plan p = mf_plan_for(sem, a.n_rows, a.n_cols, a.B, pro, pair, a.mf_part != nullptr);
    if (!p.ok) return hipErrorNotSupported;
    hipError_t r;
    switch (sem) {
    case SEM_Q4_K_GGML: r = gemv_mf_sem<SEM_Q4_K_GGML>(a, p.BM, p.n_tiles, p.S, p.lds, st); break;
    case SEM_Q6_K_SEQ: r = gemv_mf_sem<SEM_Q6_K_SEQ>(a, p.BM, p.n_tiles, p.S, p.lds, st); break;
    case SEM_Q8_0: r = gemv_mf_sem<SEM_Q8_0>(a, p.BM, p.n_tiles, p.S, p.lds, st); break;
    case SEM_Q4_0: r = gemv_mf_sem<SEM_Q4_0>(a, p.BM, p.n_tiles, p.S, p.lds, st); break;
    case SEM_MXFP4: r = gemv_mf_sem<SEM_MXFP4>(a, p.BM, p.n_tiles, p.S, p.lds, st); break;
    default: r = gemv_mf_sem<SEM_MXFP4_CLAMP>(a, p.BM, p.n_tiles, p.S, p.lds, st); break;
    }
    if (r != hipSuccess) return r;
    if (p.S > 1) {
        const dim3 rg((unsigned)(((long)a.B * a.n_rows + 255) / 256));
        if (pair) hipLaunchKernelGGL(k_mf_reduce<true>, rg, dim3(256), 0, st, a, p.S);
        else hipLaunchKernelGGL(k_mf_reduce<false>, rg, dim3(256), 0, st, a, p.S);
    }
    return hipGetLastError();
}
