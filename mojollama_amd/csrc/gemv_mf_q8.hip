// gemv_mf_q8.hip — batch 2..8 MFMA decode GEMV instantiations: SEM_Q8_0, SEM_Q4_0.
#include "gemv_mf.h"

namespace mllm_gemv {

// Workgroups resident per CU for one instantiation at this LDS size (asked
// of the runtime, which accounts for the kernel's registers too).
template <class K>
static int mf_per_cu(K kernel, size_t lds)
{
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, kMfThreads, lds) != hipSuccess || n < 1) n = 1;
    return n;
}

// The grid is persistent: no more workgroups per split than stay resident,
// each walking row tiles x, x + gridDim.x, ...
template <int SEM, int BM, bool PRO, bool PAIR>
static void launch_mf(const mllm_gemv_args &a, int n_tiles, int S, size_t lds, hipStream_t st)
{
    const auto kernel = k_gemv_mf<SEM, BM, PRO, PAIR>;
    const int gx = std::max(1, std::min(n_tiles, device_cus() * mf_per_cu(kernel, lds) / S));
    hipLaunchKernelGGL(kernel, dim3(gx, S), dim3(kMfThreads), lds, st, a);
}

template <int SEM, int BM>
static void launch_mf_bm(const mllm_gemv_args &a, int n_tiles, int S, size_t lds, hipStream_t st)
{
    const bool pro = mllm_has_prologue(a), pair = a.silu_pair != 0;
    if (pro && pair) launch_mf<SEM, BM, true, true>(a, n_tiles, S, lds, st);
    else if (pro) launch_mf<SEM, BM, true, false>(a, n_tiles, S, lds, st);
    else if (pair) launch_mf<SEM, BM, false, true>(a, n_tiles, S, lds, st);
    else launch_mf<SEM, BM, false, false>(a, n_tiles, S, lds, st);
}

template <int SEM> hipError_t gemv_mf_sem(const mllm_gemv_args &a, int BM, int n_tiles, int S, size_t lds, hipStream_t st);

template <>
hipError_t gemv_mf_sem<SEM_Q8_0>(const mllm_gemv_args &a, int BM, int n_tiles, int S, size_t lds, hipStream_t st)
{
    if (BM == 2) launch_mf_bm<SEM_Q8_0, 2>(a, n_tiles, S, lds, st);
    else if (BM == 4) launch_mf_bm<SEM_Q8_0, 4>(a, n_tiles, S, lds, st);
    else launch_mf_bm<SEM_Q8_0, 8>(a, n_tiles, S, lds, st);
    return hipGetLastError();
}

template <>
hipError_t gemv_mf_sem<SEM_Q4_0>(const mllm_gemv_args &a, int BM, int n_tiles, int S, size_t lds, hipStream_t st)
{
    if (BM == 2) launch_mf_bm<SEM_Q4_0, 2>(a, n_tiles, S, lds, st);
    else if (BM == 4) launch_mf_bm<SEM_Q4_0, 4>(a, n_tiles, S, lds, st);
    else launch_mf_bm<SEM_Q4_0, 8>(a, n_tiles, S, lds, st);
    return hipGetLastError();
}

} // namespace mllm_gemv
