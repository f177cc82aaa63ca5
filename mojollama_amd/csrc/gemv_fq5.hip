// gemv_fq5.hip — fused decode GEMV instantiations (prologue / paired rows): SEM_Q5_0_F32, SEM_Q5_0_Q8.
#include "gemv_impl.h"

namespace mllm_gemv {
MLLM_GEMV_FUSED_INSTANTIATE(SEM_Q5_0_F32)
MLLM_GEMV_FUSED_INSTANTIATE(SEM_Q5_0_Q8)
} // namespace mllm_gemv
