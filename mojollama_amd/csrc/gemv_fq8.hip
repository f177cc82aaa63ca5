// gemv_fq8.hip — fused decode GEMV instantiations (prologue / paired rows): SEM_Q8_0, SEM_Q4_0, SEM_Q4_1.
#include "gemv_impl.h"

namespace mllm_gemv {
MLLM_GEMV_FUSED_INSTANTIATE(SEM_Q8_0)
MLLM_GEMV_FUSED_INSTANTIATE(SEM_Q4_0)
MLLM_GEMV_FUSED_INSTANTIATE(SEM_Q4_1)
} // namespace mllm_gemv
