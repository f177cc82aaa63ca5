// gemv_fkq.hip — fused decode GEMV instantiations (prologue / paired rows): SEM_Q4_K_GGML, SEM_Q4_K_Q8.
#include "gemv_impl.h"

namespace mllm_gemv {
MLLM_GEMV_FUSED_INSTANTIATE(SEM_Q4_K_GGML)
MLLM_GEMV_FUSED_INSTANTIATE(SEM_Q4_K_Q8)
} // namespace mllm_gemv
