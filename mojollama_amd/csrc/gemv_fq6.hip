// gemv_fq6.hip — fused decode GEMV instantiations (prologue / paired rows): SEM_Q6_K_GGML, SEM_Q6_K_LOWNIB, SEM_Q6_K_SEQ.
#include "gemv_impl.h"

namespace mllm_gemv {
MLLM_GEMV_FUSED_INSTANTIATE(SEM_Q6_K_GGML)
MLLM_GEMV_FUSED_INSTANTIATE(SEM_Q6_K_LOWNIB)
MLLM_GEMV_FUSED_INSTANTIATE(SEM_Q6_K_SEQ)
} // namespace mllm_gemv
