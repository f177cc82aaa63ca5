// gemv_fk5.hip — fused decode GEMV instantiations (prologue / paired rows): SEM_Q5_K_GGML, SEM_Q5_K_CE.
#include "gemv_impl.h"

namespace mllm_gemv {
MLLM_GEMV_FUSED_INSTANTIATE(SEM_Q5_K_GGML)
MLLM_GEMV_FUSED_INSTANTIATE(SEM_Q5_K_CE)
} // namespace mllm_gemv
