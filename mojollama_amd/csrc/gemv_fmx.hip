// gemv_fmx.hip — fused decode GEMV instantiations (prologue / paired rows): SEM_MXFP4, SEM_MXFP4_CLAMP, SEM_MXFP4_Q8.
#include "gemv_impl.h"

namespace mllm_gemv {
MLLM_GEMV_FUSED_INSTANTIATE(SEM_MXFP4)
MLLM_GEMV_FUSED_INSTANTIATE(SEM_MXFP4_CLAMP)
MLLM_GEMV_FUSED_INSTANTIATE(SEM_MXFP4_Q8)
} // namespace mllm_gemv
