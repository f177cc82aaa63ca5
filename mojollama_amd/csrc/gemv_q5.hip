// gemv_q5.hip — decode GEMV instantiations: Q5_0_F32, Q5_0_Q8.
#include "gemv_impl.h"

namespace mllm_gemv {
MLLM_GEMV_INSTANTIATE(SEM_Q5_0_F32)
MLLM_DEQUANT_INSTANTIATE(SEM_Q5_0_F32)
MLLM_GEMV_INSTANTIATE(SEM_Q5_0_Q8)
} // namespace mllm_gemv
