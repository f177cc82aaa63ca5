// dropin.h — the drop-in entry points' shared host-side services (capi.hip),
// used by the model drivers in other translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <shared_mutex>
#include "mllm_common.h"

// Packed device copy of a raw host matrix (GGUF block bytes, rows x cols)
// under semantic `sem`, uploaded once per host pointer through the weight
// cache and re-uploaded when a fingerprint of its bytes changes.  The device
// copy stays until mllm_cache_clear().  gemv_only (optional): the matrix's
// block scales keep it on the GEMV path at every batch
// (mllm_scales_need_gemv).  Returns 0, or -1 with the error recorded.
int mllm_dropin_weight(const void *host, int sem, int rows, int cols, mllm_packed *view, bool *gemv_only);

// The semantic the reference gives GGUF code qt on quant_matmul_omp (QK:1355-1388), -1 if none.
int mllm_qmm_sem(int qt);

// Drop-in calls hold this shared for their whole duration; mllm_cache_clear
// takes it exclusively before it frees anything.
std::shared_mutex &mllm_api_mutex();

// Frees the models and mirrors qwen36_batch_forward and the SSM drop-ins keep (part of mllm_cache_clear).
void mllm_qwen36_cache_clear();
