// dense16.h — the prefill GEMM over a load-time fp16 copy of a quantised
// matrix (dense16.hip).
#pragma once
#include <string>
#include <hip/hip_runtime.h>
#include "mllm_common.h"

long mllm_d16_bytes(int n_rows, int n_cols);
// Dequantise (the fp32-weight semantics' *_dequantize_row arithmetic) and round
// to fp16 into w16 [n_rows][n_cols]; synchronises `st`.  Fails when a weight
// is not finite in fp16.
int mllm_d16_make(int sem, const mllm_packed &W, int n_rows, int n_cols, void *w16, hipStream_t st, std::string &err);
long mllm_d16_workspace_bytes(int n_rows, int n_cols, int M);
// out[t][r] (stride ldo) = w16 row r . x[t] (stride ldx), t < M.  The first call
// per shape on a device builds the hipBLASLt plan (not capturable); later
// calls launch only.
int mllm_d16_gemm(const void *w16, const float *x, int ldx, int M, float *out, int ldo, int n_rows, int n_cols,
                  void *ws, long ws_bytes, hipStream_t st, std::string &err);
