// gemm.h — launch interface of the quantised-weight MFMA GEMM (gemm.hip).
#pragma once
#include <hip/hip_runtime.h>
#include "mllm_common.h"

// Activation source of the GEMM's B operand.
enum { XM_F32 = 0,   // fp32 rows x[row][k] (split into bf16 hi + lo)
       XM_Q8 = 1,    // Q8_0 quants, exact in bf16 (Q4_K_Q8)
       XM_Q8D = 2 }; // Q8_0 quants times their block scale (MXFP4_Q8)

// out[out_row(p)][n] = sum_k w[n][k] * b[row_of(p)][k] for entries p of each
// work tile and weight rows n < n_rows.  Work tiles are either the
// consecutive 64-entry slices of [0, n_entries) (tile_expert == nullptr), or
// the device list (tile_expert[t], tile_begin[t], tile_end[t]) for t < *n_tiles
// that picks table[tile_expert[t]] as the weight matrix (grouped expert GEMM).
// dual: two matrices (gate W/table, up W2/table2) share the tile and the
// epilogue stores silu(gate) * up (gate clamped to +-80 when clamp_silu).
struct qgemm_args {
    mllm_packed W, W2;
    const mllm_packed *table, *table2;
    const float *x;        // XM_F32 rows
    int ldx;
    mllm_xq xq;            // XM_Q8 / XM_Q8D rows (row stride n_cols rounded down to 32)
    const int *row_of;     // entry -> activation row (nullptr: identity)
    float *out;
    int ldo;
    const int *out_row;    // entry -> output row (nullptr: identity)
    int n_rows, n_cols;
    int n_entries;
    const int *tile_expert, *tile_begin, *tile_end, *n_tiles;
    int clamp_silu;
};

hipError_t mllm_launch_qgemm(int sem, int xmode, bool dual, const qgemm_args &a, int max_tiles, hipStream_t st);
bool mllm_qgemm_supported(int sem);
