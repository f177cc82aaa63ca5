// gemm.h — launch interface of the quantised-weight MFMA GEMM (gemm.hip).
#pragma once
#include <hip/hip_runtime.h>
#include "mllm_common.h"

// Activation source of the GEMM's B operand.
enum { XM_PLANES = 0, // fp32 rows pre-split into bf16 hi + lo planes (mllm_launch_act_split)
       XM_Q8 = 1,     // Q8_0 quants, exact in bf16 (Q4_K_Q8)
       XM_Q8D = 2 };  // Q8_0 quants times their block scale (MXFP4_Q8)

// Split-activation planes of `rows` fp32 rows of K columns: x = p0 + p1 (+ p2),
// each plane the bf16 rounding of what the previous ones leave.  Plane p at
// base + p * plane elements, row r at r * ldp, ldp = K rounded up to 64 (zero
// padded), so a row's planes are 16-byte aligned; lo_nz[r] != 0 when row r is
// not bf16-exact (a plane past the first has a non-zero element).  Weights
// exact in one bf16 (MXFP4) take three planes, which makes their products
// exact; the others two.
struct act_planes {
    const __bf16 *base;
    long plane;
    int ldp;
    const int *lo_nz;
};
inline int act_planes_ld(int K) { return (K + 63) / 64 * 64; }
inline long act_planes_elems(long rows, int K) { return rows * (long)act_planes_ld(K); }
inline int act_nplanes(int sem) { return (sem == SEM_MXFP4 || sem == SEM_MXFP4_CLAMP) ? 3 : 2; }
hipError_t mllm_launch_act_split(const float *x, int ldx, int rows, int K, int nplanes, __bf16 *base, long plane,
                                 int *lo_nz, hipStream_t st);

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
    act_planes xp;         // XM_PLANES rows
    mllm_xq xq;            // XM_Q8 / XM_Q8D rows (row stride n_cols rounded down to 32)
    const int *row_of;     // entry -> activation row (nullptr: identity)
    float *out;
    int ldo;
    const int *out_row;    // entry -> output row (nullptr: identity)
    int n_rows, n_cols;
    int n_entries;
    const int *tile_expert, *tile_begin, *tile_end, *n_tiles;
    int clamp_silu;
    // split K (dense launches): ksplit > 1 workgroups per output tile each sum a
    // contiguous range of K steps into part[z][entry][row]; a second kernel adds
    // the ksplit partials in order into out.
    int ksplit;
    float *part;
    // dense_ld > 0: W / W2 / table entries hold p[0] = the matrix's bf16 planes
    // (mllm_launch_dense_planes: [planes][n_rows][dense_ld], dense_ld a
    // multiple of 64, zero padded), copied into the tiles instead of decoded.
    int dense_ld;
};

hipError_t mllm_launch_qgemm(int sem, int xmode, bool dual, const qgemm_args &a, int max_tiles, hipStream_t st);
// Split count chosen for a dense launch and the partial buffer it needs (floats).
int mllm_qgemm_ksplit(int sem, int n_rows, int n_cols, int n_entries);
inline long mllm_qgemm_part_floats(int sem, int n_rows, int n_cols, int n_entries)
{
    const int ks = mllm_qgemm_ksplit(sem, n_rows, n_cols, n_entries);
    return ks > 1 ? (long)ks * n_entries * n_rows : 0;
}
bool mllm_qgemm_supported(int sem);
// Dense bf16 copies for the tiles (qgemm_args.dense_ld): the number of planes
// a semantic's copy holds (0: not offered), and the copy itself, [planes]
// [n_rows][ldw] (ldw a multiple of 64 >= n_cols; columns past the last block
// are not written: clear the buffer first).
int mllm_dense_planes(int sem);
hipError_t mllm_launch_dense_planes(int sem, const mllm_packed &W, int n_rows, int n_cols, int ldw, __bf16 *out,
                                    hipStream_t st);
