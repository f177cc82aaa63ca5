// gemm16.h — the K-quant GEMM on one exact fp16 weight plane (gemm16.hip).
//
// For Q4_K (ggml: CE:255-313; and dot_q4_k_q8_0's integer term: QK:1647-1735)
// and Q6_K (sequential: CE:315-378; low-nibble: QK:1778-1903) the weight of
// element k of super-block b is d_b * c_k - dmin_b * m_j(k) (Q4_K ggml) or
// d_b * c_k (Q6_K, and Q4_K's integer term), where the integer c_k =
// sc_j * q_k (Q4_K: <= 63 * 15 = 945) or sc_j * (q_k - 32) (Q6_K: |.| <= 1024)
// is exact in fp16.  The GEMM multiplies those integers on
// v_mfma_f32_32x32x16_f16 against fp16 activation planes, sums each
// super-block's products in fp32, then applies d_b per row in fp32; Q4_K
// ggml's min term, sum_j dmin_b m_j S_j with S_j the activation's sum over
// sub-block j, and dot_q4_k_q8_0's, sum_b dmin_b u_b, run as a second small
// MFMA product over those sums.  One MFMA per weight-activation pair where
// the activation is exact in one fp16 plane (bf16 or Q8_0 inputs), two
// otherwise -- against two bf16 planes on each side before.
//
// MXFP4 (one 32-element block per lane and step, its E8M0 scale folded into
// the fp16 weights) runs on the same loop without per-super-block scales.
//
// Activations (mllm_launch_act16) are rows of fp16 in the MFMA's K order for
// the semantic (each 64-position step of a row holds the elements a lane's
// decoded weights meet, so weights decode straight into MFMA registers), the
// fp32 rows scaled by a power of two per row so the largest element lies in
// [2^8, 2^9): x*s = h0 + h1 (h1 the fp16 rounding of the remainder; lo_nz[r]
// when some h1 of row r is non-zero), with the min-term sums beside them.
#pragma once
#include <hip/hip_runtime.h>
#include "mllm_common.h"

// Whether the fp16-plane GEMM serves a semantic.
bool mllm_q16_supported(int sem);

// MXFP4 on the fp16 plane (grouped expert GEMMs): a weight v 2^(E-127)
// (QK:683-720, 629-678) decodes as the fp16 v 2^(E + eoff), exact when every
// non-zero exponent E of the launch's matrices lies in [emax - 25, emax] with
// eoff = 5 - emax; the result is scaled by wscale = 2^(-127 - eoff).
// mllm_q16_mx: the MXFP4 semantics the GEMM serves (SEM_MXFP4 against fp32
// activations, SEM_MXFP4_Q8 against the dequantised Q8_0 pack).
bool mllm_q16_mx(int sem);
// ORs the exponent range of n_mats MXFP4 matrices (device table) into
// range[0] (smallest non-zero E, start at 255) and range[1] (largest, start at 0).
hipError_t mllm_launch_mx_erange(const mllm_packed *tab_dev, int n_mats, int n_rows, int n_cols, int *range,
                                 hipStream_t st);
// eoff / wscale for an exponent range; false when the range does not fit.
bool mllm_q16_mx_shift(int emin, int emax, int *eoff, float *wscale);
// Step-major metadata: a matrix's per-block metadata transposed so the rows of one
// super-block are contiguous (a wave's 32 rows read one short run instead of 32 scattered
// lines).  Records (b, row) at (b * n_rows + row) * R: Q4_K its 16-byte d / dmin / scales
// record (R = 16); Q6_K its 16 sub-block scales (R = 16), then at sm_doff its d (R = 2);
// MXFP4 per 64-element step b the E bytes of blocks 2b, 2b+1 (R = 2).  Bytes per matrix
// (256-aligned) and the d offset; 0 for semantics without a form.
long mllm_q16_smeta_bytes(int sem, int n_rows, int n_cols, long *doff);
// The copies of n_mats matrices (device table), matrix m at dst + m * stride.
hipError_t mllm_launch_q16_smeta(int sem, const mllm_packed *tab_dev, int n_mats, int n_rows, int n_cols, uint8_t *dst,
                                 long stride, hipStream_t st);

// The activation rows of the fp16-plane GEMM (a workspace carve).
struct act16 {
    _Float16 *h;       // [nplanes][rows][ldh]: K positions in the semantic's MFMA order
    long hplane;
    int ldh;
    _Float16 *m;       // [2][rows][ldm]: min-term sums (Q4_K ggml: sub-blocks; Q4_K x Q8_0: super-blocks), or null
    long mplane;
    int ldm;
    float *inv_s;      // [rows]: 1 / the row's power-of-two scale (Q4_K x Q8_0: 1)
    float *inv_m;      // [rows]: 1 / the min-term planes' scale (Q4_K x Q8_0)
    int *lo_nz;        // [rows]: the second plane holds a non-zero element
    _Float16 *zero;    // [ldh] zeros: the second-plane row of rows whose lo_nz is 0 (whose row may be unwritten)
};
size_t mllm_act16_bytes(int sem, long rows, int K);
act16 mllm_act16_carve(int sem, void *ws, long rows, int K);
// fp32 rows x[r * ldx + k] (fp32-activation semantics; MXFP4 x Q8_0: their Q8_0
// quantisation, quants times block scales), or the Q8_0 pack xq (Q4_K x Q8_0:
// mllm_launch_quantize_q8_0's quants and min-term sums) -> act.
hipError_t mllm_launch_act16(int sem, const float *x, int ldx, const mllm_xq *xq, int rows, int K, const act16 &act,
                             hipStream_t st);

// out[out_row(p)][n] = W[n] . x[row_of(p)] over the entries p of each work
// tile: the consecutive slices of [0, n_entries) (tile_expert == nullptr), or
// the bucketing's expert tiles (tile_expert[t], tile_begin[t], tile_end[t],
// t < *n_tiles) with W = table[tile_expert[t]].  dual: gate (W / table) and
// up (W2 / table2) share the tile; out = silu(gate) * up (gate clamped to
// +-80 when clamp_silu).  ksplit > 1 (dense, not dual): partial sums of K
// ranges into part[z][entry][row], added in order afterwards.
struct q16_args {
    mllm_packed W, W2;
    const mllm_packed *table, *table2;
    act16 x;
    const int *row_of;
    float *out;
    int ldo;
    const int *out_row;
    int n_rows, n_cols, n_entries;
    const int *tile_expert, *tile_begin, *tile_end, *n_tiles;
    int clamp_silu;
    int ksplit;
    float *part;
    int eoff;        // MXFP4: weights decode as v 2^(E + eoff) (mllm_q16_mx_shift)
    float wscale;    // MXFP4: 2^(-127 - eoff), applied to the result
    int rows_fast;   // set by the launch: work tiles ordered row block fastest
    // step-major metadata (mllm_launch_q16_smeta) of W / table[e] at sm + e * sm_stride and of
    // W2 / table2[e] at sm2 + e * sm_stride, or null (K-quants then read the packed planes;
    // MXFP4 needs it)
    const uint8_t *sm, *sm2;
    long sm_stride, sm_doff;
};
// Entries per work tile of a launch (grouped launches: the bucketing's tile).
int mllm_q16_tile_entries(bool grouped, int n_entries);
int mllm_q16_ksplit(int sem, int n_rows, int n_cols, int n_entries);
inline long mllm_q16_part_floats(int sem, int n_rows, int n_cols, int n_entries)
{
    const int ks = mllm_q16_ksplit(sem, n_rows, n_cols, n_entries);
    return ks > 1 ? (long)ks * n_entries * n_rows : 0;
}
hipError_t mllm_launch_q16(int sem, bool dual, const q16_args &a, int max_tiles, hipStream_t st);
