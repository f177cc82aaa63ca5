// mllm_common.h — definitions shared by host and device code of libmllm_gpu.
//
// Semantics.  The reference gives one GGUF quant type different meanings on
// different exported symbols (e.g. Q6_K is ggml order in q6_k_dequantize_row,
// low-nibble-only through quant_matmul_omp, sequential order in
// q6_k_batch_matmul).  Every kernel here is keyed by a *semantic* id that
// names one of those meanings; the C ABI maps (entry point, GGUF code) to it
// exactly as the reference's dispatch does.
//
// Packed weight layout.  Raw GGUF blocks (34 B Q8_0, 17 B MXFP4, 210 B Q6_K,
// ...) are not 16-byte multiples, so the device copy of a weight matrix is
// split into planes: the bulk quant bytes of every block, row-major, in one
// plane (16-byte aligned, so a lane streams them with dwordx4 loads) and the
// per-block scales in small side planes.  The total byte count equals the
// raw GGUF size; only the order changes.
#pragma once
#include <stdint.h>

enum mllm_sem {
    SEM_F32 = 0,          // f32_matmul_omp                                QK:884-913
    SEM_Q4_0 = 1,         // q4_0_matmul_omp / q4_0_batch_matmul           QK:77-95,135-154; CE:68-110
    SEM_Q4_1 = 2,         // q4_1_matmul_omp                               QK:97-117,160-177
    SEM_Q5_0_F32 = 3,     // q5_0_row_dot (fp32 x)                         QK:1245-1266
    SEM_Q5_0_Q8 = 4,      // q5_0_matmul_omp via Q8_0(x)                   QK:1232-1237,1268-1353
    SEM_Q8_0 = 5,         // q8_0_matmul_omp / q8_0_batch_matmul           QK:376-416; CE:216-253
    SEM_Q4_K_GGML = 6,    // q4_k_batch_matmul / q4_k_row_dot_avx2          CE:255-313; QK:1980-2063
    SEM_Q4_K_Q8 = 7,      // quant_matmul_omp(12): dot_q4_k_q8_0            QK:199-209,1647-1758
    SEM_Q5_K_GGML = 8,    // q5_k_row_dot_avx2 / q5_k_dequantize_row        QK:249-364,830-866
    SEM_Q5_K_CE = 9,      // q5_k_batch_matmul (engine's own struct)        CE:46-52,380-425
    SEM_Q6_K_GGML = 10,   // q6_k_dequantize_row                            QK:762-800
    SEM_Q6_K_LOWNIB = 11, // quant_matmul_omp(14): q6k_dequant_8            QK:1778-1903
    SEM_Q6_K_SEQ = 12,    // q6_k_batch_matmul                              CE:315-378
    SEM_MXFP4 = 13,       // mxfp4_matmul_omp / mxfp4_row_dot_f32           QK:502-627,683-720
    SEM_MXFP4_CLAMP = 14, // mxfp4_batch_matmul (scale clamped to 1e20)     CE:427-534
    SEM_MXFP4_Q8 = 15,    // mxfp4_row_dot_q8                               QK:629-678
    SEM_COUNT = 16
};

// Packed layouts.  Q5_K has two source layouts (ggml / engine struct) that
// pack to the same planes.
enum mllm_layout {
    LY_F32 = 0, LY_Q4_0, LY_Q4_1, LY_Q5_0, LY_Q8_0, LY_Q4_K, LY_Q5_K_GGML, LY_Q5_K_CE,
    LY_Q6_K, LY_MXFP4, LY_COUNT
};

#define MLLM_MAX_PLANES 4

struct mllm_layout_desc {
    int block_elems;                 // elements per quant block
    int block_bytes;                 // raw GGUF bytes per block
    int n_planes;
    int plane_bytes[MLLM_MAX_PLANES];// bytes per block in each plane (sum == block_bytes)
};

// Plane contents per layout (bytes per block):
//   Q4_0  : qs[16] | d[2]             Q4_1 : qs[16] | d,m[4]
//   Q5_0  : ql[16] | qh[4] | d[2]     Q8_0 : qs[32] | d[2]
//   Q4_K  : qs[128] | d,dmin,scales[16]
//   Q5_K  : ql[128] | qh[32] | d,dmin,scales[16]
//   Q6_K  : ql[128] | qh[64] | scales[16] | d[2]
//   MXFP4 : q[16] | e8m0[1]           F32 : 32 floats per "block"
static inline __host__ __device__ mllm_layout_desc mllm_layout_info(int ly)
{
    switch (ly) {
    case LY_F32:       return {32, 128, 1, {128, 0, 0, 0}};
    case LY_Q4_0:      return {32, 18, 2, {16, 2, 0, 0}};
    case LY_Q4_1:      return {32, 20, 2, {16, 4, 0, 0}};
    case LY_Q5_0:      return {32, 22, 3, {16, 4, 2, 0}};
    case LY_Q8_0:      return {32, 34, 2, {32, 2, 0, 0}};
    case LY_Q4_K:      return {256, 144, 2, {128, 16, 0, 0}};
    case LY_Q5_K_GGML:
    case LY_Q5_K_CE:   return {256, 176, 3, {128, 32, 16, 0}};
    case LY_Q6_K:      return {256, 210, 4, {128, 64, 16, 2}};
    case LY_MXFP4:     return {32, 17, 2, {16, 1, 0, 0}};
    }
    return {0, 0, 0, {0, 0, 0, 0}};
}

static inline __host__ __device__ int mllm_sem_layout(int sem)
{
    switch (sem) {
    case SEM_F32: return LY_F32;
    case SEM_Q4_0: return LY_Q4_0;
    case SEM_Q4_1: return LY_Q4_1;
    case SEM_Q5_0_F32: case SEM_Q5_0_Q8: return LY_Q5_0;
    case SEM_Q8_0: return LY_Q8_0;
    case SEM_Q4_K_GGML: case SEM_Q4_K_Q8: return LY_Q4_K;
    case SEM_Q5_K_GGML: return LY_Q5_K_GGML;
    case SEM_Q5_K_CE: return LY_Q5_K_CE;
    case SEM_Q6_K_GGML: case SEM_Q6_K_LOWNIB: case SEM_Q6_K_SEQ: return LY_Q6_K;
    default: return LY_MXFP4;
    }
}

// Semantics whose activation is first quantised to Q8_0 (QK:1406-1455).
static constexpr inline __host__ __device__ bool mllm_sem_uses_q8(int sem)
{
    return sem == SEM_Q4_K_Q8 || sem == SEM_MXFP4_Q8 || sem == SEM_Q5_0_Q8;
}

// Device view of one packed matrix: plane base pointers.
struct mllm_packed {
    const uint8_t *p[MLLM_MAX_PLANES];
};

// Packed byte size of an n_rows x n_cols matrix, plane offsets 256-byte aligned.
static inline __host__ __device__ long mllm_packed_bytes(int ly, int n_rows, int n_cols, long *offs)
{
    mllm_layout_desc L = mllm_layout_info(ly);
    long nblk = (long)n_rows * (n_cols / L.block_elems);
    long off = 0;
    for (int i = 0; i < L.n_planes; i++) {
        if (offs) offs[i] = off;
        off += ((nblk * L.plane_bytes[i]) + 255) / 256 * 256;
    }
    return off > 0 ? off : 256;
}

// Activation pack written by the Q8_0 quantiser for the Q8 semantics, per
// token b and 32-element block j (nb32 = n_cols/32 blocks per token):
//   q  : int8  [B][nb32*32]  quants
//   d  : float [B][nb32]     fp16 scale, decoded
//   s4 : float [B][nb32]     d * (sum q[0..7] + sum q[16..23])   (Q4_K min term, QK:1714-1732)
//   sq : int   [B][nb32]     sum of all 32 quants
struct mllm_xq {
    const int8_t *q;
    const float *d;
    const float *s4;
    const int *sq;
};
