// gemv.h — host-side launch interfaces of the kernels in libmllm_gpu.
#pragma once
#include <hip/hip_runtime.h>
#include "mllm_common.h"

// One decode GEMV launch.  A "job" is one matrix-vector product; blockIdx.y
// walks the jobs.  Matrix of job j: `W` when `table` is null, otherwise
// table[idx ? idx[j] : j] (device arrays).  x / out of job j start at
// x + (j / job_div)*x_job_stride / out + j*out_job_stride (elements; job_div
// 0 or 1 = one x per job); token b of a job reads x + b*ldx and writes
// out + b*ldo.  With job_split > 0, jobs j >= job_split run as job
// j - job_split of a second list (table2, out2), so two projections of the
// same activations (MoE gate and up) share one launch.
struct mllm_gemv_args {
    mllm_packed W;
    const mllm_packed *table;
    const int *idx;
    const float *x;
    long x_job_stride;
    int ldx;
    float *out;
    long out_job_stride;
    int ldo;
    int n_rows, n_cols, B;
    int k_tile;   // activation elements staged in LDS per pass (set by the launcher)
    mllm_xq xq;   // Q8_0 activation pack (Q8 semantics); job/token strides follow x's.
                  // xq.q == nullptr: each workgroup quantises x (fp32) itself.
    int job_div;
    int job_split;
    const mllm_packed *table2;
    float *out2;
    // The activation is silu(x) * x_up (mllm_silu_mul, same offsets as x)
    // instead of x: fp32-activation semantics at B == 1, and Q8 semantics
    // quantising in the kernel.  silu_noclamp: the gate is not clamped
    // (moe_ffn CE:649-652, the dense FFN's silu).
    const float *x_up;
    int silu_noclamp;
    // Fused prologue (single-matrix launches, no job table): token b's
    // activation is v = x[b] + x_res[b] (x_res optional, same strides as x),
    // res_out[b] = v when res_out is given (the new residual stream), then
    // with rms_w the RMS norm of v over its n_cols elements times rms_w:
    //   rms_div == 0: v * (1 / sqrtf(mean(v^2) + eps)) * rms_w   (simd_ops rms_norm, TE:1516,1641)
    //   rms_div == 1: (v / sqrtf(mean(v^2) + eps)) * rms_w       (gptoss_batch_forward.c GO:29-34)
    const float *x_res;
    float *res_out;
    const float *rms_w;
    float rms_eps;
    int rms_div;
    // Fused epilogue: out[b][r] = out_add[b][r] + (W x)[b][r] (same strides as
    // out; may alias out): the residual add after a projection.
    const float *out_add;
    int pro_lds;   // byte offset of the prologue's LDS scratch (set by the launcher)
    // Paired rows (batch 1): output row r is silu(g_r . x) * (u_r . x) (the
    // gate clamped to +-80 unless silu_noclamp), g_r = row r and u_r = row
    // r + n_rows of the matrix, or with table2 row r of table2's matrix for the
    // job's expert: gate, up and the SiLU product in one launch.
    int silu_pair;
    // Split-K partials of the batch 2..8 MFMA GEMV (mllm_gemv_mf_part_floats
    // floats; optional: without it that kernel runs unsplit or not at all).
    float *mf_part;
};

// moe_forward_omp's SiLU product (QK:2157-2164): the gate clamped to +-80,
// then silu(g) * u.  Every kernel that forms it uses this one expression;
// clamp = false gives the unclamped form of moe_ffn and the dense FFN.
__device__ __forceinline__ float mllm_silu_mul(float g, float u, bool clamp = true)
{
    if (clamp) {
        g = g < -80.0f ? -80.0f : g;
        g = g > 80.0f ? 80.0f : g;
    }
    return (g / (1.0f + expf(-g))) * u;
}

// vmaxps(a, b): a if a > b, else b, so a NaN in either operand gives b.
__device__ __forceinline__ float mllm_maxps(float a, float b) { return a > b ? a : b; }

// quantize_row_q8_0's amax over one 32-block in the reference's vector order
// (QK:1417-1425): eight lanes m_j fold |v[8i+j]|, i = 0..3, as
// maxps(m_j, |v|); then maxps(m_j, m_j^4), (., j^2), (., j^1), lane 0 read.
// Without a NaN this is max|v|; with one, amax is NaN exactly when the
// reference's is.  fn(i) returns |v[i]|.
__device__ __forceinline__ float mllm_q8_amax_tree(const float (&m)[8])
{
    const float t0 = mllm_maxps(m[0], m[4]), t1 = mllm_maxps(m[1], m[5]);
    const float t2 = mllm_maxps(m[2], m[6]), t3 = mllm_maxps(m[3], m[7]);
    return mllm_maxps(mllm_maxps(t0, t2), mllm_maxps(t1, t3));
}

template <class F>
__device__ __forceinline__ float mllm_q8_amax_ref(F fn)
{
    float m[8];
#pragma unroll
    for (int j = 0; j < 8; j++) m[j] = mllm_maxps(0.0f, fn(j));
#pragma unroll
    for (int i = 1; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) m[j] = mllm_maxps(m[j], fn(8 * i + j));
    return mllm_q8_amax_tree(m);
}

// Whether a launch asks for the fused activation prologue.
inline __host__ __device__ bool mllm_has_prologue(const mllm_gemv_args &a) { return a.x_res || a.rms_w || a.res_out; }
// Whether the persistent kernel's fused forms (prologue, paired rows) stage
// this launch's activation at once; paired rows need B == 1.
bool mllm_gemv_fused_fits(int sem, int n_cols, int B, bool prologue);

// n_cols below one quant block (no whole block per row): every output is 0, as
// the reference's dot over n_cols / block = 0 blocks; no weight is read.
hipError_t mllm_launch_gemv(int sem, const mllm_gemv_args &a, int n_jobs, hipStream_t st);
// Elements per quant block of a semantic's weight layout (1 for fp32 rows).
int mllm_sem_block_elems(int sem);
// Whether mllm_launch_gemv takes the fused prologue for this shape (the
// persistent kernel stages all of K; else the caller runs the prologue first).
bool mllm_gemv_prologue_fits(int sem, int n_cols, int B);

// The batch 2..8 decode GEMV on the matrix cores (gemv_mf.h): Q4_K ggml and
// Q6_K sequential weights, fp32 activations, with the prologue, the paired
// gate/up rows and out_add fused.  have_part: an mf_part buffer of
// mllm_gemv_mf_part_floats floats is given (short matrices then split K).
bool mllm_gemv_mf_fits(int sem, int n_rows, int n_cols, int B, bool pro, bool pair, bool have_part);
long mllm_gemv_mf_part_floats(int sem, int n_rows, int n_cols, int B, bool pro, bool pair);
// hipErrorNotSupported: this launch has no MFMA form (the caller takes the VALU kernel).
hipError_t mllm_launch_gemv_mf(int sem, const mllm_gemv_args &a, hipStream_t st);

// Repack raw GGUF blocks (device) into the plane layout `ly`.
hipError_t mllm_launch_pack(int ly, const uint8_t *raw, uint8_t *packed, int n_rows, int n_cols, hipStream_t st);
mllm_packed mllm_packed_view(int ly, const uint8_t *packed, int n_rows, int n_cols);

// quantize_row_q8_0 over T rows of n_cols floats (QK:1406-1455), bit-exact.
// Writes the raw 34-byte blocks to q8_raw (if non-null) and the activation
// pack (q / d / s4 / sq) to the xq arrays (if non-null).  With x_up, the
// rows quantised are mllm_silu_mul(x, x_up).
hipError_t mllm_launch_quantize_q8_0(const float *x, int T, int n_cols, uint8_t *q8_raw,
                                     int8_t *xq_q, float *xq_d, float *xq_s4, int *xq_sq, hipStream_t st,
                                     const float *x_up = nullptr);

// Router: logits by a sequential fp32 FMA chain (CE:614-618), softmax with
// expf, insertion top-k with strict '>' (CE:628-638), optional renormalise
// (GO:88-92).  router_t is the router transposed to [N][E].
long mllm_router_packed_floats(int N, int E);
hipError_t mllm_launch_router_pack(const float *router, int N, int E, float *out, hipStream_t st);
// logits_ws (optional, mllm_route_workspace_floats floats): lets T <= 8 tokens spread over expert slices.
long mllm_route_workspace_floats(int T, int E);
hipError_t mllm_launch_route(const float *router_p, const float *x, int T, int N, int E, int K, int renorm,
                             int *top_idx, float *top_w, float *logits_ws, hipStream_t st);

// Softmax and top-K (CE:614-638, renormalised when `renorm`) of logits [T][E]
// computed elsewhere: k_route_finish on its own.
hipError_t mllm_launch_route_finish(const float *logits, int T, int E, int K, int renorm, int *top_idx, float *top_w,
                                    hipStream_t st);

// The fused GEMV activation on its own, T rows of n (one workgroup each):
// v = (x_up ? silu(x) * x_up : x) + x_res; res_out = v; with rms_w the RMS
// norm of v (div: (v / rms) * w, else v * (1 / rms) * w).  Any pointer but x
// and out may be null.
hipError_t mllm_launch_act_prologue(const float *x, const float *x_res, float *res_out, const float *rms_w, float eps,
                                    int div, const float *x_up, int clamp, int T, int n, int ldx, float *out,
                                    hipStream_t st);
// Plain streaming read of bytes / 16 words (mllm_read_probe).
hipError_t mllm_launch_read_probe(const void *p, long bytes, void *sink, hipStream_t st);
// TE:620-666 Q8_0 requantisation of fp32 rows [n_rows][n_cols] into raw 34-byte blocks.
hipError_t mllm_launch_requant_q8_0(const float *w, int n_rows, int n_cols, uint8_t *out, hipStream_t st);
// p[i] = v, i < n (a fill kernel: nothing here records a memset node).
hipError_t mllm_launch_fill(float *p, long n, float v, hipStream_t st);
// out[i] = (float)u[i]: TE:643-645's F16 conversion (the patterns' integer values)
hipError_t mllm_launch_u16_value_f32(const uint16_t *u, long n, float *out, hipStream_t st);
// ORs into *flags (device int): 1 = some block scale of the n_mats matrices in
// tab_dev (device array; or the single host-side view `one` when tab_dev is
// null) is inf/NaN, 2 = some E8M0 exponent is >= 178 (see k_scale_scan).
hipError_t mllm_launch_scale_scan(const mllm_packed *tab_dev, const mllm_packed *one, int n_mats, int sem, int n_rows,
                                  int n_cols, int *flags, hipStream_t st);
// Whether a matrix of semantic sem whose scan gave `flags` must stay on the
// GEMV path: the MFMA GEMMs fold block scales into bf16 weights, so a
// non-finite scale meets zero activation planes (inf * 0 = NaN where the
// reference's per-element product is +-inf), and the MXFP4 scale clamps
// (QK:648-650, CE:454-456) are not applied there.
bool mllm_scales_need_gemv(int sem, int flags);
// out[i] += add[i], i < n.
hipError_t mllm_launch_add(float *out, const float *add, long n, hipStream_t st);
// out[b][r] = silu(y[b][r]) * y[b][n + r] (+ add[b][r]); y is [B][2n].
hipError_t mllm_launch_silu_pair(const float *y, int B, int n, int clamp, float *out, const float *add, hipStream_t st);

// h[i] = silu(g[i]) * u[i] (clamp g to +-80 when clamp != 0), i < n.
hipError_t mllm_launch_silu_mul(const float *g, const float *u, float *h, long n, int clamp, hipStream_t st);

// out[t][i] = sum_k (in k order) w[t][k] * d[t][k][i]; fused selects fmaf (moe_ffn CE:662) or
// add-of-product (moe_forward_omp QK:2243-2244).  d == nullptr: every d term is 0.  Slots whose
// expert idx[t][k] is negative (left empty by the routing) are skipped; idx == nullptr: none are.
hipError_t mllm_launch_combine(const float *d, const float *w, const int *idx, int T, int K, int N, float *out,
                               int fused, hipStream_t st);

// fp32 rows of a packed matrix under a fp32-weight semantic; returns 0 or -1
// (semantic without an fp32 weight form, or launch failure).
int mllm_launch_dequant(int sem, const mllm_packed &W, int n_rows, int n_cols, float *out, hipStream_t st);

// moe_ffn engine for T tokens (host activations in/out); see capi.hip.
int mllm_moe_ffn_dev_tokens(const float *router, const uint8_t *const bases[3], const int qts[3], int N, int E, int K,
                            int M, const float *x_host, float *out_host, int T);
