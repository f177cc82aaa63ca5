// ops.hip — the small kernels around the GEMVs: weight repack, Q8_0
// activation quantisation, MoE routing, SiLU-gate and the weighted combine.
#include <math.h>
#include "decode.h"
#include "gemv.h"

namespace {

// ------------------------------------------------------------------ repack
// Source byte offsets of each plane inside a raw GGUF block.
struct pack_src { int n; int off[4]; int len[4]; int plane[4]; };

__host__ __device__ pack_src pack_plan(int ly)
{
    switch (ly) {
    case LY_Q4_0: return {2, {2, 0}, {16, 2}, {0, 1}};
    case LY_Q4_1: return {2, {4, 0}, {16, 4}, {0, 1}};
    case LY_Q5_0: return {3, {6, 2, 0}, {16, 4, 2}, {0, 1, 2}};
    case LY_Q8_0: return {2, {2, 0}, {32, 2}, {0, 1}};
    // K-quant meta planes get d, dmin here; the scale pairs are re-laid below.
    case LY_Q4_K: return {2, {16, 0}, {128, 4}, {0, 1}};
    // block_q5_K (ggml, QK:211-246): d dmin scales[12] qh[32] qs[128]
    case LY_Q5_K_GGML: return {3, {48, 16, 0}, {128, 32, 4}, {0, 1, 2}};
    // the engine's block_q5_K (CE:46-52): d dmin qh[32] ql[128] scales[12]
    case LY_Q5_K_CE: return {3, {36, 4, 0}, {128, 32, 4}, {0, 1, 2}};
    // block_q6_K (CE:34-39): ql[128] qh[64] scales[16] d
    case LY_Q6_K: return {4, {0, 128, 192, 208}, {128, 64, 16, 2}, {0, 1, 2, 3}};
    case LY_MXFP4: return {2, {0, 16}, {16, 1}, {0, 1}};
    }
    return {0, {0}, {0}, {0}};
}

// 6-bit (scale, min) pair j of a K-quant scale array (get_scale_min_k4 QK:62-71).
__device__ void k4_pair(int j, const uint8_t *q, uint32_t &sc, uint32_t &m)
{
    if (j < 4) { sc = q[j] & 63; m = q[j + 4] & 63; }
    else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m  = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

__global__ void k_pack(int ly, const uint8_t *__restrict__ raw, uint8_t *__restrict__ packed, long nblk,
                       long off0, long off1, long off2, long off3)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    const mllm_layout_desc L = mllm_layout_info(ly);
    const pack_src ps = pack_plan(ly);
    const long offs[4] = {off0, off1, off2, off3};
    const uint8_t *src = raw + i * L.block_bytes;
    for (int s = 0; s < ps.n; s++) {
        const int p = ps.plane[s];
        uint8_t *dst = packed + offs[p] + i * L.plane_bytes[p];
        for (int j = 0; j < ps.len[s]; j++) dst[j] = src[ps.off[s] + j];
    }
    if (ly == LY_Q4_K || ly == LY_Q5_K_GGML || ly == LY_Q5_K_CE) {
        // meta = [d | dmin] [sc_0..7 as 6-bit fields, 48 bits] [m_0..7, 48 bits]
        const uint8_t *sc = src + (ly == LY_Q5_K_CE ? 164 : 4);
        uint64_t S = 0, M = 0;
        for (int j = 0; j < 8; j++) {
            uint32_t a, b;
            k4_pair(j, sc, a, b);
            S |= (uint64_t)a << (6 * j);
            M |= (uint64_t)b << (6 * j);
        }
        uint32_t *meta = reinterpret_cast<uint32_t *>(packed + offs[ly == LY_Q4_K ? 1 : 2] + i * 16);
        meta[1] = (uint32_t)S;
        meta[2] = (uint32_t)(S >> 32) | ((uint32_t)M << 16);
        meta[3] = (uint32_t)(M >> 16);
    }
}

// ---------------------------------------------------------------- quantise
// One thread per 32-element block.  Mirrors quantize_row_q8_0 (QK:1406-1455):
// amax, d = amax/127 (1 if 0), id = 1/d, q = RNE(clamp(x*id, +-127)) with a
// NaN product clamped to -127 (maxps returns its second operand), scale
// stored as fp16 RNE.
__global__ void k_quantize_q8_0(const float *__restrict__ x, int T, int n_cols, uint8_t *__restrict__ q8_raw,
                                int8_t *__restrict__ xq_q, float *__restrict__ xq_d, float *__restrict__ xq_s4,
                                int *__restrict__ xq_sq)
{
    const int nb = n_cols / 32;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)T * nb) return;
    const long t = i / nb, j = i % nb;
    const float *s = x + t * (long)n_cols + 32 * j;
    float v[32];
#pragma unroll
    for (int k = 0; k < 32; k++) v[k] = s[k];
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; k++) { float a = fabsf(v[k]); amax = (a > amax) ? a : amax; }
    float d = amax / 127.0f;
    if (d == 0.0f) d = 1.0f;
    const float id = 1.0f / d;
    const uint16_t dh = __builtin_bit_cast(uint16_t, (_Float16)d);  // RNE
    int q[32];
    int sq = 0, s4 = 0;
#pragma unroll
    for (int k = 0; k < 32; k++) {
        float p = v[k] * id;
        p = (p > -127.0f) ? p : -127.0f;
        p = (p < 127.0f) ? p : 127.0f;
        q[k] = (int)rintf(p);
        sq += q[k];
        if ((k & 16) == 0 ? k < 8 : k < 24) s4 += q[k];
    }
    if (q8_raw) {
        uint8_t *dst = q8_raw + i * 34;
        dst[0] = dh & 0xFF;
        dst[1] = dh >> 8;
#pragma unroll
        for (int k = 0; k < 32; k++) dst[2 + k] = (uint8_t)(int8_t)q[k];
    }
    if (xq_q) {
        uint32_t w[8];
#pragma unroll
        for (int k = 0; k < 8; k++)
            w[k] = (uint32_t)(q[4 * k] & 0xFF) | ((uint32_t)(q[4 * k + 1] & 0xFF) << 8) |
                   ((uint32_t)(q[4 * k + 2] & 0xFF) << 16) | ((uint32_t)(q[4 * k + 3] & 0xFF) << 24);
        uint4 *dq = reinterpret_cast<uint4 *>(xq_q + i * 32);
        dq[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dq[1] = make_uint4(w[4], w[5], w[6], w[7]);
        const float dd = h2f(dh);
        xq_d[i] = dd;
        xq_s4[i] = dd * (float)s4;
        xq_sq[i] = sq;
    }
}

// ------------------------------------------------------------------ routing
// exp rounded from double: within half an ulp of the exact value, as the
// host libm's expf is, so the probabilities (and every comparison on them)
// match the reference's except where the two roundings straddle a midpoint.
__device__ __forceinline__ float expf_cr(float v) { return (float)exp((double)v); }

// One workgroup per token; thread e computes logit e as a sequential FMA
// chain over i = 0..N-1 (CE:614-618 compiles to scalar vfmadd231ss), then
// thread 0 runs the softmax and insertion top-k exactly as CE:620-638.
__global__ __launch_bounds__(256) void k_route(const float *__restrict__ router_t, const float *__restrict__ x,
                                               int N, int E, int K, int renorm, int *__restrict__ top_idx,
                                               float *__restrict__ top_w)
{
    __shared__ float p[256];
    const int t = blockIdx.x, e = threadIdx.x;
    const float *xt = x + (long)t * N;
    if (e < E) {
        float dot = 0.0f;
        for (int i = 0; i < N; i++) dot = fmaf(xt[i], router_t[(long)i * E + e], dot);
        p[e] = dot;
    }
    __syncthreads();
    if (e != 0) return;
    float mx = p[0];
    for (int j = 1; j < E; j++) if (p[j] > mx) mx = p[j];
    float sum = 0.0f;
    for (int j = 0; j < E; j++) { p[j] = expf_cr(p[j] - mx); sum += p[j]; }
    const float inv = 1.0f / (sum + 1e-10f);
    for (int j = 0; j < E; j++) p[j] *= inv;
    float tv[16];
    int ti[16];
    for (int k = 0; k < K; k++) { tv[k] = -1e30f; ti[k] = -1; }
    for (int j = 0; j < E; j++) {
        const float v = p[j];
        for (int k = 0; k < K; k++) {
            if (v > tv[k]) {
                for (int k2 = K - 1; k2 > k; k2--) { tv[k2] = tv[k2 - 1]; ti[k2] = ti[k2 - 1]; }
                tv[k] = v; ti[k] = j;
                break;
            }
        }
    }
    if (renorm) {
        float s = 0.0f;
        for (int k = 0; k < K; k++) s += tv[k];
        const float r = 1.0f / (s + 1e-10f);
        for (int k = 0; k < K; k++) tv[k] *= r;
    }
    for (int k = 0; k < K; k++) { top_idx[(long)t * K + k] = ti[k]; top_w[(long)t * K + k] = tv[k]; }
}

// ---------------------------------------------------------------- MoE glue
__global__ void k_silu_mul(const float *__restrict__ g, const float *__restrict__ u, float *__restrict__ h, long n,
                           int clamp)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float gv = g[i];
    if (clamp) { gv = gv < -80.0f ? -80.0f : gv; gv = gv > 80.0f ? 80.0f : gv; }
    h[i] = (gv / (1.0f + expf(-gv))) * u[i];
}

__global__ void k_combine(const float *__restrict__ d, const float *__restrict__ w, int K, int N,
                          float *__restrict__ out, int fused)
{
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    float acc = 0.0f;
    for (int k = 0; k < K; k++) {
        const float wk = w[(long)t * K + k], dv = d[((long)t * K + k) * N + i];
        acc = fused ? fmaf(wk, dv, acc) : acc + wk * dv;
    }
    out[(long)t * N + i] = acc;
}

} // namespace

mllm_packed mllm_packed_view(int ly, const uint8_t *packed, int n_rows, int n_cols)
{
    long offs[MLLM_MAX_PLANES] = {0, 0, 0, 0};
    mllm_packed_bytes(ly, n_rows, n_cols, offs);
    mllm_packed v;
    const mllm_layout_desc L = mllm_layout_info(ly);
    for (int i = 0; i < MLLM_MAX_PLANES; i++) v.p[i] = i < L.n_planes ? packed + offs[i] : nullptr;
    if (ly == LY_F32) v.p[0] = packed;
    return v;
}

hipError_t mllm_launch_pack(int ly, const uint8_t *raw, uint8_t *packed, int n_rows, int n_cols, hipStream_t st)
{
    if (ly == LY_F32)
        return hipMemcpyAsync(packed, raw, (size_t)n_rows * n_cols * 4, hipMemcpyDeviceToDevice, st);
    long offs[MLLM_MAX_PLANES] = {0, 0, 0, 0};
    mllm_packed_bytes(ly, n_rows, n_cols, offs);
    const mllm_layout_desc L = mllm_layout_info(ly);
    const long nblk = (long)n_rows * (n_cols / L.block_elems);
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL(k_pack, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, st, ly, raw, packed, nblk,
                       offs[0], offs[1], offs[2], offs[3]);
    return hipGetLastError();
}

hipError_t mllm_launch_quantize_q8_0(const float *x, int T, int n_cols, uint8_t *q8_raw, int8_t *xq_q, float *xq_d,
                                     float *xq_s4, int *xq_sq, hipStream_t st)
{
    const long n = (long)T * (n_cols / 32);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_quantize_q8_0, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, st, x, T, n_cols, q8_raw,
                       xq_q, xq_d, xq_s4, xq_sq);
    return hipGetLastError();
}

hipError_t mllm_launch_route(const float *router_t, const float *x, int T, int N, int E, int K, int renorm,
                             int *top_idx, float *top_w, hipStream_t st)
{
    if (E > 256 || K > 16 || K > E || T <= 0) return hipErrorInvalidValue;
    const int threads = (E + 63) / 64 * 64;
    hipLaunchKernelGGL(k_route, dim3(T), dim3(threads), 0, st, router_t, x, N, E, K, renorm, top_idx, top_w);
    return hipGetLastError();
}

hipError_t mllm_launch_silu_mul(const float *g, const float *u, float *h, long n, int clamp, hipStream_t st)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, h, n, clamp);
    return hipGetLastError();
}

hipError_t mllm_launch_combine(const float *d, const float *w, int T, int K, int N, float *out, int fused,
                               hipStream_t st)
{
    if (T <= 0 || N <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_combine, dim3((N + 255) / 256, T), dim3(256), 0, st, d, w, K, N, out, fused);
    return hipGetLastError();
}
