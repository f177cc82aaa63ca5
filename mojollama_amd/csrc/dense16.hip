// dense16.hip — prefill GEMM over a load-time fp16 copy of a quantised matrix.
//
// The weights are dequantised once, with the reference's *_dequantize_row
// arithmetic (QK:762-878: w = fl(s*q) + o), and rounded to fp16; each call
// rounds its fp32 activations to fp16 under one power-of-two scale chosen
// from the batch's largest finite element (in one pass at scale 1, redone at
// another scale only when that element falls outside [1/4, 2^15)), and the
// product runs as a plain
// GEMM on hipBLASLt (fp16 operands, fp32 accumulation and output, the scale
// undone through its per-row device alpha).  The copy costs 2 bytes per weight in HBM (3.6x a
// Q4_K matrix); in exchange the per-tile dequantisation leaves the prefill's
// critical path.  Relative rounding of weights and activations is at most
// 2^-11 each, so y = W.x keeps ~3e-4 of the output scale.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>
#include <algorithm>
#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <tuple>
#include "gemv.h"
#include "dense16.h"

namespace {

constexpr int kPartMax = 1024;           // amax partials of the activation pass
constexpr size_t kBlasWs = 32u << 20;    // hipBLASLt workspace cap

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// fp32 -> fp16 (round to nearest even); bad = some |w| rounds to inf or is not finite.
__global__ __launch_bounds__(256) void k_w16(const float4 *__restrict__ w, long n4, uint2 *__restrict__ out,
                                             int *__restrict__ bad)
{
    const long G = (long)gridDim.x * 256;
    int b = 0;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += G) {
        const float4 v = w[i];
        b |= !(fabsf(v.x) < 65520.f) | !(fabsf(v.y) < 65520.f) | !(fabsf(v.z) < 65520.f) | !(fabsf(v.w) < 65520.f);
        const _Float16 h0 = (_Float16)v.x, h1 = (_Float16)v.y, h2 = (_Float16)v.z, h3 = (_Float16)v.w;
        out[i] = make_uint2((uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16),
                            (uint32_t)__builtin_bit_cast(uint16_t, h2) | ((uint32_t)__builtin_bit_cast(uint16_t, h3) << 16));
    }
    if (b) *bad = 1;
}

__device__ float block_max(float v, float *red)
{
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return v;
}

// Element offset of float4 i of the M x K activations (rows at stride ldx).
__device__ __forceinline__ long x4_off(long i, int k4, int ldx, bool flat)
{
    if (flat) return i * 4;
    const int r = (int)(i / k4), c = (int)(i - (long)r * k4);
    return (long)r * ldx + 4 * c;
}

__device__ __forceinline__ float amax4(float m, float4 v)
{
    const float a[4] = {fabsf(v.x), fabsf(v.y), fabsf(v.z), fabsf(v.w)};
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (a[j] < INFINITY) m = fmaxf(m, a[j]);   // finite elements only (NaN compares false)
    return m;
}

__device__ __forceinline__ uint2 pack_h4(float4 v, float sc)
{
    const _Float16 h0 = (_Float16)(v.x * sc), h1 = (_Float16)(v.y * sc), h2 = (_Float16)(v.z * sc),
                   h3 = (_Float16)(v.w * sc);
    return make_uint2((uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16),
                      (uint32_t)__builtin_bit_cast(uint16_t, h2) | ((uint32_t)__builtin_bit_cast(uint16_t, h3) << 16));
}

// Largest finite |x| lands in [kScale1Lo, kScale1Hi): fp16(x) at scale 1 rounds
// every element as fp16(x * 2^E) does at the scale below, except elements
// under 2^-14 (fp16 subnormals at scale 1), which keep an absolute error under
// 2^-25, below 2^-23 of the largest element; the one-pass conversion stands.
constexpr float kScale1Lo = 0.25f, kScale1Hi = 32768.f;

// x16 = fp16(x) (scale 1) and alpha = 1, with the largest finite |x| of each
// block to part[]; each thread keeps four 16-byte loads in flight (K is a
// multiple of 4).
__global__ __launch_bounds__(256) void k_x16_cvt1(const float *__restrict__ x, int K, int ldx, long n4,
                                                  float *__restrict__ part, uint2 *__restrict__ x16,
                                                  float *__restrict__ alpha, int n_rows)
{
    __shared__ float red[4];
    const long G = (long)gridDim.x * 256;
    const int k4 = K / 4;
    const bool flat = ldx == K;
    float m = 0.f;
    long i = (long)blockIdx.x * 256 + threadIdx.x;
    for (; i + 3 * G < n4; i += 4 * G) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = *(const float4 *)(x + x4_off(i + u * G, k4, ldx, flat));
#pragma unroll
        for (int u = 0; u < 4; u++) {
            m = amax4(m, v[u]);
            x16[i + u * G] = pack_h4(v[u], 1.f);
        }
    }
    for (; i < n4; i += G) {
        const float4 v = *(const float4 *)(x + x4_off(i, k4, ldx, flat));
        m = amax4(m, v);
        x16[i] = pack_h4(v, 1.f);
    }
    for (long r = (long)blockIdx.x * 256 + threadIdx.x; r < n_rows; r += G) alpha[r] = 1.f;
    m = block_max(m, red);
    if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// Where the batch's largest finite |x| falls outside [kScale1Lo, kScale1Hi):
// x16 = fp16(x * 2^E) again, E such that it lands in [2^14, 2^15), and
// alpha[r] = 2^-E for the GEMM's n_rows output rows (its per-row device
// alpha); otherwise every workgroup returns at once.
__global__ __launch_bounds__(256) void k_x16_fix(const float *__restrict__ x, int K, int ldx, long n4,
                                                 const float *__restrict__ part, int n_part, uint2 *__restrict__ x16,
                                                 float *__restrict__ alpha, int n_rows)
{
    __shared__ float red[4];
    const long G = (long)gridDim.x * 256;
    const int k4 = K / 4;
    const bool flat = ldx == K;
    float m = 0.f;
    for (int j = threadIdx.x; j < n_part; j += 256) m = fmaxf(m, part[j]);
    m = block_max(m, red);
    if (m == 0.f || (m >= kScale1Lo && m < kScale1Hi)) return;
    int e = 0;
    frexpf(m, &e);   // m < 2^e
    e = max(-120, min(120, 15 - e));
    const float sc = ldexpf(1.f, e);
    for (long r = (long)blockIdx.x * 256 + threadIdx.x; r < n_rows; r += G) alpha[r] = ldexpf(1.f, -e);
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += G)
        x16[i] = pack_h4(*(const float4 *)(x + x4_off(i, k4, ldx, flat)), sc);
}

constexpr int kAlgoCands = 8;   // heuristic candidates timed at plan time

// A shape's GEMM: its descriptors and the heuristic's candidates (fixed once
// made); `chosen` is the candidate calls use, -1 until timed (calls then use
// the heuristic's first), published once by the timing call.
struct plan {
    hipblasLtMatmulDesc_t op;
    hipblasLtMatrixLayout_t a, b, d;
    hipblasLtMatmulHeuristicResult_t cand[kAlgoCands];
    int n_cand;
    std::atomic<int> chosen{-1};
};

std::mutex g_mu, g_tune_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<std::tuple<int, int, int, int, int>, std::unique_ptr<plan>> g_plans;

int device_cus_d16()
{
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 256;
    return cus;
}

// The GEMM out[M][ldo] = x16[M][K] . w16[N][K]^T in hipBLASLt's column-major
// terms: D (N x M, ld ldo) = op(A) B with A = w16 stored K x N (transposed) and
// B = x16 stored K x M.
plan *get_plan(int N, int K, int M, int ldo, std::string &err)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) { err = "hipGetDevice failed"; return nullptr; }
    std::lock_guard<std::mutex> lk(g_mu);
    const auto key = std::make_tuple(dev, N, K, M, ldo);
    auto it = g_plans.find(key);
    if (it != g_plans.end()) return it->second.get();
    hipblasLtHandle_t h;
    auto hi = g_handles.find(dev);
    if (hi == g_handles.end()) {
        if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) { err = "hipblasLtCreate failed"; return nullptr; }
        g_handles[dev] = h;
    } else {
        h = hi->second;
    }
    auto pp = std::make_unique<plan>();
    plan &p = *pp;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    const int32_t pm = HIPBLASLT_POINTER_MODE_ALPHA_DEVICE_VECTOR_BETA_HOST;
    const uint64_t wsmax = kBlasWs;
    hipblasLtMatmulPreference_t pref = nullptr;
    int n = 0;
    bool ok = hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_POINTER_MODE, &pm, sizeof pm) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16F, K, N, K) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16F, K, M, K) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&p.d, HIP_R_32F, N, M, ldo) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsmax, sizeof wsmax) ==
                  HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulAlgoGetHeuristic(h, p.op, p.a, p.b, p.d, p.d, pref, kAlgoCands, p.cand, &n) ==
                  HIPBLAS_STATUS_SUCCESS &&
              n > 0;
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (!ok) {
        err = "hipBLASLt has no fp16 x fp16 -> fp32 algorithm for this shape";
        return nullptr;
    }
    p.n_cand = n;
    return g_plans.emplace(key, std::move(pp)).first->second.get();
}

hipblasLtHandle_t handle_for_current()
{
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lk(g_mu);
    return g_handles[dev];
}

// The heuristic's candidates timed on the call's own operands (the better of
// two rounds of 5 runs, after a warm-up) the first time a shape runs outside a
// graph capture; the fastest is kept, the heuristic's first unless another is
// 3% faster.  Every candidate computes the same product.
void time_candidates(plan *p, hipblasLtHandle_t h, const float *alpha, const void *w16, const void *x16, float *out,
                     void *bws, hipStream_t st)
{
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return;
    int best_c = 0;
    float best = 1e30f;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (p->n_cand < 2 || hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        if (e0) (void)hipEventDestroy(e0);
        p->chosen.store(0, std::memory_order_release);
        return;
    }
    const float beta = 0.f;
    for (int c = 0; c < p->n_cand; c++) {
        const hipblasLtMatmulHeuristicResult_t &r = p->cand[c];
        if (r.state != HIPBLAS_STATUS_SUCCESS || r.workspaceSize > kBlasWs) continue;
        auto run = [&] {
            return hipblasLtMatmul(h, p->op, alpha, w16, p->a, x16, p->b, &beta, out, p->d, out, p->d, &r.algo, bws,
                                   r.workspaceSize, st) == HIPBLAS_STATUS_SUCCESS;
        };
        if (!run()) continue;
        float ms = 1e30f;
        bool ok = true;
        for (int round = 0; round < 2 && ok; round++) {
            ok = hipEventRecord(e0, st) == hipSuccess;
            for (int k = 0; k < 5 && ok; k++) ok = run();
            float t = 0.f;
            ok = ok && hipEventRecord(e1, st) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
                 hipEventElapsedTime(&t, e0, e1) == hipSuccess;
            if (ok) ms = std::min(ms, t);
        }
        if (!ok) continue;
        // the heuristic's first candidate unless another is clearly faster
        if (c == 0 ? ms < best : ms < 0.97f * best) {
            best = ms;
            best_c = c;
        }
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    p->chosen.store(best_c, std::memory_order_release);
}

} // namespace

long mllm_d16_bytes(int n_rows, int n_cols) { return (long)n_rows * n_cols * 2; }

int mllm_d16_make(int sem, const mllm_packed &W, int n_rows, int n_cols, void *w16, hipStream_t st, std::string &err)
{
    const long n = (long)n_rows * n_cols;
    if (n <= 0 || n_cols % 4) { err = "n_cols must be a positive multiple of 4"; return -1; }
    float *tmp = nullptr;
    int *bad = nullptr;
    int bad_h = 0;
    if (hipMalloc(&tmp, n * 4) != hipSuccess || hipMalloc(&bad, 4) != hipSuccess) {
        (void)hipFree(tmp);
        err = "hipMalloc of the fp32 staging copy failed";
        return -1;
    }
    int rc = -1;
    // columns past the last whole block stay zero (the reference ignores a ragged tail)
    if (hipMemsetAsync(bad, 0, 4, st) != hipSuccess || hipMemsetAsync(tmp, 0, n * 4, st) != hipSuccess)
        err = "hipMemsetAsync failed";
    else if (mllm_launch_dequant(sem, W, n_rows, n_cols, tmp, st) != 0) err = "semantic has no fp32 weight form";
    else {
        const long n4 = n / 4;
        const unsigned g = (unsigned)std::min<long>((n4 + 255) / 256, 8L * device_cus_d16());
        hipLaunchKernelGGL(k_w16, dim3(g), dim3(256), 0, st, (const float4 *)tmp, n4, (uint2 *)w16, bad);
        if (hipGetLastError() != hipSuccess || hipMemcpyAsync(&bad_h, bad, 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
            err = "fp16 conversion failed";
        else if (bad_h)
            err = "matrix holds weights outside fp16's finite range (|w| >= 65520, inf or NaN): keep it on the quantised path";
        else
            rc = 0;
    }
    (void)hipStreamSynchronize(st);
    (void)hipFree(tmp);
    (void)hipFree(bad);
    return rc;
}

long mllm_d16_workspace_bytes(int n_rows, int n_cols, int M)
{
    return (long)(align256((size_t)M * n_cols * 2) + align256(kPartMax * 4) + align256((size_t)n_rows * 4) + kBlasWs);
}

int mllm_d16_gemm(const void *w16, const float *x, int ldx, int M, float *out, int ldo, int n_rows, int n_cols,
                  void *ws, long ws_bytes, hipStream_t st, std::string &err)
{
    if (M <= 0 || n_rows <= 0 || n_cols <= 0 || n_cols % 4 || ldx % 4 || ldx < n_cols || ldo < n_rows ||
        ((uintptr_t)x & 15) || ((uintptr_t)w16 & 15) || ((uintptr_t)ws & 255)) {
        err = "shape or alignment (n_cols, ldx multiples of 4, 16-byte aligned x and weights, 256-byte aligned workspace)";
        return -1;
    }
    if (!ws || ws_bytes < mllm_d16_workspace_bytes(n_rows, n_cols, M)) { err = "workspace too small"; return -1; }
    plan *p = get_plan(n_rows, n_cols, M, ldo, err);
    if (!p) return -1;
    uint8_t *base = (uint8_t *)ws;
    uint2 *x16 = (uint2 *)base;
    float *part = (float *)(base + align256((size_t)M * n_cols * 2));
    float *alpha = (float *)((uint8_t *)part + align256(kPartMax * 4));
    void *bws = (uint8_t *)alpha + align256((size_t)n_rows * 4);
    const long n4 = (long)M * n_cols / 4;
    const int np = (int)std::min<long>(kPartMax, std::max<long>(1, (n4 + 1023) / 1024));
    hipLaunchKernelGGL(k_x16_cvt1, dim3(np), dim3(256), 0, st, x, n_cols, ldx, n4, part, x16, alpha, n_rows);
    // one workgroup per CU: in the common case each only reads the partials and returns
    const unsigned gc = (unsigned)std::min<long>((n4 + 1023) / 1024, (long)device_cus_d16());
    hipLaunchKernelGGL(k_x16_fix, dim3(gc), dim3(256), 0, st, x, n_cols, ldx, n4, part, np, x16, alpha, n_rows);
    if (hipGetLastError() != hipSuccess) { err = "activation conversion launch failed"; return -1; }
    const hipblasLtHandle_t h = handle_for_current();
    if (p->chosen.load(std::memory_order_acquire) < 0) {
        std::lock_guard<std::mutex> lk(g_tune_mu);
        if (p->chosen.load(std::memory_order_acquire) < 0) time_candidates(p, h, alpha, w16, x16, out, bws, st);
    }
    const int c = std::max(0, p->chosen.load(std::memory_order_acquire));
    const float beta = 0.f;
    const hipblasStatus_t s = hipblasLtMatmul(h, p->op, alpha, w16, p->a, x16, p->b, &beta, out, p->d, out, p->d,
                                              &p->cand[c].algo, bws, p->cand[c].workspaceSize, st);
    if (s != HIPBLAS_STATUS_SUCCESS) { err = "hipblasLtMatmul failed"; return -1; }
    return 0;
}
