// capi.hip — the C ABI of libmllm_gpu.
//
// Two faces:
//   * drop-in entry points with the reference engine's names and signatures
//     (host pointers in, results in the caller's host buffers on return), so
//     the reference's ctypes caller can load this library instead of its
//     combined_engine.so;
//   * mllm_* device-pointer entry points (inputs already in HBM, work queued
//     on a caller stream) used by the benchmarks and by callers that keep
//     activations on the GPU.
//
// Drop-in calls upload each weight matrix once, keyed by its host pointer,
// into the packed plane layout (weights are immutable for an engine's
// lifetime, TE:461-463; mllm_cache_clear() drops the cache).  Each calling
// thread gets its own HIP stream and staging buffers, so concurrent calls
// from ctypes threads (which release the GIL) do not share state.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <map>
#include <mutex>
#include <shared_mutex>
#include <string>
#include <tuple>
#include <vector>
#include "gemm.h"
#include "gemm16.h"
#include "gemv.h"
#include "mllm.h"
#include "moe.h"
#include "dropin.h"

namespace {

thread_local std::string g_last_error;
std::mutex g_log_mu;
std::map<std::string, int> g_logged;

void set_error(const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    std::lock_guard<std::mutex> lk(g_log_mu);
    if (g_logged[buf]++ == 0) fprintf(stderr, "[mllm_gpu] %s\n", buf);
}

#define HIP_OK(expr)                                                                                  \
    do {                                                                                              \
        hipError_t e_ = (expr);                                                                       \
        if (e_ != hipSuccess) {                                                                       \
            set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, __LINE__);    \
            return -1;                                                                                \
        }                                                                                             \
    } while (0)

// ----------------------------------------------------------- entry → semantic
// Which semantic a reference entry point gives each GGUF code.
enum { ENT_QMM = 0, ENT_BMM = 1, ENT_ROWS = 2, ENT_MOE_GU = 3, ENT_MOE_DOWN = 4 };

int sem_for(int entry, int qt)
{
    switch (entry) {
    case ENT_QMM:  // quant_matmul_omp QK:1355-1388
        switch (qt) {
        case 0: return SEM_F32; case 2: return SEM_Q4_0; case 3: return SEM_Q4_1; case 6: return SEM_Q5_0_Q8;
        case 8: return SEM_Q8_0; case 12: return SEM_Q4_K_Q8; case 13: return SEM_Q5_K_GGML;
        case 14: return SEM_Q6_K_LOWNIB; case 39: return SEM_MXFP4;
        }
        return -1;
    case ENT_BMM:  // *_batch_matmul CE:68,216,256,316,381,435
        switch (qt) {
        case 2: return SEM_Q4_0; case 8: return SEM_Q8_0; case 12: return SEM_Q4_K_GGML; case 13: return SEM_Q5_K_CE;
        case 14: return SEM_Q6_K_SEQ; case 39: return SEM_MXFP4_CLAMP;
        }
        return -1;
    case ENT_ROWS:  // batch_qkv_omp / batch_gate_up_omp via matmul_row_range QK:1095-1222
        switch (qt) {
        case 2: return SEM_Q4_0; case 3: return SEM_Q4_1; case 6: return SEM_Q5_0_F32; case 8: return SEM_Q8_0;
        case 12: return SEM_Q4_K_Q8; case 13: return SEM_Q5_K_GGML; case 14: return SEM_Q6_K_LOWNIB;
        case 39: return SEM_MXFP4;
        }
        return -1;
    case ENT_MOE_GU:  // moe_forward_omp gate/up when not both MXFP4, QK:2114-2152
        switch (qt) {
        case 12: return SEM_Q4_K_Q8; case 14: return SEM_Q6_K_LOWNIB; case 2: return SEM_Q4_0;
        case 3: return SEM_Q4_1; case 6: return SEM_Q5_0_Q8;
        }
        return -1;
    case ENT_MOE_DOWN:  // moe_forward_omp down QK:2192-2245 (Q4_K down yields zeros there)
        switch (qt) {
        case 39: return SEM_MXFP4_Q8; case 14: return SEM_Q6_K_LOWNIB; case 2: return SEM_Q4_0;
        case 6: return SEM_Q5_0_F32;
        }
        return -1;
    }
    return -1;
}

long raw_row_bytes(int ly, int n_cols)
{
    if (ly == LY_F32) return (long)n_cols * 4;
    mllm_layout_desc L = mllm_layout_info(ly);
    return (long)(n_cols / L.block_elems) * L.block_bytes;
}

// ----------------------------------------------------------------- device context
struct dev_buf {
    void *p = nullptr;
    size_t n = 0;
    int ensure(size_t bytes)
    {
        if (bytes <= n) return 0;
        if (p) (void)hipFree(p);
        p = nullptr; n = 0;
        size_t want = bytes < 4096 ? 4096 : bytes + bytes / 4;
        if (hipMalloc(&p, want) != hipSuccess) { p = nullptr; return -1; }
        n = want;
        return 0;
    }
};

struct host_buf {
    void *p = nullptr;
    void *dp = nullptr;   // the same memory as a device address (kernels write it over PCIe), or null
    size_t n = 0;
    int ensure(size_t bytes)
    {
        if (bytes <= n) return 0;
        if (p) (void)hipHostFree(p);
        p = dp = nullptr; n = 0;
        size_t want = bytes < 4096 ? 4096 : bytes + bytes / 4;
        if (hipHostMalloc(&p, want, hipHostMallocDefault) != hipSuccess) { p = nullptr; return -1; }
        if (hipHostGetDevicePointer(&dp, p, 0) != hipSuccess) dp = nullptr;
        n = want;
        return 0;
    }
};

// Drop-in results up to this size are written by the kernels straight into the
// pinned staging buffer (posted PCIe writes) instead of device memory plus a
// device-to-host copy: one DMA transfer fewer per call (Q8_0 5632x2048 B=1:
// ~31 -> ~19 us per quant_matmul_omp call on MI355X).
constexpr size_t kDirectOutMax = 256u << 10;

// Per-thread state: stream plus staging/scratch buffers.  Freed only at
// process end (a thread's buffers are reused by its later calls).
struct thread_ctx {
    hipStream_t st = nullptr;
    int device = -1;
    dev_buf d_in, d_out, d_scr, d_tab;
    host_buf h_in, h_out;
    int init()
    {
        if (st) return 0;
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) { set_error("no HIP device"); return -1; }
        if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) {
            set_error("hipStreamCreate failed");
            st = nullptr;
            return -1;
        }
        device = dev;
        return 0;
    }
};
thread_local thread_ctx t_ctx;

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Weight cache: (host pointer, layout, rows, cols, host row stride) -> packed device copy.
struct wkey {
    const void *host;
    int ly, rows, cols;
    long stride;   // 0: rows are contiguous
    bool operator<(const wkey &o) const
    {
        return std::tie(host, ly, rows, cols, stride) < std::tie(o.host, o.ly, o.rows, o.cols, o.stride);
    }
};
struct wentry {
    uint8_t *dev = nullptr;
    long bytes = 0;
    uint64_t fp = 0;
    mllm_packed view;
    int scale_flags = 0;   // mllm_launch_scale_scan of the packed copy
};
std::mutex g_cache_mu;
std::map<wkey, wentry> g_cache;
std::vector<uint8_t *> g_retired;  // replaced device copies, freed by mllm_cache_clear()

// Fingerprint of a host buffer: 64 words sampled across it.  A cache hit
// whose fingerprint changed (the caller freed a matrix and a new one landed
// at the same address) re-uploads instead of using stale weights.
uint64_t fingerprint(const void *p, long n)
{
    const uint8_t *b = (const uint8_t *)p;
    uint64_t h = 1469598103934665603ull ^ (uint64_t)n;
    if (n <= 0) return h;
    for (int i = 0; i < 64; i++) {
        long off = (long)((__int128)n * i / 64);
        uint64_t w = 0;
        memcpy(&w, b + off, (size_t)(n - off < 8 ? n - off : 8));
        h = (h ^ w) * 1099511628211ull;
    }
    uint64_t w = 0;
    memcpy(&w, b + (n >= 8 ? n - 8 : 0), (size_t)(n >= 8 ? 8 : n));
    return (h ^ w) * 1099511628211ull;
}
// (host, E, N) -> routing-layout copy and the fingerprint of the host router it was made from
std::map<std::tuple<const void *, int, int>, std::pair<float *, uint64_t>> g_router_cache;

// Drop-in calls hold this shared for their whole duration; mllm_cache_clear
// takes it exclusively, so it never frees a device copy that a call in flight
// has looked up and not yet finished using.
std::shared_mutex g_api_mu;
#define API_GUARD std::shared_lock<std::shared_mutex> api_guard_(g_api_mu)

// Upload + pack a raw host matrix (once).  Returns its packed view and, with
// scale_flags, the scale scan of the packed copy (mllm_launch_scale_scan, any
// semantic of the layout: the flags depend on the bytes only).
//
// row_stride (bytes, 0 = contiguous rows): row r of the matrix starts at
// host + r * row_stride and holds raw_row_bytes(ly, cols) bytes; the rows are
// gathered on the host before the upload (moe_forward_omp's Q5_0 down rows).
int get_weight(const void *host, int ly, int rows, int cols, mllm_packed &view, int *scale_flags = nullptr,
               long row_stride = 0)
{
    const long rrb = raw_row_bytes(ly, cols);
    if (row_stride == rrb) row_stride = 0;
    wkey k{host, ly, rows, cols, row_stride};
    const long raw = rrb * rows;
    const long span = row_stride && rows > 0 ? (long)(rows - 1) * row_stride + rrb : raw;
    const uint64_t fpr = fingerprint(host, span);
    {
        std::lock_guard<std::mutex> lk(g_cache_mu);
        auto it = g_cache.find(k);
        if (it != g_cache.end()) {
            if (it->second.fp == fpr) {
                view = it->second.view;
                if (scale_flags) *scale_flags = it->second.scale_flags;
                return 0;
            }
            g_retired.push_back(it->second.dev);
            g_cache.erase(it);
        }
    }
    thread_ctx &c = t_ctx;
    const long packed = ly == LY_F32 ? (raw > 0 ? raw : 256) : mllm_packed_bytes(ly, rows, cols, nullptr);
    wentry e;
    e.bytes = packed;
    HIP_OK(hipMalloc(&e.dev, packed));
    e.view = mllm_packed_view(ly, e.dev, rows, cols);
    uint8_t *tmp = nullptr;
    if (raw > 0) {
        const long fo = align256(raw);   // the scan's flag word after the raw bytes
        if (hipMalloc(&tmp, fo + 256) != hipSuccess) { (void)hipFree(e.dev); set_error("hipMalloc(raw %ld) failed", raw); return -1; }
        int *fl = (int *)(tmp + fo);
        const int sem_any = ly == LY_MXFP4 ? SEM_MXFP4 : ly == LY_Q6_K ? SEM_Q6_K_GGML : ly == LY_Q4_K ? SEM_Q4_K_GGML
                          : ly == LY_Q5_K_GGML ? SEM_Q5_K_GGML : ly == LY_Q5_K_CE ? SEM_Q5_K_CE : ly == LY_Q8_0 ? SEM_Q8_0
                          : ly == LY_Q4_0 ? SEM_Q4_0 : ly == LY_Q4_1 ? SEM_Q4_1 : ly == LY_Q5_0 ? SEM_Q5_0_F32 : SEM_F32;
        std::vector<uint8_t> gathered;
        const void *src = host;
        if (row_stride) {
            gathered.resize((size_t)raw);
            for (int r = 0; r < rows; r++)
                memcpy(gathered.data() + (size_t)r * rrb, (const uint8_t *)host + (size_t)r * row_stride, (size_t)rrb);
            src = gathered.data();
        }
        hipError_t r = hipMemcpyAsync(tmp, src, raw, hipMemcpyHostToDevice, c.st);
        if (r == hipSuccess) r = mllm_launch_pack(ly, tmp, e.dev, rows, cols, c.st);
        if (r == hipSuccess) r = mllm_launch_fill((float *)fl, 1, 0.0f, c.st);
        if (r == hipSuccess) r = mllm_launch_scale_scan(nullptr, &e.view, 1, sem_any, rows, cols, fl, c.st);
        if (r == hipSuccess) r = hipMemcpyAsync(&e.scale_flags, fl, sizeof(int), hipMemcpyDeviceToHost, c.st);
        if (r == hipSuccess) r = hipStreamSynchronize(c.st);
        (void)hipFree(tmp);
        if (r != hipSuccess) { (void)hipFree(e.dev); set_error("weight upload failed: %s", hipGetErrorString(r)); return -1; }
    }
    e.fp = fpr;
    std::lock_guard<std::mutex> lk(g_cache_mu);
    auto ins = g_cache.emplace(k, e);
    if (!ins.second) (void)hipFree(e.dev);  // another thread uploaded it first
    view = ins.first->second.view;
    if (scale_flags) *scale_flags = ins.first->second.scale_flags;
    return 0;
}

} // namespace

int mllm_dropin_weight(const void *host, int sem, int rows, int cols, mllm_packed *view, bool *gemv_only)
{
    if (sem < 0 || sem >= SEM_COUNT || !host || rows <= 0 || cols <= 0) { set_error("weight: bad matrix"); return -1; }
    int flags = 0;
    if (get_weight(host, mllm_sem_layout(sem), rows, cols, *view, &flags)) return -1;
    if (gemv_only) *gemv_only = mllm_scales_need_gemv(sem, flags);
    return 0;
}

int mllm_qmm_sem(int qt) { return sem_for(ENT_QMM, qt); }

std::shared_mutex &mllm_api_mutex() { return g_api_mu; }

namespace {

// Several host matrices of one layout and width stacked row-wise into one
// packed device matrix (the q/k/v or gate/up matrices of batch_qkv_omp /
// batch_gate_up_omp, so one GEMV launch covers them), cached by the tuple of
// host pointers and row counts and checked by each matrix's fingerprint.
std::map<std::vector<long>, wentry> g_concat_cache;

int get_weight_concat(const uint8_t *const *hosts, const int *rows, int n, int ly, int cols, mllm_packed &view)
{
    std::vector<long> key;
    uint64_t fp = 1469598103934665603ull;
    long total_rows = 0, total_raw = 0;
    for (int i = 0; i < n; i++) {
        key.push_back((long)(uintptr_t)hosts[i]);
        key.push_back(rows[i]);
        const long raw = raw_row_bytes(ly, cols) * rows[i];
        fp = (fp ^ fingerprint(hosts[i], raw)) * 1099511628211ull;
        total_rows += rows[i];
        total_raw += raw;
    }
    key.push_back(ly);
    key.push_back(cols);
    {
        std::lock_guard<std::mutex> lk(g_cache_mu);
        auto it = g_concat_cache.find(key);
        if (it != g_concat_cache.end()) {
            if (it->second.fp == fp) { view = it->second.view; return 0; }
            g_retired.push_back(it->second.dev);
            g_concat_cache.erase(it);
        }
    }
    thread_ctx &c = t_ctx;
    wentry e;
    e.bytes = mllm_packed_bytes(ly, (int)total_rows, cols, nullptr);
    HIP_OK(hipMalloc(&e.dev, e.bytes));
    uint8_t *tmp = nullptr;
    if (total_raw > 0) {
        if (hipMalloc(&tmp, total_raw) != hipSuccess) { (void)hipFree(e.dev); set_error("hipMalloc(raw %ld) failed", total_raw); return -1; }
        hipError_t r = hipSuccess;
        long off = 0;
        for (int i = 0; i < n && r == hipSuccess; i++) {
            const long raw = raw_row_bytes(ly, cols) * rows[i];
            if (raw > 0) r = hipMemcpyAsync(tmp + off, hosts[i], raw, hipMemcpyHostToDevice, c.st);
            off += raw;
        }
        if (r == hipSuccess) r = mllm_launch_pack(ly, tmp, e.dev, (int)total_rows, cols, c.st);
        if (r == hipSuccess) r = hipStreamSynchronize(c.st);
        (void)hipFree(tmp);
        if (r != hipSuccess) { (void)hipFree(e.dev); set_error("weight upload failed: %s", hipGetErrorString(r)); return -1; }
    }
    e.view = mllm_packed_view(ly, e.dev, (int)total_rows, cols);
    e.fp = fp;
    std::lock_guard<std::mutex> lk(g_cache_mu);
    auto ins = g_concat_cache.emplace(key, e);
    if (!ins.second) (void)hipFree(e.dev);
    view = ins.first->second.view;
    return 0;
}

// Router [E][N] fp32 on the host -> device copy in the routing layout
// (mllm_router_pack: element (i, e) at ((i/4)*E + e)*4 + i%4, zero pad
// rows), cached like the weights: a hit whose host contents changed (a new
// router at a freed one's address) is packed again, the old copy retired.
int get_router(const float *host, int E, int N, const float **dev_out)
{
    auto key = std::make_tuple((const void *)host, E, N);
    const uint64_t fp = fingerprint(host, (long)E * N * 4);
    {
        std::lock_guard<std::mutex> lk(g_cache_mu);
        auto it = g_router_cache.find(key);
        if (it != g_router_cache.end() && it->second.second == fp) { *dev_out = it->second.first; return 0; }
    }
    std::vector<float> t((size_t)mllm_router_packed_floats(N, E), 0.0f);
    for (int e = 0; e < E; e++)
        for (int i = 0; i < N; i++) t[((size_t)(i >> 2) * E + e) * 4 + (i & 3)] = host[(size_t)e * N + i];
    float *d = nullptr;
    HIP_OK(hipMalloc(&d, t.size() * 4));
    HIP_OK(hipMemcpy(d, t.data(), t.size() * 4, hipMemcpyHostToDevice));
    std::lock_guard<std::mutex> lk(g_cache_mu);
    auto it = g_router_cache.find(key);
    if (it == g_router_cache.end()) {
        it = g_router_cache.emplace(key, std::make_pair(d, fp)).first;
    } else if (it->second.second != fp) {
        // another thread may still be reading the old copy: retire it
        g_retired.push_back((uint8_t *)it->second.first);
        it->second = std::make_pair(d, fp);
    } else {
        (void)hipFree(d);   // another thread packed the same contents meanwhile
    }
    *dev_out = it->second.first;
    return 0;
}


long moe_ffn_stride(int which, int qt, int N, int M);

// moe_ffn's per-layer expert table: the three expert tensors of a layer
// (gate, up, down, E experts each at the strides of CE:593-605) -> a device
// array of 3*E packed views, built once per (tensors, shape, types) and
// checked on each call by one fingerprint per tensor (a tensor freed and
// another allocated at its address has other contents), instead of looking
// up and fingerprinting each of the 3*E expert matrices per call.
struct layer_key {
    const void *b[3];
    int qt[3], sem[3], N, E, M;
    bool operator<(const layer_key &o) const
    {
        return std::tie(b[0], b[1], b[2], qt[0], qt[1], qt[2], sem[0], sem[1], sem[2], N, E, M) <
               std::tie(o.b[0], o.b[1], o.b[2], o.qt[0], o.qt[1], o.qt[2], o.sem[0], o.sem[1], o.sem[2], o.N, o.E, o.M);
    }
};
struct layer_entry {
    mllm_packed *dtab = nullptr;
    uint64_t fp[3] = {0, 0, 0};
    int gemv_only = 0;   // mllm_moe_needs_gemv of dtab
};
std::map<layer_key, layer_entry> g_layer_cache;

int get_layer_table(const uint8_t *const bases[3], const int qts[3], const int sems[3], int N, int E, int M,
                    const mllm_packed **dtab_out, int *gemv_only = nullptr)
{
    layer_key k{};
    uint64_t fp[3];
    for (int w = 0; w < 3; w++) {
        k.b[w] = bases[w]; k.qt[w] = qts[w]; k.sem[w] = sems[w];
        fp[w] = fingerprint(bases[w], moe_ffn_stride(w, qts[w], N, M) * E);
    }
    k.N = N; k.E = E; k.M = M;
    {
        std::lock_guard<std::mutex> lk(g_cache_mu);
        auto it = g_layer_cache.find(k);
        if (it != g_layer_cache.end() && !memcmp(it->second.fp, fp, sizeof fp)) {
            *dtab_out = it->second.dtab;
            if (gemv_only) *gemv_only = it->second.gemv_only;
            return 0;
        }
    }
    std::vector<mllm_packed> tab(3 * (size_t)E);
    for (int w = 0; w < 3; w++) {
        const long stride = moe_ffn_stride(w, qts[w], N, M);
        const int rows = w < 2 ? M : N, cols = w < 2 ? N : M;
        for (int e = 0; e < E; e++)
            if (get_weight(bases[w] + (long)e * stride, mllm_sem_layout(sems[w]), rows, cols, tab[(size_t)w * E + e])) return -1;
    }
    mllm_packed *d = nullptr;
    HIP_OK(hipMalloc(&d, tab.size() * sizeof(mllm_packed)));
    HIP_OK(hipMemcpy(d, tab.data(), tab.size() * sizeof(mllm_packed), hipMemcpyHostToDevice));
    const int go = mllm_moe_needs_gemv(d, sems[0], sems[1], sems[2], N, M, E);
    if (go < 0) { (void)hipFree(d); set_error("MoE layer: scale scan failed"); return -1; }
    std::lock_guard<std::mutex> lk(g_cache_mu);
    auto it = g_layer_cache.find(k);
    if (it != g_layer_cache.end()) g_retired.push_back((uint8_t *)it->second.dtab);   // a call in flight may read it
    layer_entry &en = g_layer_cache[k];
    en.dtab = d;
    en.gemv_only = go;
    memcpy(en.fp, fp, sizeof fp);
    *dtab_out = d;
    if (gemv_only) *gemv_only = go;
    return 0;
}

// Scratch layout for the Q8_0 activation pack of T rows x n_cols.
struct xq_bufs {
    int8_t *q; float *d; float *s4; int *sq;
};
size_t xq_bytes(long T, int n_cols)
{
    const long nb = n_cols / 32;
    return align256(T * nb * 32) + 3 * align256(T * nb * 4);
}
xq_bufs xq_carve(void *base, long T, int n_cols)
{
    const long nb = n_cols / 32;
    uint8_t *p = (uint8_t *)base;
    xq_bufs b;
    b.q = (int8_t *)p; p += align256(T * nb * 32);
    b.d = (float *)p; p += align256(T * nb * 4);
    b.s4 = (float *)p; p += align256(T * nb * 4);
    b.sq = (int *)p;
    return b;
}

// The GEMM's activation mode for a semantic.
int gemm_xmode(int sem) { return sem == SEM_Q4_K_Q8 ? XM_Q8 : sem == SEM_MXFP4_Q8 ? XM_Q8D : XM_PLANES; }

// B > 8 tokens run the MFMA GEMM; fp32-activation semantics then need split planes.
bool uses_planes(int sem, int B) { return B > 8 && mllm_qgemm_supported(sem) && gemm_xmode(sem) == XM_PLANES; }
size_t planes_bytes(int sem, long rows, int n_cols)
{
    return align256((size_t)act_nplanes(sem) * act_planes_elems(rows, n_cols) * 2) + align256(rows * 4);
}

// Scratch of run_gemv's GEMM path (B > 8): Q8_0 activation pack, split
// planes, split-K partials.  The GEMV path needs none (Q8_0 activations are
// quantised by the GEMV workgroups).
// The fp16-plane K-quant GEMM (gemm16.hip) serves B > 8 tokens of its
// semantics over whole super-blocks.
bool uses_q16(int sem, int n_cols, int B) { return B > 8 && mllm_q16_supported(sem) && n_cols % 256 == 0; }

size_t gemv_required_bytes(int sem, int n_rows, int n_cols, int B)
{
    if (!(B > 8 && mllm_qgemm_supported(sem) && n_cols >= mllm_sem_block_elems(sem))) return 0;
    if (uses_q16(sem, n_cols, B))
        return (mllm_sem_uses_q8(sem) ? xq_bytes(B, n_cols) : 0) + mllm_act16_bytes(sem, B, n_cols) +
               align256((size_t)mllm_q16_part_floats(sem, n_rows, n_cols, B) * 4);
    return (mllm_sem_uses_q8(sem) ? xq_bytes(B, n_cols) : 0) + (uses_planes(sem, B) ? planes_bytes(sem, B, n_cols) : 0) +
           align256((size_t)mllm_qgemm_part_floats(sem, n_rows, n_cols, B) * 4);
}

// Optional scratch of the batch 2..8 MFMA GEMV: its split-K partials (without
// them short matrices run unsplit, or on the VALU kernel).
size_t gemv_mf_bytes(int sem, int n_rows, int n_cols, int B, bool pro = false, bool pair = false)
{
    if (B < 2 || B > 8) return 0;
    return align256((size_t)mllm_gemv_mf_part_floats(sem, n_rows, n_cols, B, pro, pair) * 4);
}

size_t gemv_scratch_bytes(int sem, int n_rows, int n_cols, int B)
{
    return std::max(gemv_required_bytes(sem, n_rows, n_cols, B), gemv_mf_bytes(sem, n_rows, n_cols, B));
}

// Queue GEMV(s) over B tokens (any B: split into groups of 8) on device data;
// out_add (optional, same layout as out, not overlapping it on the MFMA path)
// is added to the result.
int run_gemv(int sem, const mllm_packed &W, const float *x, float *out, int n_rows, int n_cols, int B,
             void *scratch, hipStream_t st, const float *out_add = nullptr, bool gemm_ok = true)
{
    const bool q8 = mllm_sem_uses_q8(sem);
    if (gemm_ok && uses_q16(sem, n_cols, B)) {
        // prefill / batched K-quants: the fp16-plane MFMA GEMM
        uint8_t *ws = (uint8_t *)scratch;
        mllm_xq xq{};
        if (q8) {
            const xq_bufs xb = xq_carve(ws, B, n_cols);
            HIP_OK(mllm_launch_quantize_q8_0(x, B, n_cols, nullptr, xb.q, xb.d, xb.s4, xb.sq, st));
            xq = {xb.q, xb.d, xb.s4, xb.sq};
            ws += xq_bytes(B, n_cols);
        }
        const act16 ac = mllm_act16_carve(sem, ws, B, n_cols);
        ws += mllm_act16_bytes(sem, B, n_cols);
        HIP_OK(mllm_launch_act16(sem, x, n_cols, q8 ? &xq : nullptr, B, n_cols, ac, st));
        q16_args g{};
        g.W = W;
        g.x = ac;
        g.out = out; g.ldo = n_rows;
        g.n_rows = n_rows; g.n_cols = n_cols; g.n_entries = B;
        g.ksplit = mllm_q16_ksplit(sem, n_rows, n_cols, B);
        if (g.ksplit > 1) g.part = (float *)ws;
        HIP_OK(mllm_launch_q16(sem, false, g, 0, st));
        if (out_add) HIP_OK(mllm_launch_add(out, out_add, (long)B * n_rows, st));
        return 0;
    }
    if (gemm_ok && B > 8 && mllm_qgemm_supported(sem) && n_cols >= mllm_sem_block_elems(sem)) {
        // prefill / batched: quantised-weight MFMA GEMM over the B tokens
        xq_bufs xb{};
        if (q8) {
            xb = xq_carve(scratch, B, n_cols);
            HIP_OK(mllm_launch_quantize_q8_0(x, B, n_cols, nullptr, xb.q, xb.d, xb.s4, xb.sq, st));
        }
        qgemm_args g{};
        g.W = W;
        if (q8) g.xq = {xb.q, xb.d, xb.s4, xb.sq};
        if (uses_planes(sem, B)) {
            uint8_t *pb = (uint8_t *)scratch + (q8 ? xq_bytes(B, n_cols) : 0);
            const long pe = act_planes_elems(B, n_cols);
            int *lo_nz = (int *)(pb + align256((size_t)act_nplanes(sem) * pe * 2));
            HIP_OK(mllm_launch_act_split(x, n_cols, B, n_cols, act_nplanes(sem), (__bf16 *)pb, pe, lo_nz, st));
            g.xp = {(const __bf16 *)pb, pe, act_planes_ld(n_cols), lo_nz};
        }
        g.out = out; g.ldo = n_rows;
        g.n_rows = n_rows; g.n_cols = n_cols; g.n_entries = B;
        g.ksplit = mllm_qgemm_ksplit(sem, n_rows, n_cols, B);
        if (g.ksplit > 1)
            g.part = (float *)((uint8_t *)scratch + (q8 ? xq_bytes(B, n_cols) : 0) +
                               (uses_planes(sem, B) ? planes_bytes(sem, B, n_cols) : 0));
        HIP_OK(mllm_launch_qgemm(sem, gemm_xmode(sem), false, g, 0, st));
        if (out_add) HIP_OK(mllm_launch_add(out, out_add, (long)B * n_rows, st));
        return 0;
    }
    for (int b0 = 0; b0 < B; b0 += 8) {
        mllm_gemv_args a{};
        a.W = W;
        a.x = x + (long)b0 * n_cols;
        a.ldx = n_cols;
        a.out = out + (long)b0 * n_rows;
        a.ldo = n_rows;
        a.n_rows = n_rows; a.n_cols = n_cols; a.B = B - b0 < 8 ? B - b0 : 8;
        a.out_add = out_add ? out_add + (long)b0 * n_rows : nullptr;
        // scratch sized by gemv_scratch_bytes holds the MFMA GEMV's partials at B <= 8
        if (B <= 8 && scratch && gemv_mf_bytes(sem, n_rows, n_cols, B)) a.mf_part = (float *)scratch;
        HIP_OK(mllm_launch_gemv(sem, a, 1, st));
    }
    return 0;
}

// Drop-in GEMV: host W/x/out, B tokens.
int host_gemv(int sem, const uint8_t *W, const float *x, float *out, int n_rows, int n_cols, int B)
{
    if (n_rows <= 0 || B <= 0) return 0;
    thread_ctx &c = t_ctx;
    if (c.init()) return -1;
    const int ly = mllm_sem_layout(sem);
    mllm_packed view;
    int scale_flags = 0;
    if (get_weight(W, ly, n_rows, n_cols, view, &scale_flags)) return -1;
    const size_t xbytes = (size_t)B * n_cols * 4, obytes = (size_t)B * n_rows * 4;
    if (c.d_in.ensure(xbytes) || c.d_out.ensure(obytes) || c.h_in.ensure(xbytes) || c.h_out.ensure(obytes) ||
        c.d_scr.ensure(gemv_scratch_bytes(sem, n_rows, n_cols, B))) {
        set_error("staging allocation failed");
        return -1;
    }
    memcpy(c.h_in.p, x, xbytes);
    HIP_OK(hipMemcpyAsync(c.d_in.p, c.h_in.p, xbytes, hipMemcpyHostToDevice, c.st));
    // B <= 8 runs the GEMV kernels, which write each output once: straight into the pinned buffer
    const bool direct = B <= 8 && obytes <= kDirectOutMax && c.h_out.dp;
    if (run_gemv(sem, view, (const float *)c.d_in.p, (float *)(direct ? c.h_out.dp : c.d_out.p), n_rows, n_cols, B,
                 c.d_scr.p, c.st, nullptr, !mllm_scales_need_gemv(sem, scale_flags)))
        return -1;
    if (!direct) HIP_OK(hipMemcpyAsync(c.h_out.p, c.d_out.p, obytes, hipMemcpyDeviceToHost, c.st));
    HIP_OK(hipStreamSynchronize(c.st));
    memcpy(out, c.h_out.p, obytes);
    return 0;
}

// n matrices applied to one host activation (batch_qkv_omp / batch_gate_up_omp,
// QK:1139-1222): x uploaded once; consecutive matrices of one semantic
// stacked into one packed matrix and run as one GEMV launch; results
// copied back with one transfer and one synchronisation.  A matrix whose
// type the reference's row path does not know (sems[i] < 0) leaves its
// output untouched.
int host_multi_gemv(const int *sems, const uint8_t *const *Ws, float *const *outs, const int *rows, int n,
                    const float *x, int n_cols)
{
    thread_ctx &c = t_ctx;
    if (c.init()) return -1;
    long total = 0;
    for (int i = 0; i < n; i++) total += rows[i] > 0 && sems[i] >= 0 ? rows[i] : 0;
    if (total == 0) return 0;
    const size_t xbytes = (size_t)n_cols * 4, obytes = (size_t)total * 4;
    if (c.d_in.ensure(xbytes) || c.d_out.ensure(obytes) || c.h_in.ensure(xbytes) || c.h_out.ensure(obytes)) {
        set_error("staging allocation failed");
        return -1;
    }
    memcpy(c.h_in.p, x, xbytes);
    HIP_OK(hipMemcpyAsync(c.d_in.p, c.h_in.p, xbytes, hipMemcpyHostToDevice, c.st));
    const bool direct = obytes <= kDirectOutMax && c.h_out.dp;   // B = 1: GEMV kernels write the pinned buffer
    long at = 0;
    for (int i = 0; i < n;) {
        if (sems[i] < 0 || rows[i] <= 0) { i++; continue; }
        int j = i + 1;
        while (j < n && sems[j] == sems[i] && rows[j] > 0) j++;
        int grp_rows = 0;
        for (int k = i; k < j; k++) grp_rows += rows[k];
        mllm_packed view;
        if (j - i == 1 ? get_weight(Ws[i], mllm_sem_layout(sems[i]), rows[i], n_cols, view)
                       : get_weight_concat(Ws + i, rows + i, j - i, mllm_sem_layout(sems[i]), n_cols, view))
            return -1;
        if (run_gemv(sems[i], view, (const float *)c.d_in.p, (float *)(direct ? c.h_out.dp : c.d_out.p) + at, grp_rows,
                     n_cols, 1, nullptr, c.st))
            return -1;
        at += grp_rows;
        i = j;
    }
    if (!direct) HIP_OK(hipMemcpyAsync(c.h_out.p, c.d_out.p, obytes, hipMemcpyDeviceToHost, c.st));
    HIP_OK(hipStreamSynchronize(c.st));
    at = 0;
    for (int i = 0; i < n; i++) {
        if (sems[i] < 0 || rows[i] <= 0) continue;
        memcpy(outs[i], (const float *)c.h_out.p + at, (size_t)rows[i] * 4);
        at += rows[i];
    }
    return 0;
}

int layout_for_qt_bmm(int qt)
{
    int s = sem_for(ENT_BMM, qt);
    return s < 0 ? -1 : mllm_sem_layout(s);
}

// moe_ffn (CE:591-665) reads these fields of the engine's BC struct (x86-64 offsets of CE:536-589).
enum { BC_N = 4, BC_NE = 224, BC_NK = 228, BC_M = 232, BC_ROUTER = 240, BC_GATE = 248, BC_UP = 256, BC_DOWN = 264,
       BC_QG = 272, BC_QU = 276, BC_QD = 280 };

template <class T> static T bc_field(const void *c, int off)
{
    T v;
    memcpy(&v, (const uint8_t *)c + off, sizeof v);
    return v;
}

// moe_ffn's expert strides (CE:593-605): gate/up default to the Q4_K size and
// down to the Q6_K size; only codes 12/13/14/39 change them.
long moe_ffn_stride(int which, int qt, int N, int M)
{
    if (which < 2) {
        long s = (long)M * (N / 256) * 144;
        if (qt == 13) s = (long)M * (N / 256) * 176;
        if (qt == 14) s = (long)M * (N / 256) * 210;
        if (qt == 39) s = (long)M * (N / 32) * 17;
        return s;
    }
    long s = (long)N * (M / 256) * 210;
    if (qt == 12) s = (long)N * (M / 256) * 144;
    if (qt == 13) s = (long)N * (M / 256) * 176;
    if (qt == 39) s = (long)N * (M / 32) * 17;
    return s;
}

} // namespace

// Error reporting for the other translation units of the library.
void mllm_set_error(const char *msg) { set_error("%s", msg); }

// =============================================================== drop-in ABI
extern "C" {

MLLM_API void quant_matmul_omp(const uint8_t *W, const float *x, float *out, int n_rows, int n_cols, int quant_type)
{
    API_GUARD;
    const int sem = sem_for(ENT_QMM, quant_type);
    if (sem < 0) { set_error("quant_matmul_omp: unknown quant type %d (output untouched)", quant_type); return; }
    host_gemv(sem, W, x, out, n_rows, n_cols, 1);
}

MLLM_API void f32_matmul_omp(const float *W, const float *x, float *out, int n_rows, int n_cols)
{
    API_GUARD;
    host_gemv(SEM_F32, (const uint8_t *)W, x, out, n_rows, n_cols, 1);
}

#define MLLM_BMM(name, qt)                                                                           \
    MLLM_API void name(const uint8_t *W, const float *x, float *out, int n_rows, int nc, int B)     \
    {                                                                                                \
        API_GUARD;                                                                                   \
        host_gemv(sem_for(ENT_BMM, qt), W, x, out, n_rows, nc, B);                                 \
    }
MLLM_BMM(q4_0_batch_matmul, 2)
MLLM_BMM(q8_0_batch_matmul, 8)
MLLM_BMM(q4_k_batch_matmul, 12)
MLLM_BMM(q6_k_batch_matmul, 14)
MLLM_BMM(q5_k_batch_matmul, 13)
MLLM_BMM(mxfp4_batch_matmul, 39)
#undef MLLM_BMM

MLLM_API void batch_qkv_omp(const uint8_t *Wq, const uint8_t *Wk, const uint8_t *Wv, const float *x, float *out_q,
                            float *out_k, float *out_v, int nq, int nk, int nv, int n_cols, int qtype_q, int qtype_k,
                            int qtype_v)
{
    API_GUARD;
    const uint8_t *Ws[3] = {Wq, Wk, Wv};
    float *outs[3] = {out_q, out_k, out_v};
    const int ns[3] = {nq, nk, nv}, qts[3] = {qtype_q, qtype_k, qtype_v};
    int sems[3];
    for (int i = 0; i < 3; i++) {
        sems[i] = sem_for(ENT_ROWS, qts[i]);
        if (sems[i] < 0) set_error("batch_qkv_omp: unknown quant type %d (output untouched)", qts[i]);
    }
    host_multi_gemv(sems, Ws, outs, ns, 3, x, n_cols);
}

MLLM_API void batch_gate_up_omp(const uint8_t *Wg, const uint8_t *Wu, const float *x, float *out_gate, float *out_up,
                                int ng, int nu, int n_cols, int qtype_g, int qtype_u)
{
    API_GUARD;
    const uint8_t *Ws[2] = {Wg, Wu};
    float *outs[2] = {out_gate, out_up};
    const int ns[2] = {ng, nu}, qts[2] = {qtype_g, qtype_u};
    int sems[2];
    for (int i = 0; i < 2; i++) {
        sems[i] = sem_for(ENT_ROWS, qts[i]);
        if (sems[i] < 0) set_error("batch_gate_up_omp: unknown quant type %d (output untouched)", qts[i]);
    }
    host_multi_gemv(sems, Ws, outs, ns, 2, x, n_cols);
}

MLLM_API int quantize_row_q8_0(const float *x, uint8_t *q8, int n_cols)
{
    const int nb = n_cols / 32;
    if (nb <= 0) return nb;
    thread_ctx &c = t_ctx;
    if (c.init()) return nb;
    const size_t xb = (size_t)n_cols * 4, qb = (size_t)nb * 34;
    if (c.d_in.ensure(xb) || c.d_out.ensure(qb) || c.h_in.ensure(xb) || c.h_out.ensure(qb)) { set_error("staging allocation failed"); return nb; }
    memcpy(c.h_in.p, x, xb);
    if (hipMemcpyAsync(c.d_in.p, c.h_in.p, xb, hipMemcpyHostToDevice, c.st) != hipSuccess ||
        mllm_launch_quantize_q8_0((const float *)c.d_in.p, 1, n_cols, (uint8_t *)c.d_out.p, nullptr, nullptr, nullptr,
                                  nullptr, c.st) != hipSuccess ||
        hipMemcpyAsync(c.h_out.p, c.d_out.p, qb, hipMemcpyDeviceToHost, c.st) != hipSuccess ||
        hipStreamSynchronize(c.st) != hipSuccess) {
        set_error("quantize_row_q8_0 failed");
        return nb;
    }
    memcpy(q8, c.h_out.p, qb);
    return nb;
}

// *_dequantize_row (QK:762-878): the ggml definitions, rounded as the reference rounds them.
static void dequant_row(int sem, const uint8_t *W, float *out, int n_values)
{
    API_GUARD;
    if (n_values <= 0) return;
    thread_ctx &c = t_ctx;
    if (c.init()) return;
    mllm_packed view;
    if (get_weight(W, mllm_sem_layout(sem), 1, n_values, view)) return;
    const size_t ob = (size_t)n_values * 4;
    if (c.d_out.ensure(ob) || c.h_out.ensure(ob)) { set_error("staging allocation failed"); return; }
    if (mllm_launch_dequant(sem, view, 1, n_values, (float *)c.d_out.p, c.st) != 0) return;
    if (hipMemcpyAsync(c.h_out.p, c.d_out.p, ob, hipMemcpyDeviceToHost, c.st) != hipSuccess ||
        hipStreamSynchronize(c.st) != hipSuccess) { set_error("dequantize_row failed"); return; }
    memcpy(out, c.h_out.p, ob);
}
MLLM_API void q4_k_dequantize_row(const uint8_t *W, float *out, int n_values) { dequant_row(SEM_Q4_K_GGML, W, out, n_values); }
MLLM_API void q5_k_dequantize_row(const uint8_t *W, float *out, int n_values) { dequant_row(SEM_Q5_K_GGML, W, out, n_values); }
MLLM_API void q6_k_dequantize_row(const uint8_t *W, float *out, int n_values) { dequant_row(SEM_Q6_K_GGML, W, out, n_values); }
MLLM_API void q8_0_dequantize_row(const uint8_t *W, float *out, int n_values) { dequant_row(SEM_Q8_0, W, out, n_values); }

MLLM_API void set_num_threads(int n) { (void)n; }
MLLM_API int get_max_threads(void)
{
    int dev = 0, cus = 1;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    return cus;
}

// moe_forward_omp (QK:2066-2250): caller-supplied routing; gate/up per
// type, SiLU clamped to +-80, down per type (MXFP4 through Q8_0(h)), and
// combined[row] = sum_k w_k * down_k in k order (the reference sums with
// an OpenMP atomic in no fixed order).  prealloc_buf is not written.
MLLM_API void moe_forward_omp(const uint8_t **gate_raw, const uint8_t **up_raw, const uint8_t **down_raw,
                              const float *x_norm, int n_ff_expert, int n_embd, int qt_gate, int qt_up, int qt_down,
                              const int *top_indices, const float *top_weights, int top_k, float *combined,
                              float *prealloc_buf, uint8_t *prealloc_q8)
{
    API_GUARD;
    (void)prealloc_buf;
    if (n_embd <= 0) return;
    if (top_k <= 0) { memset(combined, 0, (size_t)n_embd * 4); return; }   // the reference clears combined (QK:2179)
    if (top_k > 64) { set_error("moe_forward_omp: top_k %d > 64", top_k); return; }
    thread_ctx &c = t_ctx;
    if (c.init()) return;
    const bool pair_mx = qt_gate == 39 && qt_up == 39;  // QK:2094
    const int sg = pair_mx ? SEM_MXFP4 : sem_for(ENT_MOE_GU, qt_gate);
    const int su = pair_mx ? SEM_MXFP4 : sem_for(ENT_MOE_GU, qt_up);
    int sd = sem_for(ENT_MOE_DOWN, qt_down);
    if (qt_down == 39 && !prealloc_q8) {
        set_error("moe_forward_omp: MXFP4 down projection needs prealloc_q8 (the reference dereferences NULL); down treated as zero");
        sd = -1;
    }
    // Q5_0 down rows start row * ((n_embd+31)/32)*22 bytes in (QK:2216, 2230): a
    // stride from n_embd, not from the n_ff-wide rows.  Followed where every row
    // stays inside the n_embd x n_ff matrix (n_embd < n_ff); where the reference
    // reads past the matrix (n_embd > n_ff) the matrix's own rows are used.
    long q5_stride = 0;
    if (qt_down == 6 && n_ff_expert > 0) {
        const long s_ref = (long)((n_embd + 31) / 32) * 22, s_own = (long)((n_ff_expert + 31) / 32) * 22;
        if (s_ref != s_own && (long)(n_embd - 1) * s_ref + (long)(n_ff_expert / 32) * 22 <= (long)n_embd * s_own)
            q5_stride = s_ref;
    }
    // slots with a negative expert id (left empty by a routing) add nothing and are dropped;
    // the remaining slots keep their order, so the k-order combine is unchanged
    std::vector<int> sel;
    std::vector<float> selw;
    for (int k = 0; k < top_k; k++)
        if (top_indices[k] >= 0) { sel.push_back(top_indices[k]); selw.push_back(top_weights[k]); }
    if (sel.empty()) { memset(combined, 0, (size_t)n_embd * 4); return; }
    const int K = (int)sel.size(), F = n_ff_expert, N = n_embd;
    // tables of the selected experts' packed views: [0,K) gate, [K,2K) up, [2K,3K) down
    std::vector<mllm_packed> tab(3 * K);
    for (int k = 0; k < K; k++) {
        const int e = sel[k];
        if (sg >= 0 && get_weight(gate_raw[e], mllm_sem_layout(sg), F, N, tab[k])) return;
        if (su >= 0 && get_weight(up_raw[e], mllm_sem_layout(su), F, N, tab[K + k])) return;
        if (sd >= 0 && get_weight(down_raw[e], mllm_sem_layout(sd), N, F, tab[2 * K + k], nullptr, q5_stride)) return;
    }
    // device scratch: x | g[K][F] | u[K][F] | h[K][F] | dn[K][N] | w[K]
    // device scratch: tab | x | w (one upload from the same layout in the pinned buffer) | g[K][F] | u[K][F] |
    // h[K][F] | dn[K][N]; tables: [0,K) gate, [K,2K) up, [2K,3K) down
    const size_t tab_b = tab.size() * sizeof(mllm_packed);
    size_t o_x = align256(tab_b), o_w = o_x + (size_t)N * 4, in_b = o_w + (size_t)K * 4,
           o_g = align256(in_b), o_u = align256(o_g + (size_t)K * F * 4), o_h = align256(o_u + (size_t)K * F * 4),
           o_dn = align256(o_h + (size_t)K * F * 4), total = align256(o_dn + (size_t)K * N * 4);
    if (c.d_scr.ensure(total) || c.h_in.ensure(in_b) || c.h_out.ensure(N * 4)) {
        set_error("moe_forward_omp: scratch allocation failed");
        return;
    }
    uint8_t *S = (uint8_t *)c.d_scr.p;
    float *dx = (float *)(S + o_x), *dg = (float *)(S + o_g), *du = (float *)(S + o_u), *dh = (float *)(S + o_h),
          *ddn = (float *)(S + o_dn), *dw = (float *)(S + o_w);
    uint8_t *hin = (uint8_t *)c.h_in.p;
    memcpy(hin, tab.data(), tab_b);
    memcpy(hin + o_x, x_norm, N * 4);
    memcpy(hin + o_w, selw.data(), K * 4);
    mllm_packed *dtab = (mllm_packed *)S;
    hipStream_t st = c.st;
    // the combine writes its N outputs straight into the pinned buffer (dx is read by the GEMVs before it)
    const bool direct = (size_t)N * 4 <= kDirectOutMax && c.h_out.dp;
    float *cdst = direct ? (float *)c.h_out.dp : dx;
#define CK(expr) do { if ((expr) != hipSuccess) { set_error("moe_forward_omp: %s failed", #expr); return; } } while (0)
    CK(hipMemcpyAsync(S, hin, in_b, hipMemcpyHostToDevice, st));
    // gate and up in one launch when their semantics agree; Q8_0 activations
    // quantised by the GEMV workgroups; silu(g) * u formed by the down
    // projection's staging (fp32 activations) or its quantisation (Q8_0)
    mllm_gemv_args a{};
    a.table = dtab; a.x = dx; a.x_job_stride = 0; a.ldx = N;
    a.out = dg; a.out_job_stride = F; a.ldo = F;
    a.n_rows = F; a.n_cols = N; a.B = 1;
    if (sg >= 0 && sg == su && sd >= 0 && sd != SEM_F32 && mllm_gemv_fused_fits(sg, N, 1, false)) {
        // gate, up and the clamped SiLU product in one launch (paired rows), then the down projection of h
        a.table2 = dtab + K; a.silu_pair = 1; a.out = dh;
        CK(mllm_launch_gemv(sg, a, K, st));
        mllm_gemv_args b{};
        b.table = dtab + 2 * K; b.x = dh; b.x_job_stride = F; b.ldx = F;
        b.out = ddn; b.out_job_stride = N; b.ldo = N;
        b.n_rows = N; b.n_cols = F; b.B = 1;
        CK(mllm_launch_gemv(sd, b, K, st));
        CK(mllm_launch_combine(ddn, dw, nullptr, 1, K, N, cdst, 0, st));
        if (!direct) CK(hipMemcpyAsync(c.h_out.p, dx, N * 4, hipMemcpyDeviceToHost, st));
        CK(hipStreamSynchronize(st));
        memcpy(combined, c.h_out.p, N * 4);
        return;
    }
    if (sg >= 0 && sg == su) {
        a.job_split = K; a.table2 = dtab + K; a.out2 = du;
        CK(mllm_launch_gemv(sg, a, 2 * K, st));
    } else {
        if (sg >= 0) CK(mllm_launch_gemv(sg, a, K, st));
        else CK(hipMemsetAsync(dg, 0, (size_t)K * F * 4, st));
        a.table = dtab + K; a.out = du;
        if (su >= 0) CK(mllm_launch_gemv(su, a, K, st));
        else CK(hipMemsetAsync(du, 0, (size_t)K * F * 4, st));
    }
    if (sd >= 0) {
        mllm_gemv_args b{};
        b.table = dtab + 2 * K; b.x = dg; b.x_job_stride = F; b.ldx = F;
        b.out = ddn; b.out_job_stride = N; b.ldo = N;
        b.n_rows = N; b.n_cols = F; b.B = 1;
        if (sd == SEM_F32) {
            CK(mllm_launch_silu_mul(dg, du, dh, (long)K * F, 1, st));
            b.x = dh;
        } else {
            b.x_up = du;
        }
        CK(mllm_launch_gemv(sd, b, K, st));
    }
    CK(mllm_launch_combine(sd >= 0 ? ddn : nullptr, dw, nullptr, 1, K, N, cdst, 0, st));
    if (!direct) CK(hipMemcpyAsync(c.h_out.p, dx, N * 4, hipMemcpyDeviceToHost, st));
    CK(hipStreamSynchronize(st));
#undef CK
    memcpy(combined, c.h_out.p, N * 4);
}

int mllm_moe_ffn_host_batched(const float *router, const uint8_t *const bases[3], const int qts[3], int N, int E, int K,
                              int M, const float *x_host, float *out_host, int T);

MLLM_API void moe_ffn(const void *c, int l, float *x, float *gate_buf, float *up_buf, float *ffn_buf, int B)
{
    API_GUARD;
    (void)gate_buf; (void)up_buf;
    if (B <= 0) return;
    const int N = bc_field<int>(c, BC_N), E = bc_field<int>(c, BC_NE), K = bc_field<int>(c, BC_NK),
              M = bc_field<int>(c, BC_M);
    const int qts[3] = {bc_field<int>(c, BC_QG), bc_field<int>(c, BC_QU), bc_field<int>(c, BC_QD)};
    const float *router = bc_field<const float **>(c, BC_ROUTER)[l];
    const uint8_t *bases[3] = {bc_field<const uint8_t **>(c, BC_GATE)[l], bc_field<const uint8_t **>(c, BC_UP)[l],
                               bc_field<const uint8_t **>(c, BC_DOWN)[l]};
    // With B > 1 the reference clears ffn_buf per token, so only the last token's result survives (CE:610-643).
    mllm_moe_ffn_dev_tokens(router, bases, qts, N, E, K, M, x + (long)(B - 1) * N, ffn_buf, 1);
}

// moe_ffn (CE:591-665) applied to each of B tokens, every token's result kept:
// ffn_out[b*N + n].  No scratch of the caller's is used.
MLLM_API void moe_ffn_batched(const void *c, int l, const float *x, float *ffn_out, int B)
{
    API_GUARD;
    if (B <= 0) return;
    const int N = bc_field<int>(c, BC_N), E = bc_field<int>(c, BC_NE), K = bc_field<int>(c, BC_NK),
              M = bc_field<int>(c, BC_M);
    const int qts[3] = {bc_field<int>(c, BC_QG), bc_field<int>(c, BC_QU), bc_field<int>(c, BC_QD)};
    const float *router = bc_field<const float **>(c, BC_ROUTER)[l];
    const uint8_t *bases[3] = {bc_field<const uint8_t **>(c, BC_GATE)[l], bc_field<const uint8_t **>(c, BC_UP)[l],
                               bc_field<const uint8_t **>(c, BC_DOWN)[l]};
    mllm_moe_ffn_host_batched(router, bases, qts, N, E, K, M, x, ffn_out, B);
}


MLLM_API const char *mllm_last_error(void) { return g_last_error.c_str(); }

MLLM_API void mllm_cache_clear(void)
{
    std::unique_lock<std::shared_mutex> api(g_api_mu);   // waits for drop-in calls in flight
    std::lock_guard<std::mutex> lk(g_cache_mu);
    (void)hipDeviceSynchronize();
    for (auto &kv : g_layer_cache) (void)hipFree(kv.second.dtab);
    g_layer_cache.clear();
    for (auto &kv : g_concat_cache) (void)hipFree(kv.second.dev);
    g_concat_cache.clear();
    for (auto &kv : g_cache) (void)hipFree(kv.second.dev);
    g_cache.clear();
    for (uint8_t *p : g_retired) (void)hipFree(p);
    g_retired.clear();
    for (auto &kv : g_router_cache) (void)hipFree(kv.second.first);
    g_router_cache.clear();
    mllm_gptoss_cache_clear();
    mllm_qwen36_cache_clear();
}

// ====================================================== device-pointer ABI
MLLM_API int mllm_sem_for(int entry, int quant_type) { return sem_for(entry, quant_type); }

MLLM_API long mllm_packed_size(int sem, int n_rows, int n_cols)
{
    if (sem < 0 || sem >= SEM_COUNT || n_rows < 0 || n_cols < 0) return -1;
    const int ly = mllm_sem_layout(sem);
    if (ly == LY_F32) return (long)n_rows * n_cols * 4;
    return mllm_packed_bytes(ly, n_rows, n_cols, nullptr);
}

MLLM_API long mllm_raw_size(int sem, int n_rows, int n_cols)
{
    if (sem < 0 || sem >= SEM_COUNT) return -1;
    return raw_row_bytes(mllm_sem_layout(sem), n_cols) * n_rows;
}

MLLM_API int mllm_pack(int sem, const void *raw_dev, void *packed_dev, int n_rows, int n_cols, void *stream)
{
    if (sem < 0 || sem >= SEM_COUNT) { set_error("mllm_pack: bad semantic %d", sem); return -1; }
    HIP_OK(mllm_launch_pack(mllm_sem_layout(sem), (const uint8_t *)raw_dev, (uint8_t *)packed_dev, n_rows, n_cols,
                            (hipStream_t)stream));
    return 0;
}

MLLM_API long mllm_gemv_workspace_size(int sem, int n_rows, int n_cols, int B)
{
    return (long)gemv_scratch_bytes(sem, n_rows, n_cols, B);
}

MLLM_API int mllm_gemv(int sem, const void *packed_dev, const float *x_dev, float *out_dev, int n_rows, int n_cols,
                       int B, void *workspace, void *stream)
{
    if (sem < 0 || sem >= SEM_COUNT) { set_error("mllm_gemv: bad semantic %d", sem); return -1; }
    if (((uintptr_t)x_dev & 15) || ((uintptr_t)packed_dev & 255)) { set_error("mllm_gemv: misaligned pointer"); return -1; }
    if (gemv_required_bytes(sem, n_rows, n_cols, B) && !workspace) { set_error("mllm_gemv: semantic %d needs a workspace", sem); return -1; }
    mllm_packed view = mllm_packed_view(mllm_sem_layout(sem), (const uint8_t *)packed_dev, n_rows, n_cols);
    return run_gemv(sem, view, x_dev, out_dev, n_rows, n_cols, B, workspace, (hipStream_t)stream);
}

// --------------------------------------------------- fused decode GEMV (f1)
static bool fusion_has_pro(const mllm_gemv_fusion *f) { return f && (f->x_res || f->res_out || f->rms_w); }
static int fusion_ld(const mllm_gemv_fusion *f, int n_cols) { return f && f->x_ld ? f->x_ld : n_cols; }
static bool fusion_pair(const mllm_gemv_fusion *f) { return f && f->silu_pair; }

// Whether one decode-GEMV launch takes the whole fusion.  Otherwise the
// activation is formed by its own kernel into the workspace, paired rows run
// as one GEMV over both halves followed by the SiLU product, and on the MFMA
// path the residual is added after the GEMM.
static bool fusion_direct(int sem, int n_rows, int n_cols, int B, const mllm_gemv_fusion *f)
{
    if (B > 8 || sem == SEM_F32 || n_cols < mllm_sem_block_elems(sem)) return false;
    const bool pro = fusion_has_pro(f), pair = fusion_pair(f);
    if (pro && (n_cols % 4 || fusion_ld(f, n_cols) % 4)) return false;
    // batch 2..8 on the matrix cores: prologue, paired rows and residual in one launch
    if (B >= 2 && !(f && f->x_up) && mllm_gemv_mf_fits(sem, n_rows, n_cols, B, pro, pair, true)) return true;
    if (pair && B != 1) return false;
    if (pro || pair) return mllm_gemv_fused_fits(sem, n_cols, B, pro);
    if (f && f->x_up) return mllm_sem_uses_q8(sem) || B == 1;
    return true;
}

// workspace: [activation B x n_cols] [residual copy B x n_rows] [pair output B x 2 n_rows] [GEMV scratch];
// on the one-launch path only the MFMA GEMV's split-K partials
struct fused_ws { size_t keep, pair, gemv, total; };
static fused_ws fused_layout(int sem, int n_rows, int n_cols, int B, const mllm_gemv_fusion *f)
{
    fused_ws w{0, 0, 0, 0};
    if (fusion_direct(sem, n_rows, n_cols, B, f)) {
        w.total = gemv_mf_bytes(sem, n_rows, n_cols, B, fusion_has_pro(f), fusion_pair(f));
        return w;
    }
    const bool pair = fusion_pair(f);
    size_t o = 0;
    if (f && (fusion_has_pro(f) || f->x_up)) o += align256((size_t)B * n_cols * 4);
    w.keep = o;
    if (f && f->out_add && B > 8 && !pair) o += align256((size_t)B * n_rows * 4);
    w.pair = o;
    if (pair) o += align256((size_t)B * 2 * n_rows * 4);
    w.gemv = o;
    w.total = o + gemv_scratch_bytes(sem, pair ? 2 * n_rows : n_rows, n_cols, B);
    return w;
}

MLLM_API long mllm_gemv_fused_workspace_size(int sem, int n_rows, int n_cols, int B, const mllm_gemv_fusion *f)
{
    if (sem < 0 || sem >= SEM_COUNT || B <= 0) return -1;
    return (long)fused_layout(sem, n_rows, n_cols, B, f).total;
}

MLLM_API int mllm_gemv_fused(int sem, const void *packed_dev, const float *x_dev, float *out_dev, int n_rows,
                             int n_cols, int B, const mllm_gemv_fusion *f, void *workspace, void *stream)
{
    if (sem < 0 || sem >= SEM_COUNT) { set_error("mllm_gemv_fused: bad semantic %d", sem); return -1; }
    if (n_rows <= 0 || B <= 0) return 0;
    if (((uintptr_t)x_dev & 15) || ((uintptr_t)packed_dev & 255)) { set_error("mllm_gemv_fused: misaligned pointer"); return -1; }
    const bool pro = fusion_has_pro(f), pair = fusion_pair(f);
    if ((pro || pair) && f->x_up) {
        set_error("mllm_gemv_fused: x_up excludes the residual/norm prologue and paired rows");
        return -1;
    }
    if (f && (((uintptr_t)f->x_up | (uintptr_t)f->x_res | (uintptr_t)f->res_out | (uintptr_t)f->rms_w |
               (uintptr_t)f->out_add) & 15)) {
        set_error("mllm_gemv_fused: fusion vectors must be 16-byte aligned");
        return -1;
    }
    const int ldx = fusion_ld(f, n_cols);
    if (ldx < n_cols) { set_error("mllm_gemv_fused: x_ld %d < n_cols %d", ldx, n_cols); return -1; }
    if (f && f->res_out) {
        // res_out is written while other workgroups still read x and x_res
        const size_t span = ((size_t)(B - 1) * ldx + n_cols) * 4;
        const uintptr_t ro = (uintptr_t)f->res_out, re = ro + span;
        auto overlaps = [&](const void *p) {
            const uintptr_t a = (uintptr_t)p, b = a + span;
            return p && a < re && ro < b;
        };
        if (overlaps(x_dev) || overlaps(f->x_res)) { set_error("mllm_gemv_fused: res_out overlaps x or x_res"); return -1; }
    }
    const fused_ws L = fused_layout(sem, n_rows, n_cols, B, f);
    const bool direct = fusion_direct(sem, n_rows, n_cols, B, f);
    // one launch: the MFMA GEMV's partials are optional where it also runs unsplit,
    // or where the VALU kernel takes the same fusion
    const bool ws_optional = direct && (mllm_gemv_mf_fits(sem, n_rows, n_cols, B, pro, pair, false) ||
                                        !(pair && B != 1));
    if (L.total && !workspace && !ws_optional) {
        set_error("mllm_gemv_fused: needs a workspace of %zu bytes", L.total);
        return -1;
    }
    hipStream_t st = (hipStream_t)stream;
    const int mrows = pair ? 2 * n_rows : n_rows;   // rows of the matrix (the stacked gate/up pair)
    mllm_packed view = mllm_packed_view(mllm_sem_layout(sem), (const uint8_t *)packed_dev, mrows, n_cols);
    const float *out_add = f ? f->out_add : nullptr;
    if (direct) {
        mllm_gemv_args a{};
        a.W = view;
        a.mf_part = L.total ? (float *)workspace : nullptr;
        a.x = x_dev; a.ldx = ldx;
        a.out = out_dev; a.ldo = n_rows;
        a.n_rows = n_rows; a.n_cols = n_cols; a.B = B;
        if (f) {
            a.x_up = f->x_up; a.silu_noclamp = !f->silu_clamp;
            a.x_res = f->x_res; a.res_out = f->res_out; a.rms_w = f->rms_w; a.rms_eps = f->rms_eps;
            a.rms_div = f->rms_div;
            a.out_add = out_add;
            a.silu_pair = f->silu_pair ? 1 : 0;
        }
        HIP_OK(mllm_launch_gemv(sem, a, 1, st));
        return 0;
    }
    uint8_t *ws = (uint8_t *)workspace;
    const float *xa = x_dev;
    if (f && (pro || f->x_up)) {
        float *xe = (float *)ws;
        HIP_OK(mllm_launch_act_prologue(x_dev, f->x_res, f->res_out, f->rms_w, f->rms_eps, f->rms_div, f->x_up,
                                        f->silu_clamp, B, n_cols, ldx, xe, st));
        xa = xe;
    } else if (ldx != n_cols) {
        set_error("mllm_gemv_fused: a strided x (x_ld) needs a fused activation step on this path");
        return -1;
    }
    if (pair) {
        float *y = (float *)(ws + L.pair);
        if (run_gemv(sem, view, xa, y, mrows, n_cols, B, ws + L.gemv, st)) return -1;
        HIP_OK(mllm_launch_silu_pair(y, B, n_rows, f->silu_clamp, out_dev, out_add, st));
        return 0;
    }
    if (out_add && B > 8) {
        // the MFMA path writes out before the residual is added: add from a copy
        float *keep = (float *)(ws + L.keep);
        HIP_OK(hipMemcpyAsync(keep, out_add, (size_t)B * n_rows * 4, hipMemcpyDeviceToDevice, st));
        out_add = keep;
    }
    return run_gemv(sem, view, xa, out_dev, n_rows, n_cols, B, ws + L.gemv, st, out_add);
}

// ------------------------------------------------ lm_head requantisation (f2)
static int requant_sem(int qt) { return qt == 12 ? SEM_Q4_K_GGML : qt == 14 ? SEM_Q6_K_GGML : -1; }
constexpr int kQtF16 = 1;   // TE:519-522: F16 output matrices are requantised too

MLLM_API long mllm_requantize_workspace_size(int quant_type, int n_rows, int n_cols)
{
    if (n_rows <= 0 || n_cols <= 0) return -1;
    if (quant_type == kQtF16) return (long)align256((size_t)n_rows * n_cols * 4);
    const int sem = requant_sem(quant_type);
    if (sem < 0) return -1;
    return (long)(align256(mllm_packed_bytes(mllm_sem_layout(sem), n_rows, n_cols, nullptr)) +
                  align256((size_t)n_rows * n_cols * 4));
}

MLLM_API int mllm_requantize_q8_0(int quant_type, const void *raw_dev, int n_rows, int n_cols, void *q8_dev,
                                  void *workspace, void *stream)
{
    const int sem = requant_sem(quant_type);
    if (sem < 0 && quant_type != kQtF16) {
        set_error("mllm_requantize_q8_0: type %d is not requantised (Q4_K, Q6_K and F16 only, TE:515-522)", quant_type);
        return -1;
    }
    if (quant_type == kQtF16 && n_cols % 32) {
        set_error("mllm_requantize_q8_0: F16 rows of whole 32-element blocks only (TE:650-651 reshapes by 32)");
        return -1;
    }
    if (n_rows <= 0 || n_cols < 32) return 0;
    if (!workspace) { set_error("mllm_requantize_q8_0: needs a workspace"); return -1; }
    hipStream_t st = (hipStream_t)stream;
    if (quant_type == kQtF16) {
        // TE:643-645: the patterns' integer values, then TE's Q8_0 statements
        float *f32 = (float *)workspace;
        HIP_OK(mllm_launch_u16_value_f32((const uint16_t *)raw_dev, (long)n_rows * n_cols, f32, st));
        HIP_OK(mllm_launch_requant_q8_0(f32, n_rows, n_cols, (uint8_t *)q8_dev, st));
        return 0;
    }
    const int ly = mllm_sem_layout(sem);
    uint8_t *packed = (uint8_t *)workspace;
    float *f32 = (float *)(packed + align256(mllm_packed_bytes(ly, n_rows, n_cols, nullptr)));
    HIP_OK(mllm_launch_pack(ly, (const uint8_t *)raw_dev, packed, n_rows, n_cols, st));
    // columns past the last whole super-block stay 0 (TE's np.zeros buffer)
    if (n_cols % 256) HIP_OK(mllm_launch_fill(f32, (long)n_rows * n_cols, 0.0f, st));
    if (n_cols >= 256 &&
        mllm_launch_dequant(sem, mllm_packed_view(ly, packed, n_rows, n_cols), n_rows, n_cols, f32, st) != 0) {
        set_error("mllm_requantize_q8_0: dequantisation failed");
        return -1;
    }
    HIP_OK(mllm_launch_requant_q8_0(f32, n_rows, n_cols, (uint8_t *)q8_dev, st));
    return 0;
}

MLLM_API int requantize_output_q8_0(const uint8_t *W, int n_rows, int n_cols, int quant_type, uint8_t *out)
{
    API_GUARD;
    const int sem = requant_sem(quant_type);
    if (sem < 0 && quant_type != kQtF16) {
        set_error("requantize_output_q8_0: type %d is not requantised (Q4_K, Q6_K and F16 only)", quant_type);
        return -1;
    }
    if (quant_type == kQtF16 && n_cols % 32) {
        set_error("requantize_output_q8_0: F16 rows of whole 32-element blocks only (TE:650-651 reshapes by 32)");
        return -1;
    }
    if (n_rows <= 0 || n_cols < 32) return 0;
    thread_ctx &c = t_ctx;
    if (c.init()) return -1;
    const size_t raw = quant_type == kQtF16 ? (size_t)n_rows * n_cols * 2
                                            : (size_t)raw_row_bytes(mllm_sem_layout(sem), n_cols) * n_rows;
    const size_t q8 = (size_t)n_rows * (n_cols / 32) * 34;
    const long ws = mllm_requantize_workspace_size(quant_type, n_rows, n_cols);
    // a load-time conversion: its buffers are allocated for the call and freed after it
    void *d_raw = nullptr, *d_q8 = nullptr, *d_ws = nullptr;
    int rc = -1;
    if (hipMalloc(&d_raw, raw ? raw : 256) == hipSuccess && hipMalloc(&d_q8, q8) == hipSuccess &&
        hipMalloc(&d_ws, ws) == hipSuccess && hipMemcpyAsync(d_raw, W, raw, hipMemcpyHostToDevice, c.st) == hipSuccess &&
        mllm_requantize_q8_0(quant_type, d_raw, n_rows, n_cols, d_q8, d_ws, c.st) == 0 &&
        hipMemcpyAsync(out, d_q8, q8, hipMemcpyDeviceToHost, c.st) == hipSuccess && hipStreamSynchronize(c.st) == hipSuccess)
        rc = 0;
    (void)hipFree(d_raw); (void)hipFree(d_q8); (void)hipFree(d_ws);
    if (rc) set_error("requantize_output_q8_0 failed");
    return rc;
}

// gqa_attention.c:93: one token's attention through mllm_gqa_decode (mode 1)
// on uploaded copies of q, K and V; workspace is not written.
MLLM_API void gqa_attention_decode(const float *q, const float *k_cache, const float *v_cache, float *out, int seq_len,
                                   int n_head, int n_kv_head, int head_dim, float *workspace)
{
    API_GUARD;
    (void)workspace;
    if (n_head <= 0 || head_dim <= 0) return;
    if (n_kv_head <= 0 || n_head % n_kv_head || n_head / n_kv_head > 16 || head_dim > 256 || head_dim % 4) {
        set_error("gqa_attention_decode: n_head %% n_kv_head == 0, n_head / n_kv_head <= 16 and head_dim <= 256, a "
                  "multiple of 4, are served (output untouched)");
        return;
    }
    const size_t qo = (size_t)n_head * head_dim * 4;
    if (seq_len <= 0) { memset(out, 0, qo); return; }
    thread_ctx &c = t_ctx;
    if (c.init()) return;
    const size_t kvb = (size_t)seq_len * n_kv_head * head_dim * 4;
    const size_t o_k = align256(qo), o_v = o_k + align256(kvb), o_l = o_v + align256(kvb), in_b = o_l + 256;
    const long ws = mllm_gqa_workspace_size(1, n_head, head_dim, seq_len);
    if (c.d_in.ensure(in_b) || c.h_in.ensure(in_b) || c.d_out.ensure(qo) || c.h_out.ensure(qo) || c.d_scr.ensure(ws)) {
        set_error("gqa_attention_decode: staging allocation failed");
        return;
    }
    uint8_t *h = (uint8_t *)c.h_in.p, *d = (uint8_t *)c.d_in.p;
    memcpy(h, q, qo);
    memcpy(h + o_k, k_cache, kvb);
    memcpy(h + o_v, v_cache, kvb);
    memcpy(h + o_l, &seq_len, sizeof(int));
    mllm_kv_view kv{(float *)(d + o_k), (float *)(d + o_v), 0, nullptr, 0, 0, 0};
    if (hipMemcpyAsync(d, h, in_b, hipMemcpyHostToDevice, c.st) != hipSuccess ||
        mllm_gqa_decode(1, (const float *)d, &kv, (const int *)(d + o_l), seq_len, 1, n_head, n_kv_head, head_dim,
                        (float *)c.d_out.p, c.d_scr.p, ws, c.st) != 0 ||
        hipMemcpyAsync(c.h_out.p, c.d_out.p, qo, hipMemcpyDeviceToHost, c.st) != hipSuccess ||
        hipStreamSynchronize(c.st) != hipSuccess) {
        set_error("gqa_attention_decode failed");
        return;
    }
    memcpy(out, c.h_out.p, qo);
}

MLLM_API int mllm_read_probe(const void *dev, long bytes, void *sink, void *stream)
{
    if (((uintptr_t)dev & 15) || (bytes & 15) || !sink) { set_error("mllm_read_probe: 16-byte aligned, multiple of 16"); return -1; }
    HIP_OK(mllm_launch_read_probe(dev, bytes, sink, (hipStream_t)stream));
    return 0;
}

MLLM_API int mllm_quantize_q8_0(const float *x_dev, int T, int n_cols, uint8_t *q8_dev, void *stream)
{
    HIP_OK(mllm_launch_quantize_q8_0(x_dev, T, n_cols, q8_dev, nullptr, nullptr, nullptr, nullptr, (hipStream_t)stream));
    return 0;
}

MLLM_API long mllm_router_packed_size(int N, int E)
{
    return (N > 0 && E > 0) ? mllm_router_packed_floats(N, E) * 4 : -1;
}

MLLM_API int mllm_router_pack(const float *router_dev, int N, int E, float *out_dev, void *stream)
{
    hipError_t r = mllm_launch_router_pack(router_dev, N, E, out_dev, (hipStream_t)stream);
    if (r != hipSuccess) { set_error("mllm_router_pack: %s", hipGetErrorString(r)); return -1; }
    return 0;
}

MLLM_API long mllm_route_workspace_size(int T, int E)
{
    return (T > 0 && E > 0) ? mllm_route_workspace_floats(T, E) * 4 : -1;
}

MLLM_API int mllm_route(const float *router_p_dev, const float *x_dev, int T, int N, int E, int K, int renorm,
                        int *idx_dev, float *w_dev, void *workspace, void *stream)
{
    hipError_t r = mllm_launch_route(router_p_dev, x_dev, T, N, E, K, renorm, idx_dev, w_dev, (float *)workspace,
                                     (hipStream_t)stream);
    if (r != hipSuccess) { set_error("mllm_route: %s (E<=256, K<=16 required)", hipGetErrorString(r)); return -1; }
    return 0;
}

MLLM_API int mllm_dequant(int sem, const void *packed_dev, int n_rows, int n_cols, float *out_dev, void *stream)
{
    mllm_packed view = mllm_packed_view(mllm_sem_layout(sem), (const uint8_t *)packed_dev, n_rows, n_cols);
    return mllm_launch_dequant(sem, view, n_rows, n_cols, out_dev, (hipStream_t)stream);
}

} // extern "C"

// ---------------------------------------------------------- moe_ffn engine
// Decode MoE for T tokens with moe_ffn semantics (A11): C routing without
// renormalisation, quant_matmul_omp semantics per expert, unclamped SiLU,
// ffn = fma(p_k, down_k, ffn) in k order.  Experts are addressed at
// base + e*stride exactly as CE:593-605 computes them.
int mllm_moe_ffn_dev_tokens(const float *router, const uint8_t *const bases[3], const int qts[3], int N, int E, int K,
                            int M, const float *x_host, float *out_host, int T)
{
    thread_ctx &c = t_ctx;
    if (c.init()) return -1;
    const int sems[3] = {sem_for(ENT_QMM, qts[0]), sem_for(ENT_QMM, qts[1]), sem_for(ENT_QMM, qts[2])};
    if (sems[0] < 0 || sems[1] < 0 || sems[2] < 0) {
        // the reference's quant_matmul_omp leaves buffers untouched for unknown codes; we zero the output
        set_error("moe_ffn: unknown expert quant type (%d,%d,%d)", qts[0], qts[1], qts[2]);
        memset(out_host, 0, (size_t)N * T * 4);
        return -1;
    }
    if (K > 16 || E > 256) { set_error("moe_ffn: E<=256 and K<=16 required"); return -1; }
    // per-expert packed views: the layer's device table (cached per layer)
    const mllm_packed *dtab = nullptr;
    if (get_layer_table(bases, qts, sems, N, E, M, &dtab)) return -1;
    const float *rt = nullptr;
    if (get_router(router, E, N, &rt)) return -1;
    // scratch: x[T][N] | idx[T][K] | w[T][K] | g,u,h [T*K][M] | dn [T*K][N] | out[T][N] | routing logits
    const size_t TK = (size_t)T * K;
    size_t o_x = 0, o_i = align256(o_x + (size_t)T * N * 4), o_w = align256(o_i + TK * 4), o_g = align256(o_w + TK * 4),
           o_u = align256(o_g + TK * M * 4), o_h = align256(o_u + TK * M * 4), o_dn = align256(o_h + TK * M * 4),
           o_o = align256(o_dn + TK * N * 4), o_l = align256(o_o + (size_t)T * N * 4),
           total = align256(o_l + (size_t)mllm_route_workspace_floats(T, E) * 4);
    if (c.d_scr.ensure(total) || c.h_in.ensure((size_t)T * N * 4) || c.h_out.ensure((size_t)T * N * 4)) {
        set_error("moe_ffn: scratch allocation failed");
        return -1;
    }
    uint8_t *S = (uint8_t *)c.d_scr.p;
    float *dx = (float *)(S + o_x), *dwt = (float *)(S + o_w), *dg = (float *)(S + o_g), *du = (float *)(S + o_u),
          *dh = (float *)(S + o_h), *ddn = (float *)(S + o_dn), *dout = (float *)(S + o_o);
    int *didx = (int *)(S + o_i);
    hipStream_t st = c.st;
    memcpy(c.h_in.p, x_host, (size_t)T * N * 4);
    HIP_OK(hipMemcpyAsync(dx, c.h_in.p, (size_t)T * N * 4, hipMemcpyHostToDevice, st));
    HIP_OK(mllm_launch_route(rt, dx, T, N, E, K, 0, didx, dwt, (float *)(S + o_l), st));
    // one GEMV launch per projection over the T*K (token, slot) jobs, gate
    // and up together when their semantics agree; Q8_0 activations quantised
    // by the GEMV workgroups.  The SiLU here is unclamped (CE:649-652).
    mllm_gemv_args a{};
    a.table = dtab; a.idx = didx; a.job_div = K;
    a.x = dx; a.x_job_stride = N; a.ldx = N;
    a.out = dg; a.out_job_stride = M; a.ldo = M;
    a.n_rows = M; a.n_cols = N; a.B = 1;
    if (sems[0] == sems[1] && mllm_gemv_fused_fits(sems[0], N, 1, false)) {
        // gate, up and the unclamped SiLU product (CE:649-652) in one launch (paired rows)
        a.table2 = dtab + E; a.silu_pair = 1; a.silu_noclamp = 1; a.out = dh;
        HIP_OK(mllm_launch_gemv(sems[0], a, (int)TK, st));
    } else if (sems[0] == sems[1]) {
        a.job_split = (int)TK; a.table2 = dtab + E; a.out2 = du;
        HIP_OK(mllm_launch_gemv(sems[0], a, 2 * (int)TK, st));
    } else {
        HIP_OK(mllm_launch_gemv(sems[0], a, (int)TK, st));
        a.table = dtab + E; a.out = du;
        HIP_OK(mllm_launch_gemv(sems[1], a, (int)TK, st));
    }
    if (!a.silu_pair) HIP_OK(mllm_launch_silu_mul(dg, du, dh, (long)TK * M, 0, st));
    mllm_gemv_args b{};
    b.table = dtab + 2 * (size_t)E; b.idx = didx;
    b.x = dh; b.x_job_stride = M; b.ldx = M;
    b.out = ddn; b.out_job_stride = N; b.ldo = N;
    b.n_rows = N; b.n_cols = M; b.B = 1;
    HIP_OK(mllm_launch_gemv(sems[2], b, (int)TK, st));
    // small results: the combine writes them straight into the pinned buffer
    const bool direct = (size_t)T * N * 4 <= kDirectOutMax && c.h_out.dp;
    HIP_OK(mllm_launch_combine(ddn, dwt, didx, T, K, N, direct ? (float *)c.h_out.dp : dout, 1, st));
    if (!direct) HIP_OK(hipMemcpyAsync(c.h_out.p, dout, (size_t)T * N * 4, hipMemcpyDeviceToHost, st));
    HIP_OK(hipStreamSynchronize(st));
    memcpy(out_host, c.h_out.p, (size_t)T * N * 4);
    return 0;
}

// moe_ffn over T tokens of host data, every token's result kept: T > 8 tokens
// whose expert types the grouped GEMM serves run the MoE layer (decode GEMVs up
// to 24 tokens, then GPU bucketing and grouped MFMA GEMMs) with moe_ffn's semantics (quant_matmul_omp
// per projection, unclamped SiLU, no renormalisation); the rest the token path.
int mllm_moe_ffn_host_batched(const float *router, const uint8_t *const bases[3], const int qts[3], int N, int E, int K,
                              int M, const float *x_host, float *out_host, int T)
{
    const int sems[3] = {sem_for(ENT_QMM, qts[0]), sem_for(ENT_QMM, qts[1]), sem_for(ENT_QMM, qts[2])};
    if (T <= 8 || sems[0] < 0 || sems[1] < 0 || sems[2] < 0 || K > 16 || E > 256 || K > E ||
        !mllm_moe_batched_supported(sems[0], sems[1], sems[2]))
        return mllm_moe_ffn_dev_tokens(router, bases, qts, N, E, K, M, x_host, out_host, T);
    thread_ctx &c = t_ctx;
    if (c.init()) return -1;
    const mllm_packed *dtab = nullptr;
    int gemv_only = 0;
    if (get_layer_table(bases, qts, sems, N, E, M, &dtab, &gemv_only)) return -1;
    const float *rt = nullptr;
    if (get_router(router, E, N, &rt)) return -1;
    mllm_moe_layer *L = mllm_moe_layer_from_views(sems[0], sems[1], sems[2], N, M, E, K, dtab, rt, 0, 0, gemv_only);
    if (!L) { set_error("moe_ffn_batched: bad layer shape"); return -1; }
    // scratch: x[T][N] | out[T][N] | layer workspace
    const size_t ws = (size_t)mllm_moe_workspace_size(L, T);
    const size_t o_o = align256((size_t)T * N * 4), o_ws = align256(o_o + (size_t)T * N * 4), total = o_ws + ws;
    if (c.d_scr.ensure(total) || c.h_in.ensure((size_t)T * N * 4) || c.h_out.ensure((size_t)T * N * 4)) {
        mllm_moe_release(L);
        set_error("moe_ffn_batched: scratch allocation failed");
        return -1;
    }
    uint8_t *S = (uint8_t *)c.d_scr.p;
    float *dx = (float *)S, *dout = (float *)(S + o_o);
    hipStream_t st = c.st;
    memcpy(c.h_in.p, x_host, (size_t)T * N * 4);
    int rc = -1;
    if (hipMemcpyAsync(dx, c.h_in.p, (size_t)T * N * 4, hipMemcpyHostToDevice, st) == hipSuccess &&
        mllm_moe_forward(L, dx, T, dout, S + o_ws, (long)ws, nullptr, nullptr, st) == 0 &&
        hipMemcpyAsync(c.h_out.p, dout, (size_t)T * N * 4, hipMemcpyDeviceToHost, st) == hipSuccess &&
        hipStreamSynchronize(st) == hipSuccess)
        rc = 0;
    mllm_moe_release(L);
    if (rc) { set_error("moe_ffn_batched: launch failed"); return -1; }
    memcpy(out_host, c.h_out.p, (size_t)T * N * 4);
    return 0;
}
