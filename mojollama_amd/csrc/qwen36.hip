// qwen36.hip — the engine's Qwen3.6 hybrid drivers on the GPU, as drop-ins on
// host buffers: qwen36_batch_forward (CE:859-1231), ssm_layer_fused
// (CE:803-849) and ssm_decode_step (CE:736-802).
//
// qwen36_batch_forward runs B tokens through L layers, each an SSM block
// (layer_types[l] == 1 with its conv weights given) or an attention block,
// then an MoE FFN with an optional shared expert, then the output head.  Every
// matmul has quant_matmul_omp's semantics (QK:1355-1388).  Per layer, on one
// stream:
//   attention  xn = rms(x); qkv = Wqkv xn; q, k, v taken from the fused buffer
//              at 0, inner and inner + N (CE:1001-1009: v at inner + N, the
//              caller's layout of inner + 2N rows, TE:1533-1543; positions
//              past the layer's rows hold what the workspace slice held
//              there, which the driver keeps as the reference leaves it);
//              RoPE on q and k; per token b in order: K/V row kv_lens[l] :=
//              k_b, v_b, then attention over kv_lens[l] + 1 rows (CE:141-158)
//              -- every token of the batch writes the same row, so token b
//              sees its own K/V there, as the reference's loop does;
//              x += Wo att
//   SSM        xn = rms(x); g = Wgate xn; att = g * silu(x conv_g) * (x conv_s)
//              and the per-group state update (ssm_decode_step); x += Wout att
//   FFN        xn = rms(x); router (f32_matmul_omp's summation order for
//              fp32 routers, so the top-K selection is the reference's),
//              softmax, top-K, renormalised (CE:1113-1152); experts with
//              moe_forward_omp's semantics (QK:2066-2250); shared expert
//              added with weight dot(xn, r) where that is > 0 (CE:1178-1210);
//              x += ffn
// rms is RMS_NORM_SIMD (CE:950-970): inputs clipped to +-1000 (NaN -> -1000
// in whole 8-groups, 0 in the tail), squares summed per 8-group in hsum_ps
// order, then sequentially, x / sqrt(ss / n + eps) * w.
//
// Host state the reference reads and writes is mirrored: the KV caches (a
// device copy per attention layer, rows uploaded when the caller's kv_lens
// passes them; the new row written back), the SSM state (uploaded and written
// back each call), and the workspace slice of the fused QKV buffer (uploaded
// and written back each call; the other workspace slices are not written).
#include <stdio.h>
#include <string.h>
#include <algorithm>
#include <map>
#include <mutex>
#include <vector>
#include "dropin.h"
#include "gemv.h"
#include "moe.h"

namespace {

__device__ __forceinline__ float clip1000(float v) { return fminf(fmaxf(v, -1000.0f), 1000.0f); }   // NaN -> -1000
__device__ __forceinline__ float expf_ref(float v) { return (float)exp((double)v); }
__device__ __forceinline__ float logf_ref(float v) { return (float)log((double)v); }
__device__ __forceinline__ float h2f_dev(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// RMS_NORM_SIMD (CE:950-970), one workgroup per token.  gs: N/8 + 1 floats of LDS.
__global__ __launch_bounds__(256) void k_q36_rms(const float *__restrict__ x, const float *__restrict__ w, int N,
                                                 float eps, float *__restrict__ out)
{
    extern __shared__ float gs[];
    const int b = blockIdx.x, ng = N / 8;
    x += (long)b * N;
    out += (long)b * N;
    for (int g = threadIdx.x; g < ng; g += blockDim.x) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            v[k] = clip1000(x[8 * g + k]);
            out[8 * g + k] = v[k];
        }
        // hsum_ps(v * v) (CE:63-66): (lo + hi) per lane, then two horizontal adds
        const float l0 = __fadd_rn(__fmul_rn(v[0], v[0]), __fmul_rn(v[4], v[4]));
        const float l1 = __fadd_rn(__fmul_rn(v[1], v[1]), __fmul_rn(v[5], v[5]));
        const float l2 = __fadd_rn(__fmul_rn(v[2], v[2]), __fmul_rn(v[6], v[6]));
        const float l3 = __fadd_rn(__fmul_rn(v[3], v[3]), __fmul_rn(v[7], v[7]));
        gs[g] = __fadd_rn(__fadd_rn(l0, l1), __fadd_rn(l2, l3));
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float ss = 0.0f;
        for (int g = 0; g < ng; g++) ss = __fadd_rn(ss, gs[g]);
        for (int i = 8 * ng; i < N; i++) {
            float v = x[i];
            v = v != v ? 0.0f : clip1000(v);
            out[i] = v;
            ss = fmaf(v, v, ss);
        }
        gs[ng] = __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)N), eps));
    }
    __syncthreads();
    const float r = gs[ng];
    for (int i = threadIdx.x; i < N; i += blockDim.x) out[i] = __fmul_rn(__fdiv_rn(out[i], r), w[i]);
}

// emb_lookup of a Q4_K embedding row (CE:714-733, its own formula: scales and
// mins offset by 32 and divided by 8, elements 2i / 2i+1 from the low / high
// nibble of byte i).  One workgroup of 256 per (super-block, token).
__global__ __launch_bounds__(256) void k_q36_embed_q4k(const uint8_t *__restrict__ rows, int N, float *__restrict__ x)
{
    const int bi = blockIdx.x, b = blockIdx.y, j = threadIdx.x, bpr = N / 256;
    const uint8_t *bp = rows + ((long)b * bpr + bi) * 144;
    const float d = h2f_dev((uint16_t)(bp[0] | bp[1] << 8)), dm = h2f_dev((uint16_t)(bp[2] | bp[3] << 8));
    const uint8_t *q = bp + 4;
    const int g = j >> 5;
    int sc, mn;
    if (g < 4) { sc = q[g] & 63; mn = q[g + 4] & 63; }
    else { sc = (q[g + 4] & 0xF) | ((q[g - 4] >> 6) << 4); mn = (q[g + 4] >> 4) | ((q[g] >> 6) << 4); }
    const float d_sc = __fdiv_rn(__fmul_rn(d, (float)(sc - 32)), 8.0f);
    const float d_mn = __fdiv_rn(__fmul_rn(dm, (float)(mn - 32)), 8.0f);
    const int s = (bp[16 + j / 2] >> ((j & 1) * 4)) & 0xF;
    x[(long)b * N + bi * 256 + j] = fmaf(d_sc, (float)(s - 8), -__fmul_rn(d_mn, 6.0f));
}

// ssm_decode_step's intermediate (CE:747-757, 788-792), optionally times the
// gate matmul's output (CE:1026-1030 / CE:831-834):
// out[b][i] = [gate[b][i] *] (cg / (1 + exp(-cg))) * cs, cg = x[i % N] conv[i],
// cs = x[(inner + i) % N] conv[inner + i].
__global__ __launch_bounds__(256) void k_q36_ssm_interm(const float *__restrict__ x, int N, const float *__restrict__ conv,
                                                        int inner, const float *__restrict__ gate, int ldg,
                                                        float *__restrict__ out, int ldo)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x, b = blockIdx.y;
    if (i >= inner) return;
    const float *xb = x + (long)b * N;
    const float cg = __fmul_rn(xb[i % N], conv[i]);
    const float cs = __fmul_rn(xb[(inner + i) % N], conv[inner + i]);
    float s = __fmul_rn(__fdiv_rn(cg, __fadd_rn(1.0f, expf_ref(-cg))), cs);
    if (gate) s = __fmul_rn(gate[(long)b * ldg + i], s);
    out[(long)b * ldo + i] = s;
}

// ssm_decode_step's state update (CE:759-786) for B tokens in order, one
// thread per (group, state element): dt = softplus(dt_bias + alpha . x),
// a = exp(A dt), bx = (beta . x) dt, h = a h + (s == 0 ? bx : 0).
__global__ __launch_bounds__(256) void k_q36_ssm_state(const float *__restrict__ x, int N, int B,
                                                       const float *__restrict__ alpha, const float *__restrict__ beta,
                                                       const float *__restrict__ dt_bias, const float *__restrict__ a_par,
                                                       int G, int Sz, int dtr, float *__restrict__ state)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= G * Sz) return;
    const int g = t / Sz, s = t - g * Sz;
    float h = state[t];
    for (int b = 0; b < B; b++) {
        const float *xb = x + (long)b * N;
        float dt = dt_bias[g];
        for (int j = 0; j < dtr; j++) dt = fmaf(alpha[g * dtr + j], xb[j % N], dt);
        dt = dt > 20.0f ? dt : logf_ref(__fadd_rn(1.0f, expf_ref(dt)));
        const float ad = expf_ref(__fmul_rn(a_par[g], dt));
        float bx = 0.0f;
        for (int j = 0; j < dtr; j++) bx = fmaf(beta[g * dtr + j], xb[j % N], bx);
        bx = __fmul_rn(bx, dt);
        h = fmaf(ad, h, s == 0 ? bx : 0.0f);
    }
    state[t] = h;
}

// q, k, v of each token from the fused QKV output (CE:1001-1009): position p
// of the fused buffer is the layer's output where p < n_qkv, else the
// workspace slice's value.
__global__ __launch_bounds__(256) void k_q36_split(const float *__restrict__ qkv, int n_qkv, const float *__restrict__ slice,
                                                   int inner, int N, int nkv, float *__restrict__ q,
                                                   float *__restrict__ k, float *__restrict__ v)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x, b = blockIdx.y;
    const float *row = qkv + (long)b * n_qkv;
    auto at = [&](int p) { return p < n_qkv ? row[p] : slice[p]; };
    if (i < inner) q[(long)b * inner + i] = at(i);
    if (i < nkv) {
        k[(long)b * nkv + i] = at(inner + i);
        v[(long)b * nkv + i] = at(inner + N + i);
    }
}

// The fused buffer as the reference's loop leaves it: the last token's output,
// its q rows rotated (rope_apply works in place there, CE:1012).
__global__ __launch_bounds__(256) void k_q36_commit(const float *__restrict__ qkv, int n_qkv, const float *__restrict__ q,
                                                    int inner, int B, float *__restrict__ slice)
{
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= n_qkv) return;
    slice[p] = p < inner ? q[(long)(B - 1) * inner + p] : qkv[(long)(B - 1) * n_qkv + p];
}

// f32_matmul_omp (QK:884-913) rows in its own summation order: 16 FMA chains
// (column c feeds chain c % 16), chain i + 8 added to chain i, then
// ((t0+t1)+(t2+t3)) + ((t4+t5)+(t6+t7)) (the hadd sequence), then the tail
// columns past the last multiple of 16 as one FMA chain.  16 lanes per row.
__global__ __launch_bounds__(256) void k_q36_f32mm(const float *__restrict__ W, const float *__restrict__ x, int rows,
                                                   int cols, float *__restrict__ out)
{
    const int lane = threadIdx.x & 63, sl = lane & 15;
    const int r = (blockIdx.x * blockDim.x + threadIdx.x) >> 4, b = blockIdx.y;
    const int rr = r < rows ? r : rows - 1;
    const float *w = W + (long)rr * cols, *xb = x + (long)b * cols;
    const int c16 = cols / 16 * 16;
    float acc = 0.0f;
    for (int c = sl; c < c16; c += 16) acc = fmaf(w[c], xb[c], acc);
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; i++) t[i] = __shfl(acc, (lane & ~15) + i, 64);
    if (sl != 0 || r >= rows) return;
    float u[8];
#pragma unroll
    for (int i = 0; i < 8; i++) u[i] = __fadd_rn(t[i], t[i + 8]);
    float res = __fadd_rn(__fadd_rn(__fadd_rn(u[0], u[1]), __fadd_rn(u[2], u[3])),
                          __fadd_rn(__fadd_rn(u[4], u[5]), __fadd_rn(u[6], u[7])));
    for (int c = c16; c < cols; c++) res = fmaf(w[c], xb[c], res);
    out[(long)b * rows + r] = res;
}

// The shared expert's weight (CE:1185-1186): a sequential FMA chain over N.
__global__ void k_q36_dot_chain(const float *__restrict__ x, const float *__restrict__ r, int N, int B,
                                float *__restrict__ out)
{
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    const float *xb = x + (long)b * N;
    float s = 0.0f;
    for (int i = 0; i < N; i++) s = fmaf(xb[i], r[i], s);
    out[b] = s;
}

// x += ffn, ffn = the experts' combine (+ sh * shared expert where sh > 0, CE:1187-1210).
__global__ __launch_bounds__(256) void k_q36_ffn_add(float *__restrict__ x, const float *__restrict__ moe,
                                                     const float *__restrict__ shd, const float *__restrict__ shs, int N)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x, b = blockIdx.y;
    if (i >= N) return;
    const long o = (long)b * N + i;
    float f = moe[o];
    if (shd) {
        const float s = shs[b];
        if (s > 0.0f) f = fmaf(s, shd[o], f);
    }
    x[o] = __fadd_rn(x[o], f);
}

// o[i] = g[i] * o[i], i < n (ssm_layer_fused step 3 for one token, CE:831-834).
__global__ void k_q36_mul(float *__restrict__ o, const float *__restrict__ g, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = __fmul_rn(g[i], o[i]);
}

// o[i] = r[i] + p[i], i < n.
__global__ void k_q36_add2(float *__restrict__ o, const float *__restrict__ r, const float *__restrict__ p, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = __fadd_rn(r[i], p[i]);
}

long a256(long n) { return (n + 255) / 256 * 256; }

// Raw GGUF bytes of a rows x cols matrix under semantic sem.
long raw_bytes(int sem, int rows, int cols)
{
    if (sem == SEM_F32) return (long)rows * cols * 4;
    const mllm_layout_desc L = mllm_layout_info(mllm_sem_layout(sem));
    return (long)rows * (cols / L.block_elems) * L.block_bytes;
}

uint64_t fp_bytes(const void *p, long n)
{
    const uint8_t *b = (const uint8_t *)p;
    uint64_t h = 1469598103934665603ull ^ (uint64_t)n;
    for (int i = 0; i < 32 && n > 0; i++) {
        const long off = (long)((__int128)(n - 1) * i / 31);
        h = (h ^ b[off]) * 1099511628211ull;
    }
    return h;
}

// --------------------------------------------------------------- model
struct q36_layer {
    int ssm = 0;                                   // SSM block (else attention)
    float *an = nullptr, *fn = nullptr;            // RMS weights
    // attention
    mllm_packed qkv{}, wo{};
    int sem_qkv = -1, sem_o = -1, n_qkv = 0, kv_slot = -1;
    // SSM
    mllm_packed gate{}, so{};
    int sem_gate = -1, sem_so = -1, gate_nr = 0;
    float *conv = nullptr, *alpha = nullptr, *beta = nullptr, *dtb = nullptr, *a = nullptr;
    // MoE
    int moe = 0, sem_router = -1;
    mllm_packed router{};                          // fp32 rows (code 0) or a packed matrix
    mllm_packed *tab = nullptr;                    // device [3E]
    mllm_moe_layer *ml = nullptr;
    // shared expert
    int sh = 0, si = 0, sem_sg = -1, sem_su = -1, sem_sd = -1;
    mllm_packed sg{}, su{}, sd{};
    float *shr = nullptr;
};

struct q36_dims {
    int L, N, NH, NKH, HD, E, K, M, rope_dim, max_ctx, si_ssm, G, Sz, dtr, emb_q, out_nr, sem_out;
    float eps;
};

struct q36_model {
    q36_dims d{};
    std::vector<q36_layer> layers;
    std::vector<void *> allocs;
    std::vector<std::pair<const void *, long>> fp_src;   // host arrays checked by fingerprint each call
    uint64_t fp = 0;
    float *out_norm = nullptr, *cos_t = nullptr, *sin_t = nullptr;
    mllm_packed out_w{};
    int n_attn = 0, P = 0;                               // attention layers; fused-slice floats mirrored
    long ws_gemv = 0, ws_attn = 0, ws_moe = 0;
    int B_cap = 0;
    // per-call device buffers (B_cap tokens)
    float *x = nullptr, *xn = nullptr, *qkvo = nullptr, *q = nullptr, *kt = nullptr, *vt = nullptr, *att = nullptr,
          *gate = nullptr, *lg = nullptr, *wk = nullptr, *mo = nullptr, *shs = nullptr, *shg = nullptr,
          *shu = nullptr, *shd = nullptr, *logits = nullptr, *slice = nullptr, *state = nullptr;
    int *idx = nullptr, *pos = nullptr;
    uint8_t *ws = nullptr, *emb_rows = nullptr;
    std::vector<void *> call_allocs;

    void *dalloc(std::vector<void *> &v, size_t bytes)
    {
        void *p = nullptr;
        if (hipMalloc(&p, bytes ? a256(bytes) : 256) != hipSuccess) return nullptr;
        v.push_back(p);
        return p;
    }
    float *upload(const float *h, long n)
    {
        float *p = (float *)dalloc(allocs, (size_t)n * 4);
        if (!p || hipMemcpy(p, h, (size_t)n * 4, hipMemcpyHostToDevice) != hipSuccess) return nullptr;
        fp_src.push_back({h, n * 4});
        return p;
    }
    void free_call()
    {
        for (void *p : call_allocs) (void)hipFree(p);
        call_allocs.clear();
        B_cap = 0;
    }
    ~q36_model()
    {
        for (auto &l : layers)
            if (l.ml) mllm_moe_release(l.ml);
        free_call();
        for (void *p : allocs) (void)hipFree(p);
    }
};

struct q36_kv {
    std::vector<float *> k, v;          // per attention layer [max_ctx][nkv]
    std::vector<int> rows;
    std::vector<uint64_t> seal;
    int max_ctx = 0, nkv = 0;
    ~q36_kv()
    {
        for (float *p : k) (void)hipFree(p);
        for (float *p : v) (void)hipFree(p);
    }
};

std::mutex g_q36_mu;
std::map<std::vector<uintptr_t>, q36_model *> g_q36_models;
std::map<std::vector<uintptr_t>, q36_kv *> g_q36_kv;
hipStream_t g_q36_st = nullptr;
void *g_q36_hin = nullptr, *g_q36_hout = nullptr;
size_t g_q36_hin_n = 0, g_q36_hout_n = 0;

int host_ensure(void **p, size_t *n, size_t want)
{
    if (want <= *n) return 0;
    if (*p) (void)hipHostFree(*p);
    *p = nullptr;
    *n = 0;
    if (hipHostMalloc(p, want + want / 4, hipHostMallocDefault) != hipSuccess) { *p = nullptr; return -1; }
    *n = want + want / 4;
    return 0;
}

int ensure_stream()
{
    if (g_q36_st) return 0;
    if (hipStreamCreateWithFlags(&g_q36_st, hipStreamNonBlocking) != hipSuccess) {
        g_q36_st = nullptr;
        mllm_set_error("qwen36: hipStreamCreate failed");
        return -1;
    }
    return 0;
}

uint64_t kv_rows_seal(const float *base, int n, int nkv)
{
    if (n <= 0) return 0;
    const int pick[3] = {0, n / 2, n - 1};
    uint64_t h = 0;
    for (int r : pick) h = h * 31 + fp_bytes(base + (long)r * nkv, (long)nkv * 4);
    return h;
}

// quant_matmul_omp on device rows: out [B][rows] (+ out_add), x [B][cols].
int gemv(const q36_model &m, int sem, const mllm_packed &W, const float *x, float *out, int rows, int cols, int B,
         const float *out_add, const float *x_up, hipStream_t st)
{
    mllm_gemv_fusion f{};
    f.out_add = out_add;
    f.x_up = x_up;
    f.silu_clamp = 1;
    return mllm_gemv_fused(sem, W.p[0], x, out, rows, cols, B, &f, m.ws, st);
}

long gemv_ws(int sem, int rows, int cols, int B, bool add, bool up)
{
    mllm_gemv_fusion f{};
    float dummy_ptr_holder = 0.0f;
    if (add) f.out_add = &dummy_ptr_holder;
    if (up) { f.x_up = &dummy_ptr_holder; f.silu_clamp = 1; }
    return mllm_gemv_fused_workspace_size(sem, rows, cols, B, &f);
}

} // namespace

void mllm_qwen36_cache_clear()
{
    std::lock_guard<std::mutex> lk(g_q36_mu);
    if (g_q36_st) (void)hipStreamSynchronize(g_q36_st);
    for (auto &e : g_q36_models) delete e.second;
    g_q36_models.clear();
    for (auto &e : g_q36_kv) delete e.second;
    g_q36_kv.clear();
}

namespace {

// Per-call buffers for B tokens.
int q36_buffers(q36_model &m, int B)
{
    if (B <= m.B_cap) return 0;
    m.free_call();
    const q36_dims &d = m.d;
    const int inner = d.NH * d.HD, nkv = d.NKH * d.HD;
    int nq = 0, gnr = 0, si = 0, bi = std::max(inner, d.si_ssm);
    for (auto &l : m.layers) {
        nq = std::max(nq, l.n_qkv);
        gnr = std::max(gnr, l.gate_nr);
        si = std::max(si, l.si);
    }
    auto A = [&](size_t bytes) { return m.dalloc(m.call_allocs, bytes); };
    m.x = (float *)A((size_t)B * d.N * 4);
    m.xn = (float *)A((size_t)B * d.N * 4);
    m.qkvo = (float *)A((size_t)B * std::max(nq, 1) * 4);
    m.q = (float *)A((size_t)B * inner * 4);
    m.kt = (float *)A((size_t)B * nkv * 4);
    m.vt = (float *)A((size_t)B * nkv * 4);
    m.att = (float *)A((size_t)B * bi * 4);
    m.gate = (float *)A((size_t)B * std::max(gnr, 1) * 4);
    m.lg = (float *)A((size_t)B * std::max(d.E, 1) * 4);
    m.idx = (int *)A((size_t)B * std::max(d.K, 1) * 4);
    m.wk = (float *)A((size_t)B * std::max(d.K, 1) * 4);
    m.mo = (float *)A((size_t)B * d.N * 4);
    m.shs = (float *)A((size_t)B * 4);
    m.shg = (float *)A((size_t)B * std::max(si, 1) * 4);
    m.shu = (float *)A((size_t)B * std::max(si, 1) * 4);
    m.shd = (float *)A((size_t)B * d.N * 4);
    m.logits = (float *)A((size_t)B * d.out_nr * 4);
    m.pos = (int *)A((size_t)d.L * (B + 1) * 4);
    m.slice = (float *)A((size_t)std::max(m.P, 1) * 4);
    m.state = (float *)A((size_t)d.L * std::max(d.G * d.Sz, 1) * 4);
    m.emb_rows = (uint8_t *)A((size_t)B * d.N * 4);
    // workspaces: the largest any launch of the pass asks for
    long wg = 256;
    for (auto &l : m.layers) {
        if (l.ssm) {
            wg = std::max(wg, gemv_ws(l.sem_gate, l.gate_nr, d.N, B, false, false));
            wg = std::max(wg, gemv_ws(l.sem_so, d.N, d.si_ssm, B, true, false));
        } else {
            wg = std::max(wg, gemv_ws(l.sem_qkv, l.n_qkv, d.N, B, false, false));
            wg = std::max(wg, gemv_ws(l.sem_o, d.N, inner, B, true, false));
        }
        if (l.moe && l.sem_router > 0) wg = std::max(wg, gemv_ws(l.sem_router, d.E, d.N, B, false, false));
        if (l.sh) {
            wg = std::max(wg, gemv_ws(l.sem_sg, l.si, d.N, B, false, false));
            wg = std::max(wg, gemv_ws(l.sem_su, l.si, d.N, B, false, false));
            wg = std::max(wg, gemv_ws(l.sem_sd, d.N, l.si, B, false, true));
        }
    }
    wg = std::max(wg, gemv_ws(d.sem_out, d.out_nr, d.N, B, false, false));
    long wm = 0;
    for (auto &l : m.layers)
        if (l.ml) wm = std::max(wm, mllm_moe_workspace_size(l.ml, B));
    const long wa = m.n_attn ? mllm_gqa_workspace_size(1, d.NH, d.HD, d.max_ctx) : 0;
    if (wg < 0 || wm < 0 || wa < 0) { mllm_set_error("qwen36: workspace size query failed"); return -1; }
    m.ws_gemv = a256(wg);
    m.ws_attn = a256(wa);
    m.ws_moe = a256(wm);
    m.ws = (uint8_t *)A((size_t)(m.ws_gemv + m.ws_attn + m.ws_moe));
    // dalloc records only the allocations that succeeded: 22 buffers above
    if (m.call_allocs.size() != 22) { mllm_set_error("qwen36: device allocation failed"); m.free_call(); return -1; }
    m.B_cap = B;
    return 0;
}

} // namespace

extern "C" {

// qwen36_batch_forward (CE:859-1231) on host buffers.  See the file comment.
MLLM_API void qwen36_batch_forward(
    int B, int L, int N, int NH, int n_kv_h, int HD, int FF, int n_experts, int top_k, int n_ff_expert, float eps,
    int rope_dim, int max_ctx, int ssm_inner, int ssm_groups, int ssm_state_size, int ssm_conv_kernel, int ssm_dt_rank,
    const float *emb, int emb_quant, const int *layer_types, const int *tokens, float *logits, const float **attn_norm_w,
    const float **ffn_norm_w, const uint8_t **attn_qkv_raw, const int *qkv_nr, const int *qkv_nc, const int *qkv_qt,
    const uint8_t **attn_gate_raw, const int *gate_nr, const int *gate_nc, const int *gate_qt,
    const uint8_t **ssm_out_raw, const int *ssm_out_nr, const int *ssm_out_nc, const int *ssm_out_qt,
    const uint8_t **attn_out_raw, const int *out_nr, const int *out_nc, const int *out_qt, uint8_t **gate_exp_raw,
    const int *gate_exp_qt, uint8_t **up_exp_raw, const int *up_exp_qt, uint8_t **down_exp_raw,
    const int *down_exp_qt, const float **shexp_gate_raw, const float **shexp_up_raw, const float **shexp_down_raw,
    const float **shexp_router, const int *shexp_int, const uint8_t **moe_router_raw, const int *moe_router_qt,
    const int *shexp_gate_qt, const int *shexp_up_qt, const int *shexp_down_qt, const float *out_norm_w,
    const uint8_t *out_w, int out_nr_final, int out_nc_final, int out_qt_final, const float **ssm_conv1d,
    const float **ssm_a, const float **ssm_dt_bias, const float **ssm_alpha, const float **ssm_beta,
    const float **ssm_norm, float *ssm_state, float *kv_k, float *kv_v, int *kv_lens, const float *cos_table,
    const float *sin_table, float *ws, uint8_t *q8_ws)
{
    (void)ssm_conv_kernel; (void)ssm_norm;
    std::shared_lock<std::shared_mutex> api(mllm_api_mutex());
#define Q36_FAIL(...) do { char m_[256]; snprintf(m_, sizeof m_, __VA_ARGS__); mllm_set_error(m_); return; } while (0)
    if (B <= 0 || L <= 0) return;
    const int inner = NH * HD, nkv = n_kv_h * HD;
    if (N <= 0 || N % 32 || !emb || !tokens || !logits || !out_w || !out_norm_w || !attn_norm_w || !ffn_norm_w)
        Q36_FAIL("qwen36_batch_forward: N must be a positive multiple of 32 and the embedding, tokens, logits, "
                 "norms and output head given (outputs untouched)");
    if (emb_quant != 0 && !(emb_quant == 12 && N % 256 == 0))
        Q36_FAIL("qwen36_batch_forward: emb_quant %d not served (0: fp32, 12: the engine's Q4_K rows)", emb_quant);
    if (out_nc_final != N || out_nr_final <= 0 || mllm_qmm_sem(out_qt_final) < 0)
        Q36_FAIL("qwen36_batch_forward: output head must be out_nr x N of a quant_matmul_omp type");
    // ---- which blocks each layer runs, and their shapes (the reference's own conditions)
    auto is_ssm = [&](int l) { return layer_types && layer_types[l] == 1 && ssm_conv1d && ssm_conv1d[l]; };
    auto has_moe = [&](int l) {
        return n_experts > 0 && top_k > 0 && gate_exp_raw && gate_exp_raw[l] && moe_router_raw && moe_router_raw[l];
    };
    int n_attn = 0, n_ssm = 0, any_moe = 0;
    long P = 0;
    for (int l = 0; l < L; l++) {
        if (!attn_norm_w[l] || !ffn_norm_w[l]) Q36_FAIL("qwen36_batch_forward: layer %d norm weights missing", l);
        if (is_ssm(l)) {
            n_ssm++;
            if (!attn_gate_raw || !attn_gate_raw[l] || !ssm_out_raw || !ssm_out_raw[l] || !ssm_a || !ssm_a[l] ||
                !ssm_dt_bias || !ssm_dt_bias[l] || !ssm_alpha || !ssm_alpha[l] || !ssm_beta || !ssm_beta[l] || !ssm_state)
                Q36_FAIL("qwen36_batch_forward: SSM layer %d weights or state missing", l);
            if (gate_nc[l] != N || gate_nr[l] < ssm_inner || ssm_out_nr[l] != N || ssm_out_nc[l] != ssm_inner ||
                mllm_qmm_sem(gate_qt[l]) < 0 || mllm_qmm_sem(ssm_out_qt[l]) < 0)
                Q36_FAIL("qwen36_batch_forward: SSM layer %d: gate must be >= ssm_inner x N, ssm_out N x ssm_inner, "
                         "of quant_matmul_omp types", l);
        } else {
            n_attn++;
            if (!attn_qkv_raw || !attn_qkv_raw[l] || !attn_out_raw || !attn_out_raw[l])
                Q36_FAIL("qwen36_batch_forward: attention layer %d weights missing", l);
            if (qkv_nc[l] != N || qkv_nr[l] < inner + nkv || out_nr[l] != N || out_nc[l] != inner ||
                mllm_qmm_sem(qkv_qt[l]) < 0 || mllm_qmm_sem(out_qt[l]) < 0)
                Q36_FAIL("qwen36_batch_forward: attention layer %d: QKV must hold >= NH*HD + n_kv_h*HD rows of N, "
                         "o N x NH*HD, of quant_matmul_omp types", l);
            if (kv_lens[l] < 0 || kv_lens[l] >= max_ctx)
                Q36_FAIL("qwen36_batch_forward: kv_lens[%d] = %d outside [0, max_ctx) (the reference writes past "
                         "its cache)", l, kv_lens[l]);
            P = std::max(P, (long)std::max(qkv_nr[l], inner + N + nkv));
        }
        any_moe |= has_moe(l);
    }
    if (n_attn && (NH <= 0 || n_kv_h <= 0 || NH % n_kv_h || NH / n_kv_h > 16 || HD <= 0 || HD > 256 || HD % 4 ||
                   !kv_k || !kv_v || !kv_lens || !cos_table || !sin_table || !ws || inner % 32))
        Q36_FAIL("qwen36_batch_forward: attention shape not served (NH %% n_kv_h == 0, NH/n_kv_h <= 16, HD <= 256 "
                 "and a multiple of 4) or KV / RoPE / workspace missing");
    const int rd = rope_dim <= 0 ? HD : rope_dim;
    if (n_attn && (rd > HD || (rd & 1))) Q36_FAIL("qwen36_batch_forward: rope_dim must be even and <= HD");
    if (n_ssm && (ssm_inner <= 0 || 2 * ssm_inner > 8192 || ssm_inner % 32 || ssm_groups < 0 || ssm_state_size < 0 ||
                  ssm_dt_rank < 0))
        Q36_FAIL("qwen36_batch_forward: ssm_inner must be a multiple of 32 with 2*ssm_inner <= 8192 (the "
                 "reference's conv buffer)");
    if (any_moe && (n_experts > 256 || top_k > 16 || top_k > n_experts || n_ff_expert <= 0))
        Q36_FAIL("qwen36_batch_forward: MoE needs n_experts <= 256, top_k <= 16 and <= n_experts");
    // the workspace layout of CE:906-927
    const int shexp_inner0 = shexp_int ? shexp_int[0] : 512;
    long S = std::max({(long)N, (long)inner, (long)FF, (long)nkv, (long)(inner + 2 * nkv), (long)n_ff_expert,
                       (long)shexp_inner0, 8192L});
    if (n_attn && P > (long)B * S)
        Q36_FAIL("qwen36_batch_forward: the fused QKV reads past its workspace slice (not served)");

    std::lock_guard<std::mutex> lk(g_q36_mu);
    if (ensure_stream()) return;
    hipStream_t st = g_q36_st;
    // ---- the model: keyed by every pointer and shape the pass reads
    std::vector<uintptr_t> key;
    auto K = [&](auto v) { key.push_back((uintptr_t)v); };
    for (int v : {L, N, NH, n_kv_h, HD, n_experts, top_k, n_ff_expert, rope_dim, max_ctx, ssm_inner, ssm_groups,
                  ssm_state_size, ssm_dt_rank, emb_quant, out_nr_final, out_qt_final})
        K((unsigned)v);
    K(__builtin_bit_cast(uint32_t, eps));
    K(out_norm_w); K(out_w); K(cos_table); K(sin_table);
    struct lay_src {
        int ssm, moe, sh, si, qts[3], sqts[3], rqt;
        const void *p[16];
        int ints[8];
    };
    std::vector<lay_src> src(L);
    for (int l = 0; l < L; l++) {
        lay_src &s = src[l];
        memset(&s, 0, sizeof s);
        s.ssm = is_ssm(l);
        s.moe = has_moe(l);
        s.p[0] = attn_norm_w[l]; s.p[1] = ffn_norm_w[l];
        if (s.ssm) {
            s.p[2] = attn_gate_raw[l]; s.p[3] = ssm_out_raw[l]; s.p[4] = ssm_conv1d[l]; s.p[5] = ssm_a[l];
            s.p[6] = ssm_dt_bias[l]; s.p[7] = ssm_alpha[l]; s.p[8] = ssm_beta[l];
            s.ints[0] = gate_nr[l]; s.ints[1] = gate_qt[l]; s.ints[2] = ssm_out_qt[l];
        } else {
            s.p[2] = attn_qkv_raw[l]; s.p[3] = attn_out_raw[l];
            s.ints[0] = qkv_nr[l]; s.ints[1] = qkv_qt[l]; s.ints[2] = out_qt[l];
        }
        if (s.moe) {
            s.qts[0] = gate_exp_qt ? gate_exp_qt[l] : 12;
            s.qts[1] = up_exp_qt ? up_exp_qt[l] : 12;
            s.qts[2] = down_exp_qt ? down_exp_qt[l] : 14;
            s.rqt = moe_router_qt ? moe_router_qt[l] : 0;
            s.p[9] = gate_exp_raw[l]; s.p[10] = up_exp_raw[l]; s.p[11] = down_exp_raw[l]; s.p[12] = moe_router_raw[l];
            s.sh = shexp_router && shexp_router[l];
            if (s.sh) {
                s.si = shexp_int ? shexp_int[l] : 512;
                s.sqts[0] = shexp_gate_qt ? shexp_gate_qt[l] : 39;
                s.sqts[1] = shexp_up_qt ? shexp_up_qt[l] : 39;
                s.sqts[2] = shexp_down_qt ? shexp_down_qt[l] : 39;
                s.p[13] = shexp_gate_raw[l]; s.p[14] = shexp_up_raw[l]; s.p[15] = shexp_down_raw[l];
                key.push_back((uintptr_t)shexp_router[l]);
            }
        }
        for (int i = 0; i < 16; i++) K(s.p[i]);
        for (int i = 0; i < 8; i++) K((unsigned)s.ints[i]);
        for (int v : {s.ssm, s.moe, s.sh, s.si, s.qts[0], s.qts[1], s.qts[2], s.sqts[0], s.sqts[1], s.sqts[2], s.rqt})
            K((unsigned)v);
    }
    q36_model *&mp = g_q36_models[key];
    if (mp) {
        uint64_t f = 0;
        for (auto &fs : mp->fp_src) f = f * 1099511628211ull + fp_bytes(fs.first, fs.second);
        if (f != mp->fp) { (void)hipStreamSynchronize(st); delete mp; mp = nullptr; }
    }
    if (!mp) {
        q36_model *m = new q36_model;
        q36_dims &d = m->d;
        d.L = L; d.N = N; d.NH = NH; d.NKH = n_kv_h; d.HD = HD; d.E = n_experts; d.K = top_k; d.M = n_ff_expert;
        d.rope_dim = rope_dim; d.max_ctx = max_ctx; d.si_ssm = ssm_inner; d.G = ssm_groups; d.Sz = ssm_state_size;
        d.dtr = ssm_dt_rank; d.emb_q = emb_quant; d.out_nr = out_nr_final; d.eps = eps;
        d.sem_out = mllm_qmm_sem(out_qt_final);
        m->P = (int)P;
        bool ok = true;
        auto weight = [&](const void *h, int sem, int rows, int cols, mllm_packed &v) {
            if (ok && mllm_dropin_weight(h, sem, rows, cols, &v, nullptr)) ok = false;
            if (ok) m->fp_src.push_back({h, raw_bytes(sem, rows, cols)});
        };
        m->out_norm = m->upload(out_norm_w, N);
        weight(out_w, d.sem_out, out_nr_final, N, m->out_w);
        if (n_attn) {
            m->cos_t = m->upload(cos_table, (long)max_ctx * (rd / 2));
            m->sin_t = m->upload(sin_table, (long)max_ctx * (rd / 2));
            ok = ok && m->cos_t && m->sin_t;
        }
        ok = ok && m->out_norm;
        m->layers.resize(L);
        for (int l = 0; l < L && ok; l++) {
            q36_layer &y = m->layers[l];
            const lay_src &s = src[l];
            y.ssm = s.ssm;
            y.an = m->upload(attn_norm_w[l], N);
            y.fn = m->upload(ffn_norm_w[l], N);
            ok = y.an && y.fn;
            if (y.ssm) {
                y.sem_gate = mllm_qmm_sem(gate_qt[l]);
                y.sem_so = mllm_qmm_sem(ssm_out_qt[l]);
                y.gate_nr = gate_nr[l];
                weight(attn_gate_raw[l], y.sem_gate, gate_nr[l], N, y.gate);
                weight(ssm_out_raw[l], y.sem_so, N, ssm_inner, y.so);
                if (ok) {
                    y.conv = m->upload(ssm_conv1d[l], 2L * ssm_inner);
                    y.a = m->upload(ssm_a[l], std::max(ssm_groups, 1));
                    y.dtb = m->upload(ssm_dt_bias[l], std::max(ssm_groups, 1));
                    y.alpha = m->upload(ssm_alpha[l], std::max((long)ssm_groups * ssm_dt_rank, 1L));
                    y.beta = m->upload(ssm_beta[l], std::max((long)ssm_groups * ssm_dt_rank, 1L));
                    ok = y.conv && y.a && y.dtb && y.alpha && y.beta;
                }
            } else {
                y.sem_qkv = mllm_qmm_sem(qkv_qt[l]);
                y.sem_o = mllm_qmm_sem(out_qt[l]);
                y.n_qkv = qkv_nr[l];
                y.kv_slot = m->n_attn++;
                weight(attn_qkv_raw[l], y.sem_qkv, qkv_nr[l], N, y.qkv);
                weight(attn_out_raw[l], y.sem_o, N, inner, y.wo);
            }
            if (!ok || !s.moe) continue;
            y.moe = 1;
            // router: fp32 rows (code 0) in f32_matmul_omp's order, else quant_matmul_omp's GEMV
            y.sem_router = mllm_qmm_sem(s.rqt);
            if (y.sem_router < 0) { mllm_set_error("qwen36_batch_forward: MoE router type not served"); ok = false; break; }
            if (y.sem_router == SEM_F32) {
                float *r = m->upload((const float *)moe_router_raw[l], (long)n_experts * N);
                ok = r != nullptr;
                y.router.p[0] = (const uint8_t *)r;
            } else {
                weight(moe_router_raw[l], y.sem_router, n_experts, N, y.router);
            }
            // experts at the reference's per-type stride (CE:977-984; 0 for other types)
            auto stride = [&](int rows, int cols, int qt) -> long {
                switch (qt) {
                case 12: return (long)rows * (cols / 256) * 144;
                case 13: return (long)rows * (cols / 256) * 176;
                case 14: return (long)rows * (cols / 256) * 210;
                case 39: return (long)rows * (cols / 32) * 17;
                case 2: return (long)rows * (cols / 32) * 18;
                case 8: return (long)rows * (cols / 32) * 34;
                }
                return 0;
            };
            int sg, su, sd;
            mllm_moe_codes_sems(s.qts[0], s.qts[1], s.qts[2], &sg, &su, &sd);
            if (sg < 0 || su < 0) {
                mllm_set_error("qwen36_batch_forward: MoE gate/up types the expert path does not compute");
                ok = false;
                break;
            }
            const long gs = stride(n_ff_expert, N, s.qts[0]), us = stride(n_ff_expert, N, s.qts[1]),
                       ds = stride(N, n_ff_expert, s.qts[2]);
            std::vector<mllm_packed> tab(3 * (size_t)n_experts);
            for (int e = 0; e < n_experts && ok; e++) {
                weight(gate_exp_raw[l] + e * gs, sg, n_ff_expert, N, tab[e]);
                weight(up_exp_raw[l] + e * us, su, n_ff_expert, N, tab[n_experts + e]);
                if (sd >= 0) weight(down_exp_raw[l] + e * ds, sd, N, n_ff_expert, tab[2 * n_experts + e]);
            }
            if (!ok) break;
            y.tab = (mllm_packed *)m->dalloc(m->allocs, tab.size() * sizeof(mllm_packed));
            ok = y.tab && hipMemcpy(y.tab, tab.data(), tab.size() * sizeof(mllm_packed), hipMemcpyHostToDevice) ==
                              hipSuccess;
            if (ok) {
                y.ml = mllm_moe_layer_for_codes(s.qts[0], s.qts[1], s.qts[2], N, n_ff_expert, n_experts, top_k, y.tab);
                ok = y.ml != nullptr;
            }
            if (ok && s.qts[2] == 39 && !q8_ws) {
                mllm_set_error("qwen36_batch_forward: an MXFP4 down projection needs q8_ws (the reference "
                               "dereferences it)");
                ok = false;
            }
            if (ok && s.sh) {
                y.sh = 1;
                y.si = s.si;
                y.sem_sg = mllm_qmm_sem(s.sqts[0]);
                y.sem_su = mllm_qmm_sem(s.sqts[1]);
                y.sem_sd = mllm_qmm_sem(s.sqts[2]);
                if (y.si <= 0 || y.sem_sg < 0 || y.sem_su < 0 || y.sem_sd < 0 || !shexp_gate_raw || !shexp_up_raw ||
                    !shexp_down_raw) {
                    mllm_set_error("qwen36_batch_forward: shared expert shape or types not served");
                    ok = false;
                    break;
                }
                weight(shexp_gate_raw[l], y.sem_sg, y.si, N, y.sg);
                weight(shexp_up_raw[l], y.sem_su, y.si, N, y.su);
                weight(shexp_down_raw[l], y.sem_sd, N, y.si, y.sd);
                y.shr = ok ? m->upload(shexp_router[l], N) : nullptr;
                ok = ok && y.shr;
            }
        }
        if (!ok) {
            if (!*mllm_last_error()) mllm_set_error("qwen36_batch_forward: model upload failed");
            delete m;
            g_q36_models.erase(key);
            return;
        }
        uint64_t f = 0;
        for (auto &fs : m->fp_src) f = f * 1099511628211ull + fp_bytes(fs.first, fs.second);
        m->fp = f;
        mp = m;
    }
    q36_model &m = *mp;
    if (q36_buffers(m, B)) return;
    const q36_dims &d = m.d;
    // ---- KV mirror of the caller's caches (attention layers)
    q36_kv *kvp = nullptr;
    if (n_attn) {
        std::vector<uintptr_t> kk = {(uintptr_t)kv_k, (uintptr_t)kv_v, (uintptr_t)max_ctx, (uintptr_t)nkv, (uintptr_t)L};
        for (int l = 0; l < L; l++) kk.push_back((uintptr_t)m.layers[l].kv_slot);
        q36_kv *&kv = g_q36_kv[kk];
        if (!kv) {
            kv = new q36_kv;
            kv->max_ctx = max_ctx;
            kv->nkv = nkv;
            bool ok = true;
            for (int i = 0; i < n_attn && ok; i++) {
                float *a = nullptr, *b = nullptr;
                ok = hipMalloc(&a, (size_t)max_ctx * nkv * 4) == hipSuccess;
                if (ok) kv->k.push_back(a);
                ok = ok && hipMalloc(&b, (size_t)max_ctx * nkv * 4) == hipSuccess;
                if (ok) kv->v.push_back(b);
            }
            kv->rows.assign(n_attn, 0);
            kv->seal.assign(n_attn, 0);
            if (!ok) {
                delete kv;
                g_q36_kv.erase(kk);
                mllm_set_error("qwen36_batch_forward: KV mirror allocation failed");
                return;
            }
        }
        kvp = kv;
    }
    // ---- host staging: embedding rows, positions, SSM state, fused slice in; logits, state, KV rows, slice out
    const long GS = (long)d.G * d.Sz;
    const size_t row_b = emb_quant == 12 ? (size_t)(N / 256) * 144 : (size_t)N * 4;
    const long ws_slice = 3L * B * S;
    const size_t o_pos = a256((long)B * row_b), o_state = o_pos + a256((long)L * (B + 1) * 4),
                 o_slice = o_state + a256((long)L * GS * 4), in_total = o_slice + a256((long)m.P * 4);
    const size_t oo_state = a256((long)B * out_nr_final * 4), oo_kv = oo_state + a256((long)L * GS * 4),
                 oo_slice = oo_kv + a256((long)n_attn * 2 * nkv * 4), out_total = oo_slice + a256((long)m.P * 4);
    if (host_ensure(&g_q36_hin, &g_q36_hin_n, in_total) || host_ensure(&g_q36_hout, &g_q36_hout_n, out_total)) {
        mllm_set_error("qwen36_batch_forward: pinned staging allocation failed");
        return;
    }
    uint8_t *hin = (uint8_t *)g_q36_hin, *hout = (uint8_t *)g_q36_hout;
    for (int b = 0; b < B; b++) memcpy(hin + b * row_b, (const uint8_t *)emb + (size_t)tokens[b] * row_b, row_b);
    int *hpos = (int *)(hin + o_pos);
    for (int l = 0; l < L; l++) {
        const int p = m.layers[l].ssm ? 0 : kv_lens[l];
        for (int b = 0; b < B; b++) hpos[l * (B + 1) + b] = p;
        hpos[l * (B + 1) + B] = p + 1;
    }
    float *hstate = (float *)(hin + o_state);
    for (int l = 0; l < L; l++)
        if (m.layers[l].ssm) memcpy(hstate + l * GS, ssm_state + l * GS, (size_t)GS * 4);
    if (n_attn) memcpy(hin + o_slice, ws + ws_slice, (size_t)m.P * 4);
#define CK(e) do { if ((e) != hipSuccess) { mllm_set_error("qwen36_batch_forward: HIP call failed: " #e); return; } } while (0)
#define CKI(e) do { if ((e) != 0) { if (!*mllm_last_error()) mllm_set_error("qwen36_batch_forward: " #e " failed"); return; } } while (0)
    // inputs: one copy of the staging block's parts
    CK(hipMemcpyAsync(m.emb_rows, hin, (size_t)B * row_b, hipMemcpyHostToDevice, st));
    CK(hipMemcpyAsync(m.pos, hin + o_pos, (size_t)L * (B + 1) * 4, hipMemcpyHostToDevice, st));
    if (n_ssm) CK(hipMemcpyAsync(m.state, hin + o_state, (size_t)L * GS * 4, hipMemcpyHostToDevice, st));
    if (n_attn) CK(hipMemcpyAsync(m.slice, hin + o_slice, (size_t)m.P * 4, hipMemcpyHostToDevice, st));
    // KV rows the mirror lacks (rewritten rows, found by a sampled seal, are uploaded again)
    for (int l = 0; l < L; l++) {
        const q36_layer &y = m.layers[l];
        if (y.ssm) continue;
        const int s = y.kv_slot, hl = kv_lens[l];
        const size_t lo = (size_t)l * max_ctx * nkv;
        int from = std::min(kvp->rows[s], hl);
        if (from > 0 && kv_rows_seal(kv_k + lo, from, nkv) * 3 + kv_rows_seal(kv_v + lo, from, nkv) != kvp->seal[s])
            from = 0;
        if (hl > from) {
            CK(hipMemcpyAsync(kvp->k[s] + (size_t)from * nkv, kv_k + lo + (size_t)from * nkv,
                              (size_t)(hl - from) * nkv * 4, hipMemcpyHostToDevice, st));
            CK(hipMemcpyAsync(kvp->v[s] + (size_t)from * nkv, kv_v + lo + (size_t)from * nkv,
                              (size_t)(hl - from) * nkv * 4, hipMemcpyHostToDevice, st));
        }
        kvp->rows[s] = hl;
    }
    // ---- the pass
    uint8_t *ws_a = m.ws + m.ws_gemv, *ws_m = ws_a + m.ws_attn;
    const dim3 tb(256);
    if (emb_quant == 12) {
        hipLaunchKernelGGL(k_q36_embed_q4k, dim3(N / 256, B), tb, 0, st, m.emb_rows, N, m.x);
        CK(hipGetLastError());
    } else {
        CK(hipMemcpyAsync(m.x, m.emb_rows, (size_t)B * N * 4, hipMemcpyDeviceToDevice, st));
    }
    const size_t rms_lds = (size_t)(N / 8 + 1) * 4;
    auto rms = [&](const float *w) {
        hipLaunchKernelGGL(k_q36_rms, dim3(B), tb, rms_lds, st, m.x, w, N, eps, m.xn);
        return hipGetLastError();
    };
    for (int l = 0; l < L; l++) {
        const q36_layer &y = m.layers[l];
        CK(rms(y.an));
        if (y.ssm) {
            const int si = ssm_inner;
            CKI(gemv(m, y.sem_gate, y.gate, m.xn, m.gate, y.gate_nr, N, B, nullptr, nullptr, st));
            hipLaunchKernelGGL(k_q36_ssm_interm, dim3((si + 255) / 256, B), tb, 0, st, m.xn, N, y.conv, si, m.gate,
                               y.gate_nr, m.att, si);
            CK(hipGetLastError());
            if (GS > 0) {
                hipLaunchKernelGGL(k_q36_ssm_state, dim3((unsigned)((GS + 255) / 256)), tb, 0, st, m.xn, N, B, y.alpha,
                                   y.beta, y.dtb, y.a, d.G, d.Sz, d.dtr, m.state + l * GS);
                CK(hipGetLastError());
            }
            CKI(gemv(m, y.sem_so, y.so, m.att, m.x, N, si, B, m.x, nullptr, st));
        } else {
            const int nq = y.n_qkv, s = y.kv_slot;
            int *pos_l = m.pos + l * (B + 1), *seq1 = pos_l + B;
            CKI(gemv(m, y.sem_qkv, y.qkv, m.xn, m.qkvo, nq, N, B, nullptr, nullptr, st));
            hipLaunchKernelGGL(k_q36_split, dim3((std::max(inner, nkv) + 255) / 256, B), tb, 0, st, m.qkvo, nq,
                               m.slice, inner, N, nkv, m.q, m.kt, m.vt);
            CK(hipGetLastError());
            CKI(mllm_rope(m.q, B, NH, HD, pos_l, m.cos_t, m.sin_t, rope_dim, st));
            CKI(mllm_rope(m.kt, B, n_kv_h, HD, pos_l, m.cos_t, m.sin_t, rope_dim, st));
            hipLaunchKernelGGL(k_q36_commit, dim3((nq + 255) / 256), tb, 0, st, m.qkvo, nq, m.q, inner, B, m.slice);
            CK(hipGetLastError());
            mllm_kv_view kv{kvp->k[s], kvp->v[s], 0, nullptr, 0, 0, 0};
            for (int b = 0; b < B; b++) {
                CKI(mllm_kv_append(&kv, pos_l + b, m.kt + (long)b * nkv, m.vt + (long)b * nkv, 1, n_kv_h, HD, st));
                CKI(mllm_gqa_decode(0, m.q + (long)b * inner, &kv, seq1, max_ctx, 1, NH, n_kv_h, HD,
                                    m.att + (long)b * inner, ws_a, m.ws_attn, st));
            }
            CKI(gemv(m, y.sem_o, y.wo, m.att, m.x, N, inner, B, m.x, nullptr, st));
        }
        if (!y.moe) continue;
        CK(rms(y.fn));
        if (y.sem_router == SEM_F32) {
            const int thr = n_experts * 16;
            hipLaunchKernelGGL(k_q36_f32mm, dim3((thr + 255) / 256, B), tb, 0, st, (const float *)y.router.p[0], m.xn,
                               n_experts, N, m.lg);
            CK(hipGetLastError());
        } else {
            CKI(gemv(m, y.sem_router, y.router, m.xn, m.lg, n_experts, N, B, nullptr, nullptr, st));
        }
        CK(mllm_launch_route_finish(m.lg, B, n_experts, top_k, 1, m.idx, m.wk, st));
        CKI(mllm_moe_forward_routed(y.ml, m.xn, B, m.mo, ws_m, m.ws_moe, m.idx, m.wk, st));
        if (y.sh) {
            hipLaunchKernelGGL(k_q36_dot_chain, dim3((B + 63) / 64), dim3(64), 0, st, m.xn, y.shr, N, B, m.shs);
            CK(hipGetLastError());
            CKI(gemv(m, y.sem_sg, y.sg, m.xn, m.shg, y.si, N, B, nullptr, nullptr, st));
            CKI(gemv(m, y.sem_su, y.su, m.xn, m.shu, y.si, N, B, nullptr, nullptr, st));
            CKI(gemv(m, y.sem_sd, y.sd, m.shg, m.shd, N, y.si, B, nullptr, m.shu, st));
        }
        hipLaunchKernelGGL(k_q36_ffn_add, dim3((N + 255) / 256, B), tb, 0, st, m.x, m.mo, y.sh ? m.shd : nullptr,
                           m.shs, N);
        CK(hipGetLastError());
    }
    CK(rms(m.out_norm));
    CKI(gemv(m, d.sem_out, m.out_w, m.xn, m.logits, out_nr_final, N, B, nullptr, nullptr, st));
    // ---- results back
    CK(hipMemcpyAsync(hout, m.logits, (size_t)B * out_nr_final * 4, hipMemcpyDeviceToHost, st));
    if (n_ssm) CK(hipMemcpyAsync(hout + oo_state, m.state, (size_t)L * GS * 4, hipMemcpyDeviceToHost, st));
    for (int l = 0; l < L; l++) {
        const q36_layer &y = m.layers[l];
        if (y.ssm) continue;
        float *hk = (float *)(hout + oo_kv) + (size_t)y.kv_slot * 2 * nkv;
        CK(hipMemcpyAsync(hk, kvp->k[y.kv_slot] + (size_t)kv_lens[l] * nkv, (size_t)nkv * 4, hipMemcpyDeviceToHost, st));
        CK(hipMemcpyAsync(hk + nkv, kvp->v[y.kv_slot] + (size_t)kv_lens[l] * nkv, (size_t)nkv * 4,
                          hipMemcpyDeviceToHost, st));
    }
    if (n_attn) CK(hipMemcpyAsync(hout + oo_slice, m.slice, (size_t)m.P * 4, hipMemcpyDeviceToHost, st));
    CK(hipStreamSynchronize(st));
    memcpy(logits, hout, (size_t)B * out_nr_final * 4);
    for (int l = 0; l < L; l++) {
        const q36_layer &y = m.layers[l];
        if (y.ssm) {
            memcpy(ssm_state + l * GS, (float *)(hout + oo_state) + l * GS, (size_t)GS * 4);
            continue;
        }
        const size_t lo = (size_t)l * max_ctx * nkv;
        const float *hk = (const float *)(hout + oo_kv) + (size_t)y.kv_slot * 2 * nkv;
        memcpy(kv_k + lo + (size_t)kv_lens[l] * nkv, hk, (size_t)nkv * 4);
        memcpy(kv_v + lo + (size_t)kv_lens[l] * nkv, hk + nkv, (size_t)nkv * 4);
        const int s = y.kv_slot, n = kv_lens[l] + 1;
        kvp->rows[s] = n;
        kvp->seal[s] = kv_rows_seal(kv_k + lo, n, nkv) * 3 + kv_rows_seal(kv_v + lo, n, nkv);
    }
    if (n_attn) memcpy(ws + ws_slice, hout + oo_slice, (size_t)m.P * 4);
#undef CK
#undef CKI
#undef Q36_FAIL
}

} // extern "C"

// ============================================================ SSM drop-ins
namespace {

// Grow-only device and pinned buffers of the SSM drop-ins (under g_q36_mu).
void *g_ssm_dev = nullptr;
size_t g_ssm_dev_n = 0;

int dev_ensure(size_t want)
{
    if (want <= g_ssm_dev_n) return 0;
    if (g_ssm_dev) (void)hipFree(g_ssm_dev);
    g_ssm_dev = nullptr;
    g_ssm_dev_n = 0;
    if (hipMalloc(&g_ssm_dev, want + want / 4) != hipSuccess) { g_ssm_dev = nullptr; return -1; }
    g_ssm_dev_n = want + want / 4;
    return 0;
}

struct ssm_io {
    // device offsets of the parameters and activations, in floats
    size_t x, conv, a, dtb, alpha, beta, state, total;
};

ssm_io ssm_layout(int B, int N, int inner, int G, int Sz, int dtr)
{
    ssm_io o{};
    size_t at = 0;
    auto take = [&](long n) { size_t r = at; at += (size_t)a256(std::max(n, 1L) * 4) / 4; return r; };
    o.x = take((long)B * N);
    o.conv = take(2L * inner);
    o.a = take(G);
    o.dtb = take(G);
    o.alpha = take((long)G * dtr);
    o.beta = take((long)G * dtr);
    o.state = take((long)G * Sz);
    o.total = at;
    return o;
}

// Stage the SSM parameters, x and the state into the pinned buffer at io's offsets.
void ssm_stage(float *h, const ssm_io &io, const float *x, int B, int N, const float *conv, int inner, const float *a,
               const float *dtb, const float *alpha, const float *beta, int G, int dtr, const float *state, int Sz)
{
    memcpy(h + io.x, x, (size_t)B * N * 4);
    memcpy(h + io.conv, conv, (size_t)2 * inner * 4);
    if (G > 0) {
        memcpy(h + io.a, a, (size_t)G * 4);
        memcpy(h + io.dtb, dtb, (size_t)G * 4);
        if (dtr > 0) {
            memcpy(h + io.alpha, alpha, (size_t)G * dtr * 4);
            memcpy(h + io.beta, beta, (size_t)G * dtr * 4);
        }
        if (Sz > 0) memcpy(h + io.state, state, (size_t)G * Sz * 4);
    }
}

} // namespace

extern "C" {

// ssm_decode_step (CE:736-802) on host buffers: ssm_intermediate[b] =
// silu(x_b conv_gate) * (x_b conv_in) and the per-group state update for the
// B tokens in order (state modified in place).  ssm_norm_w and conv_kernel are
// unused, as in the reference.
MLLM_API void ssm_decode_step(const float *x, float *ssm_intermediate, const float *conv1d_w, const float *a_param,
                              const float *dt_bias, const float *alpha, const float *beta, const float *ssm_norm_w,
                              float *state, int B, int N, int inner, int groups, int state_size, int conv_kernel,
                              int dt_rank)
{
    (void)ssm_norm_w; (void)conv_kernel;
    std::shared_lock<std::shared_mutex> api(mllm_api_mutex());
    if (B <= 0) return;
    const bool has_state = groups > 0 && state_size > 0;
    if (N <= 0 || inner <= 0 || 2 * inner > 8192 || groups < 0 || state_size < 0 || dt_rank < 0 || !x ||
        !ssm_intermediate || !conv1d_w || (groups > 0 && (!a_param || !dt_bias || (dt_rank > 0 && (!alpha || !beta)))) ||
        (has_state && !state)) {
        mllm_set_error("ssm_decode_step: bad shape or null argument (2*inner must fit the reference's 8192-float "
                       "conv buffer; outputs untouched)");
        return;
    }
    std::lock_guard<std::mutex> lk(g_q36_mu);
    if (ensure_stream()) return;
    hipStream_t st = g_q36_st;
    const ssm_io io = ssm_layout(B, N, inner, groups, state_size, dt_rank);
    const size_t o_int = io.total, total = io.total + (size_t)a256((long)B * inner * 4) / 4;
    const size_t out_n = (size_t)B * inner + (size_t)groups * state_size;
    if (dev_ensure(total * 4) || host_ensure(&g_q36_hin, &g_q36_hin_n, io.total * 4) ||
        host_ensure(&g_q36_hout, &g_q36_hout_n, out_n * 4)) {
        mllm_set_error("ssm_decode_step: allocation failed");
        return;
    }
    float *h = (float *)g_q36_hin, *ho = (float *)g_q36_hout, *dv = (float *)g_ssm_dev;
    ssm_stage(h, io, x, B, N, conv1d_w, inner, a_param, dt_bias, alpha, beta, groups, dt_rank, state, state_size);
#define CK(e) do { if ((e) != hipSuccess) { mllm_set_error("ssm_decode_step: HIP call failed: " #e); return; } } while (0)
    CK(hipMemcpyAsync(dv, h, io.total * 4, hipMemcpyHostToDevice, st));
    hipLaunchKernelGGL(k_q36_ssm_interm, dim3((inner + 255) / 256, B), dim3(256), 0, st, dv + io.x, N, dv + io.conv,
                       inner, nullptr, 0, dv + o_int, inner);
    CK(hipGetLastError());
    if (has_state) {
        hipLaunchKernelGGL(k_q36_ssm_state, dim3((groups * state_size + 255) / 256), dim3(256), 0, st, dv + io.x, N,
                           B, dv + io.alpha, dv + io.beta, dv + io.dtb, dv + io.a, groups, state_size, dt_rank,
                           dv + io.state);
        CK(hipGetLastError());
    }
    CK(hipMemcpyAsync(ho, dv + o_int, (size_t)B * inner * 4, hipMemcpyDeviceToHost, st));
    if (has_state) CK(hipMemcpyAsync(ho + (size_t)B * inner, dv + io.state, (size_t)groups * state_size * 4,
                                     hipMemcpyDeviceToHost, st));
    CK(hipStreamSynchronize(st));
#undef CK
    memcpy(ssm_intermediate, ho, (size_t)B * inner * 4);
    if (has_state) memcpy(state, ho + (size_t)B * inner, (size_t)groups * state_size * 4);
}

// ssm_layer_fused (CE:803-849) on host buffers: ssm_decode_step into
// `output` (used as the intermediate, B x inner floats), then per token b in
// order: interm_b *= gate_raw . x_b, output[b*N ..] = residual_b +
// ssm_out_raw . interm_b.  output must hold max(B*N, B*inner) floats; where
// N > inner a token's result overwrites later tokens' intermediates before
// they are used, as in the reference, and that order is reproduced.
MLLM_API void ssm_layer_fused(const float *x, float *residual, float *output, const float *conv1d_w,
                              const float *a_param, const float *dt_bias, const float *alpha, const float *beta,
                              const float *ssm_norm_w, float *state, const uint8_t *gate_raw, int gate_nr, int gate_nc,
                              int gate_qt, const uint8_t *ssm_out_raw, int ssm_out_nr, int ssm_out_nc, int ssm_out_qt,
                              int B, int N, int inner, int groups, int state_size, int conv_kernel, int dt_rank)
{
    (void)ssm_norm_w; (void)conv_kernel;
    std::shared_lock<std::shared_mutex> api(mllm_api_mutex());
    if (B <= 0) return;
    const int sem_g = mllm_qmm_sem(gate_qt), sem_o = mllm_qmm_sem(ssm_out_qt);
    const bool has_state = groups > 0 && state_size > 0;
    if (N <= 0 || N > 8192 || inner <= 0 || 2 * inner > 8192 || groups < 0 || state_size < 0 || dt_rank < 0 || !x ||
        !residual || !output || !conv1d_w || !gate_raw || !ssm_out_raw ||
        (groups > 0 && (!a_param || !dt_bias || (dt_rank > 0 && (!alpha || !beta)))) || (has_state && !state) ||
        gate_nc != N || gate_nr < inner || gate_nr > 8192 || ssm_out_nr != N || ssm_out_nc != inner || sem_g < 0 ||
        sem_o < 0) {
        mllm_set_error("ssm_layer_fused: shapes not served (gate >= inner x N and <= 8192 rows, ssm_out N x inner, "
                       "quant_matmul_omp types, N <= 8192 and 2*inner <= 8192 as the reference's stack buffers) or "
                       "null argument (outputs untouched)");
        return;
    }
    std::lock_guard<std::mutex> lk(g_q36_mu);
    if (ensure_stream()) return;
    hipStream_t st = g_q36_st;
    mllm_packed wg, wo;
    if (mllm_dropin_weight(gate_raw, sem_g, gate_nr, N, &wg, nullptr) ||
        mllm_dropin_weight(ssm_out_raw, sem_o, N, inner, &wo, nullptr))
        return;
    const ssm_io io = ssm_layout(B, N, inner, groups, state_size, dt_rank);
    const long on = std::max((long)B * N, (long)B * inner);
    const size_t o_res = io.total, o_out = o_res + a256((long)B * N * 4) / 4, o_gate = o_out + a256(on * 4) / 4,
                 o_op = o_gate + a256((long)B * gate_nr * 4) / 4, o_ws = o_op + a256((long)B * N * 4) / 4;
    const long wsg = std::max(mllm_gemv_workspace_size(sem_g, gate_nr, N, B), 256L);
    mllm_gemv_fusion fa{};
    float dummy = 0.0f;
    fa.out_add = &dummy;
    const long wso = std::max({mllm_gemv_fused_workspace_size(sem_o, N, inner, B, &fa),
                               mllm_gemv_fused_workspace_size(sem_o, N, inner, 1, &fa), 256L});
    const size_t total = o_ws + (size_t)a256(std::max(wsg, wso)) / 4;
    const size_t in_n = o_out, out_n = (size_t)on + (size_t)groups * state_size;
    if (dev_ensure(total * 4) || host_ensure(&g_q36_hin, &g_q36_hin_n, in_n * 4) ||
        host_ensure(&g_q36_hout, &g_q36_hout_n, out_n * 4)) {
        mllm_set_error("ssm_layer_fused: allocation failed");
        return;
    }
    float *h = (float *)g_q36_hin, *ho = (float *)g_q36_hout, *dv = (float *)g_ssm_dev;
    ssm_stage(h, io, x, B, N, conv1d_w, inner, a_param, dt_bias, alpha, beta, groups, dt_rank, state, state_size);
    memcpy(h + o_res, residual, (size_t)B * N * 4);
    float *X = dv + io.x, *RES = dv + o_res, *O = dv + o_out, *GATE = dv + o_gate, *OP = dv + o_op;
    void *WS = dv + o_ws;
#define CK(e) do { if ((e) != hipSuccess) { mllm_set_error("ssm_layer_fused: HIP call failed: " #e); return; } } while (0)
#define CKI(e) do { if ((e) != 0) return; } while (0)
    CK(hipMemcpyAsync(dv, h, in_n * 4, hipMemcpyHostToDevice, st));
    if (has_state) {
        hipLaunchKernelGGL(k_q36_ssm_state, dim3((groups * state_size + 255) / 256), dim3(256), 0, st, X, N, B,
                           dv + io.alpha, dv + io.beta, dv + io.dtb, dv + io.a, groups, state_size, dt_rank,
                           dv + io.state);
        CK(hipGetLastError());
    }
    CKI(mllm_gemv(sem_g, wg.p[0], X, GATE, gate_nr, N, B, WS, st));
    mllm_gemv_fusion f{};
    f.out_add = RES;
    if (N <= inner) {
        // no token's result reaches another token's intermediate: all tokens at once
        hipLaunchKernelGGL(k_q36_ssm_interm, dim3((inner + 255) / 256, B), dim3(256), 0, st, X, N, dv + io.conv,
                           inner, GATE, gate_nr, O, inner);
        CK(hipGetLastError());
        CKI(mllm_gemv_fused(sem_o, wo.p[0], O, OP, N, inner, B, &f, WS, st));
        CK(hipMemcpyAsync(O, OP, (size_t)B * N * 4, hipMemcpyDeviceToDevice, st));
    } else {
        hipLaunchKernelGGL(k_q36_ssm_interm, dim3((inner + 255) / 256, B), dim3(256), 0, st, X, N, dv + io.conv,
                           inner, nullptr, 0, O, inner);
        CK(hipGetLastError());
        for (int b = 0; b < B; b++) {
            hipLaunchKernelGGL(k_q36_mul, dim3((inner + 255) / 256), dim3(256), 0, st, O + (long)b * inner,
                               GATE + (long)b * gate_nr, inner);
            CK(hipGetLastError());
            CKI(mllm_gemv(sem_o, wo.p[0], O + (long)b * inner, OP, N, inner, 1, WS, st));
            hipLaunchKernelGGL(k_q36_add2, dim3((N + 255) / 256), dim3(256), 0, st, O + (long)b * N,
                               RES + (long)b * N, OP, N);
            CK(hipGetLastError());
        }
    }
    CK(hipMemcpyAsync(ho, O, (size_t)on * 4, hipMemcpyDeviceToHost, st));
    if (has_state) CK(hipMemcpyAsync(ho + on, dv + io.state, (size_t)groups * state_size * 4, hipMemcpyDeviceToHost, st));
    CK(hipStreamSynchronize(st));
#undef CK
#undef CKI
    memcpy(output, ho, (size_t)on * 4);
    if (has_state) memcpy(state, ho + on, (size_t)groups * state_size * 4);
}

} // extern "C"
