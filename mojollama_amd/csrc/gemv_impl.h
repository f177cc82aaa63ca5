// gemv_impl.h — decode GEMV kernels for batch 1..8 on gfx950 (instantiated per
// semantic in gemv_*.hip so the library compiles in parallel).
//
// out[b][row] = sum_k w[row][k] * x[b][k] for one weight matrix, or for a list
// of "jobs" (expert matrices picked through a device-side index array, as the
// MoE layer needs).  The path is HBM-bound, so the kernel is built around the
// weight stream:
//   * a workgroup (4 wave64s) first stages its activations into LDS, tiling
//     K when B*K does not fit in 48 KB;
//   * a wave owns R rows per group of LPR lanes; the lanes of a group walk the
//     row's 32-weight chunks, so one wave-wide load reads consecutive 16-byte
//     pieces of a row; a lane issues the loads of all R rows before decoding;
//   * fp32 activations are staged as three int8 digit planes per 16-element
//     group (see "activation digits"), so a run of 16 byte codes costs 12
//     v_dot4_i32_i8 and the per-run scale and offset are applied once in fp32;
//   * lane groups reduce with DPP row operations and two cross-row swaps.
#pragma once
#include <algorithm>
#include "decode.h"
#include "gemv.h"

namespace mllm_gemv {

constexpr int kLdsFloats = 12288;   // 48 KB of activations per workgroup

template <int W>
MLLM_DEV float group_sum(float v)
{
    // Sum over aligned groups of W lanes; every lane of the group ends with the total.
    if constexpr (W >= 2)  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false)); // quad_perm 1,0,3,2
    if constexpr (W >= 4)  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false)); // quad_perm 2,3,0,1
    if constexpr (W >= 8)  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false)); // row_half_mirror
    if constexpr (W >= 16) v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false)); // row_mirror
    if constexpr (W >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (W >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// Matrix, output and activation offsets of job `job` (blockIdx.y).
struct job_view {
    mllm_packed W;
    float *out;
    long xj;   // activation row index: x starts at xj * x_job_stride
};

MLLM_DEV job_view view_job(const mllm_gemv_args &a, int job)
{
    job_view v;
    const bool second = a.job_split > 0 && job >= a.job_split;
    if (second) job -= a.job_split;
    v.out = (second ? a.out2 : a.out) + job * a.out_job_stride;
    v.xj = a.job_div > 1 ? job / a.job_div : job;
    // W is taken from the argument block only on the table-less path, so no
    // address choice mixes the argument block with a table (which would put
    // the kernel arguments in scratch memory)
    if (a.table) {
        // job-uniform reads through the constant address space: scalar loads, which
        // leave the vector memory counter to the activation and weight loads (a
        // generic load here makes the compiler drain every vector load before the
        // first weight load is issued)
        typedef const __attribute__((address_space(4))) int cint;
        typedef const __attribute__((address_space(4))) uint64_t cu64;
        const int e = a.idx ? *(cint *)(a.idx + job) : job;
        cu64 *tp = (cu64 *)((second ? a.table2 : a.table) + (e < 0 ? 0 : e));
#pragma unroll
        for (int i = 0; i < MLLM_MAX_PLANES; i++) v.W.p[i] = (const uint8_t *)tp[i];
    } else {
        v.W = a.W;
    }
    return v;
}

// ---------------------------------------------------------------- activation digits
//
// fp32-activation semantics run their dot products on integers.  Each
// 16-element group of x is written as P * (d0 + d1/2^7 + d2/2^14) with P a
// power of two (max|x| / P in [32, 64), so |d0| <= 64) and d1, d2 in [-64, 64]:
// all of it exact in fp32 except the discarded remainder, at most 2^-15 of P,
// i.e. below 2^-20 of the group's largest element.  A run of 16 weight codes
// u then dots each digit plane with v_dot4_i32_i8 (exact in int32), and
//   sum_i (s*(u_i - bias) + o) * x_i = s*P*(I0 + I1/2^7 + I2/2^14) + (o - s*bias) * sum_i x_i.
// LDS per token: three digit planes of PL = KT + KT/16 bytes (16 bytes of
// padding per 256, so the lanes' 16-byte reads spread over the banks), then
// a float2 record (P, sum x) per group.  Digit bytes are stored in the
// format's code order (byte t of word j holds element code_pos(j, t)), so a
// code word and a digit word line up byte for byte.  A group holding an inf
// or NaN gets P = NaN: every row then falls to the per-element path below
// and comes out NaN.
MLLM_DEV int dpad(int i) { return i + ((i >> 8) << 4); }

struct digit_geom {
    int PL;        // bytes per digit plane
    int tstride;   // bytes per token (16-byte multiple)
};

__host__ __device__ inline digit_geom digit_geom_for(int KT)
{
    digit_geom g;
    g.PL = KT + (KT >> 4);
    g.tstride = (3 * g.PL + 8 * (KT >> 4) + 15) & ~15;
    return g;
}

// Staging is split in two so that a workgroup can issue its activation loads
// ahead of its first weight loads (loads complete in order, so x then does
// not wait behind the weights) and turn them into digits while the weights
// are in flight.  Each thread takes half-groups of 8 elements (kStageSlots
// per pass); the two halves of a group sit in adjacent lanes and exchange
// their max and sum over DPP.
constexpr int kStageSlots = 4;

template <bool SILU> struct x_stage {
    float4 v[kStageSlots][2];
};
// SiLU-product staging: the gate half in v, the up half in u.
template <> struct x_stage<true> {
    float4 v[kStageSlots][2];
    float4 u[kStageSlots][2];
};

template <bool SILU, int NT = 256>
MLLM_DEV void stage_load(x_stage<SILU> &st, const float *__restrict__ x, const float *__restrict__ xu, int ldx, int B,
                         int k0, int kn, int pass)
{
    // Branch-free per lane: a slot some lane of the workgroup uses is loaded by
    // every lane (indices past the end clamped to the last half-group; such
    // lanes store nothing), so the loads stay in flight while the caller issues
    // its weight loads behind them.
    const int nh = kn >> 3, n = B * nh;
    const bool vec = (ldx & 3) == 0;
#pragma unroll
    for (int q = 0; q < kStageSlots; q++) {
        const int base = NT * (q + pass * kStageSlots);
        if (base >= n) break;
        const int idx = min(base + (int)threadIdx.x, n - 1);
        const int b = idx / nh, h = idx - b * nh;
        const float *src = x + (long)b * ldx + k0 + 8 * h;
        if (vec) {
            st.v[q][0] = gld<float4>(src);
            st.v[q][1] = gld<float4>(src + 4);
        } else {
            st.v[q][0] = make_float4(gld<float>(src), gld<float>(src + 1), gld<float>(src + 2), gld<float>(src + 3));
            st.v[q][1] = make_float4(gld<float>(src + 4), gld<float>(src + 5), gld<float>(src + 6), gld<float>(src + 7));
        }
        if constexpr (SILU) {
            const float *su = xu + (long)b * ldx + k0 + 8 * h;
            if (vec) {
                st.u[q][0] = gld<float4>(su);
                st.u[q][1] = gld<float4>(su + 4);
            } else {
                st.u[q][0] = make_float4(gld<float>(su), gld<float>(su + 1), gld<float>(su + 2), gld<float>(su + 3));
                st.u[q][1] = make_float4(gld<float>(su + 4), gld<float>(su + 5), gld<float>(su + 6), gld<float>(su + 7));
            }
        }
    }
}

// Value of the partner lane (lane ^ 1).
MLLM_DEV float lane_pair(float v) { return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false)); }

// ---------------------------------------------------------------- fused prologue
//
// Residual add and RMS norm fused into the staging (mllm_gemv_args: x_res,
// res_out, rms_w).  RMSNorm scales a token's whole activation by one scalar
// s (1/rms, or rms with rms_div), so W . (v * s * w) = s * (W . (v * w)):
// the kernel stages v * w at once, records sum(v^2) of each 8-element piece
// in LDS, and each wave folds s into its outputs in the epilogue, after the
// barrier that follows the staging anyway -- no extra pass over x and no
// extra barrier.  (The product is reassociated relative to the reference's
// (v * s) * w: one fp32 rounding apart.)
struct pro_regs {
    float4 r[kStageSlots][2];   // residual
    float4 w[kStageSlots][2];   // RMS weight
};

MLLM_DEV void f4x2_to8(const float4 (&p)[2], float (&v)[8])
{
    v[0] = p[0].x; v[1] = p[0].y; v[2] = p[0].z; v[3] = p[0].w;
    v[4] = p[1].x; v[5] = p[1].y; v[6] = p[1].z; v[7] = p[1].w;
}

// v (8 elements of token b at column k): + residual; res_out = v (writer
// workgroup); part = sum v^2; v * rms weight.
MLLM_DEV void prologue8(float (&v)[8], const float4 (&r)[2], const float4 (&w)[2], const mllm_gemv_args &a, int b,
                        int k, bool writer, float *part)
{
    if (a.x_res) {
        float rr[8];
        f4x2_to8(r, rr);
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] += rr[e];
    }
    if (writer) {
        float *o = a.res_out + (long)b * a.ldx + k;
        *reinterpret_cast<float4 *>(o) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4 *>(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
    if (a.rms_w) {
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) ss = fmaf(v[e], v[e], ss);
        *part = ss;
        float ww[8];
        f4x2_to8(w, ww);
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] *= ww[e];
    }
}

// Residual and RMS-weight loads of the half-groups stage_load loads (same
// indices, clamped the same way; elements from k0 on).
MLLM_DEV void pro_load(pro_regs &pr, const mllm_gemv_args &a, int B, int kn, int pass, int k0 = 0)
{
    const int nh = kn >> 3, n = B * nh;
#pragma unroll
    for (int q = 0; q < kStageSlots; q++) {
        const int base = 256 * (q + pass * kStageSlots);
        if (base >= n) break;
        const int idx = min(base + (int)threadIdx.x, n - 1);
        const int b = idx / nh, h = idx - b * nh;
        if (a.x_res) {
            const float *src = a.x_res + (long)b * a.ldx + k0 + 8 * h;
            pr.r[q][0] = gld<float4>(src);
            pr.r[q][1] = gld<float4>(src + 4);
        }
        if (a.rms_w) {
            pr.w[q][0] = gld<float4>(a.rms_w + k0 + 8 * h);
            pr.w[q][1] = gld<float4>(a.rms_w + k0 + 8 * h + 4);
        }
    }
}

// Byte 0 of a, b, c, d packed into one word (a lowest).
MLLM_DEV uint32_t pack_b0(uint32_t a, uint32_t b, uint32_t c, uint32_t d)
{
    const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);   // [a0, b0, 0, 0]
    const uint32_t hi = __builtin_amdgcn_perm(d, c, 0x04000c0cu);   // [0, 0, c0, d0]
    return lo | hi;
}

template <int SEM, bool SILU, bool PRO = false, int NT = 256>
MLLM_DEV bool stage_store(const x_stage<SILU> &st, uint8_t *lds, const digit_geom &dg, int B, int kn, int pass,
                          bool clamp, const pro_regs *pr = nullptr, const mllm_gemv_args *pa = nullptr,
                          float *part = nullptr)
{
    const int nh = kn >> 3;
    constexpr float M = 12582912.0f;   // 1.5 * 2^23: t = y + M holds rne(y) in its low mantissa bits
    bool any_bad = false;
#pragma unroll
    for (int q = 0; q < kStageSlots; q++) {
        const int idx = threadIdx.x + NT * (q + pass * kStageSlots);
        if (idx >= B * nh) continue;       // B * nh is even: both halves of a group take the same path
        const int b = idx / nh, h = idx - b * nh, g = h >> 1, half = h & 1;
        float v[8] = {st.v[q][0].x, st.v[q][0].y, st.v[q][0].z, st.v[q][0].w,
                      st.v[q][1].x, st.v[q][1].y, st.v[q][1].z, st.v[q][1].w};
        if constexpr (SILU) {
            const float u[8] = {st.u[q][0].x, st.u[q][0].y, st.u[q][0].z, st.u[q][0].w,
                                st.u[q][1].x, st.u[q][1].y, st.u[q][1].z, st.u[q][1].w};
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = mllm_silu_mul(v[e], u[e], clamp);
        }
        if constexpr (PRO)
            prologue8(v, pr->r[q], pr->w[q], *pa, b, 8 * h, pa->res_out && blockIdx.x == 0, part + idx);
        float m = 0.0f, sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) { m = fmaxf(m, fabsf(v[e])); sum += v[e]; }
        m = fmaxf(m, lane_pair(m));
        sum += lane_pair(sum);
        const bool bad = !isfinite(sum);
        any_bad |= bad;
        // P = 2^E with |x| / P < 64: E from m's exponent field
        const int E = (int)((__float_as_uint(m) >> 23) & 0xFF) - 132;
        uint32_t t[3][8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float y = ldexpf(v[e], -E);          // exact (|y| < 64)
            const float t0 = y + M, r0 = y - (t0 - M);
            const float t1 = fmaf(r0, 128.0f, M), r1 = fmaf(r0, 128.0f, M - t1);
            const float t2 = fmaf(r1, 128.0f, M);
            t[0][e] = __float_as_uint(t0); t[1][e] = __float_as_uint(t1); t[2][e] = __float_as_uint(t2);
        }
        // this half's 8 elements are words 2*half, 2*half+1 of the group
        uint8_t *tb = lds + b * dg.tstride;
#pragma unroll
        for (int p = 0; p < 3; p++) {
            // word jj of this half holds, in both code orders, its elements code_pos(jj, 0..3)
            uint32_t w[2];
#pragma unroll
            for (int jj = 0; jj < 2; jj++)
                w[jj] = pack_b0(t[p][code_pos<SEM>(jj, 0)], t[p][code_pos<SEM>(jj, 1)], t[p][code_pos<SEM>(jj, 2)],
                                t[p][code_pos<SEM>(jj, 3)]);
            *reinterpret_cast<uint2 *>(tb + p * dg.PL + dpad(16 * g) + 8 * half) = make_uint2(w[0], w[1]);
        }
        if (half == 0) {
            const float P = bad ? __int_as_float(0x7FC00000) : ldexpf(1.0f, E);
            reinterpret_cast<float2 *>(tb + 3 * dg.PL)[g] = make_float2(P, bad ? P : sum);
        }
    }
    return any_bad;
}


// The rare path of the digit staging: a group whose 16 values hold an inf or
// NaN (or overflow their sum) was staged under P = NaN, which makes every
// output NaN; the reference gives +-inf wherever no NaN arises.  A wave with
// such a group stages its groups again from memory keeping each element's
// class: a group holding +-inf gets digit +-64 for each infinite element and
// 0 for the finite ones (their products are finite, the group's sum is not)
// under P = +inf, which sends every chunk reading it to chunk_value's
// per-element path; a NaN keeps P = NaN; an all-finite group whose sum
// overflowed is staged as usual.  v = silu(x, xu) with xu, + x_res with x_res.
template <int SEM, int NT = 256>
MLLM_DEV void stage_fix(uint8_t *lds, const digit_geom &dg, const float *__restrict__ x, const float *__restrict__ xu,
                        const float *__restrict__ x_res, int ldx, int B, int k0, int kn, bool clamp)
{
    constexpr float M = 12582912.0f;
    const int nh = kn >> 3, n = B * nh;
    for (int base = 0; base < n; base += NT) {       // n even: both halves of a group stay in step
        const int idx = base + (int)threadIdx.x;
        if (idx >= n) break;
        const int b = idx / nh, h = idx - b * nh, g = h >> 1, half = h & 1;
        const long o = (long)b * ldx + k0 + 8 * h;
        float v[8];
        for (int e = 0; e < 8; e++) {
            v[e] = x[o + e];
            if (xu) v[e] = mllm_silu_mul(v[e], xu[o + e], clamp);
            if (x_res) v[e] += x_res[o + e];
        }
        float m = 0.0f, sum = 0.0f, nf = 0.0f;     // nf: 1 per infinite element, 256 per NaN
        for (int e = 0; e < 8; e++) {
            m = fmaxf(m, fabsf(v[e]));
            sum += v[e];
            nf += v[e] != v[e] ? 256.0f : isinf(v[e]) ? 1.0f : 0.0f;
        }
        m = fmaxf(m, lane_pair(m));
        sum += lane_pair(sum);
        nf += lane_pair(nf);
        const int E = (int)((__float_as_uint(m) >> 23) & 0xFF) - 132;
        uint32_t t[3][8];
        for (int e = 0; e < 8; e++) {
            if (nf == 0.0f) {
                const float y = ldexpf(v[e], -E);
                const float t0 = y + M, r0 = y - (t0 - M);
                const float t1 = fmaf(r0, 128.0f, M), r1 = fmaf(r0, 128.0f, M - t1);
                t[0][e] = __float_as_uint(t0); t[1][e] = __float_as_uint(t1);
                t[2][e] = __float_as_uint(fmaf(r1, 128.0f, M));
            } else {
                t[0][e] = __float_as_uint(M + (isinf(v[e]) ? copysignf(64.0f, v[e]) : 0.0f));
                t[1][e] = t[2][e] = __float_as_uint(M);
            }
        }
        uint8_t *tb = lds + b * dg.tstride;
        for (int p = 0; p < 3; p++) {
            uint32_t w[2];
            for (int jj = 0; jj < 2; jj++)
                w[jj] = pack_b0(t[p][code_pos<SEM>(jj, 0)], t[p][code_pos<SEM>(jj, 1)], t[p][code_pos<SEM>(jj, 2)],
                                t[p][code_pos<SEM>(jj, 3)]);
            *reinterpret_cast<uint2 *>(tb + p * dg.PL + dpad(16 * g) + 8 * half) = make_uint2(w[0], w[1]);
        }
        if (half == 0) {
            const float P = nf == 0.0f ? ldexpf(1.0f, E) : nf < 256.0f ? __builtin_inff() : __int_as_float(0x7FC00000);
            reinterpret_cast<float2 *>(tb + 3 * dg.PL)[g] = make_float2(P, nf == 0.0f ? sum : 0.0f);
        }
    }
}

// Stage tokens b < B, elements [k0, k0+kn), as digits; load_first = a pass-0
// load already issued by the caller.
template <int SEM, bool SILU, int NT = 256>
MLLM_DEV void stage_digits(x_stage<SILU> &st, bool load_first, uint8_t *lds, const digit_geom &dg,
                           const float *__restrict__ x, const float *__restrict__ xu, int ldx, int B, int k0, int kn,
                           bool clamp = true)
{
    // pass 0 stays out of the pass loop: there the wait before the digits
    // covers the activation loads only, not weight loads the caller issued
    // behind them (at a loop head the wait would cover every load in flight)
    const int passes = (B * (kn >> 3) + NT * kStageSlots - 1) / (NT * kStageSlots);
    if (!load_first) stage_load<SILU, NT>(st, x, xu, ldx, B, k0, kn, 0);
    bool bad = stage_store<SEM, SILU, false, NT>(st, lds, dg, B, kn, 0, clamp);
    for (int pass = 1; pass < passes; pass++) {
        stage_load<SILU, NT>(st, x, xu, ldx, B, k0, kn, pass);
        bad |= stage_store<SEM, SILU, false, NT>(st, lds, dg, B, kn, pass, clamp);
    }
    if (__any(bad)) stage_fix<SEM, NT>(lds, dg, x, SILU ? xu : nullptr, nullptr, ldx, B, k0, kn, clamp);
}

// The digit words of the run starting at tile-relative element e.
struct run_digits {
    uint32_t w[3][4];
    float P, sum;
};

MLLM_DEV void load_run(const uint8_t *tb, const digit_geom &dg, int e, run_digits &r)
{
#pragma unroll
    for (int p = 0; p < 3; p++) {
        const uint4 q = *reinterpret_cast<const uint4 *>(tb + p * dg.PL + dpad(e));
        r.w[p][0] = q.x; r.w[p][1] = q.y; r.w[p][2] = q.z; r.w[p][3] = q.w;
    }
    const float2 rec = reinterpret_cast<const float2 *>(tb + 3 * dg.PL)[e >> 4];
    r.P = rec.x;
    r.sum = rec.y;
}

template <int SEM> constexpr int digit_bias() { return SEM == SEM_Q8_0 ? 0 : sem_traits<SEM>::kBias; }

// Code t of word U as a value (Q8_0 codes are signed bytes here).
template <int SEM>
MLLM_DEV float code_f(uint32_t U, int t)
{
    if constexpr (SEM == SEM_Q8_0) return (float)(int8_t)((U >> (8 * t)) & 0xFF);
    else return ubyte_f(U, t);
}

// sum over one run of u_i * x_i in units of P: I0 + I1/2^7 + I2/2^14.  Codes
// |u| <= 64 (every format but Q8_0): the one integer (I0*2^7 + I1)*2^7 + I2,
// formed by a single v_dot4 chain that shifts its accumulator between planes
// and converted once; |d0|, |d1|, |d2| <= 64 over 16 elements bound it by
// 16*64*64*(2^14 + 2^7 + 1) < 2^31.  Q8_0's codes reach -128, which could
// carry the chain to 2^31: three accumulators there.
template <int SEM>
MLLM_DEV float run_idot(const uint32_t *U, const run_digits &x)
{
    if constexpr (SEM == SEM_Q8_0) {
        int I[3];
#pragma unroll
        for (int p = 0; p < 3; p++) {
            int acc = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) acc = __builtin_amdgcn_sdot4((int)U[j], (int)x.w[p][j], acc, false);
            I[p] = acc;
        }
        return fmaf((float)I[2], 0x1p-14f, fmaf((float)I[1], 0x1p-7f, (float)I[0]));
    } else {
        int acc = 0;
#pragma unroll
        for (int p = 0; p < 3; p++) {
            if (p) acc <<= 7;
#pragma unroll
            for (int j = 0; j < 4; j++) acc = __builtin_amdgcn_sdot4((int)U[j], (int)x.w[p][j], acc, false);
        }
        return (float)acc * 0x1p-14f;
    }
}

// Contribution of one decoded chunk to one token.
template <int SEM>
MLLM_DEV float chunk_value(const chunk_codes &k, const run_digits &x0, const run_digits &x1)
{
    constexpr int ibias = digit_bias<SEM>();
    constexpr float bias = (float)ibias;
    constexpr bool need_sum = ibias != 0 || sem_traits<SEM>::kOffset;
    float t = fmaf(k.s0 * x0.P, run_idot<SEM>(k.U, x0), (k.s1 * x1.P) * run_idot<SEM>(k.U + 4, x1));
    // (with no bias the offset term is o * sum x: an infinite s already makes the first term non-finite)
    if constexpr (need_sum && ibias == 0) t = fmaf(k.o0, x0.sum, fmaf(k.o1, x1.sum, t));
    else if constexpr (need_sum) t = fmaf(fmaf(-k.s0, bias, k.o0), x0.sum, fmaf(fmaf(-k.s1, bias, k.o1), x1.sum, t));
    if (!isfinite(t)) {
        // inf/NaN somewhere (scale, activation or an overflowing partial): weigh each
        // element as the reference does (w = s*q first, then w*x), x rebuilt from its digits.
        // The empty volatile asm keeps this a branch: without it the compiler
        // speculates the whole per-element path (~230 VALU ops per chunk) into
        // straight-line code that every lane runs.
        asm volatile("");
        t = 0.f;
        // a group holding +-inf is staged under P = +inf with digits +-64 / 0:
        // at P = 2^127 they rebuild +-inf / 0 (a NaN group keeps P = NaN)
        const float P0 = x0.P > 0x1p127f ? 0x1p127f : x0.P, P1 = x1.P > 0x1p127f ? 0x1p127f : x1.P;
        if constexpr (SEM == SEM_Q5_K_GGML) {
            // q5_k_row_dot_avx2 factors the min out of each 32-element sub-block
            // (QK:300, 338): d1 * sum(q x) - m1 * sum(x), here per 16-element run
            // (o = -m1), which gives the same inf / NaN outcome
            float qx0 = 0.f, sx0 = 0.f, qx1 = 0.f, sx1 = 0.f;
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float e0 = fmaf((float)(int8_t)(x0.w[2][j] >> (8 * q)), 0x1p-14f,
                                          fmaf((float)(int8_t)(x0.w[1][j] >> (8 * q)), 0x1p-7f, (float)(int8_t)(x0.w[0][j] >> (8 * q))));
                    const float e1 = fmaf((float)(int8_t)(x1.w[2][j] >> (8 * q)), 0x1p-14f,
                                          fmaf((float)(int8_t)(x1.w[1][j] >> (8 * q)), 0x1p-7f, (float)(int8_t)(x1.w[0][j] >> (8 * q))));
                    const float a0 = P0 * e0, a1 = P1 * e1;
                    qx0 = fmaf(code_f<SEM>(k.U[j], q), a0, qx0);
                    qx1 = fmaf(code_f<SEM>(k.U[4 + j], q), a1, qx1);
                    sx0 += a0;
                    sx1 += a1;
                }
            return fmaf(k.s0, qx0, k.o0 * sx0) + fmaf(k.s1, qx1, k.o1 * sx1);
        }
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float w0 = fmaf(k.s0, code_f<SEM>(k.U[j], q) - bias, k.o0);
                const float w1 = fmaf(k.s1, code_f<SEM>(k.U[4 + j], q) - bias, k.o1);
                const float e0 = fmaf((float)(int8_t)(x0.w[2][j] >> (8 * q)), 0x1p-14f,
                                      fmaf((float)(int8_t)(x0.w[1][j] >> (8 * q)), 0x1p-7f, (float)(int8_t)(x0.w[0][j] >> (8 * q))));
                const float e1 = fmaf((float)(int8_t)(x1.w[2][j] >> (8 * q)), 0x1p-14f,
                                      fmaf((float)(int8_t)(x1.w[1][j] >> (8 * q)), 0x1p-7f, (float)(int8_t)(x1.w[0][j] >> (8 * q))));
                t = fmaf(w0, P0 * e0, t);
                t = fmaf(w1, P1 * e1, t);
            }
    }
    return t;
}

// The run at digit offset dp (dpad of its first element) with its record at rec.
MLLM_DEV void load_run_at(const uint8_t *tb, const digit_geom &dg, int dp, int rec, run_digits &r)
{
#pragma unroll
    for (int p = 0; p < 3; p++) {
        const uint4 q = *reinterpret_cast<const uint4 *>(tb + p * dg.PL + dp);
        r.w[p][0] = q.x; r.w[p][1] = q.y; r.w[p][2] = q.z; r.w[p][3] = q.w;
    }
    const float2 v = *reinterpret_cast<const float2 *>(tb + 3 * dg.PL + rec);
    r.P = v.x;
    r.sum = v.y;
}

// Batch 1: chunk cc of block blk of R rows (already fetched into raw), activation
// digits from LDS (tile starting at element k0); SET: acc = the value, else +=.
// WHOLE: the tile is the whole row (k0 = 0); a chunk's two runs then lie in one
// 256-element segment of it, so their padded offsets follow from the segment
// and the chunk's place in it without the general dpad.
template <int SEM, int R, bool SET = false, bool WHOLE = false>
MLLM_DEV void accumulate_at(const raw_chunk (&raw)[R], int blk, int cc, const uint8_t *xl, const digit_geom &dg,
                            int k0, float (&acc)[R][1])
{
    // activation digits once per chunk, reused by the R rows
    chunk_codes k;
    codes_at<SEM, true>(raw[0], blk, cc, k);
    run_digits x0, x1;
    if constexpr (WHOLE) {
        constexpr int EPB = sem_traits<SEM>::kBlockElems;
        static_assert(EPB == 256 || EPB == 32, "blocks of 32 or 256 elements");
        const int seg = EPB == 256 ? blk : blk >> 3;
        const int f0 = k.x0 - 256 * seg, d1 = k.x1 - k.x0;    // f0 + d1 + 16 <= 256 in every format
        const int dp = 272 * seg + f0, rec = 128 * seg + 8 * (f0 >> 4);
        load_run_at(xl, dg, dp, rec, x0);
        load_run_at(xl, dg, dp + d1, rec + d1 / 2, x1);
    } else {
        load_run(xl, dg, k.x0 - k0, x0);
        load_run(xl, dg, k.x1 - k0, x1);
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        if (r) codes_at<SEM, true>(raw[r], blk, cc, k);
        const float v = chunk_value<SEM>(k, x0, x1);
        acc[r][0] = SET ? v : acc[r][0] + v;
    }
}

// Add chunk c of R rows (already fetched into raw) to acc, activation digits
// from LDS (tile starting at element k0).
template <int SEM, int BM, int R>
MLLM_DEV void accumulate(const raw_chunk (&raw)[R], int c, const uint8_t *xl, const digit_geom &dg, int k0, int B,
                         float (&acc)[R][BM])
{
    chunk_codes k;
    if constexpr (BM == 1) {
        constexpr int CPB = sem_traits<SEM>::kChunksPerBlock;
        accumulate_at<SEM, R>(raw, (int)((unsigned)c / CPB), (int)((unsigned)c % CPB), xl, dg, k0, acc);
    } else {
#pragma unroll
        for (int r = 0; r < R; r++) {
            codes<SEM, true>(raw[r], c, k);
#pragma unroll
            for (int b = 0; b < BM; b++) {
                if (b < B) {
                    run_digits x0, x1;
                    load_run(xl + b * dg.tstride, dg, k.x0 - k0, x0);
                    load_run(xl + b * dg.tstride, dg, k.x1 - k0, x1);
                    acc[r][b] += chunk_value<SEM>(k, x0, x1);
                }
            }
        }
    }
}

// fp32-activation semantics, K tiled through LDS (used when B*K does not fit)
template <int SEM, int BM, int R, int LPR, bool SILU>
__global__ __launch_bounds__(256) void k_gemv(mllm_gemv_args a)
{
    extern __shared__ uint4 xl4[];
    uint8_t *xl = reinterpret_cast<uint8_t *>(xl4);
    constexpr int BE = sem_traits<SEM>::kBlockElems, CPB = sem_traits<SEM>::kChunksPerBlock;
    const job_view jv = view_job(a, blockIdx.y);
    const mllm_packed W = jv.W;
    const float *__restrict__ x = a.x + jv.xj * a.x_job_stride;
    const float *__restrict__ xu = SILU ? a.x_up + jv.xj * a.x_job_stride : nullptr;
    float *__restrict__ out = jv.out;

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = lane / LPR, sl = lane % LPR;
    const int row0 = ((blockIdx.x * 4 + wave) * (64 / LPR) + grp) * R;
    const int nb = a.n_cols / BE;
    const int kused = nb * BE;
    const int B = a.B;
    const int KT = a.k_tile;
    const digit_geom dg = digit_geom_for(KT);

    float acc[R][BM];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < BM; b++) acc[r][b] = 0.0f;

    for (int k0 = 0; k0 < kused; k0 += KT) {
        const int kn = min(KT, kused - k0);
        if (k0) __syncthreads();
        x_stage<SILU> xst;
        stage_digits<SEM, SILU>(xst, false, xl, dg, x, xu, a.ldx, B, k0, kn, !a.silu_noclamp);
        __syncthreads();
        const int c_end = (k0 + kn) / BE * CPB;
        for (int c = k0 / BE * CPB + sl; c < c_end; c += LPR) {
            raw_chunk raw[R];
#pragma unroll
            for (int r = 0; r < R; r++) fetch<SEM>(W, nb, min(row0 + r, a.n_rows - 1), c, raw[r]);
            accumulate<SEM, BM, R>(raw, c, xl, dg, k0, B, acc);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int b = 0; b < BM; b++) {
            const float v = group_sum<LPR>(acc[r][b]);
            const int row = row0 + r;
            if (sl == 0 && row < a.n_rows && b < B)
                out[(long)b * a.ldo + row] = a.out_add ? a.out_add[(long)b * a.ldo + row] + v : v;
        }
    }
}

// Add chunk c of R rows to acc against the Q8_0 activation staged in LDS
// (per token: quant bytes padded 16 B per 256, then KT/32 scales, KT/32 min sums).
template <int SEM, int BM, int R>
MLLM_DEV void accumulate_q8(const raw_chunk (&raw)[R], int c, const float *xl, int tstride, int qstride, int KT,
                            int k0, int B, float (&acc)[R][BM])
{
    const uint8_t *lq = reinterpret_cast<const uint8_t *>(xl);
    // tile-relative 32-block indices of the chunk's two 16-byte activation pieces
    int ja, jb, qoa, qob;
    if constexpr (SEM == SEM_Q4_K_Q8) {
        ja = 8 * (c >> 2) + 2 * (c & 3) - k0 / 32; jb = ja + 1;
        qoa = 32 * ja; qob = 32 * jb;
    } else {
        ja = jb = c - k0 / 32;
        qoa = 32 * ja; qob = qoa + 16;
    }
#pragma unroll
    for (int b = 0; b < BM; b++) {
        if (b < B) {
            const uint8_t *tq = lq + b * tstride * 4;
            const float *tf = xl + b * tstride + qstride / 4;
            const uint4 qa = *reinterpret_cast<const uint4 *>(tq + qoa + ((qoa >> 8) << 4));
            const uint4 qb = *reinterpret_cast<const uint4 *>(tq + qob + ((qob >> 8) << 4));
            const float d8 = tf[ja];
            const float s4 = tf[KT / 32 + ja] + tf[KT / 32 + jb];
#pragma unroll
            for (int r = 0; r < R; r++) acc[r][b] += q8_dot<SEM>(raw[r], c, qa, qb, d8, s4);
        }
    }
}

// Copy the Q8_0 activation pack of tokens b < B, elements [k0, k0+kn), into LDS.
MLLM_DEV void stage_q8(float *xl, const mllm_xq &xq, long q_job, long b_job, int ldx, int B, int KT, int tstride,
                       int qstride, int k0, int kn)
{
    uint8_t *lq = reinterpret_cast<uint8_t *>(xl);
    const int n16 = kn >> 4, nbk = kn >> 5;
    for (int i = threadIdx.x; i < B * n16; i += blockDim.x) {
        const int b = i / n16, e = (i - b * n16) << 4;
        const uint4 v = gld<uint4>(xq.q + q_job + (long)b * (ldx / 32) * 32 + k0 + e);
        *reinterpret_cast<uint4 *>(lq + b * tstride * 4 + e + ((e >> 8) << 4)) = v;
    }
    for (int i = threadIdx.x; i < B * nbk; i += blockDim.x) {
        const int b = i / nbk, j = i - b * nbk;
        const long src = b_job + (long)b * (ldx / 32) + k0 / 32 + j;
        float *tb = xl + b * tstride + qstride / 4;
        tb[j] = gld<float>(xq.d + src);
        tb[KT / 32 + j] = gld<float>(xq.s4 + src);
    }
}

// Quantise the activation of tokens b < B, elements [k0, k0+kn), straight
// into the LDS form stage_q8 copies, with the arithmetic of
// quantize_row_q8_0 (QK:1406-1455, k_quantize_q8_0): per 32-block amax,
// d = amax/127 (1 when 0), q = rint(clamp(x * (1/d), +-127)), the scale kept
// as its fp16 rounding, and the Q4_K min-term sum over elements 0-7 and
// 16-23.  The activation is mllm_silu_mul(x, xu) when xu is given.  Four
// lanes share a block (8 elements each) and combine amax and the sum over
// DPP; a pass covers 256 quarter-blocks and its loads are issued first
// (q8f_load), the caller placing the weight prefetch between the two halves.
struct q8f_stage {
    float4 v[2], u[2];
    float4 r[2], w[2];   // residual and RMS weight (fused prologue)
};

MLLM_DEV void q8f_load(q8f_stage &st, const float *__restrict__ x, const float *__restrict__ xu, int ldx, int B,
                       int k0, int kn, int pass)
{
    const int nq = kn >> 3, i = threadIdx.x + 256 * pass;
    if (i >= B * nq) return;
    const int b = i / nq, e = (i - b * nq) << 3;
    const float *src = x + (long)b * ldx + k0 + e;
    const float *su = xu ? xu + (long)b * ldx + k0 + e : nullptr;
    if ((ldx & 3) == 0) {
        st.v[0] = gld<float4>(src);
        st.v[1] = gld<float4>(src + 4);
        if (su) { st.u[0] = gld<float4>(su); st.u[1] = gld<float4>(su + 4); }
    } else {
        st.v[0] = make_float4(gld<float>(src), gld<float>(src + 1), gld<float>(src + 2), gld<float>(src + 3));
        st.v[1] = make_float4(gld<float>(src + 4), gld<float>(src + 5), gld<float>(src + 6), gld<float>(src + 7));
        if (su) {
            st.u[0] = make_float4(gld<float>(su), gld<float>(su + 1), gld<float>(su + 2), gld<float>(su + 3));
            st.u[1] = make_float4(gld<float>(su + 4), gld<float>(su + 5), gld<float>(su + 6), gld<float>(su + 7));
        }
    }
}

// The fused prologue's residual / RMS-weight loads for q8f_load's elements.
MLLM_DEV void q8f_pro_load(q8f_stage &st, const mllm_gemv_args &a, int B, int kn, int pass)
{
    const int nq = kn >> 3, i = threadIdx.x + 256 * pass;
    if (i >= B * nq) return;
    const int b = i / nq, e = (i - b * nq) << 3;
    if (a.x_res) {
        const float *src = a.x_res + (long)b * a.ldx + e;
        st.r[0] = gld<float4>(src);
        st.r[1] = gld<float4>(src + 4);
    }
    if (a.rms_w) {
        st.w[0] = gld<float4>(a.rms_w + e);
        st.w[1] = gld<float4>(a.rms_w + e + 4);
    }
}

MLLM_DEV void q8f_store(const q8f_stage &st, bool silu, float *xl, int B, int KT, int tstride, int qstride, int kn,
                        int pass, bool clamp = true, const mllm_gemv_args *pa = nullptr, float *part = nullptr)
{
    const int nq = kn >> 3, i = threadIdx.x + 256 * pass;
    if (i >= B * nq) return;           // B * nq is a multiple of 4: a block's four lanes take the same path
    const int b = i / nq, qi = i - b * nq, e = qi << 3;
    float v[8] = {st.v[0].x, st.v[0].y, st.v[0].z, st.v[0].w, st.v[1].x, st.v[1].y, st.v[1].z, st.v[1].w};
    if (silu) {
        const float u[8] = {st.u[0].x, st.u[0].y, st.u[0].z, st.u[0].w, st.u[1].x, st.u[1].y, st.u[1].z, st.u[1].w};
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = mllm_silu_mul(v[k], u[k], clamp);
    } else if (pa) {
        prologue8(v, st.r, st.w, *pa, b, e, pa->res_out && blockIdx.x == 0, part + i);
    }
    // prescale (the fused RMS norm): the block's unrounded scale d and its min-term
    // quant count go to LDS; the caller turns them into fp16(s * d) once s is known
    const bool prescale = pa && pa->rms_w;
    float amax = 0.0f;
    bool nan = false;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float a = fabsf(v[k]);
        amax = (a > amax) ? a : amax;
        nan |= a != a;
    }
    if (__any(nan)) {
        // the reference's vmaxps order decides whether a NaN reaches amax: lane l
        // of the quad holds elements 8l..8l+7, so its v[j] is the reference's
        // lane j at step l; every lane folds the four steps from DPP broadcasts
        float m[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int a = __float_as_int(fabsf(v[j]));
            m[j] = mllm_maxps(0.0f, __int_as_float(__builtin_amdgcn_mov_dpp(a, 0x00, 0xF, 0xF, false)));
            m[j] = mllm_maxps(m[j], __int_as_float(__builtin_amdgcn_mov_dpp(a, 0x55, 0xF, 0xF, false)));
            m[j] = mllm_maxps(m[j], __int_as_float(__builtin_amdgcn_mov_dpp(a, 0xAA, 0xF, 0xF, false)));
            m[j] = mllm_maxps(m[j], __int_as_float(__builtin_amdgcn_mov_dpp(a, 0xFF, 0xF, 0xF, false)));
        }
        amax = mllm_q8_amax_tree(m);
    } else {
        amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0xB1, 0xF, 0xF, false)));
        amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0x4E, 0xF, 0xF, false)));
    }
    float d = amax / 127.0f;
    if (d == 0.0f) d = 1.0f;
    const float id = 1.0f / d;
    uint32_t w[2] = {0, 0};
    int sum = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        float p = v[k] * id;
        p = (p > -127.0f) ? p : -127.0f;
        p = (p < 127.0f) ? p : 127.0f;
        const int q = (int)rintf(p);
        sum += q;
        w[k >> 2] |= (uint32_t)(q & 0xFF) << (8 * (k & 3));
    }
    // min-term sum: quarters 0 and 2 of the block (elements 0-7, 16-23)
    int s4 = (qi & 1) ? 0 : sum;
    s4 += __builtin_amdgcn_mov_dpp(s4, 0xB1, 0xF, 0xF, false);
    s4 += __builtin_amdgcn_mov_dpp(s4, 0x4E, 0xF, 0xF, false);
    uint8_t *lq = reinterpret_cast<uint8_t *>(xl) + b * tstride * 4;
    *reinterpret_cast<uint2 *>(lq + e + ((e >> 8) << 4)) = make_uint2(w[0], w[1]);
    if ((qi & 3) == 0) {
        const float dd = h2f(__builtin_bit_cast(uint16_t, (_Float16)d));
        float *tf = xl + b * tstride + qstride / 4;
        tf[e >> 5] = prescale ? d : dd;
        tf[KT / 32 + (e >> 5)] = prescale ? (float)s4 : dd * (float)s4;
    }
}

// Q8_0-activation semantics: the quantised activation (int8 quants, decoded
// scales, Q4_K min-term sums) is staged in LDS the same way.
template <int SEM, int BM, int R, int LPR>
__global__ __launch_bounds__(256) void k_gemv_q8(mllm_gemv_args a)
{
    extern __shared__ float xl[];
    constexpr int BE = q8_traits<SEM>::kBlockElems, CPB = q8_traits<SEM>::kChunksPerBlock;
    const job_view jv = view_job(a, blockIdx.y);
    const mllm_packed W = jv.W;
    float *__restrict__ out = jv.out;
    const long q_job = jv.xj * a.x_job_stride;          // elements
    const long b_job = jv.xj * (a.x_job_stride / 32);   // 32-blocks

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = lane / LPR, sl = lane % LPR;
    const int row0 = ((blockIdx.x * 4 + wave) * (64 / LPR) + grp) * R;
    const int nb = a.n_cols / BE;
    const int kused = nb * BE;
    const int B = a.B;
    const int KT = a.k_tile;
    // LDS per token: KT quant bytes (+16 B per 256), then KT/32 scales and KT/32 min sums
    const int qstride = KT + (KT >> 4);
    const int tstride = qstride / 4 + 2 * (KT / 32);   // in floats

    float acc[R][BM];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < BM; b++) acc[r][b] = 0.0f;

    const float *xf = a.x + jv.xj * a.x_job_stride;
    const float *xuf = a.x_up ? a.x_up + jv.xj * a.x_job_stride : nullptr;
    for (int k0 = 0; k0 < kused; k0 += KT) {
        const int kn = min(KT, kused - k0);
        if (k0) __syncthreads();
        if (a.xq.q) {
            stage_q8(xl, a.xq, q_job, b_job, a.ldx, B, KT, tstride, qstride, k0, kn);
        } else {
            for (int pass = 0; pass * 256 < B * (kn >> 3); pass++) {
                q8f_stage qs;
                q8f_load(qs, xf, xuf, a.ldx, B, k0, kn, pass);
                q8f_store(qs, xuf != nullptr, xl, B, KT, tstride, qstride, kn, pass, !a.silu_noclamp);
            }
        }
        __syncthreads();
        const int c_end = (k0 + kn) / BE * CPB;
        for (int c = k0 / BE * CPB + sl; c < c_end; c += LPR) {
            raw_chunk raw[R];
#pragma unroll
            for (int r = 0; r < R; r++) q8_fetch<SEM>(W, nb, min(row0 + r, a.n_rows - 1), c, raw[r]);
            accumulate_q8<SEM, BM, R>(raw, c, xl, tstride, qstride, KT, k0, B, acc);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int b = 0; b < BM; b++) {
            const float v = group_sum<LPR>(acc[r][b]);
            const int row = row0 + r;
            if (sl == 0 && row < a.n_rows && b < B)
                out[(long)b * a.ldo + row] = a.out_add ? a.out_add[(long)b * a.ldo + row] + v : v;
        }
    }
}

// Persistent variant used whenever all of x fits in LDS: a workgroup stages
// x once, then its waves walk row groups (stride = all waves of the grid),
// prefetching the next step's weight chunks while the current step computes,
// so every lane keeps two rounds of 16-byte loads in flight.  A step is one
// pass of the lane group over LPR chunks of its R rows; the last step of a
// row group reduces and writes it.  Q8 selects the Q8_0-activation form.
template <int SEM, bool Q8> struct gemv_geom {
    static constexpr int BE = Q8 ? q8_traits<SEM>::kBlockElems : sem_traits<SEM>::kBlockElems;
    static constexpr int CPB = Q8 ? q8_traits<SEM>::kChunksPerBlock : sem_traits<SEM>::kChunksPerBlock;
};

// FUSE bits of the persistent kernel (mllm_gemv_args): kFusePro = the
// residual / RMS-norm prologue; kFusePair = paired rows with the SiLU product
// in the epilogue: adjacent lane groups compute a gate row (even group) and
// its up row (odd group: row o + n_rows of the same matrix, or row o of
// table2's matrix in a job launch -- the gate/up pair of an MoE expert), and
// the even group writes silu(gate) * up after one cross-lane exchange.
constexpr int kFusePro = 1, kFusePair = 2;

// Waves per workgroup of the persistent kernel: eight on the ring path (64
// lanes per row, batch 1, no fusion), four elsewhere.  The ring path serves
// long rows, whose whole-K staging holds a workgroup to up to ~60 KB of LDS
// (two workgroups per CU): eight waves per workgroup keep four waves per SIMD
// in flight instead of two, sharing one staged copy of the activation.
template <int SEM, bool Q8, int BM, int R, int LPR, int FUSE>
constexpr int gemv_p_waves()
{
    return (R == 1 && BM == 1 && LPR == 64 && FUSE == 0 && !Q8 && kFetchLin<SEM>) ? 8 : 4;
}

template <int SEM, bool Q8, int BM, int R, int LPR, bool SILU, int FUSE>
__global__ __launch_bounds__((64 * gemv_p_waves<SEM, Q8, BM, R, LPR, FUSE>())) void k_gemv_p(mllm_gemv_args a)
{
    static_assert(!(Q8 && SILU), "the SiLU product of Q8_0 activations is formed by the quantiser");
    static_assert(!(SILU && FUSE), "the SiLU staging and the fusions are exclusive");
    constexpr bool PRO = (FUSE & kFusePro) != 0, PAIR = (FUSE & kFusePair) != 0;
    static_assert(!PAIR || (R == 1 && LPR <= 32), "paired rows: one row per lane group, two groups per pair");
    extern __shared__ float xl[];
    constexpr int BE = gemv_geom<SEM, Q8>::BE, CPB = gemv_geom<SEM, Q8>::CPB;
    constexpr int GPW = 64 / LPR;                       // lane groups per wave
    constexpr int OPW = PAIR ? GPW / 2 : GPW * R;       // output rows per wave and step
    constexpr int NW = gemv_p_waves<SEM, Q8, BM, R, LPR, FUSE>(), NT = 64 * NW;
    static_assert(NT == 256 || (!PRO && !Q8), "the prologue and Q8_0 staging take 256 threads");
    const job_view jv = view_job(a, blockIdx.y);
    const mllm_packed W = jv.W;
    // the "up" rows of a pair: table2's matrix of the job's expert, else the same matrix n_rows further
    mllm_packed W2 = W;
    int up_off = a.n_rows;
    if constexpr (PAIR) {
        if (a.table2) {
            typedef const __attribute__((address_space(4))) int cint;
            typedef const __attribute__((address_space(4))) uint64_t cu64;
            const int e = a.idx ? *(cint *)(a.idx + blockIdx.y) : (int)blockIdx.y;
            cu64 *tp = (cu64 *)(a.table2 + (e < 0 ? 0 : e));
#pragma unroll
            for (int i = 0; i < MLLM_MAX_PLANES; i++) W2.p[i] = (const uint8_t *)tp[i];
            up_off = 0;
        }
    }
    float *__restrict__ out = jv.out;

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = lane / LPR, sl = lane % LPR;
    const int nb = a.n_cols / BE, kused = nb * BE, nch = nb * CPB;
    const int iters = (nch + LPR - 1) / LPR;
    if (iters == 0) return;   // no whole block per row: the launcher writes zeros instead of launching this
    const int n_out = a.n_rows;
    const int nrg = (n_out + OPW - 1) / OPW;
    const int wstride = gridDim.x * NW;
    const int rg0 = blockIdx.x * NW + wave;
    const int B = a.B;
    // LDS geometry (whole K staged): activation digits, or the Q8_0 pack
    const int KT = (kused + 255) / 256 * 256;
    const digit_geom dg = digit_geom_for(KT);
    const int qstride = KT + (KT >> 4), tstride = qstride / 4 + 2 * (KT / 32);

    // A step is (row group rg, chunk pass it); the next step advances it, then rg.
    // Output row of lane group grp, row r: o0 + r; with PAIR, o0 + grp / 2 of the gate (even) or up (odd) rows.
    auto out_row = [&](int rg, int r) __attribute__((always_inline)) {
        return PAIR ? rg * OPW + (grp >> 1) : rg * OPW + grp * R + r;
    };
    // the ring path's formats with a linear chunk layout: buffer-resource loads (fetch_lin)
    constexpr bool LIN = R == 1 && BM == 1 && LPR == 64 && FUSE == 0 && !Q8 && kFetchLin<SEM>;
    lin_planes lp{};
    if constexpr (LIN) lp = lin_make<SEM>(W, (uint32_t)n_out * (uint32_t)nb);
    auto fetch_step = [&](int rg, int it, raw_chunk (&buf)[R]) __attribute__((always_inline)) {
        if constexpr (LIN) {
            const uint32_t ublk = (uint32_t)min(out_row(rg, 0), n_out - 1) * (uint32_t)nb + (uint32_t)(it * (64 / CPB));
            fetch_lin<SEM>(lp, ublk, sl, buf[0]);
            return;
        }
        const int c = min(it * LPR + sl, nch - 1);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int o = min(out_row(rg, r), n_out - 1);
            if constexpr (PAIR) {
                const bool up = grp & 1;
                if constexpr (Q8) q8_fetch<SEM>(up ? W2 : W, nb, up ? o + up_off : o, c, buf[r]);
                else fetch<SEM>(up ? W2 : W, nb, up ? o + up_off : o, c, buf[r]);
            } else {
                if constexpr (Q8) q8_fetch<SEM>(W, nb, o, c, buf[r]);
                else fetch<SEM>(W, nb, o, c, buf[r]);
            }
        }
    };
    float acc[R][BM];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < BM; b++) acc[r][b] = 0.0f;
    float scale[BM];   // RMSNorm scale per token (prologue)
#pragma unroll
    for (int b = 0; b < BM; b++) scale[b] = 1.0f;
    auto run_step = [&](int rg, int it, const raw_chunk (&buf)[R]) __attribute__((always_inline)) {
        // a lane past the row's last chunk recomputes the last one and discards it
        const int c = min(it * LPR + sl, nch - 1);
        const bool live = it * LPR + sl < nch;
        float part[R][BM];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int b = 0; b < BM; b++) part[r][b] = 0.0f;
        if constexpr (Q8) {
            accumulate_q8<SEM, BM, R>(buf, c, xl, tstride, qstride, KT, 0, B, part);
        } else if constexpr (BM == 1 && LPR % CPB == 0) {
            // a lane's chunk within its block is the same at every step (sl % CPB) and
            // its block advances by LPR / CPB: the digit addresses and the scale
            // selection follow from the lane and the step (a lane past the row's
            // end takes the last block and is discarded)
            const int blk = min(it * (LPR / CPB) + sl / CPB, nb - 1);
            accumulate_at<SEM, R, true, true>(buf, blk, sl % CPB, reinterpret_cast<const uint8_t *>(xl), dg, 0, part);
        } else {
            accumulate<SEM, BM, R>(buf, c, reinterpret_cast<const uint8_t *>(xl), dg, 0, B, part);
        }
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int b = 0; b < BM; b++) acc[r][b] += live ? part[r][b] : 0.0f;
        if (it == iters - 1) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int o = out_row(rg, r);
#pragma unroll
                for (int b = 0; b < BM; b++) {
                    float v = group_sum<LPR>(acc[r][b]);
                    acc[r][b] = 0.0f;
                    if constexpr (PRO && !Q8) v = a.rms_div ? v / scale[b] : v * scale[b];
                    bool writes = sl == 0 && o < n_out && b < B;
                    if constexpr (PAIR) {
                        // the odd group's up value to the even group's lanes
                        const float u = __shfl_xor(v, LPR, 64);
                        v = mllm_silu_mul(v, u, !a.silu_noclamp);
                        writes = writes && (grp & 1) == 0;
                    }
                    if (writes) {
                        const long oi = (long)b * a.ldo + o;
                        out[oi] = a.out_add ? a.out_add[oi] + v : v;
                    }
                }
            }
        }
    };
    auto advance = [&](int &rg, int &it) __attribute__((always_inline)) {
        if (++it == iters) { it = 0; rg += wstride; }
    };

    // Every prefetch is issued unconditionally (clamped to the last row group):
    // with the same loads outstanding on every path, the compiler waits only
    // for the oldest slot instead of draining all loads.  A ring of NR steps:
    // slot u holds the chunks of step s + u, so NR - 1 steps of weight loads
    // stay in flight while a step computes (one in flight, 32 bytes a lane,
    // leaves a long matrix bound by memory latency, not bandwidth)
    // (the ring on long rows only -- 64 lanes per row, batch 1, no fusion: on the short
    // matrices of a decode chain its prologue and tail cost more than it hides)
    constexpr int NR = (R == 1 && BM == 1 && LPR == 64 && FUSE == 0) ? 4 : 2;
    raw_chunk ring[NR][R];
    int rg = rg0, it = 0;
    int rgf = rg0, itf = 0;   // the fetch cursor, NR - 1 steps ahead once the prologue has run
    auto prefetch = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NR - 1; j++) {
            fetch_step(min(rgf, nrg - 1), itf, ring[j]);
            advance(rgf, itf);
        }
    };
    // prologue: sum(v^2) of each staged 8-element piece, past the staged activation
    float *part = xl + a.pro_lds / 4;
    if constexpr (Q8) {
        if (a.xq.q) {
            prefetch();
            stage_q8(xl, a.xq, jv.xj * a.x_job_stride, jv.xj * (a.x_job_stride / 32), a.ldx, B, KT, tstride, qstride,
                     0, kused);
        } else {
            // quantise in the workgroup: activation loads first, then the weights
            const float *xf = a.x + jv.xj * a.x_job_stride;
            const float *xuf = a.x_up ? a.x_up + jv.xj * a.x_job_stride : nullptr;
            q8f_stage qs;
            q8f_load(qs, xf, xuf, a.ldx, B, 0, kused, 0);
            if constexpr (PRO) q8f_pro_load(qs, a, B, kused, 0);
            prefetch();
            for (int pass = 0;;) {
                q8f_store(qs, xuf != nullptr, xl, B, KT, tstride, qstride, kused, pass, !a.silu_noclamp,
                          PRO ? &a : nullptr, part);
                if (++pass * 256 >= B * (kused >> 3)) break;
                q8f_load(qs, xf, xuf, a.ldx, B, 0, kused, pass);
                if constexpr (PRO) q8f_pro_load(qs, a, B, kused, pass);
            }
        }
    } else {
        // activation loads first, then the weights; the digits are computed while the weights are in flight
        x_stage<SILU> xst;
        const float *xj = a.x + jv.xj * a.x_job_stride;
        const float *xuj = SILU ? a.x_up + jv.xj * a.x_job_stride : nullptr;
        stage_load<SILU, NT>(xst, xj, xuj, a.ldx, B, 0, kused, 0);
        if constexpr (PRO) {
            pro_regs pr;
            pro_load(pr, a, B, kused, 0);
            prefetch();
            // pass 0 out of the pass loop (see stage_digits)
            const int passes = (B * (kused >> 3) + 256 * kStageSlots - 1) / (256 * kStageSlots);
            bool bad = stage_store<SEM, false, true>(xst, reinterpret_cast<uint8_t *>(xl), dg, B, kused, 0, true, &pr,
                                                     &a, part);
            for (int pass = 1; pass < passes; pass++) {
                stage_load<false>(xst, xj, nullptr, a.ldx, B, 0, kused, pass);
                pro_load(pr, a, B, kused, pass);
                bad |= stage_store<SEM, false, true>(xst, reinterpret_cast<uint8_t *>(xl), dg, B, kused, pass, true,
                                                     &pr, &a, part);
            }
            // with the RMS norm a non-finite value makes every output NaN, as the
            // reference's normalised vector holds inf * 0 = NaN; without it the
            // residual sum is staged again keeping its infinities
            if (!a.rms_w && __any(bad))
                stage_fix<SEM>(reinterpret_cast<uint8_t *>(xl), dg, xj, nullptr, a.x_res, a.ldx, B, 0, kused, true);
        } else {
            prefetch();
            stage_digits<SEM, SILU, NT>(xst, true, reinterpret_cast<uint8_t *>(xl), dg, xj, xuj, a.ldx, B, 0, kused,
                                    !a.silu_noclamp);
        }
    }
    __syncthreads();
    if constexpr (PRO) {
        if (a.rms_w) {
            // each wave sums every token's pieces (deterministic order) for its outputs' scale
            const int nh = kused >> 3;
#pragma unroll
            for (int b = 0; b < BM; b++) {
                if (b >= B) break;
                float t = 0.0f;
                for (int h = lane; h < nh; h += 64) t += part[b * nh + h];
                t = group_sum<64>(t);
                const float r = sqrtf(t / (float)a.n_cols + a.rms_eps);
                scale[b] = a.rms_div ? r : 1.0f / r;
            }
            if constexpr (Q8) {
                // Q8_0 activations: the quants of v * w equal those of the normalised
                // activation (a common factor per token); its block scale is
                // fp16(d * s), the scale quantize_row_q8_0 stores for the normalised
                // values (QK:1406-1455) -- the dots (Q4_K x Q8_0 drops that scale from
                // one of its terms, QK:1714-1723) then see the normalised activation
                const int nbk = KT / 32;
                for (int j = threadIdx.x; j < B * nbk; j += 256) {
                    const int b = j / nbk, jj = j - b * nbk;
                    float sb = scale[0];
#pragma unroll
                    for (int bb = 1; bb < BM; bb++) sb = b == bb ? scale[bb] : sb;
                    float *tf = xl + b * tstride + qstride / 4;
                    const float d = a.rms_div ? tf[jj] / sb : tf[jj] * sb;
                    const float dd = h2f(__builtin_bit_cast(uint16_t, (_Float16)d));
                    tf[jj] = dd;
                    tf[nbk + jj] = dd * tf[nbk + jj];
                }
                __syncthreads();
            }
        }
    }
    if (rg >= nrg) return;
    if constexpr (NR == 2) {
        // two buffers, alternating
        for (;;) {
            int rg1 = rg, it1 = it;
            advance(rg1, it1);
            fetch_step(min(rg1, nrg - 1), it1, ring[1]);
            run_step(rg, it, ring[0]);
            if (rg1 >= nrg) break;
            int rg2 = rg1, it2 = it1;
            advance(rg2, it2);
            fetch_step(min(rg2, nrg - 1), it2, ring[0]);
            run_step(rg1, it1, ring[1]);
            if (rg2 >= nrg) break;
            rg = rg2; it = it2;
        }
        return;
    }
    // the wave's steps: its row groups rg0, rg0 + wstride, ... times iters; whole units of NR
    // steps in the loop (one exit, so the ring stays in its registers), the rest after it,
    // already in the ring
    const int nsteps = ((nrg - 1 - rg0) / wstride + 1) * iters;
    int s = 0;
    for (; s + NR <= nsteps; s += NR) {
#pragma unroll
        for (int u = 0; u < NR; u++) {
            fetch_step(min(rgf, nrg - 1), itf, ring[(u + NR - 1) % NR]);
            advance(rgf, itf);
            run_step(rg, it, ring[u]);
            advance(rg, it);
        }
    }
#pragma unroll
    for (int u = 0; u < NR - 1; u++) {
        if (s + u >= nsteps) break;
        run_step(rg, it, ring[u]);
        advance(rg, it);
    }
}

// f32_matmul_omp (QK:884-913): plain fp32 rows, any n_cols.
template <int BM>
__global__ __launch_bounds__(256) void k_gemv_f32(mllm_gemv_args a)
{
    const job_view jv = view_job(a, blockIdx.y);
    const float *Wf = reinterpret_cast<const float *>(jv.W.p[0]);
    const float *x = a.x + jv.xj * a.x_job_stride;
    float *out = jv.out;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row = blockIdx.x * 4 + wave;
    if (row >= a.n_rows) return;
    const float *w = Wf + (long)row * a.n_cols;
    float acc[BM];
#pragma unroll
    for (int b = 0; b < BM; b++) acc[b] = 0.f;
    for (int i = lane; i < a.n_cols; i += 64) {
        float wv = w[i];
#pragma unroll
        for (int b = 0; b < BM; b++)
            if (b < a.B) acc[b] = fmaf(wv, x[(long)b * a.ldx + i], acc[b]);
    }
#pragma unroll
    for (int b = 0; b < BM; b++) {
        float v = group_sum<64>(acc[b]);
        if (lane == 0 && b < a.B) out[(long)b * a.ldo + row] = a.out_add ? a.out_add[(long)b * a.ldo + row] + v : v;
    }
}

// Dequantise rows to fp32 the way the reference's *_dequantize_row functions
// round: w = fl(s*q) + o, two roundings (QK:762-878).
template <int SEM>
__global__ __launch_bounds__(256) void k_dequant(mllm_packed W, int n_rows, int n_cols, float *__restrict__ out)
{
    constexpr int CPB = sem_traits<SEM>::kChunksPerBlock;
    constexpr int bias = sem_traits<SEM>::kBias;
    const int nb = n_cols / sem_traits<SEM>::kBlockElems, nch = nb * CPB;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)n_rows * nch) return;
    const int row = (int)(i / nch), c = (int)(i % nch);
    raw_chunk raw;
    fetch<SEM>(W, nb, row, c, raw);
    chunk_codes k;
    codes<SEM>(raw, c, k);
    float *o = out + (long)row * n_cols;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float q0 = (float)((int)((k.U[j] >> (8 * t)) & 0xFF) - bias);
            const float q1 = (float)((int)((k.U[4 + j] >> (8 * t)) & 0xFF) - bias);
            o[k.x0 + code_pos<SEM>(j, t)] = __fadd_rn(__fmul_rn(k.s0, q0), k.o0);
            o[k.x1 + code_pos<SEM>(j, t)] = __fadd_rn(__fmul_rn(k.s1, q1), k.o1);
        }
}

template <int SEM>
hipError_t launch_dequant(const mllm_packed &W, int n_rows, int n_cols, float *out, hipStream_t st)
{
    const long n = (long)n_rows * (n_cols / sem_traits<SEM>::kBlockElems) * sem_traits<SEM>::kChunksPerBlock;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_dequant<SEM>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, W, n_rows, n_cols, out);
    return hipGetLastError();
}

inline int device_cus()
{
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return cus;
}

constexpr size_t kPersistentLds = 72 * 1024;

template <int SEM, bool Q8, int BM, int R, int LPR, bool SILU>
void launch_lpr(bool persistent, dim3 grid, size_t lds, const mllm_gemv_args &a, hipStream_t st)
{
    if (persistent)
        hipLaunchKernelGGL((k_gemv_p<SEM, Q8, BM, R, LPR, SILU, 0>), grid, dim3(64 * gemv_p_waves<SEM, Q8, BM, R, LPR, 0>()),
                           lds, st, a);
    else if constexpr (Q8) hipLaunchKernelGGL((k_gemv_q8<SEM, BM, R, LPR>), grid, dim3(256), lds, st, a);
    else hipLaunchKernelGGL((k_gemv<SEM, BM, R, LPR, SILU>), grid, dim3(256), lds, st, a);
}

// The SiLU-product form exists for fp32-activation semantics at B == 1 only
// (the caller checks).
template <int SEM, bool Q8, int BM, int R>
void launch_shape(bool persistent, int lpr, dim3 grid, size_t lds, const mllm_gemv_args &a, hipStream_t st)
{
    if constexpr (!Q8 && BM == 1) {
        if (a.x_up) {
            if (lpr == 64) launch_lpr<SEM, Q8, BM, R, 64, true>(persistent, grid, lds, a, st);
            else if (lpr == 32) launch_lpr<SEM, Q8, BM, R, 32, true>(persistent, grid, lds, a, st);
            else launch_lpr<SEM, Q8, BM, R, 16, true>(persistent, grid, lds, a, st);
            return;
        }
    }
    if (lpr == 64) launch_lpr<SEM, Q8, BM, R, 64, false>(persistent, grid, lds, a, st);
    else if (lpr == 32) launch_lpr<SEM, Q8, BM, R, 32, false>(persistent, grid, lds, a, st);
    else launch_lpr<SEM, Q8, BM, R, 16, false>(persistent, grid, lds, a, st);
}

// Lanes per row of a launch: at batch 1, 16 lanes per row up to ~1.8 KB of
// row bytes and 32 up to ~5 KB, measured fastest on MI355X across the
// TinyLlama/GPT-OSS shapes, widened on short matrices until the launch has
// about two workgroups per CU; larger batches reuse each chunk's decode over
// R rows x B tokens.  HR = output rows per lane group.
template <int SEM, bool Q8, int BM>
int pick_lpr(const mllm_gemv_args &a, int n_jobs, int HR)
{
    constexpr int BE = gemv_geom<SEM, Q8>::BE, CPB = gemv_geom<SEM, Q8>::CPB;
    const int kused = a.n_cols / BE * BE;
    const int nch = kused / BE * CPB;
    auto waste = [&](int lpr) { int it = (nch + lpr - 1) / lpr; return (double)(it * lpr - nch) / (it * lpr); };
    int lpr = 64;
    auto wgs_at = [&](int l) { const int rpw = 4 * (64 / l) * HR; return (long)(a.n_rows + rpw - 1) / rpw * n_jobs; };
    if (BM == 1) {
        const long row_bytes = (long)kused / 32 * sem_traits<SEM>::kBytesPer32;
        lpr = row_bytes <= 1800 ? 16 : row_bytes <= 5000 ? 32 : 64;
        // short matrices: wider lane groups (fewer rows per workgroup) until
        // the launch has about two workgroups per CU
        while (lpr < 64 && wgs_at(lpr) < 2L * device_cus()) lpr *= 2;
        // 64 lanes per row read through 32-bit buffer offsets (fetch_lin): matrices
        // of 4 GiB and more take 32
        if (lpr == 64 && (long)a.n_rows * row_bytes >= (1l << 32)) lpr = 32;
    } else {
        // lanes per row: enough chunks per lane to keep every lane busy on short
        // rows; 32 where that still leaves two workgroups per CU (fewer lane-group
        // reductions per row: measured faster on the 11264-row gate+up, slower
        // on 2048-2560 rows)
        if (nch < 64 || waste(64) > waste(32) + 0.05 || wgs_at(32) >= 2L * device_cus()) lpr = 32;
        if (nch < 32 || (lpr == 32 && waste(32) > waste(16) + 0.05)) lpr = 16;
    }
    return lpr;
}

template <int SEM, int BM>
void launch_sem(mllm_gemv_args a, int n_jobs, hipStream_t st)
{
    constexpr bool Q8 = mllm_sem_uses_q8(SEM);
    constexpr int BE = gemv_geom<SEM, Q8>::BE;
    const int kused = a.n_cols / BE * BE;
    constexpr int R = (BM == 1) ? 1 : (BM == 2) ? 4 : 2;
    const int lpr = pick_lpr<SEM, Q8, BM>(a, n_jobs, R);
    const int rows_per_wg = 4 * (64 / lpr) * R;
    const int wg_needed = (a.n_rows + rows_per_wg - 1) / rows_per_wg;

    // whole-K staging for the persistent kernel (+ the prologue's reduction
    // scratch and scales past it)
    const int ktp = (kused + 255) / 256 * 256;
    const size_t lds_p = Q8 ? (size_t)BM * (ktp + ktp / 16 + 8 * (ktp / 32)) : (size_t)BM * digit_geom_for(ktp).tstride;
    if (lds_p <= kPersistentLds) {
        const int nw = lpr == 64 ? gemv_p_waves<SEM, Q8, BM, R, 64, 0>() : 4;
        const int rows_p = nw * (64 / lpr) * R;
        const int per_cu = nw == 8 ? 2 : lds_p <= 40 * 1024 ? 3 : 2;
        const int wgs = std::max(1, std::min((a.n_rows + rows_p - 1) / rows_p, device_cus() * per_cu / std::max(1, n_jobs)));
        launch_shape<SEM, Q8, BM, R>(true, lpr, dim3(wgs, n_jobs), lds_p, a, st);
        return;
    }
    // K tiled through 48 KB of LDS
    // digits: 3.6875 bytes per element and token (3 planes + 1/16 padding each + 8-byte record per 16)
    int kt = Q8 ? (kLdsFloats * 4 * 4 / (BM * 5 * 4 + BM)) / 256 * 256 : (kLdsFloats * 4 * 16 / (BM * 59)) / 256 * 256;
    if (kt > kused) kt = (kused + 255) / 256 * 256;
    if (kt < 256) kt = 256;
    a.k_tile = kt;
    const size_t lds = Q8 ? (size_t)BM * (kt + kt / 16 + 8 * (kt / 32)) : (size_t)BM * digit_geom_for(kt).tstride;
    launch_shape<SEM, Q8, BM, R>(false, lpr, dim3(wg_needed, n_jobs), lds, a, st);
}

// LDS bytes the persistent kernel stages for whole K at batch BM (the
// launcher takes it when they fit kPersistentLds), with the prologue scratch.
inline size_t persistent_lds(bool q8, int block_elems, int n_cols, int BM, bool prologue)
{
    const int kused = n_cols / block_elems * block_elems;
    const int ktp = (kused + 255) / 256 * 256;
    size_t l = q8 ? (size_t)BM * (ktp + ktp / 16 + 8 * (ktp / 32)) : (size_t)BM * digit_geom_for(ktp).tstride;
    if (prologue) l = (l + 15) / 16 * 16 + (size_t)BM * (ktp / 8) * 4;
    return l;
}

// The fused persistent kernel (prologue and / or paired rows; the caller has
// checked that the whole activation fits the kernel's LDS).  Paired rows run
// at batch 1 only; the fused launches take 32 or 64 lanes per row at B > 1.
template <int SEM, bool Q8, int BM, int R, int FUSE>
void launch_fused_lpr(int lpr, dim3 grid, size_t lds, const mllm_gemv_args &a, hipStream_t st)
{
    constexpr bool PAIR = (FUSE & kFusePair) != 0;
    static_assert(FUSE != 0, "fused launches run four-wave workgroups");
    if constexpr (!PAIR) {
        if (lpr == 64) { hipLaunchKernelGGL((k_gemv_p<SEM, Q8, BM, R, 64, false, FUSE>), grid, dim3(256), lds, st, a); return; }
    }
    if (lpr >= 32 || BM > 1) hipLaunchKernelGGL((k_gemv_p<SEM, Q8, BM, R, 32, false, FUSE>), grid, dim3(256), lds, st, a);
    else if constexpr (BM == 1) hipLaunchKernelGGL((k_gemv_p<SEM, Q8, BM, R, 16, false, FUSE>), grid, dim3(256), lds, st, a);
}

template <int SEM, int BM>
hipError_t launch_fused(mllm_gemv_args a, int n_jobs, hipStream_t st)
{
    constexpr bool Q8 = mllm_sem_uses_q8(SEM);
    const bool pro = mllm_has_prologue(a), pair = a.silu_pair != 0;
    if (pair && BM != 1) return hipErrorInvalidValue;
    constexpr int BE = gemv_geom<SEM, Q8>::BE;
    const int kused = a.n_cols / BE * BE;
    const int ktp = (kused + 255) / 256 * 256;
    size_t lds = Q8 ? (size_t)BM * (ktp + ktp / 16 + 8 * (ktp / 32)) : (size_t)BM * digit_geom_for(ktp).tstride;
    if (pro) {
        lds = (lds + 15) / 16 * 16;
        a.pro_lds = (int)lds;
        lds += (size_t)BM * (ktp / 8) * 4;   // one sum of squares per staged 8-element piece
    }
    if (lds > kPersistentLds) return hipErrorInvalidValue;
    constexpr int R = (BM == 1) ? 1 : (BM == 2) ? 4 : 2;
    int lpr;
    if (pair) {
        // a pair takes two lane groups (its gate and its up row): size the launch over 2 n_rows rows
        mllm_gemv_args rows2 = a;
        rows2.n_rows = 2 * a.n_rows;
        lpr = std::min(32, pick_lpr<SEM, Q8, BM>(rows2, n_jobs, 1));
    } else {
        lpr = pick_lpr<SEM, Q8, BM>(a, n_jobs, R);
    }
    if (BM > 1 && lpr < 32) lpr = 32;
    const int outs_per_wg = pair ? 4 * (64 / lpr) / 2 : 4 * (64 / lpr) * R;
    const int wg_needed = (a.n_rows + outs_per_wg - 1) / outs_per_wg;
    const int per_cu = lds <= 40 * 1024 ? 3 : 2;
    const dim3 grid(std::max(1, std::min(wg_needed, device_cus() * per_cu / std::max(1, n_jobs))), n_jobs);
    if constexpr (BM == 1) {
        if (pair && pro) launch_fused_lpr<SEM, Q8, 1, 1, kFusePro | kFusePair>(lpr, grid, lds, a, st);
        else if (pair) launch_fused_lpr<SEM, Q8, 1, 1, kFusePair>(lpr, grid, lds, a, st);
        else launch_fused_lpr<SEM, Q8, 1, 1, kFusePro>(lpr, grid, lds, a, st);
    } else {
        launch_fused_lpr<SEM, Q8, BM, R, kFusePro>(lpr, grid, lds, a, st);
    }
    return hipGetLastError();
}

template <int SEM>
hipError_t launch_fused_any_b(const mllm_gemv_args &a, int n_jobs, hipStream_t st)
{
    if (a.B == 1) return launch_fused<SEM, 1>(a, n_jobs, st);
    if (a.B == 2) return launch_fused<SEM, 2>(a, n_jobs, st);
    if (a.B <= 4) return launch_fused<SEM, 4>(a, n_jobs, st);
    return launch_fused<SEM, 8>(a, n_jobs, st);
}

// Launch the GEMV of one semantic for B = a.B (1..8).
template <int SEM>
void launch_sem_any_b(const mllm_gemv_args &a, int n_jobs, hipStream_t st)
{
    if (a.B == 1) launch_sem<SEM, 1>(a, n_jobs, st);
    else if (a.B == 2) launch_sem<SEM, 2>(a, n_jobs, st);
    else if (a.B <= 4) launch_sem<SEM, 4>(a, n_jobs, st);
    else launch_sem<SEM, 8>(a, n_jobs, st);
}

// Per-semantic entry points, defined in gemv_*.hip (fused forms in gemv_f*.hip).
template <int SEM> void gemv_sem(const mllm_gemv_args &a, int n_jobs, hipStream_t st);
template <int SEM> hipError_t gemv_fused_sem(const mllm_gemv_args &a, int n_jobs, hipStream_t st);
template <int SEM> hipError_t dequant_sem(const mllm_packed &W, int n_rows, int n_cols, float *out, hipStream_t st);

#define MLLM_GEMV_INSTANTIATE(SEM)                                                                   \
    template <> void gemv_sem<SEM>(const mllm_gemv_args &a, int n_jobs, hipStream_t st)              \
    {                                                                                                \
        launch_sem_any_b<SEM>(a, n_jobs, st);                                                        \
    }
#define MLLM_GEMV_FUSED_INSTANTIATE(SEM)                                                             \
    template <> hipError_t gemv_fused_sem<SEM>(const mllm_gemv_args &a, int n_jobs, hipStream_t st)  \
    {                                                                                                \
        return launch_fused_any_b<SEM>(a, n_jobs, st);                                               \
    }
#define MLLM_DEQUANT_INSTANTIATE(SEM)                                                                \
    template <> hipError_t dequant_sem<SEM>(const mllm_packed &W, int n_rows, int n_cols, float *out, \
                                            hipStream_t st)                                          \
    {                                                                                                \
        return launch_dequant<SEM>(W, n_rows, n_cols, out, st);                                      \
    }

} // namespace mllm_gemv
