/* oracle.c — CPU restatement of a730/MojoLlama's quantised-matmul + MoE path.
 *
 * TEST INFRASTRUCTURE ONLY: see oracle.h.  Plain scalar C written from the
 * reference's arithmetic (file:line cited per function); it shares no code
 * with the reference.  Built with -ffp-contract=off so every fused
 * multiply-add below is an explicit fmaf().
 *
 * Reference files:
 *   CE = src/mojollama/kernels/cengine_batch_instr.c
 *   QK = src/mojollama/kernels/quant_kernels_omp.c
 *   GO = src/mojollama/kernels/gptoss_batch_forward.c
 */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- fp16 */

/* IEEE binary16 -> binary32, exact (the reference uses F16C _cvtsh_ss, CE:54, QK:39). */
float orc_f16_to_f32(uint16_t h)
{
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 0x3ffu, bits;
    if (e == 0) {
        float v = (float)m * (1.0f / 16777216.0f);      /* m * 2^-24, exact */
        return s ? -v : v;
    }
    if (e == 31) bits = s | 0x7f800000u | (m << 13);
    else         bits = s | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16 with round-to-nearest-even (the reference's
 * _mm_cvtps_ph(.., _MM_FROUND_TO_NEAREST_INT), QK:1435-1439). */
uint16_t orc_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7e00u;              /* NaN */
    if (ax >= 0x477ff000u) return sign | 0x7c00u;             /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                                   /* < 2^-14: subnormal */
        float a;
        memcpy(&a, &ax, 4);
        return sign | (uint16_t)nearbyintf(a * 16777216.0f);  /* units of 2^-24, RNE */
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return sign | (uint16_t)h;
}

static inline float ld_f16(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* get_scale_min_k4 (QK:62-71) / k4_scale (CE:56-60): 6-bit (scale, min) pair j. */
static inline void k4_pair(int j, const uint8_t *q, int *sc, int *m)
{
    if (j < 4) { *sc = q[j] & 63; *m = q[j + 4] & 63; }
    else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m  = (q[j + 4] >> 4)  | ((q[j]     >> 6) << 4);
    }
}

/* E8M0 byte -> float with bits (E << 23) (QK:542, CE:449). */
static inline float e8m0(uint8_t e)
{
    uint32_t b = (uint32_t)e << 23;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

static inline int sext4(int n) { return n >= 8 ? n - 16 : n; }

/* ------------------------------------------------------- block geometry */

int orc_block_elems(int sem)
{
    switch (sem) {
    case ORC_F32: return 1;
    case ORC_Q4_K_GGML: case ORC_Q4_K_Q8: case ORC_Q5_K_GGML: case ORC_Q5_K_CE:
    case ORC_Q6_K_GGML: case ORC_Q6_K_LOWNIB: case ORC_Q6_K_SEQ: return 256;
    default: return 32;
    }
}

int orc_block_bytes(int sem)
{
    switch (sem) {
    case ORC_F32: return 4;
    case ORC_Q4_0: return 18;
    case ORC_Q4_1: return 20;
    case ORC_Q5_0_F32: case ORC_Q5_0_Q8: return 22;
    case ORC_Q8_0: return 34;
    case ORC_Q4_K_GGML: case ORC_Q4_K_Q8: return 144;
    case ORC_Q5_K_GGML: case ORC_Q5_K_CE: return 176;
    case ORC_Q6_K_GGML: case ORC_Q6_K_LOWNIB: case ORC_Q6_K_SEQ: return 210;
    default: return 17;                                   /* MXFP4 */
    }
}

long orc_row_bytes(int sem, int n_cols)
{
    return (long)(n_cols / orc_block_elems(sem)) * orc_block_bytes(sem);
}

/* ------------------------------------------------ fp32 weight dequant */

/* Q4_0 (QK:77-95, CE:68-110): lo nibble -> element k, hi -> 16+k; w = (n-8)*d. */
static void dq_q4_0(const uint8_t *b, float *w)
{
    float d = ld_f16(b);
    for (int k = 0; k < 16; k++) {
        w[k]      = (float)((b[2 + k] & 15) - 8) * d;
        w[16 + k] = (float)((b[2 + k] >> 4) - 8) * d;
    }
}

/* Q4_1 (QK:97-117): w = fma(n, d, m), lo nibble -> k, hi -> 16+k. */
static void dq_q4_1(const uint8_t *b, float *w)
{
    float d = ld_f16(b), m = ld_f16(b + 2);
    for (int k = 0; k < 16; k++) {
        w[k]      = fmaf((float)(b[4 + k] & 15), d, m);
        w[16 + k] = fmaf((float)(b[4 + k] >> 4), d, m);
    }
}

/* Q5_0 as the reference lays it out ([d:2][qh:4][ql:16]) with sequential
 * nibble order: element e = nibble (e&1) of ql[e/2] | qh bit e, minus 16
 * (q5_0_row_dot QK:1239-1251, dot_q5_0_q8_0 QK:1262-1316). */
static int q5_0_val(const uint8_t *b, int e)
{
    const uint8_t *qh = b + 2, *ql = b + 6;
    return (((ql[e / 2] >> ((e & 1) * 4)) & 15) | (((qh[e / 8] >> (e % 8)) & 1) << 4)) - 16;
}

static void dq_q5_0(const uint8_t *b, float *w)
{
    float d = ld_f16(b);
    for (int e = 0; e < 32; e++) w[e] = (float)q5_0_val(b, e) * d;
}

/* Q8_0 (QK:376-416, CE:216-253): w = q * d. */
static void dq_q8_0(const uint8_t *b, float *w)
{
    float d = ld_f16(b);
    for (int k = 0; k < 32; k++) w[k] = (float)(int8_t)b[2 + k] * d;
}

/* Q4_K ggml order (CE:255-313): for group g, lo nibbles of qs[32g..] are
 * elements 64g+k with pair 2g, hi nibbles 64g+32+k with pair 2g+1;
 * w = fl(fl(d*sc)*n) - fl(dmin*m). */
static void dq_q4_k(const uint8_t *b, float *w)
{
    float d = ld_f16(b), dm = ld_f16(b + 2);
    const uint8_t *sc = b + 4, *qs = b + 16;
    for (int g = 0; g < 4; g++) {
        int s1, m1, s2, m2;
        k4_pair(2 * g, sc, &s1, &m1);
        k4_pair(2 * g + 1, sc, &s2, &m2);
        float d1 = d * (float)s1, mm1 = dm * (float)m1;
        float d2 = d * (float)s2, mm2 = dm * (float)m2;
        for (int k = 0; k < 32; k++) {
            w[64 * g + k]      = (float)(qs[32 * g + k] & 15) * d1 - mm1;
            w[64 * g + 32 + k] = (float)(qs[32 * g + k] >> 4) * d2 - mm2;
        }
    }
}

/* Q5_K ggml layout d@0 dmin@2 scales@4 qh@16 qs@48 (QK:211-246, 830-866):
 * as Q4_K plus 16 when qh[k] bit 2g (lo) / 2g+1 (hi) is set. */
static void dq_q5_k_ggml(const uint8_t *b, float *w)
{
    float d = ld_f16(b), dm = ld_f16(b + 2);
    const uint8_t *sc = b + 4, *qh = b + 16, *qs = b + 48;
    for (int g = 0; g < 4; g++) {
        int s1, m1, s2, m2;
        k4_pair(2 * g, sc, &s1, &m1);
        k4_pair(2 * g + 1, sc, &s2, &m2);
        float d1 = d * (float)s1, mm1 = dm * (float)m1;
        float d2 = d * (float)s2, mm2 = dm * (float)m2;
        for (int k = 0; k < 32; k++) {
            int lo = (qs[32 * g + k] & 15) + (((qh[k] >> (2 * g)) & 1) << 4);
            int hi = (qs[32 * g + k] >> 4) + (((qh[k] >> (2 * g + 1)) & 1) << 4);
            w[64 * g + k]      = (float)lo * d1 - mm1;
            w[64 * g + 32 + k] = (float)hi * d2 - mm2;
        }
    }
}

/* Q5_K with the engine's own struct (CE:46-52: d@0 dmin@2 qh@4 ql@36
 * scales@164) and sequential element order (CE:393-407): element e is
 * nibble (e&1) of ql[e/2] | bit (e&7) of qh[e/8] << 4, pair e/32. */
static void dq_q5_k_ce(const uint8_t *b, float *w)
{
    float d = ld_f16(b), dm = ld_f16(b + 2);
    const uint8_t *qh = b + 4, *ql = b + 36, *sc = b + 164;
    for (int e = 0; e < 256; e++) {
        int s, m;
        k4_pair(e / 32, sc, &s, &m);
        int v = ((ql[e / 2] >> ((e & 1) * 4)) & 15) | (((qh[e / 8] >> (e & 7)) & 1) << 4);
        w[e] = (float)v * (d * (float)s) - dm * (float)m;
    }
}

/* Q6_K: ql@0 qh@128 int8 scales@192 d@208.
 * ggml order (q6_k_dequantize_row QK:762-800): half h, l<32, quadrant Q at
 * 128h + 32Q + l, scale sc[8h + l/16 + 2Q], 2-bit high part qh[32h+l]>>2Q;
 * low nibble from ql[64h + l + 32*(Q&1)], low half for Q<2, high for Q>=2.
 * lownib (q6k_dequant_8, QK:1778-1812): quadrants 2,3 also take the LOW nibble. */
static void dq_q6_k_quadrant(const uint8_t *b, float *w, int lownib)
{
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    float d = ld_f16(b + 208);
    for (int h = 0; h < 2; h++)
        for (int l = 0; l < 32; l++)
            for (int Q = 0; Q < 4; Q++) {
                int byte = ql[64 * h + l + 32 * (Q & 1)];
                int nib = (Q < 2 || lownib) ? (byte & 15) : (byte >> 4);
                int q = (nib | (((qh[32 * h + l] >> (2 * Q)) & 3) << 4)) - 32;
                w[128 * h + 32 * Q + l] = (d * (float)sc[8 * h + l / 16 + 2 * Q]) * (float)q;
            }
}

/* Q6_K sequential order (q6_k_batch_matmul CE:315-378): element e is
 * nibble (e&1) of ql[e/2] | ((qh[e/4] >> 2(e&3)) & 3) << 4, minus 32,
 * scale d*sc[e/16]; w = q * fl(d*sc). */
static void dq_q6_k_seq(const uint8_t *b, float *w)
{
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    float d = ld_f16(b + 208);
    for (int e = 0; e < 256; e++) {
        int q = (((ql[e / 2] >> ((e & 1) * 4)) & 15) | (((qh[e / 4] >> (2 * (e & 3))) & 3) << 4)) - 32;
        w[e] = (float)q * (d * (float)sc[e / 16]);
    }
}

/* MXFP4 as the reference defines it (QK:485-500, CE:41-44): q[16] then an
 * E8M0 byte; element e = sign-extended nibble (e&1) of q[e/2]; w = v * 2^(E-127).
 * clamp: mxfp4_batch_matmul limits the scale to 1e20 (CE:454-456). */
static void dq_mxfp4(const uint8_t *b, float *w, int clamp)
{
    float s = e8m0(b[16]);
    if (clamp && s > 1e20f) s = 1e20f;
    for (int e = 0; e < 32; e++) w[e] = (float)sext4((b[e / 2] >> ((e & 1) * 4)) & 15) * s;
}

int orc_dequant_row(int sem, const uint8_t *row, float *w, int n_cols)
{
    int be = orc_block_elems(sem), bb = orc_block_bytes(sem), nb = n_cols / be;
    for (int i = 0; i < nb; i++) {
        const uint8_t *b = row + (long)i * bb;
        float *o = w + (long)i * be;
        switch (sem) {
        case ORC_F32:         memcpy(o, b, 4); break;
        case ORC_Q4_0:        dq_q4_0(b, o); break;
        case ORC_Q4_1:        dq_q4_1(b, o); break;
        case ORC_Q5_0_F32:    dq_q5_0(b, o); break;
        case ORC_Q8_0:        dq_q8_0(b, o); break;
        case ORC_Q4_K_GGML:   dq_q4_k(b, o); break;
        case ORC_Q5_K_GGML:   dq_q5_k_ggml(b, o); break;
        case ORC_Q5_K_CE:     dq_q5_k_ce(b, o); break;
        case ORC_Q6_K_GGML:   dq_q6_k_quadrant(b, o, 0); break;
        case ORC_Q6_K_LOWNIB: dq_q6_k_quadrant(b, o, 1); break;
        case ORC_Q6_K_SEQ:    dq_q6_k_seq(b, o); break;
        case ORC_MXFP4:       dq_mxfp4(b, o, 0); break;
        case ORC_MXFP4_CLAMP: dq_mxfp4(b, o, 1); break;
        default: return -1;
        }
    }
    for (int i = nb * be; i < n_cols; i++) w[i] = 0.0f;   /* reference ignores a ragged tail */
    return 0;
}

/* --------------------------------------------- activation quantisation */

/* maxps(a, b) (vmaxps): a if a > b, else b, so a NaN in either operand
 * gives the second operand. */
static float maxps(float a, float b) { return a > b ? a : b; }

/* quantize_row_q8_0 (QK:1406-1455): per 32: amax, d = amax/127 (1 if 0),
 * id = 1/d, q = RNE(clamp(x*id, +-127)); stored scale fp16_RNE(d).
 * amax follows the reference's vector order, which only matters for NaN:
 * eight lanes m_j fold |x_{8i+j}| for i = 0..3 as maxps(m_j, |x|)
 * (QK:1417-1421), then the halves, pairs and neighbours combine as
 * maxps(m_j, m_{j^4}), maxps(., j^2), maxps(., j^1) (QK:1423-1425), lane 0
 * read.  A NaN product clamps to -127 (maxps returns its second operand). */
int orc_quantize_row_q8_0(const float *x, uint8_t *q8, int n_cols)
{
    int nb = n_cols / 32;
    for (int b = 0; b < nb; b++) {
        const float *s = x + 32 * b;
        uint8_t *dst = q8 + 34 * b;
        float m[8], t[8], u[8];
        for (int j = 0; j < 8; j++) m[j] = 0.0f;
        for (int i = 0; i < 4; i++)
            for (int j = 0; j < 8; j++) m[j] = maxps(m[j], fabsf(s[8 * i + j]));
        for (int j = 0; j < 8; j++) t[j] = maxps(m[j], m[j ^ 4]);
        for (int j = 0; j < 8; j++) u[j] = maxps(t[j], t[j ^ 2]);
        float amax = maxps(u[0], u[1]);
        float d = amax / 127.0f;
        if (d == 0.0f) d = 1.0f;
        float id = 1.0f / d;
        uint16_t h = orc_f32_to_f16(d);
        dst[0] = (uint8_t)(h & 0xff);
        dst[1] = (uint8_t)(h >> 8);
        for (int i = 0; i < 32; i++) {
            float v = s[i] * id;
            v = (v > -127.0f) ? v : -127.0f;
            v = (v < 127.0f) ? v : 127.0f;
            dst[2 + i] = (uint8_t)(int8_t)(int)nearbyintf(v);
        }
    }
    return nb;
}

/* --------------------------------------------- Q8_0-activation dots */

/* dot_q4_k_q8_0 (QK:1647-1735) on one super-block and its 8 Q8_0 blocks.
 * Its two horizontal reductions read only the low 128 bits (QK:1714-1723,
 * 1728-1732), so the integer term sees elements k<16 of each sub-block and
 * no Q8 scale, and the min term sums q8 elements 0-7 and 16-23 with no
 * sub-block min:
 *   int_sum = sum_j sc_j * sum_{k<16} nib_{j,k} q8_{j,k}
 *   sum_min = sum_j dmin*d8_j * (sum_{k<8} q8 + sum_{16<=k<24} q8)
 *   value   = d*int_sum - sum_min                                      */
static float dot_q4_k_q8_sb(const uint8_t *qk, const uint8_t *q8)
{
    float d = ld_f16(qk), dmin = ld_f16(qk + 2);
    const uint8_t *sc = qk + 4, *qs = qk + 16;
    int32_t int_sum = 0;
    float sum_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        int s, m;
        k4_pair(j, sc, &s, &m);
        const uint8_t *blk = q8 + 34 * j;
        const int8_t *q = (const int8_t *)(blk + 2);
        float d8 = ld_f16(blk);
        int32_t dot = 0, qsum = 0;
        for (int k = 0; k < 16; k++) dot += ((qs[32 * (j >> 1) + k] >> (4 * (j & 1))) & 15) * q[k];
        for (int k = 0; k < 8; k++) qsum += q[k] + q[16 + k];
        int_sum += s * dot;
        sum_min = fmaf(dmin * d8, (float)qsum, sum_min);
    }
    return fmaf(d, (float)int_sum, -sum_min);
}

/* mxfp4_row_dot_q8 (QK:629-678) on one block: cs = clamp(2^(E-127)*d8, +-1e20),
 * value = cs * sum_k v_k q8_k. */
static double dot_mxfp4_q8_blk(const uint8_t *b, const uint8_t *q8blk)
{
    float cs = e8m0(b[16]) * ld_f16(q8blk);
    if (cs > 1e20f) cs = 1e20f;
    if (cs < -1e20f) cs = -1e20f;
    const int8_t *q = (const int8_t *)(q8blk + 2);
    int32_t dot = 0;
    for (int e = 0; e < 32; e++) dot += sext4((b[e / 2] >> ((e & 1) * 4)) & 15) * q[e];
    return (double)cs * (double)dot;
}

/* dot_q5_0_q8_0 (QK:1262-1316): d5*d8*sum v*q8. */
static float dot_q5_0_q8_blk(const uint8_t *b, const uint8_t *q8blk)
{
    const int8_t *q = (const int8_t *)(q8blk + 2);
    int32_t acc = 0;
    for (int e = 0; e < 32; e++) acc += q5_0_val(b, e) * q[e];
    return ld_f16(b) * ld_f16(q8blk) * (float)acc;
}

/* ------------------------------------------------------------- GEMV */

/* q5_k_row_dot_avx2 (QK:249-344) on one super-block: per 32-element
 * sub-block d1 * sum(q x) - m1 * sum(x) with d1 = d*sc, m1 = dmin*m in fp32
 * (QK:266-269, 300, 338): the min term factored out of the sum, which is
 * what decides the result when x holds an inf (inf - inf = NaN where a
 * per-element w*x would give +-inf). */
static double dot_q5_k_ggml_sb(const uint8_t *b, const float *x)
{
    float d = ld_f16(b), dm = ld_f16(b + 2);
    const uint8_t *sc = b + 4, *qh = b + 16, *qs = b + 48;
    double acc = 0.0;
    for (int g = 0; g < 4; g++) {
        int s1, m1, s2, m2;
        k4_pair(2 * g, sc, &s1, &m1);
        k4_pair(2 * g + 1, sc, &s2, &m2);
        float d1 = d * (float)s1, mm1 = dm * (float)m1;
        float d2 = d * (float)s2, mm2 = dm * (float)m2;
        double qx1 = 0, sx1 = 0, qx2 = 0, sx2 = 0;
        for (int k = 0; k < 32; k++) {
            int lo = (qs[32 * g + k] & 15) + (((qh[k] >> (2 * g)) & 1) << 4);
            int hi = (qs[32 * g + k] >> 4) + (((qh[k] >> (2 * g + 1)) & 1) << 4);
            qx1 += (double)lo * x[64 * g + k];
            sx1 += x[64 * g + k];
            qx2 += (double)hi * x[64 * g + 32 + k];
            sx2 += x[64 * g + 32 + k];
        }
        acc += (double)d1 * qx1 - (double)mm1 * sx1;
        acc += (double)d2 * qx2 - (double)mm2 * sx2;
    }
    return acc;
}

void orc_gemv(int sem, const uint8_t *W, const float *x, float *out,
              int n_rows, int n_cols, int B)
{
    long rb = orc_row_bytes(sem, n_cols);
    int q8_sem = (sem == ORC_Q4_K_Q8 || sem == ORC_MXFP4_Q8 || sem == ORC_Q5_0_Q8);
    if (q8_sem) {
        int nb32 = n_cols / 32;
        uint8_t *xq = (uint8_t *)malloc((size_t)(nb32 > 0 ? nb32 : 1) * 34);
        for (int b = 0; b < B; b++) {
            orc_quantize_row_q8_0(x + (long)b * n_cols, xq, n_cols);
            for (int r = 0; r < n_rows; r++) {
                const uint8_t *row = W + (long)r * rb;
                double acc = 0.0;
                if (sem == ORC_Q4_K_Q8)
                    for (int s = 0; s < n_cols / 256; s++) acc += dot_q4_k_q8_sb(row + 144L * s, xq + 8L * 34 * s);
                else if (sem == ORC_MXFP4_Q8)
                    for (int k = 0; k < nb32; k++) acc += dot_mxfp4_q8_blk(row + 17L * k, xq + 34L * k);
                else
                    for (int k = 0; k < nb32; k++) acc += dot_q5_0_q8_blk(row + 22L * k, xq + 34L * k);
                out[(long)b * n_rows + r] = (float)acc;
            }
        }
        free(xq);
        return;
    }
    if (sem == ORC_Q5_K_GGML) {
        for (int r = 0; r < n_rows; r++)
            for (int b = 0; b < B; b++) {
                double acc = 0.0;
                for (int s = 0; s < n_cols / 256; s++)
                    acc += dot_q5_k_ggml_sb(W + (long)r * rb + 176L * s, x + (long)b * n_cols + 256L * s);
                out[(long)b * n_rows + r] = (float)acc;
            }
        return;
    }
    float *w = (float *)malloc((size_t)(n_cols > 0 ? n_cols : 1) * sizeof(float));
    for (int r = 0; r < n_rows; r++) {
        orc_dequant_row(sem, W + (long)r * rb, w, n_cols);
        for (int b = 0; b < B; b++) {
            const float *xb = x + (long)b * n_cols;
            double acc = 0.0;
            for (int i = 0; i < n_cols; i++) acc += (double)w[i] * (double)xb[i];
            out[(long)b * n_rows + r] = (float)acc;
        }
    }
    free(w);
}

/* ------------------------------------------- entry point -> semantic */

int orc_sem_for(int entry, int qt)
{
    switch (entry) {
    case 0:   /* quant_matmul_omp dispatch QK:1355-1388 */
        switch (qt) {
        case 0: return ORC_F32;   case 2: return ORC_Q4_0;   case 3: return ORC_Q4_1;
        case 6: return ORC_Q5_0_Q8; case 8: return ORC_Q8_0; case 12: return ORC_Q4_K_Q8;
        case 13: return ORC_Q5_K_GGML; case 14: return ORC_Q6_K_LOWNIB; case 39: return ORC_MXFP4;
        default: return -1;
        }
    case 1:   /* CE:68,216,256,316,381,435 */
        switch (qt) {
        case 2: return ORC_Q4_0; case 8: return ORC_Q8_0; case 12: return ORC_Q4_K_GGML;
        case 13: return ORC_Q5_K_CE; case 14: return ORC_Q6_K_SEQ; case 39: return ORC_MXFP4_CLAMP;
        default: return -1;
        }
    case 2:   /* batch_qkv_omp / batch_gate_up_omp QK:1139-1222 via matmul_row_range QK:1095-1133 */
        switch (qt) {
        case 2: return ORC_Q4_0; case 3: return ORC_Q4_1; case 6: return ORC_Q5_0_F32;
        case 8: return ORC_Q8_0; case 12: return ORC_Q4_K_Q8; case 13: return ORC_Q5_K_GGML;
        case 14: return ORC_Q6_K_LOWNIB; case 39: return ORC_MXFP4;
        default: return -1;
        }
    case 3:   /* moe_forward_omp gate/up, not both MXFP4 (QK:2122-2152) */
        switch (qt) {
        case 12: return ORC_Q4_K_Q8; case 14: return ORC_Q6_K_LOWNIB; case 2: return ORC_Q4_0;
        case 3: return ORC_Q4_1; case 6: return ORC_Q5_0_Q8;
        default: return -1;
        }
    case 4:   /* moe_forward_omp down (QK:2192-2245) */
        switch (qt) {
        case 39: return ORC_MXFP4_Q8; case 14: return ORC_Q6_K_LOWNIB; case 2: return ORC_Q4_0;
        case 6: return ORC_Q5_0_F32;
        default: return -1;
        }
    }
    return -1;
}

/* ------------------------------------------------------------ routing */

void orc_route(const float *router_w, const float *x, int T, int N, int E, int K,
               int renorm, int *top_idx, float *top_w)
{
    float *p = (float *)malloc((size_t)E * sizeof(float));
    for (int t = 0; t < T; t++) {
        const float *xt = x + (long)t * N;
        for (int e = 0; e < E; e++) {                 /* CE:614-618: scalar FMA chain */
            float dot = 0.0f;
            for (int i = 0; i < N; i++) dot = fmaf(xt[i], router_w[(long)e * N + i], dot);
            p[e] = dot;
        }
        float mx = p[0];                              /* CE:621-622 */
        for (int e = 1; e < E; e++) if (p[e] > mx) mx = p[e];
        float sum = 0.0f;
        for (int e = 0; e < E; e++) { p[e] = expf(p[e] - mx); sum += p[e]; }
        float inv = 1.0f / (sum + 1e-10f);
        for (int e = 0; e < E; e++) p[e] *= inv;
        int *ti = top_idx + (long)t * K;
        float *tv = top_w + (long)t * K;
        for (int k = 0; k < K; k++) { tv[k] = -1e30f; ti[k] = -1; }
        for (int e = 0; e < E; e++) {                 /* CE:628-638 insertion, strict '>' */
            float v = p[e];
            for (int k = 0; k < K; k++) {
                if (v > tv[k]) {
                    for (int k2 = K - 1; k2 > k; k2--) { tv[k2] = tv[k2 - 1]; ti[k2] = ti[k2 - 1]; }
                    tv[k] = v; ti[k] = e;
                    break;
                }
            }
        }
        if (renorm) {                                 /* GO:88-92, CE:1148-1152 */
            float s = 0.0f;
            for (int k = 0; k < K; k++) s += tv[k];
            float r = 1.0f / (s + 1e-10f);
            for (int k = 0; k < K; k++) tv[k] *= r;
        }
    }
    free(p);
}

/* ----------------------------------------------------------------- MoE */

long orc_moe_ffn_stride(int which, int qt, int N, int M)
{
    /* CE:593-605: gate/up default to the Q4_K size, down to Q6_K; only
     * codes 12/13/14/39 change it (so e.g. Q8_0 experts get a Q4_K stride). */
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

void orc_moe_ffn_token(const float *router_w, const uint8_t *gate, const uint8_t *up,
                       const uint8_t *down, int qt_gate, int qt_up, int qt_down,
                       int N, int E, int K, int M, const float *x, float *out)
{
    int idx[16];
    float wt[16];
    orc_route(router_w, x, 1, N, E, K, 0, idx, wt);
    float *g = (float *)malloc(sizeof(float) * (size_t)M);
    float *u = (float *)malloc(sizeof(float) * (size_t)M);
    float *dn = (float *)malloc(sizeof(float) * (size_t)N);
    int sg = orc_sem_for(0, qt_gate), su = orc_sem_for(0, qt_up), sd = orc_sem_for(0, qt_down);
    for (int i = 0; i < N; i++) out[i] = 0.0f;       /* CE:643 */
    for (int k = 0; k < K; k++) {
        int e = idx[k];
        if (e < 0 || sg < 0 || su < 0 || sd < 0) continue;
        orc_gemv(sg, gate + e * orc_moe_ffn_stride(0, qt_gate, N, M), x, g, M, N, 1);
        orc_gemv(su, up + e * orc_moe_ffn_stride(1, qt_up, N, M), x, u, M, N, 1);
        for (int i = 0; i < M; i++) {                 /* CE:653-657: no clamp */
            float gv = g[i];
            g[i] = (gv / (1.0f + expf(-gv))) * u[i];
        }
        orc_gemv(sd, down + e * orc_moe_ffn_stride(2, qt_down, N, M), g, dn, N, M, 1);
        for (int i = 0; i < N; i++) out[i] = fmaf(wt[k], dn[i], out[i]);   /* CE:662 */
    }
    free(g); free(u); free(dn);
}

/* Row stride in bytes of moe_forward_omp's Q5_0 down projection when it
 * differs from the matrix's own and every row it addresses lies inside the
 * n_embd x n_ff matrix (QK:2216, 2230: row * ((n_embd+31)/32)*22); else 0. */
long orc_moe_q5_down_stride(int qt_down, int n_embd, int n_ff)
{
    if (qt_down != ORC_QT_Q5_0 || n_embd <= 0 || n_ff <= 0) return 0;
    const long s_ref = (long)((n_embd + 31) / 32) * 22, s_own = (long)((n_ff + 31) / 32) * 22;
    if (s_ref == s_own) return 0;
    const long last = (long)(n_embd - 1) * s_ref + (long)(n_ff / 32) * 22;
    return last <= (long)n_embd * s_own ? s_ref : 0;
}

void orc_moe_forward_token(const uint8_t *const *gate, const uint8_t *const *up,
                           const uint8_t *const *down, const float *x, int n_ff, int n_embd,
                           int qt_gate, int qt_up, int qt_down, const int *top_idx,
                           const float *top_w, int top_k, int has_q8_scratch, float *out)
{
    float *g = (float *)malloc(sizeof(float) * (size_t)n_ff);
    float *u = (float *)malloc(sizeof(float) * (size_t)n_ff);
    float *dn = (float *)malloc(sizeof(float) * (size_t)n_embd);
    int pair_mx = (qt_gate == 39 && qt_up == 39);    /* QK:2094 */
    int sg = pair_mx ? ORC_MXFP4 : orc_sem_for(3, qt_gate);
    int su = pair_mx ? ORC_MXFP4 : orc_sem_for(3, qt_up);
    int sd = orc_sem_for(4, qt_down);
    if (qt_down == 39 && !has_q8_scratch) sd = -1;   /* reference dereferences NULL here */
    /* Q5_0 down rows (QK:2216, 2230) start row * ((n_embd+31)/32)*22 bytes in,
     * a stride taken from n_embd, not from the n_ff-wide rows; followed where
     * every row stays inside the n_embd x n_ff matrix (n_embd < n_ff), else the
     * reference reads past it and the matrix's own row stride is used. */
    const long q5_stride = orc_moe_q5_down_stride(qt_down, n_embd, n_ff);
    for (int i = 0; i < n_embd; i++) out[i] = 0.0f;   /* QK:2192 */
    for (int k = 0; k < top_k; k++) {
        int e = top_idx[k];
        if (sg >= 0) orc_gemv(sg, gate[e], x, g, n_ff, n_embd, 1); else memset(g, 0, sizeof(float) * n_ff);
        if (su >= 0) orc_gemv(su, up[e], x, u, n_ff, n_embd, 1); else memset(u, 0, sizeof(float) * n_ff);
        for (int i = 0; i < n_ff; i++) {              /* QK:2157-2164: clamp to +-80 */
            float gv = g[i];
            if (gv < -80.0f) gv = -80.0f;
            if (gv > 80.0f) gv = 80.0f;
            g[i] = (gv / (1.0f + expf(-gv))) * u[i];
        }
        if (sd >= 0 && q5_stride)
            for (int r = 0; r < n_embd; r++) orc_gemv(sd, down[e] + (long)r * q5_stride, g, dn + r, 1, n_ff, 1);
        else if (sd >= 0) orc_gemv(sd, down[e], g, dn, n_embd, n_ff, 1);
        else memset(dn, 0, sizeof(float) * n_embd);
        for (int i = 0; i < n_embd; i++) out[i] += top_w[k] * dn[i];   /* atomic add, k order here */
    }
    free(g); free(u); free(dn);
}

/* ------------------------------------------------ lm_head requantisation */

/* The reference caller's lm_head requantisation (TE:620-666,
 * _requantize_output): each row of a Q4_K / Q6_K matrix dequantised as
 * q4_k_dequantize_row / q6_k_dequantize_row do (QK:762-828; columns past the
 * last whole super-block stay 0, as TE's np.zeros buffer leaves them), or of
 * an F16 matrix (type 1) as TE:643-645 converts it,
 * raw_u16.astype(np.float32).view(np.float32): the integer value of each
 * 16-bit pattern, not its fp16 value (0x3C00 -> 15360.0f); then per 32
 * elements in float32 as TE's numpy code computes it:
 * amax = max(max|x|, 1e-10f), d = amax / 127, q = round-half-even(x / d)
 * clamped to +-127, d stored as fp16 (RNE) before the 32 quants.
 * Returns 0, or -1 for a type TE does not requantise this way (and for an F16
 * row length TE's reshape into 32-element blocks rejects). */
int orc_requant_q8_0(int qt, const uint8_t *W, int n_rows, int n_cols, uint8_t *out)
{
    const int f16 = qt == ORC_QT_F16;
    const int sem = qt == ORC_QT_Q4_K ? ORC_Q4_K_GGML : qt == ORC_QT_Q6_K ? ORC_Q6_K_GGML : -1;
    if (sem < 0 && !f16) return -1;
    if (f16 && n_cols % 32) return -1;
    const long rb = f16 ? 2L * n_cols : orc_row_bytes(sem, n_cols);
    const int nb = n_cols / 32;
    float *w = (float *)malloc((size_t)(n_cols > 0 ? n_cols : 1) * sizeof(float));
    if (!w) return -1;
    for (int r = 0; r < n_rows; r++) {
        memset(w, 0, (size_t)n_cols * sizeof(float));
        if (f16) {
            const uint8_t *src = W + (long)r * rb;
            for (int i = 0; i < n_cols; i++) w[i] = (float)(uint16_t)(src[2 * i] | (src[2 * i + 1] << 8));
        } else {
            orc_dequant_row(sem, W + (long)r * rb, w, n_cols / 256 * 256);
        }
        for (int b = 0; b < nb; b++) {
            const float *x = w + 32 * b;
            uint8_t *dst = out + ((long)r * nb + b) * 34;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) { const float a = fabsf(x[i]); if (a > amax) amax = a; }
            if (amax < 1e-10f) amax = 1e-10f;
            const float d = amax / 127.0f;
            const uint16_t h = orc_f32_to_f16(d);
            dst[0] = (uint8_t)(h & 0xff);
            dst[1] = (uint8_t)(h >> 8);
            for (int i = 0; i < 32; i++) {
                float q = nearbyintf(x[i] / d);
                q = q < -127.0f ? -127.0f : q > 127.0f ? 127.0f : q;
                dst[2 + i] = (uint8_t)(int8_t)(int)q;
            }
        }
    }
    free(w);
    return 0;
}

/* ------------------------------------------------------------ attention */

/* exp_ps_simd (gqa_attention.c:32-48), one lane: t = x*log2e, n = rne(t +
 * 0.5) (cvtps_epi32 under the default MXCSR), f = t - n, then the FMA chain
 * exactly as the source writes it (starting from 1 and adding the
 * coefficients in ascending order), times 2^n built from the clamped biased
 * exponent. */
float orc_exp_ps_simd(float x)
{
    const float t = x * 1.4426950408889634f;
    const int n = (int)nearbyintf(t + 0.5f);
    const float f = t - (float)n;
    float p = 1.0f;
    p = fmaf(p, f, 0.6931471805599453f);
    p = fmaf(p, f, 0.2402265069591007f);
    p = fmaf(p, f, 0.0555041086648216f);
    p = fmaf(p, f, 0.0096181291076285f);
    p = fmaf(p, f, 0.0013333558146428f);
    int biased = n + 127;
    biased = biased < 0 ? 0 : biased > 255 ? 255 : biased;
    uint32_t bits = (uint32_t)biased << 23;
    float two_n;
    memcpy(&two_n, &bits, 4);
    return p * two_n;
}

void orc_gqa_decode(int mode, const float *q, const float *k, const float *v, long row_stride, int seq_len,
                    int nh, int nkh, int hd, float *out)
{
    const int gr = nh / nkh;
    const float scale = 1.0f / sqrtf((float)hd);
    float *sc = (float *)malloc((size_t)(seq_len > 0 ? seq_len : 1) * sizeof(float));
    for (int h = 0; h < nh; h++) {
        const int j = h / gr;
        const float *qh = q + (long)h * hd;
        float mx = -1e30f;
        for (int s = 0; s < seq_len; s++) {
            const float *kr = k + (long)s * row_stride + (long)j * hd;
            /* one fp32 FMA chain in element order: the reference's AVX2 lane
             * order (CE:149-151) or sgemm blocking is not reproducible here,
             * and any order is within fp32 rounding; a fixed order matters
             * for exp_ps_simd, where a one-ulp change of a score can move its
             * n = rne(t + 0.5) and so the weight by a step */
            float dot = 0.0f;
            for (int d = 0; d < hd; d++) dot = fmaf(qh[d], kr[d], dot);
            sc[s] = dot * scale;                        /* CE:152 dot*=inv; sgemm alpha */
            if (sc[s] > mx) mx = sc[s];
        }
        double sum = 0.0;
        const int vec_end = mode == ORC_ATTN_GQA_C ? seq_len / 8 * 8 : 0;
        for (int s = 0; s < seq_len; s++) {
            float e;
            if (s < vec_end) {                           /* gqa_attention.c:71-77 */
                float z = sc[s] - mx;
                z = z > -80.0f ? z : -80.0f;
                z = z < 80.0f ? z : 80.0f;
                e = orc_exp_ps_simd(z);
            } else {
                e = expf(sc[s] - mx);
                if (mode == ORC_ATTN_GQA_C && e > 1e38f) e = 1e38f;
            }
            sc[s] = e;
            sum += e;
        }
        const float inv = mode == ORC_ATTN_GQA_C ? 1.0f / ((float)sum + 1e-10f) : 1.0f / (float)sum;
        for (int d = 0; d < hd; d++) {
            double acc = 0.0;
            for (int s = 0; s < seq_len; s++) acc += (double)(sc[s] * inv) * v[(long)s * row_stride + (long)j * hd + d];
            out[(long)h * hd + d] = (float)acc;
        }
    }
    free(sc);
}

void orc_rope(float *buf, int nh, int hd, int pos, const float *cos_t, const float *sin_t, int rope_dim)
{
    if (rope_dim <= 0) rope_dim = hd;
    const int hd2 = rope_dim / 2;
    const float *cr = cos_t + (long)pos * hd2, *sr = sin_t + (long)pos * hd2;
    for (int h = 0; h < nh; h++) {
        float *b = buf + (long)h * hd;
        for (int j = 0; j < hd2; j++) {
            const float a0 = b[j], a1 = b[j + hd2];
            b[j] = a0 * cr[j] - a1 * sr[j];
            b[j + hd2] = a1 * cr[j] + a0 * sr[j];
        }
    }
}

/* ----------------------------------------------------------- gptoss_forward */

/* rms_norm (GO:29-34): (x / sqrtf(ss/N + eps)) * w, ss in double. */
static void orc_rms_div(float *out, const float *x, const float *w, int n, float eps)
{
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float r = sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; i++) out[i] = (x[i] / r) * w[i];
}

void orc_gptoss_forward(const orc_gptoss *m, int token, int pos, float *k_cache, float *v_cache, int *kv_len,
                        float *logits)
{
    const int N = m->N, inner = m->NH * m->HD, kvd = m->NKH * m->HD;
    float *x = (float *)malloc(sizeof(float) * N), *xn = (float *)malloc(sizeof(float) * N);
    float *res = (float *)malloc(sizeof(float) * N), *ffn = (float *)malloc(sizeof(float) * N);
    float *q = (float *)malloc(sizeof(float) * inner), *att = (float *)malloc(sizeof(float) * inner);
    float *k = (float *)malloc(sizeof(float) * kvd), *v = (float *)malloc(sizeof(float) * kvd);
    float *op = (float *)malloc(sizeof(float) * N);
    int idx[64];
    float w[64];
    memcpy(x, m->emb + (long)token * N, sizeof(float) * N);
    for (int l = 0; l < m->L; l++) {
        memcpy(res, x, sizeof(float) * N);
        orc_rms_div(xn, x, m->wAN[l], N, m->eps);
        orc_gemv(ORC_MXFP4, m->wQ[l], xn, q, inner, N, 1);
        orc_gemv(ORC_MXFP4, m->wK[l], xn, k, kvd, N, 1);
        orc_gemv(ORC_MXFP4, m->wV[l], xn, v, kvd, N, 1);
        orc_rope(q, m->NH, m->HD, pos, m->cos_t, m->sin_t, m->rope_dim);
        orc_rope(k, m->NKH, m->HD, pos, m->cos_t, m->sin_t, m->rope_dim);
        float *kc = k_cache + (long)l * m->max_ctx * kvd, *vc = v_cache + (long)l * m->max_ctx * kvd;
        int sl = kv_len[l];
        memcpy(kc + (long)sl * kvd, k, sizeof(float) * kvd);
        memcpy(vc + (long)sl * kvd, v, sizeof(float) * kvd);
        kv_len[l]++;
        sl++;
        orc_gqa_decode(ORC_ATTN_GQA_C, q, kc, vc, kvd, sl, m->NH, m->NKH, m->HD, att);
        orc_gemv(ORC_MXFP4, m->wO[l], att, op, N, inner, 1);
        for (int i = 0; i < N; i++) x[i] = res[i] + op[i];
        orc_rms_div(xn, x, m->wFN[l], N, m->eps);
        orc_route(m->w_gate_inp[l], xn, 1, N, m->E, m->K, 1, idx, w);
        orc_moe_forward_token(m->w_gate_exps + l, m->w_up_exps + l, m->w_down_exps + l, xn, m->M, N, m->qt_gate,
                              m->qt_up, m->qt_down, idx, w, m->K, 1, ffn);
        for (int i = 0; i < N; i++) x[i] = res[i] + ffn[i];
    }
    orc_gemv(ORC_MXFP4, m->wOut, xn, logits, m->outNR, N, 1);
    free(x); free(xn); free(res); free(ffn); free(q); free(att); free(k); free(v); free(op);
}
