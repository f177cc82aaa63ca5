/* oracle.h — CPU restatement of a730/MojoLlama's quantised-matmul + MoE hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (mojollama_amd/) links,
 * loads or calls this code.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the checker.
 *
 * Each function restates one exported reference symbol's arithmetic (the
 * same quant type means different things on different reference entry
 * points, so semantics are keyed per symbol: see enum orc_sem).  Matmul
 * outputs are accumulated in double: the oracle gives the value of the
 * reference's formula on its fp32 weights, not its fp32 summation order.
 * Routing (orc_route) and activation quantisation (orc_quantize_row_q8_0)
 * are restated bit-exactly, including the fp32 FMA chain and glibc expf.
 */
#ifndef MOJOLLAMA_ORACLE_H
#define MOJOLLAMA_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Per-symbol semantics.  Values are shared with the GPU library's
 * mllm_sem enum so tests can pass one id to both. */
enum orc_sem {
    ORC_F32           = 0,  /* f32_matmul_omp            QK:884-913                    */
    ORC_Q4_0          = 1,  /* q4_0_matmul_omp / q4_0_batch_matmul  QK:77-95,135-154, CE:68-110 */
    ORC_Q4_1          = 2,  /* q4_1_matmul_omp           QK:97-117,160-177             */
    ORC_Q5_0_F32      = 3,  /* q5_0_row_dot (fp32 x)     QK:1239-1251                  */
    ORC_Q5_0_Q8       = 4,  /* q5_0_matmul_omp (Q8_0 x)  QK:1224-1237,1262-1336        */
    ORC_Q8_0          = 5,  /* q8_0_matmul_omp / q8_0_batch_matmul  QK:376-416, CE:216-253 */
    ORC_Q4_K_GGML     = 6,  /* q4_k_batch_matmul / q4_k_row_dot_avx2 / q4_k_dequantize_row  CE:255-313, QK:1980-2063, QK:804-828 */
    ORC_Q4_K_Q8       = 7,  /* quant_matmul_omp(12): dot_q4_k_q8_0  QK:199-209,1647-1758 */
    ORC_Q5_K_GGML     = 8,  /* q5_k_row_dot_avx2 / q5_k_dequantize_row  QK:249-364, QK:830-866 */
    ORC_Q5_K_CE       = 9,  /* q5_k_batch_matmul (CE struct layout)     CE:46-52,380-425 */
    ORC_Q6_K_GGML     = 10, /* q6_k_dequantize_row       QK:762-800                    */
    ORC_Q6_K_LOWNIB   = 11, /* quant_matmul_omp(14): q6k_dequant_8 uses ql&15 for all quadrants  QK:1778-1903 */
    ORC_Q6_K_SEQ      = 12, /* q6_k_batch_matmul (sequential element order)  CE:315-378 */
    ORC_MXFP4         = 13, /* mxfp4_matmul_omp / mxfp4_row_dot(_f32), no scale clamp  QK:502-627,683-720 */
    ORC_MXFP4_CLAMP   = 14, /* mxfp4_batch_matmul, scale clamped to 1e20  CE:427-534 */
    ORC_MXFP4_Q8      = 15, /* mxfp4_row_dot_q8 (Q8_0 x, clamped combined scale)  QK:629-678 */
    ORC_SEM_COUNT     = 16
};

/* GGUF type codes used by the reference (QK:6-14, TE:19-25). */
enum { ORC_QT_F32 = 0, ORC_QT_F16 = 1, ORC_QT_Q4_0 = 2, ORC_QT_Q4_1 = 3, ORC_QT_Q5_0 = 6, ORC_QT_Q8_0 = 8,
       ORC_QT_Q4_K = 12, ORC_QT_Q5_K = 13, ORC_QT_Q6_K = 14, ORC_QT_MXFP4 = 39 };

float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);                 /* round to nearest even */

int  orc_block_elems(int sem);                    /* 32 or 256 (1 for F32) */
int  orc_block_bytes(int sem);                    /* bytes per block (4 for F32) */
long orc_row_bytes(int sem, int n_cols);

/* Dequantise one row of n_cols elements under a fp32-activation semantic.
 * Returns 0, or -1 for a semantic that has no fp32 weight (the Q8_0-x ones). */
int  orc_dequant_row(int sem, const uint8_t *row, float *w, int n_cols);

/* quantize_row_q8_0 (QK:1406-1455), bit-exact.  Returns n_cols/32. */
int  orc_quantize_row_q8_0(const float *x, uint8_t *q8, int n_cols);

/* y[b*n_rows + r] = row r of W applied to x[b*n_cols ...] under semantic sem. */
void orc_gemv(int sem, const uint8_t *W, const float *x, float *out,
              int n_rows, int n_cols, int B);

/* Map a reference entry point + GGUF code to its semantic (-1: the
 * reference writes zeros / does nothing for that combination).
 * entry: 0 quant_matmul_omp, 1 *_batch_matmul, 2 batch_qkv/gate_up row path,
 *        3 moe_forward_omp gate/up (non-MXFP4 pair), 4 moe_forward_omp down. */
int  orc_sem_for(int entry, int qt);

/* Routing, bit-exact with moe_ffn CE:606-638 (renorm=0) and
 * router_topk GO:53-93 / qwen36_batch_forward CE:1148-1152 (renorm=1):
 * sequential fp32 FMA logits, max by strict '>', expf, sequential sum,
 * x 1/(sum+1e-10), insertion top-k with strict '>', optional renorm. */
void orc_route(const float *router_w, const float *x, int T, int N, int E, int K,
               int renorm, int *top_idx, float *top_w);

/* moe_ffn CE:591-665 for one token (B=1 call), fp32 in/out.
 * Expert e's tensors start at gate + e*gate_stride bytes etc. with the
 * strides moe_ffn derives from the quant codes (CE:593-605). */
void orc_moe_ffn_token(const float *router_w, const uint8_t *gate, const uint8_t *up,
                       const uint8_t *down, int qt_gate, int qt_up, int qt_down,
                       int N, int E, int K, int M, const float *x, float *out);

/* moe_forward_omp's Q5_0 down row stride (QK:2216, 2230: taken from n_embd)
 * where it differs from the matrix's own and stays inside the matrix, else 0. */
long orc_moe_q5_down_stride(int qt_down, int n_embd, int n_ff);

/* moe_forward_omp QK:2066-2250 for one token, caller-supplied routing.
 * gate/up/down are per-expert pointer arrays.  has_q8_scratch mirrors the
 * prealloc_q8 != NULL condition of QK:2167,2194. combine in k order. */
void orc_moe_forward_token(const uint8_t *const *gate, const uint8_t *const *up,
                           const uint8_t *const *down, const float *x, int n_ff, int n_embd,
                           int qt_gate, int qt_up, int qt_down, const int *top_idx,
                           const float *top_w, int top_k, int has_q8_scratch, float *out);

/* TE:620-666 _requantize_output: Q4_K / Q6_K rows (ggml dequantisation) to
 * Q8_0 blocks by TE's numpy rule (amax >= 1e-10, q = rint(x / (amax/127)),
 * clamp +-127, fp16 scale).  out: n_rows * (n_cols/32) * 34 bytes.  -1 for
 * other types. */
int orc_requant_q8_0(int qt, const uint8_t *W, int n_rows, int n_cols, uint8_t *out);

/* moe_ffn's expert strides (CE:593-605). */
long orc_moe_ffn_stride(int which, int qt, int N, int M);

/* Decode attention of one query token over seq_len cached positions.
 * q [nh][hd]; row s of kv head j at k + s*row_stride + j*hd (likewise v);
 * query head h reads kv head h / (nh/nkh); out [nh][hd].
 * mode ORC_ATTN_CE     : CE:141-158 gqa: scores dot*(1/sqrtf(hd)), max from
 *                        -1e30 by strict '>', expf(s - max), 1/sum.
 * mode ORC_ATTN_GQA_C  : gqa_attention.c:93 gqa_attention_decode: the same
 *                        scores; softmax_simd (gqa_attention.c:50-88): the
 *                        first floor(seq_len/8)*8 weights by exp_ps_simd on
 *                        (s - max) clamped to [-80, 80], the rest expf
 *                        capped at 1e38, 1/(sum + 1e-10).
 * Scores: one fp32 FMA chain per dot in element order, times the scale;
 * the weighted V sum accumulates in double. */
enum { ORC_ATTN_CE = 0, ORC_ATTN_GQA_C = 1 };
void orc_gqa_decode(int mode, const float *q, const float *k, const float *v, long row_stride, int seq_len,
                    int nh, int nkh, int hd, float *out);
/* exp_ps_simd (gqa_attention.c:32-48) on one value, as written. */
float orc_exp_ps_simd(float x);
/* rope_apply (GO:37-51): pairs (j, j + rope_dim/2) of each head rotated by
 * cos/sin rows [pos][rope_dim/2]. */
void orc_rope(float *buf, int nh, int hd, int pos, const float *cos_t, const float *sin_t, int rope_dim);

/* gptoss_forward (GO:96-189), one token, the reference's steps in order:
 * x = emb[token]; per layer l: res = x; xn = (x / rms) * wAN[l] (rms_norm,
 * GO:29-34); q, k, v = MXFP4 GEMVs (mxfp4_matmul_omp) of xn; RoPE on q and
 * k at pos; K/V row kv_len[l] of layer l's cache := k, v and kv_len[l]++;
 * att = gqa_attention_decode over kv_len[l] rows; x = res + Wo att; xn =
 * rms_norm(x, wFN[l]); router_topk (GO:53-93: fp32 chain, softmax, top-k,
 * renormalise); ffn = moe_forward_omp(w_*_exps + l, ...) -- expert e of
 * layer l is the matrix at w_*_exps[l + e], as GO:179-181 index it; x =
 * res + ffn (the attention output is not carried, GO:186).  Finally logits
 * = MXFP4 GEMV of the last xn (GO:189: no output norm).  Caches are
 * [L][max_ctx][nkh * hd]. */
typedef struct {
    int L, N, NH, NKH, HD, V, E, K, M, max_ctx, rope_dim, outNR;
    float eps;
    const float *emb;
    const uint8_t *const *wQ, *const *wK, *const *wV, *const *wO;
    const float *const *wAN, *const *wFN;
    const uint8_t *wOut;
    const float *const *w_gate_inp;
    const uint8_t *const *w_gate_exps, *const *w_up_exps, *const *w_down_exps;
    int qt_gate, qt_up, qt_down;
    const float *cos_t, *sin_t;
} orc_gptoss;
void orc_gptoss_forward(const orc_gptoss *m, int token, int pos, float *k_cache, float *v_cache, int *kv_len,
                        float *logits);

#ifdef __cplusplus
}
#endif
#endif
