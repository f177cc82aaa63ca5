/* mllm.h — C ABI of libmllm_gpu.so, the MI355X (gfx950) implementation of
 * a730/MojoLlama's quantised-matmul + MoE-FFN hot path.
 *
 * Part 1 declares drop-in replacements for the reference engine's exported
 * symbols, with identical names, argument lists and meaning, so a caller that
 * binds them through ctypes (turbo_engine_v7_moe.py, "TE") can load this
 * library in place of its combined_engine.so.  Weights and activations are
 * host pointers as in the reference; results are in the caller's buffers when
 * the call returns.  Reference files:
 *   QK = src/mojollama/kernels/quant_kernels_omp.c
 *   CE = src/mojollama/kernels/cengine_batch_instr.c
 *   TE = src/mojollama/kernels/turbo_engine_v7_moe.py
 *
 * Part 2 declares device-pointer entry points (mllm_*) that take inputs already
 * resident in HBM and queue work on a caller stream (hipStream_t passed as
 * void*; NULL = the default stream).
 *
 * Errors: no entry point aborts.  A failure is logged once to stderr and kept
 * for mllm_last_error(); drop-in calls leave the output untouched on an
 * unknown quant code (as the reference's dispatch does, QK:1385-1386);
 * mllm_* calls return -1.
 */
#ifndef MLLM_H
#define MLLM_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLLM_API __attribute__((visibility("default")))

/* ------------------------------------------------------------ Part 1: drop-in */

/* QK:1355-1388 quant_matmul_omp — out[n_rows] = W x for one token.  quant_type is
 * the GGUF code: 0 F32, 2 Q4_0, 3 Q4_1, 6 Q5_0, 8 Q8_0, 12 Q4_K, 13 Q5_K,
 * 14 Q6_K, 39 MXFP4; bound by TE:251-252. */
MLLM_API void quant_matmul_omp(const uint8_t *W, const float *x, float *out, int n_rows, int n_cols, int quant_type);

/* QK:884-913 f32_matmul_omp; bound by TE:253-254. */
MLLM_API void f32_matmul_omp(const float *W, const float *x, float *out, int n_rows, int n_cols);

/* CE:68,216,256,316,381,435 — B-batched GEMV, out[b*n_rows + r]. */
MLLM_API void q4_0_batch_matmul(const uint8_t *W, const float *x, float *out, int n_rows, int nc, int B);
MLLM_API void q8_0_batch_matmul(const uint8_t *W, const float *x, float *out, int n_rows, int nc, int B);
MLLM_API void q4_k_batch_matmul(const uint8_t *W, const float *x, float *out, int n_rows, int nc, int B);
MLLM_API void q6_k_batch_matmul(const uint8_t *W, const float *x, float *out, int n_rows, int nc, int B);
MLLM_API void q5_k_batch_matmul(const uint8_t *W, const float *x, float *out, int n_rows, int nc, int B);
MLLM_API void mxfp4_batch_matmul(const uint8_t *W, const float *x, float *out, int n_rows, int nc, int B);

/* QK:1139-1183 batch_qkv_omp and QK:1186-1222 batch_gate_up_omp (TE:255-258). */
MLLM_API void batch_qkv_omp(const uint8_t *Wq, const uint8_t *Wk, const uint8_t *Wv, const float *x, float *out_q,
                            float *out_k, float *out_v, int nq, int nk, int nv, int n_cols, int qtype_q, int qtype_k,
                            int qtype_v);
MLLM_API void batch_gate_up_omp(const uint8_t *Wg, const uint8_t *Wu, const float *x, float *out_gate, float *out_up,
                                int ng, int nu, int n_cols, int qtype_g, int qtype_u);

/* QK:1406-1455 quantize_row_q8_0 — bit-exact; returns n_cols/32. */
MLLM_API int quantize_row_q8_0(const float *x, uint8_t *q8, int n_cols);

/* QK:762-878 *_dequantize_row (TE:389-392 binds the Q6_K/Q4_K ones). */
MLLM_API void q4_k_dequantize_row(const uint8_t *W, float *out, int n_values);
MLLM_API void q5_k_dequantize_row(const uint8_t *W, float *out, int n_values);
MLLM_API void q6_k_dequantize_row(const uint8_t *W, float *out, int n_values);
MLLM_API void q8_0_dequantize_row(const uint8_t *W, float *out, int n_values);

/* QK:2066-2250 moe_forward_omp (TE:363-377, called at TE:2067).  Combine order
 * is k order (the reference's OpenMP atomic has no fixed order); prealloc_buf
 * is not written; an MXFP4 down projection with prealloc_q8 == NULL yields a
 * zero down term and an error (the reference dereferences NULL there). */
MLLM_API void moe_forward_omp(const uint8_t **gate_raw, const uint8_t **up_raw, const uint8_t **down_raw,
                              const float *x_norm, int n_ff_expert, int n_embd, int qt_gate, int qt_up, int qt_down,
                              const int *top_indices, const float *top_weights, int top_k, float *combined,
                              float *prealloc_buf, uint8_t *prealloc_q8);

/* CE:591-665 moe_ffn — `c` is the engine's BC struct (CE:536-589); fields read:
 * N, n_experts, n_experts_per_tok, moe_intermediate, w_gate_inp, w_gate_exps,
 * w_up_exps, w_down_exps, gate/up/down_exp_quant.  Writes N floats to ffn_buf
 * (the last token's result when B > 1, as in the reference); gate_buf/up_buf
 * are not used as scratch. */
MLLM_API void moe_ffn(const void *c, int l, float *x, float *gate_buf, float *up_buf, float *ffn_buf, int B);

/* moe_ffn (CE:591-665) for each of B tokens, keeping every token's result:
 * ffn_out[b*N + n] (moe_ffn itself keeps only the last token's, CE:610-643).
 * No reference counterpart: the batched form of moe_ffn for prefill-sized B.
 * B > 8 tokens run the MoE layer (grouped GEMMs above 24 tokens) with
 * moe_ffn's semantics: quant_matmul_omp per projection, unclamped SiLU, the
 * un-renormalised top-K routing, k-order combine. */
MLLM_API void moe_ffn_batched(const void *c, int l, const float *x, float *ffn_out, int B);

/* TE:515-522, 620-666 (_requantize_output): the caller's load-time conversion
 * of a Q4_K / Q6_K / F16 lm_head to Q8_0, done in numpy there and on the GPU
 * here: each row dequantised as q4_k/q6_k_dequantize_row (QK:762-828), or for
 * F16 (quant_type 1) converted as TE:643-645 does, which takes each 16-bit
 * pattern's integer value (0x3C00 -> 15360.0f) rather than its fp16 value;
 * then per 32 elements amax = max(max|x|, 1e-10), d = amax/127, q = rint(x/d)
 * clamped to +-127, d stored as fp16 -- bit-exact with TE's result.  Host
 * pointers: W is the raw GGUF matrix, out receives n_rows * (n_cols/32) * 34
 * bytes.  Returns 0, or -1 for another type (TE's Q5_K branch raises) or an
 * F16 row length that is not a multiple of 32 (TE's reshape raises).  No
 * counterpart symbol in the reference's C library: the routine TE would call
 * in place of its loop. */
MLLM_API int requantize_output_q8_0(const uint8_t *W, int n_rows, int n_cols, int quant_type, uint8_t *out);

/* gqa_attention.c:93 gqa_attention_decode: decode attention of one token.
 * q [n_head][head_dim]; k_cache / v_cache [seq_len][n_kv_head][head_dim];
 * query head h reads KV head h / (n_head / n_kv_head); out [n_head][head_dim].
 * Scores (q . k) / sqrtf(head_dim); softmax_simd (gqa_attention.c:50-88):
 * maximum from -1e30, the first floor(seq_len/8)*8 weights by the source's
 * exp_ps_simd polynomial on (s - max) clamped to [-80, 80], the rest expf
 * capped at 1e38, normalised by 1 / (sum + 1e-10).  workspace is not written
 * (the reference keeps its weights there; nothing reads them back).  Host
 * pointers: q, K and V are uploaded on every call, so the device entry
 * mllm_gqa_decode is the fast path.  seq_len <= 0 gives zeros.  Served for
 * n_head % n_kv_head == 0, n_head / n_kv_head <= 16, head_dim <= 256 and a
 * multiple of 4; other shapes leave out untouched with an error. */
MLLM_API void gqa_attention_decode(const float *q, const float *k_cache, const float *v_cache, float *out, int seq_len,
                                   int n_head, int n_kv_head, int head_dim, float *workspace);

/* gptoss_forward (GO:96-189): one decode token of gpt-oss through all
 * layers, the reference's steps in its order (see mllm_gptoss_step), on the
 * reference's host buffers: logits[outNR] written, K/V row kv_len[l] of each
 * layer written into k_cache / v_cache ([L][max_ctx][NKH*HD]) and kv_len[l]
 * incremented.  Weights are packed on the device on first use (cached by
 * their pointers and a sampled fingerprint); the caches are mirrored on the
 * device and only rows the mirror lacks (or rewritten rows) are uploaded.
 * Q/K/V/O and the output projection are MXFP4 whatever *_quant says (GO
 * calls mxfp4_matmul_omp for all of them); expert e of layer l is
 * w_*_exps[l + e] (GO:179-181), so those arrays need L - 1 + n_experts
 * entries.  workspace, moe_prealloc_* and gqa_ws are not written.  Refused
 * (error, outputs untouched) when kv_len[l] >= max_ctx (the reference writes
 * past its cache) or nQ/nK/nV/nO disagree with NH, NKH, HD, N. */
MLLM_API void gptoss_forward(const int *token, int pos, const float *emb, int V, const uint8_t **wQ,
                             const uint8_t **wK, const uint8_t **wV, const uint8_t **wO, const float **wAN,
                             const float **wFN, const int *nQ, const int *nK, const int *nV, const int *nO,
                             const int *q_quant, const int *k_quant, const int *v_quant, const int *o_quant,
                             const uint8_t *wOut, int outNR, int outNC, int outQuant, float *k_cache, float *v_cache,
                             int *kv_len, const float *cos_table, const float *sin_table, int max_ctx, int rope_dim,
                             float *workspace, int ws_size, int L, int N, int NH, int NKH, int HD, int FF, float eps,
                             int n_experts, int n_experts_per_tok, int moe_intermediate, const float **w_gate_inp,
                             const uint8_t **w_gate_exps, const uint8_t **w_up_exps, const uint8_t **w_down_exps,
                             int gate_exp_quant, int up_exp_quant, int down_exp_quant, float *logits,
                             float *moe_prealloc_buf, uint8_t *moe_prealloc_q8, float *gqa_ws);

/* QK:1029-1030: accepted and ignored / number of compute units. */
MLLM_API void set_num_threads(int n);
MLLM_API int get_max_threads(void);

/* The Qwen3.6 hybrid drivers TE binds (TE:263-311, 397-408).
 *
 * ssm_decode_step (CE:736-802): per token, the conv'd input split into gate
 * and SSM halves, ssm_intermediate[b] = silu(gate) * ssm_in; the per-group
 * state updated once per token in order (h = exp(A dt) h + [s == 0] (beta.x)
 * dt, dt = softplus(dt_bias + alpha.x)).  The intermediate does not read the
 * state (the reference's own arithmetic).  2*inner <= 8192.
 *
 * ssm_layer_fused (CE:803-849): ssm_decode_step into `output` (as scratch of
 * B*inner floats), then per token b: interm *= gate_raw.x_b, output[b*N..] =
 * residual_b + ssm_out_raw.interm (quant_matmul_omp semantics); output holds
 * max(B*N, B*inner) floats and its aliasing is reproduced in order.  Gate
 * gate_nr >= inner rows of N columns (<= 8192), ssm_out N x inner.
 *
 * qwen36_batch_forward (CE:859-1231): B tokens through L SSM / attention
 * layers with MoE FFNs and shared experts, then the output head, every
 * matmul with quant_matmul_omp semantics; logits [B][out_nr_final].  The
 * caller's state is read and written as the reference does: the SSM state
 * (per layer at l * groups * state_size), row kv_lens[l] of each attention
 * layer's caches ([L][max_ctx][n_kv_h*HD]; kv_lens not incremented), and the
 * fused-QKV slice of ws (ws + 3*B*S, S from CE:906-913), where V is read at
 * offset NH*HD + N (CE:1002-1009).  The other workspace slices are not
 * written.  The device keeps mirrors of the KV caches: rows below kv_lens
 * that the caller changes between calls must be followed by
 * mllm_cache_clear() (a changed sample of rows is detected, not every row).
 * fp32 routers (code 0) are summed in f32_matmul_omp's order, so top-K
 * selection matches the reference on its own logits.  Refused (error,
 * outputs untouched): kv_lens[l] outside [0, max_ctx), QKV rows fewer than
 * NH*HD + n_kv_h*HD, shapes that are not N x inner / inner x N, 2*ssm_inner >
 * 8192, more than 256 experts or top_k > 16, emb_quant other than 0 / 12, an
 * MXFP4 down projection with q8_ws == NULL (the reference dereferences it). */
MLLM_API void ssm_decode_step(const float *x, float *ssm_intermediate, const float *conv1d_w, const float *a_param,
                              const float *dt_bias, const float *alpha, const float *beta, const float *ssm_norm_w,
                              float *state, int B, int N, int inner, int groups, int state_size, int conv_kernel,
                              int dt_rank);
MLLM_API void ssm_layer_fused(const float *x, float *residual, float *output, const float *conv1d_w,
                              const float *a_param, const float *dt_bias, const float *alpha, const float *beta,
                              const float *ssm_norm_w, float *state, const uint8_t *gate_raw, int gate_nr, int gate_nc,
                              int gate_qt, const uint8_t *ssm_out_raw, int ssm_out_nr, int ssm_out_nc, int ssm_out_qt,
                              int B, int N, int inner, int groups, int state_size, int conv_kernel, int dt_rank);
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
    const float *sin_table, float *ws, uint8_t *q8_ws);

MLLM_API const char *mllm_last_error(void);
MLLM_API void mllm_cache_clear(void);

/* ------------------------------------------------------ Part 2: device pointers */

/* Semantic ids (mllm_sem in mojollama_amd/csrc/mllm_common.h) for a reference
 * entry point: 0 quant_matmul_omp, 1 *_batch_matmul, 2 batch_qkv/gate_up rows,
 * 3 moe_forward_omp gate/up, 4 moe_forward_omp down.  -1: reference no-op. */
MLLM_API int mllm_sem_for(int entry, int quant_type);

/* Byte sizes of a raw GGUF matrix and of its packed device layout. */
MLLM_API long mllm_raw_size(int sem, int n_rows, int n_cols);
MLLM_API long mllm_packed_size(int sem, int n_rows, int n_cols);

/* Repack raw GGUF blocks (device) into the packed layout (256-byte aligned). */
MLLM_API int mllm_pack(int sem, const void *raw_dev, void *packed_dev, int n_rows, int n_cols, void *stream);

/* out[b][r] = row r of W applied to x[b], b < B (any B), under semantic `sem`.
 * Q8_0-activation semantics, and B > 8 (run as an MFMA GEMM over split bf16
 * activation planes), need `workspace` of mllm_gemv_workspace_size bytes.
 * At 2 <= B <= 8 the Q4_K, Q6_K, Q8_0, Q4_0 and MXFP4 batch semantics run on
 * the matrix cores from the batch where that is faster; given the workspace,
 * short matrices there also split K over more workgroups (optional: NULL
 * runs unsplit or on the vector kernel). */
MLLM_API long mllm_gemv_workspace_size(int sem, int n_rows, int n_cols, int B);
MLLM_API int mllm_gemv(int sem, const void *packed_dev, const float *x_dev, float *out_dev, int n_rows, int n_cols,
                       int B, void *workspace, void *stream);

/* The decode GEMV with the work around it fused in (the RMSNorm before the
 * QKV and gate/up projections, TE:1516,1641 / GO:29-34, the residual adds
 * after the output and down projections, TE:1628-1651, the SiLU product
 * before the down projection).  Every field may be NULL / 0:
 *   x_up:     activation = silu(x) * x_up (silu_clamp: gate clamped to +-80,
 *             moe_forward_omp QK:2157-2164; else plain silu);
 *   x_res:    activation v = x + x_res;
 *   res_out:  v is written here (the new residual stream; must not overlap x
 *             or x_res);
 *   rms_w:    activation = RMSNorm(v) * rms_w over n_cols, rms_div 0:
 *             v * (1/sqrtf(mean(v^2) + eps)) (simd_ops rms_norm), 1:
 *             v / sqrtf(mean(v^2) + eps) (gptoss_batch_forward.c rms_norm);
 *   out_add:  out = out_add + W * activation (may equal out).
 * x_up excludes x_res/res_out/rms_w and silu_pair.  Shapes the decode kernel
 * can stage at once (B <= 8; paired rows at B == 1) run as one launch; others
 * form the activation in the workspace first and the SiLU product after the
 * GEMV (mllm_gemv_fused_workspace_size bytes). */
typedef struct {
    const float *x_up;
    int silu_clamp;
    const float *x_res;
    float *res_out;
    const float *rms_w;
    float rms_eps;
    int rms_div;
    const float *out_add;
    int x_ld;             /* token stride of x, x_up, x_res and res_out (0: n_cols) */
    int silu_pair;        /* the matrix holds 2*n_rows rows, gate rows then up rows (a stacked
                             gate/up pair): out[r] = silu(gate_r . v) * (up_r . v), silu_clamp as above */
} mllm_gemv_fusion;
MLLM_API long mllm_gemv_fused_workspace_size(int sem, int n_rows, int n_cols, int B, const mllm_gemv_fusion *f);
MLLM_API int mllm_gemv_fused(int sem, const void *packed_dev, const float *x_dev, float *out_dev, int n_rows,
                             int n_cols, int B, const mllm_gemv_fusion *f, void *workspace, void *stream);

/* requantize_output_q8_0 on device data: raw_dev (raw GGUF Q4_K / Q6_K, or
 * F16 patterns) -> q8_dev (raw Q8_0 blocks); workspace of
 * mllm_requantize_workspace_size bytes. */
MLLM_API long mllm_requantize_workspace_size(int quant_type, int n_rows, int n_cols);
MLLM_API int mllm_requantize_q8_0(int quant_type, const void *raw_dev, int n_rows, int n_cols, void *q8_dev,
                                  void *workspace, void *stream);

/* A plain streaming read of `bytes` (a multiple of 16) at a 16-byte aligned
 * device address, every word read once: the bandwidth ceiling a kernel that
 * reads the same bytes in one launch is measured against.  sink: 16 bytes of
 * device memory (written only if the data xor to a fixed pattern). */
MLLM_API int mllm_read_probe(const void *dev, long bytes, void *sink, void *stream);

/* quantize_row_q8_0 over T rows. */
MLLM_API int mllm_quantize_q8_0(const float *x_dev, int T, int n_cols, uint8_t *q8_dev, void *stream);

/* Routing layout of an fp32 router [E][N] (row e = expert e's weights, as the
 * reference's w_gate_inp): element (i, e) at ((i/4)*E + e)*4 + i%4, rows from N
 * up to a multiple of 32 zero; mllm_router_packed_size bytes. */
MLLM_API long mllm_router_packed_size(int N, int E);
MLLM_API int mllm_router_pack(const float *router_dev, int N, int E, float *out_dev, void *stream);

/* Routing of T tokens (CE:606-638; renormalised top-K weights when `renorm`):
 * router_p in the routing layout, x [T][N] -> idx/w [T][K].  E <= 256, K <= 16.
 * `workspace` (optional, mllm_route_workspace_size bytes) lets T <= 8 tokens
 * spread over expert slices; NULL runs one workgroup per token. */
MLLM_API long mllm_route_workspace_size(int T, int E);
MLLM_API int mllm_route(const float *router_p_dev, const float *x_dev, int T, int N, int E, int K, int renorm,
                        int *idx_dev, float *w_dev, void *workspace, void *stream);

/* fp32 weights of a packed matrix (fp32-weight semantics only). */
MLLM_API int mllm_dequant(int sem, const void *packed_dev, int n_rows, int n_cols, float *out_dev, void *stream);

/* ------------------------------------------------------- MoE layer, T tokens */

/* A prepared MoE layer: per-expert packed weights (device pointers, arrays of E
 * entries on the host) with the reference's GGUF codes, and the fp32 router
 * [E][N] (device; the layer keeps its own copy in the routing layout, so the
 * caller may free it after the call).  Per token the layer computes what
 * moe_forward_omp (QK:2066-2250) computes when fed the C routing of moe_ffn
 * (CE:606-638), renormalised when `renorm` (GO:88-92): gate/up per type,
 * SiLU with the gate clamped to +-80, down per type, k-order combine.
 * T > 24 tokens run the batched path (GPU bucketing by expert, grouped MFMA
 * GEMMs); T <= 24 the decode GEMVs, one job per (token, slot). */
typedef struct mllm_moe_layer mllm_moe_layer;
MLLM_API mllm_moe_layer *mllm_moe_prepare(int qt_gate, int qt_up, int qt_down, int N, int M, int E, int K,
                                          const void *const *gate_packed, const void *const *up_packed,
                                          const void *const *down_packed, const float *router_dev, int renorm);
MLLM_API void mllm_moe_release(mllm_moe_layer *layer);
/* Load-time bf16 copies of the layer's expert matrices whose weights are exact
 * in bf16 (the MXFP4 forms: gate/up of one semantic, down), which the batched
 * path (T > 24) then copies into its tiles instead of decoding; results are
 * bit-identical.  Matrices the batched path runs on the fp16-plane GEMM
 * (mllm_moe_layer_info bits 1 / 2) are not copied: that GEMM reads the packed
 * weights and is faster.  2 bytes per weight (3.8x MXFP4), freed with the layer.
 * Returns the bytes allocated (0: nothing qualifies, or already made), -1 on
 * error; synchronises `stream`.  No reference counterpart: the memory-for-
 * speed trade of moe_forward_omp's experts (QK:2066-2250) on 288 GB HBM. */
MLLM_API long mllm_moe_dense_experts(mllm_moe_layer *layer, void *stream);
MLLM_API long mllm_moe_workspace_size(const mllm_moe_layer *layer, int T);
/* Which GEMMs the layer's batched path runs, as bits: 1 gate/up and 2 down on
 * the fp16-plane GEMM (K-quant super-blocks; MXFP4 when the matrices' E8M0
 * exponents span at most 25 binades), 4 the whole layer on the per-token
 * GEMVs (scales the GEMMs would not reproduce).  -1 for a null layer.  No
 * reference counterpart: a query for callers and tests. */
MLLM_API int mllm_moe_layer_info(const mllm_moe_layer *layer);
/* out[T][N]; idx_out/w_out (optional, device [T][K]) receive the routing. */
MLLM_API int mllm_moe_forward(const mllm_moe_layer *layer, const float *x, int T, float *out, void *workspace,
                              long ws_bytes, int *idx_out, float *w_out, void *stream);
/* mllm_moe_forward without a workspace argument and without allocating.  No
 * counterpart in the reference: for callers that cannot call hipMalloc (code
 * under HIP graph capture, tight serving loops, harnesses that forbid it).
 * The workspace is a static device array of MLLM_MOE_NOALLOC_SCRATCH_BYTES
 * that each GPU the library runs on holds until the process ends; T whose
 * workspace (mllm_moe_workspace_size) exceeds it is rejected with -1 and an
 * error (64 tokens fit at both benchmark MoE shapes).  All calls on one GPU
 * share that GPU's array: calls that overlap on one GPU (other streams, other
 * threads) race.  Same results as mllm_moe_forward. */
#define MLLM_MOE_NOALLOC_SCRATCH_BYTES (32 * 1024 * 1024)
MLLM_API int mllm_moe_forward_noalloc(const mllm_moe_layer *layer, const float *x, int T, float *out, int *idx_out,
                                      float *w_out, void *stream);
/* The stable expert bucketing on its own: entries idx[TK] over E experts ->
 * off[E+1], perm[pos] = entry, pos_of[entry] = pos (-1 for idx < 0), and
 * tiles = 3 arrays of (TK/64 + E + 1) ints (expert, begin, end) + count. */
MLLM_API int mllm_moe_bucket(const int *idx, int TK, int E, int *off, int *perm, int *pos_of, int *tiles,
                             void *stream);

/* ------------------------------------------------ decode attention, KV cache */
/* A KV cache on the device.  Rows hold n_kv_head * head_dim floats; V mirrors
 * K's layout.  Contiguous (block_tables == NULL): row s of sequence b at
 * k + b * seq_stride + s * n_kv_head * head_dim (GO:158-161).  Paged
 * (CE:160-214, PagedAttention): sequence b's logical page s / page_size maps
 * through block_tables[b * max_blocks + s / page_size] to a physical page of
 * page_size rows at k + page * page_size * n_kv_head * head_dim; CE keeps one
 * such pool per layer, K then V ([2][L][n_pages][page_size][n_kv_head *
 * head_dim], CE:164), so k / v point at the layer's K and V pools.  A row
 * whose page is unmapped (< 0) or out of range reads as zeros (the
 * reference's gather skips it, leaving stale workspace). */
typedef struct {
    float *k;
    float *v;
    long seq_stride;
    const int *block_tables;
    int max_blocks;
    int page_size;
    int n_pages;
} mllm_kv_view;

/* Decode attention of B sequences (one query token each) over their first
 * seq_lens[b] cached rows (device array, each <= max_seq).
 * mode 0: CE:141-158 gqa (expf weights, 1 / sum); mode 1: gqa_attention.c
 * (see gqa_attention_decode).  q, out [B][NH * HD]; NH % NKH == 0,
 * NH / NKH <= 16, HD <= 256 and a multiple of 4; K and V 16-byte aligned.  Three launches on `stream`; weights and partial
 * sums go to the workspace (mllm_gqa_workspace_size). */
MLLM_API long mllm_gqa_workspace_size(int B, int NH, int HD, int max_seq);
MLLM_API int mllm_gqa_decode(int mode, const float *q, const mllm_kv_view *kv, const int *seq_lens, int max_seq, int B,
                             int NH, int NKH, int HD, float *out, void *workspace, long ws_bytes, void *stream);
/* Row pos[b] (device array) of sequence b := k_new[b], v_new[b] [NKH * HD]
 * (the KV store of CE:1363-1381 and GO:158-161); a row whose page is unmapped
 * is skipped. */
MLLM_API int mllm_kv_append(const mllm_kv_view *kv, const int *pos, const float *k_new, const float *v_new, int B,
                            int NKH, int HD, void *stream);
/* rope_apply (GO:37-51): in place on buf [T][NH * HD]; for each head the pairs
 * (j, j + r/2), r = rope_dim (HD when <= 0), rotated by cos_t / sin_t rows
 * [pos[t]][r/2] (pos a device array). */
MLLM_API int mllm_rope(float *buf, int T, int NH, int HD, const int *pos, const float *cos_t, const float *sin_t,
                       int rope_dim, void *stream);

/* gptoss_forward's model on the device.  Host pointers to the raw GGUF
 * weights (MXFP4 Q/K/V/O/output, fp32 norms and routers, experts of the given
 * types indexed [l + e] as GO:179-181); create uploads and packs them (the
 * Q/K/V rows of a layer stacked into one matrix) and builds one MoE layer per
 * layer (mllm_moe_prepare, renormalised routing). */
typedef struct {
    int L, N, NH, NKH, HD, E, K, M, max_ctx, rope_dim, outNR;
    float eps;
    const uint8_t *const *wQ, *const *wK, *const *wV, *const *wO;
    const float *const *wAN, *const *wFN;
    const uint8_t *wOut;
    const float *const *w_gate_inp;
    const uint8_t *const *w_gate_exps, *const *w_up_exps, *const *w_down_exps;
    int qt_gate, qt_up, qt_down;
    const float *cos_t, *sin_t;        /* [max_ctx][rope_dim / 2] */
} mllm_gptoss_desc;
typedef struct mllm_gptoss mllm_gptoss;
MLLM_API mllm_gptoss *mllm_gptoss_create(const mllm_gptoss_desc *desc);
MLLM_API void mllm_gptoss_release(mllm_gptoss *m);
/* Floats of one of the step's K / V caches: L * max_ctx * NKH * HD. */
MLLM_API long mllm_gptoss_kv_floats(const mllm_gptoss *m);
/* One token, device pointers only, no host synchronisation (14 launches per
 * layer; capturable): x_emb the token's embedding row [N], pos the RoPE
 * position [1], kv_len [L] (read, then incremented), caches [L][max_ctx][NKH *
 * HD], logits [outNR]. */
MLLM_API int mllm_gptoss_step(mllm_gptoss *m, const float *x_emb, const int *pos, int *kv_len, float *k_cache,
                              float *v_cache, float *logits, void *stream);

/* The page table of CE:160-201 (host side): a free list that hands out
 * pages 0, 1, 2, ... in order, returned pages reused last-in first-out, and
 * a logical -> physical map of MLLM_PAGE_TABLE_BLOCKS entries (MAX_BLOCKS,
 * CE:23), -1 when unmapped.  Upload mllm_page_table_entries to the device as
 * a sequence's block table. */
#define MLLM_PAGE_TABLE_BLOCKS 1024
typedef struct mllm_page_table mllm_page_table;
MLLM_API mllm_page_table *mllm_page_table_create(int max_pages, int page_size);
MLLM_API void mllm_page_table_destroy(mllm_page_table *pt);
MLLM_API int mllm_page_table_alloc(mllm_page_table *pt);
MLLM_API void mllm_page_table_free(mllm_page_table *pt, int page_id);
MLLM_API void mllm_page_table_map(mllm_page_table *pt, int logical_page, int physical_page);
MLLM_API int mllm_page_table_lookup(const mllm_page_table *pt, int logical_page);
MLLM_API const int *mllm_page_table_entries(const mllm_page_table *pt);

#ifdef __cplusplus
}
#endif
#endif
