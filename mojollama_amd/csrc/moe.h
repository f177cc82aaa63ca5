// moe.h — internal entry points of moe.hip used by the C ABI (capi.hip).
#pragma once
#include "mllm.h"
#include "mllm_common.h"

// A MoE layer over the given semantics and per-expert packed views (device
// array of 3*E: gate, up, down), routing from a router already in the routing
// layout; both arrays stay the caller's and must outlive the layer's use.
// clamp = 0 gives moe_ffn's unclamped SiLU; gemv_only (mllm_moe_needs_gemv
// of the same table) keeps every T on the per-token GEMV path.  Released with
// mllm_moe_release, which frees neither array; creating one allocates nothing
// on the device.
mllm_moe_layer *mllm_moe_layer_from_views(int sem_g, int sem_u, int sem_d, int N, int M, int E, int K,
                                          const mllm_packed *tab_dev, const float *router_p, int renorm, int clamp,
                                          int gemv_only);

// Whether the grouped GEMMs would depart from the reference on these weights
// (1) or not (0); -1 on a HIP error.  They fold block scales into bf16
// weights, so a non-finite scale meets zero activation planes (inf * 0 = NaN
// where the reference's per-element product is +-inf); and an MXFP4 down
// projection with Q8_0 activations whose exponent reaches 178 can meet the
// reference's +-1e20 clamp of 2^(E-127) * d8 (QK:648-650), which the GEMMs do
// not apply.  Such layers run on the per-token GEMV path.  Synchronous (a
// setup-time scan of the block scales).
int mllm_moe_needs_gemv(const mllm_packed *tab_dev, int sem_g, int sem_u, int sem_d, int N, int M, int E);

// Whether the grouped-GEMM (T > 24) path serves these semantics.
bool mllm_moe_batched_supported(int sem_g, int sem_u, int sem_d);

// Record an error for mllm_last_error() (logged once to stderr).
void mllm_set_error(const char *msg);

// Frees the models and KV mirrors gptoss_forward keeps (part of mllm_cache_clear).
void mllm_gptoss_cache_clear();

// mllm_moe_forward with the routing supplied (device idx / w [T][K], e.g.
// computed by a caller's own router): moe_forward_omp's contract (QK:2066).
int mllm_moe_forward_routed(const mllm_moe_layer *L, const float *x, int T, float *out, void *workspace,
                            long ws_bytes, const int *idx, const float *w, hipStream_t st);

// A layer for routed forwards over the expert types of moe_forward_omp (GGUF
// codes, QK:2094-2245) and the device table tab_dev ([E] gate, [E] up, [E]
// down packed views; the caller's, kept alive while the layer is used).  No
// router: only mllm_moe_forward_routed serves it.  nullptr for gate/up types
// the reference's expert path does not compute; synchronous (scans the block
// scales).  Released with mllm_moe_release.
mllm_moe_layer *mllm_moe_layer_for_codes(int qt_gate, int qt_up, int qt_down, int N, int M, int E, int K,
                                         const mllm_packed *tab_dev);

// The semantics a layer gives the codes (gate, up; down: -2 for the
// reference's Q4_K zeros, -1 unknown).
void mllm_moe_codes_sems(int qt_gate, int qt_up, int qt_down, int *sem_g, int *sem_u, int *sem_d);
