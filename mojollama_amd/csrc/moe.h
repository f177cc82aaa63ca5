// moe.h — internal entry points of moe.hip used by the C ABI (capi.hip).
#pragma once
#include "mllm.h"
#include "mllm_common.h"

// A MoE layer over the given semantics and per-expert packed views (device
// array of 3*E: gate, up, down), routing from a router already in the routing
// layout; both arrays stay the caller's and must outlive the layer's use.
// clamp = 0 gives moe_ffn's unclamped SiLU.  Released with mllm_moe_release,
// which frees neither array; creating one allocates nothing on the device.
mllm_moe_layer *mllm_moe_layer_from_views(int sem_g, int sem_u, int sem_d, int N, int M, int E, int K,
                                          const mllm_packed *tab_dev, const float *router_p, int renorm, int clamp);

// Whether the grouped-GEMM (T > 24) path serves these semantics.
bool mllm_moe_batched_supported(int sem_g, int sem_u, int sem_d);

// Record an error for mllm_last_error() (logged once to stderr).
void mllm_set_error(const char *msg);
