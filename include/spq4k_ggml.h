/* spq4k_ggml.h — ggml graph nodes that run quantised matmuls through spq4k.
 *
 * The engine adapter for the reference's graph builders: a Q4_K (or Q5_K,
 * Q6_K or Q8_0, the types a Q4_K model stores some tensors in) weight's
 * GGML_OP_MUL_MAT / GGML_OP_MUL_MAT_ID node is replaced by a ggml custom op
 * (ggml_custom_4d, ggml.h:2610-2623) whose callback runs the product on the
 * GPU through spq4k. This is the custom-op pattern the engine already uses for
 * its fp32 CRT matmul (sp_crt_mul_mat, desktop/engine/src/forward.cpp:1266-1281,
 * whose Q4_K branch is the TODO at :1270-1273) and for BURN_MOE
 * (burn_moe_op.cpp:377-430): the callback works on ith == 0 only
 * (forward.cpp:1248, burn_moe_op.cpp:203) and moves tensors with
 * ggml_backend_tensor_get / _set, or through tensor->data for tensors that
 * live in a plain ggml context.
 *
 * Weights are uploaded to the GPU the first time a weight tensor is seen and
 * stay resident (keyed by tensor, data pointer, byte count, type and shape)
 * until spq4k_ggml_forget or spq4k_ggml_free; activations and outputs cross
 * PCIe per node. Tensors that live in a device (non-host) backend buffer --
 * a HIP build of ggml on the same GPU -- are used in place instead: the
 * weight is adopted without a copy and a node whose activations, ids and
 * output are all device-resident moves nothing over PCIe. Built against the
 * host engine's ggml.h.
 */
#ifndef SPQ4K_GGML_H
#define SPQ4K_GGML_H

#include "ggml.h"
#include "spq4k.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct spq4k_ggml spq4k_ggml;

/* Create a binding on `device` (an spq4k context plus the resident-weight
 * table). Returns 0 or a negative errno (spq4k_init's codes). */
int spq4k_ggml_init(int device, spq4k_ggml **out);
void spq4k_ggml_free(spq4k_ggml *b);

/* GGML_OP_MUL_MAT (ggml_mul_mat, ggml.h:1414-1420) for a Q4_K, Q5_K, Q6_K or
 * Q8_0 weight: W [K, M], x [K, T] f32 contiguous (ne2 = ne3 = 1) -> [M, T] f32.
 * Returns NULL (build ggml's own node instead) for any other type or shape. */
struct ggml_tensor *spq4k_ggml_mul_mat(struct ggml_context *ctx, struct ggml_tensor *W, struct ggml_tensor *x,
                                       spq4k_ggml *b);

/* GGML_OP_MUL_MAT_ID (ggml_mul_mat_id, ggml.h:1434-1438) for an expert bank
 * of one of those types: as [K, M, E], x [K, ne11, T] f32 (ne11 = 1 or n_used), ids
 * [n_used, T] i32 -> [M, n_used, T] f32. */
struct ggml_tensor *spq4k_ggml_mul_mat_id(struct ggml_context *ctx, struct ggml_tensor *as, struct ggml_tensor *x,
                                          struct ggml_tensor *ids, spq4k_ggml *b);

/* The routed-expert FFN block of a MoE layer as one node, in place of the
 * reference's BURN_MOE custom op (sp_build_burn_moe_op,
 * desktop/engine/src/burn_moe_op.cpp:377-430, same sources in the same
 * order: cur [n_embd, T] f32, selected [k, T] i32, weights [1, k, T] f32,
 * gate_exps / up_exps [n_embd, n_ff, E], down_exps [n_ff, n_embd, E]) with the
 * arithmetic of the stock graph it replaces (forward.cpp:1098-1117): runs
 * spq4k_moe_ffn on the GPU -> [n_embd, T] f32. All experts resident on the
 * GPU (the op's CPU-side sub-bank split, pivot > 0, is not taken). Returns
 * NULL (build the stock graph instead) for other types or shapes. */
struct ggml_tensor *spq4k_ggml_moe_ffn(struct ggml_context *ctx, struct ggml_tensor *cur, struct ggml_tensor *selected,
                                       struct ggml_tensor *weights, struct ggml_tensor *gate_exps,
                                       struct ggml_tensor *up_exps, struct ggml_tensor *down_exps, spq4k_ggml *b);

/* Drop the resident GPU copy of weight tensor W (every copy when W is NULL),
 * e.g. before its ggml context is freed or its model reloaded; a later node
 * on W uploads it again. Returns the number of copies freed. */
int spq4k_ggml_forget(spq4k_ggml *b, const struct ggml_tensor *W);

/* The device address of the binding's resident copy of W (NULL when W has
 * none yet). For a W that lives in a device buffer it is W->data itself: the
 * binding adopted it in place. */
const void *spq4k_ggml_resident_data(const spq4k_ggml *b, const struct ggml_tensor *W);

/* Custom-op callbacks return nothing: the first failure is kept here (0 when
 * every node succeeded) and the failed node's output is filled with NaN. */
int spq4k_ggml_status(const spq4k_ggml *b);
const char *spq4k_ggml_last_error(const spq4k_ggml *b);

#ifdef __cplusplus
}
#endif

#endif /* SPQ4K_GGML_H */
