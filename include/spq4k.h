/*
 * spq4k.h — C ABI of the MI355X (gfx950) Q4_K dequant-matvec library.
 *
 * The library computes what the reference's ggml CPU backend computes for
 * GGML_TYPE_Q4_K weights (vendored ggml in nihilistau/shannon-prime-burnhard,
 * paths below relative to vendor/ggml/): activations are quantised to Q8_K
 * exactly as quantize_row_q8_K does, integer sub-block sums are exact, and
 * outputs agree with ggml_vec_dot_q4_K_q8_K to fp32 summation order.
 * GGML_TYPE_Q6_K and GGML_TYPE_Q5_K weights (the sibling K-quants that Q4_K
 * models carry for some tensors) take the same Q8_K activations and go
 * through the same entry points once uploaded with their type
 * (spq4k_weights_upload_type); their outputs agree with
 * ggml_vec_dot_q6_K_q8_K / ggml_vec_dot_q5_K_q8_K the same way.
 * GGML_TYPE_Q8_0 weights (32-value blocks; K a multiple of 32) take Q8_0
 * activations made as the CPU backend's quantize_row_q8_0 makes them, and
 * agree with ggml_vec_dot_q8_0_q8_0 the same way.
 *
 * Conventions
 *   - Every function returns 0 on success or a negative errno value:
 *     -EINVAL (bad argument: K not a multiple of 256, null or misaligned
 *     pointer, T out of range), -ENOMEM (device allocation failed),
 *     -ENODEV (no such HIP device), -EIO (a HIP runtime call failed;
 *     spq4k_last_error() has the message), -EBUSY (the call would have to
 *     grow its scratch while its stream is being captured; spq4k_reserve).
 *     This follows the reference's burnhard_residue_matmul.h:39-56
 *     (0 / -EINVAL / -ENOMEM).
 *   - Plain pointers are DEVICE pointers and the call only enqueues work on
 *     the context's stream (like a ggml backend's compute); *_host variants
 *     take host pointers, copy in and out, and return when the result is in
 *     host memory.
 *   - A context is single-writer: calls on one context must not overlap from
 *     several threads (the reference's sp_crt_dispatch.h:30-33 contract).
 *     Work on one context is ordered by its stream.
 *   - Layouts are ggml's: a Q4_K weight matrix with ne[0] = K (inputs) and
 *     ne[1] = M (outputs) is M rows of K/256 blocks of 144 bytes
 *     (ggml-common.h:317-328); an expert bank adds ne[2] = E. Activations
 *     X[T][K] fp32 (src1 with ne[0] = K, ne[1] = T); outputs Y[T][M].
 *     Device pointers to weights must be 16-byte aligned, activation rows
 *     16-byte aligned, Q8_K buffers 4-byte aligned.
 */
#ifndef SPQ4K_H
#define SPQ4K_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPQ4K_QK_K 256
#define SPQ4K_Q4K_BLOCK_BYTES 144
#define SPQ4K_Q5K_BLOCK_BYTES 176
#define SPQ4K_Q6K_BLOCK_BYTES 210
#define SPQ4K_Q8K_BLOCK_BYTES 292
#define SPQ4K_QK8_0 32
#define SPQ4K_Q8_0_BLOCK_BYTES 34
#define SPQ4K_GEMV_MAX_T 8

/* weight types, with ggml's numbers (enum ggml_type, ggml.h:398, :402-404) */
#define SPQ4K_TYPE_Q8_0 8
#define SPQ4K_TYPE_Q4_K 12
#define SPQ4K_TYPE_Q5_K 13
#define SPQ4K_TYPE_Q6_K 14

typedef struct spq4k_ctx spq4k_ctx;
typedef struct spq4k_weights spq4k_weights;

/* ---- context ----------------------------------------------------------
 * Replaces the backend bring-up of the CUDA path (ggml_backend_init_by_type,
 * desktop/engine/src/cli/main.cpp:95-110; ForwardContext::create,
 * desktop/engine/src/forward.cpp:694-705). Owns a HIP stream and the
 * scratch used by split-K GEMV, prefill GEMM and MoE routing. */
int         spq4k_init(int device, spq4k_ctx **out);
void        spq4k_free(spq4k_ctx *ctx);
/* Use the caller's hipStream_t (NULL restores the context's own stream). */
int         spq4k_set_stream(spq4k_ctx *ctx, void *hip_stream);
void       *spq4k_get_stream(spq4k_ctx *ctx);
/* the HIP device of the context */
int         spq4k_get_device(const spq4k_ctx *ctx);
int         spq4k_synchronize(spq4k_ctx *ctx);
const char *spq4k_last_error(const spq4k_ctx *ctx);
int         spq4k_device_count(void);
/* Grow the context's scratch to at least scratch_bytes (activation planes,
 * K-split partial sums, MoE routing) and its fusion scratch to at least
 * fusion_bytes (normalised rows and gate / up outputs of the unfused
 * spq4k_mul_mat_rms_norm / spq4k_mul_mat_swiglu paths), as the CUDA backend's
 * memory pool grows on demand (ggml_cuda_pool_leg::alloc,
 * ggml-cuda/ggml-cuda.cu:382). A call that needs more scratch than the
 * context holds grows it itself, except while its stream is being captured
 * into a HIP graph: it then returns -EBUSY and enqueues nothing, so reserve
 * before capturing. Buffers replaced by larger ones stay allocated until
 * spq4k_free, so graphs captured earlier stay valid. Sizes: activation
 * planes take 340 bytes per 256 values of each input row (Q8_0: 36 bytes per
 * 32), a K split up to 8 MiB of partial sums beside them; the fusion scratch
 * takes 4 bytes per input value (the norm) plus 8 per output (SwiGLU). */
int         spq4k_reserve(spq4k_ctx *ctx, size_t scratch_bytes, size_t fusion_bytes);

/* ---- weights -----------------------------------------------------------
 * Replaces the backend weight upload (ggml_backend_tensor_set of a Q4_K
 * tensor, desktop/engine/src/llama_weights.cpp:483-560). The device copy is
 * byte-identical to the host bytes. E = 1 for a dense matrix. */
int    spq4k_weights_upload(spq4k_ctx *ctx, const void *q4k_host, int64_t M, int64_t K, int64_t E,
                            spq4k_weights **out);
/* Wrap Q4_K bytes already in device memory (not copied, not freed). */
int    spq4k_weights_wrap(spq4k_ctx *ctx, const void *q4k_dev, int64_t M, int64_t K, int64_t E,
                          spq4k_weights **out);
/* Allocate an uninitialised device weight buffer (filled by
 * spq4k_quantize_q4K or a device copy). */
int    spq4k_weights_alloc(spq4k_ctx *ctx, int64_t M, int64_t K, int64_t E, spq4k_weights **out);
void   spq4k_weights_free(spq4k_weights *w);
void  *spq4k_weights_data(const spq4k_weights *w);
size_t spq4k_weights_nbytes(const spq4k_weights *w);

/* The same for a weight of ggml type `type` (SPQ4K_TYPE_Q4_K, SPQ4K_TYPE_Q5_K:
 * GGML_TYPE_Q5_K blocks of 176 bytes, ggml-common.h:334-346,
 * SPQ4K_TYPE_Q6_K: GGML_TYPE_Q6_K blocks of 210 bytes, ggml-common.h:348-357,
 * or SPQ4K_TYPE_Q8_0: GGML_TYPE_Q8_0 blocks of 34 bytes per 32 values,
 * ggml-common.h:241-245, K a multiple of 32), as ggml_backend_tensor_set
 * uploads a tensor of any type (llama_weights.cpp:483-560). The plain forms
 * above are type Q4_K. Every matmul entry point below takes weights of any
 * of these types (batches run on the matrix cores: Q4_K, Q5_K and Q6_K from
 * 4 tokens, Q8_0 from 9 tokens when K is a multiple of 256; the others on
 * the matvec kernels); matrices passed together (the *_multi forms) must
 * share it. Q6_K and Q8_0 data need 2-byte alignment, Q4_K and Q5_K 16. */
int spq4k_weights_upload_type(spq4k_ctx *ctx, int type, const void *host, int64_t M, int64_t K, int64_t E,
                              spq4k_weights **out);
int spq4k_weights_wrap_type(spq4k_ctx *ctx, int type, const void *dev, int64_t M, int64_t K, int64_t E,
                            spq4k_weights **out);
/* Whether [p, p + bytes) lies in device memory of the context's GPU
 * (hipPointerGetAttributes): 1 yes, 0 no (host memory, another GPU's, or
 * memory the runtime does not know). An engine adapter uses it before
 * passing a tensor's address to the entry points above, which read device
 * pointers in place -- the decision the reference makes from a buffer's
 * device type before dereferencing tensor->data (burn_moe_op.cpp:67-80). */
int spq4k_ptr_on_device(spq4k_ctx *ctx, const void *p, size_t bytes);
int spq4k_weights_alloc_type(spq4k_ctx *ctx, int type, int64_t M, int64_t K, int64_t E, spq4k_weights **out);
/* the ggml type id of w, or -EINVAL for NULL */
int spq4k_weights_type(const spq4k_weights *w);
/* the shape of w (rows M, inputs K, experts E); -EINVAL for NULL */
int spq4k_weights_shape(const spq4k_weights *w, int64_t *M, int64_t *K, int64_t *E);

/* ---- type traits (ggml.h:2791-2804, ggml-cpu.h:113-123) -----------------
 * spq4k_dequant      : ggml_to_float_t for Q4_K   = dequantize_row_q4_K
 *                      (ggml-quants.c:1467-1489); bit-exact fp32.
 * spq4k_quantize_q8K : ggml_from_float_t for Q8_K = quantize_row_q8_K
 *                      (ggml-cpu/arch/x86/quants.c:505 -> ggml-quants.c:2692);
 *                      bit-exact blocks (an all-zero block gets zero bsums).
 * spq4k_quantize_q4K : ggml_quantize_chunk(GGML_TYPE_Q4_K, ..., imatrix=NULL)
 *                      = quantize_q4_K -> quantize_row_q4_K_ref
 *                      (ggml-quants.c:1564-1568, :1395-1465); bit-exact bytes.
 * spq4k_vec_dot      : ggml_vec_dot_t for Q4_K x Q8_K with nrc = 1
 *                      (ggml_vec_dot_q4_K_q8_K, ggml-cpu/arch/x86/quants.c:1900);
 *                      *s is a device float. */
int spq4k_dequant(spq4k_ctx *ctx, const void *vx, float *y, int64_t k);
int spq4k_quantize_q8K(spq4k_ctx *ctx, const float *x, void *vy, int64_t k);
int spq4k_quantize_q4K(spq4k_ctx *ctx, const float *src, void *dst, int64_t nrow, int64_t n_per_row);
int spq4k_vec_dot(spq4k_ctx *ctx, int n, float *s, const void *vx, const void *vy);

/* Type traits of any supported weight type (ggml_get_type_traits(type),
 * ggml.c:768-791; ggml_get_type_traits_cpu(type), ggml-cpu.c:297-322):
 * spq4k_to_float       : to_float           (Q6_K: dequantize_row_q6_K,
 *                        ggml-quants.c:1877-1906; Q5_K: dequantize_row_q5_K,
 *                        :1669-1694; bit-exact fp32)
 * spq4k_quantize_chunk : ggml_quantize_chunk(type, ..., imatrix = NULL)
 *                        (ggml.h:2764; Q6_K: quantize_q6_K ->
 *                        quantize_row_q6_K_ref, ggml-quants.c:1992-1996,
 *                        :1807-1875; Q5_K: quantize_q5_K ->
 *                        quantize_row_q5_K_ref, :1789-1793, :1582-1667;
 *                        bit-exact bytes)
 * spq4k_vec_dot_q8K    : vec_dot with vec_dot_type Q8_K, nrc = 1 (Q6_K:
 *                        ggml_vec_dot_q6_K_q8_K, arch/x86/quants.c:2288;
 *                        Q5_K: ggml_vec_dot_q5_K_q8_K, :2078); *s is a
 *                        device float. Not for Q8_0 (see below).
 * Q8_0 (k a multiple of 32): to_float is dequantize_row_q8_0
 * (ggml-quants.c:491-505, bit-exact); quantize_chunk is quantize_q8_0 ->
 * quantize_row_q8_0_ref (ggml-quants.c:2219, :234-257; bit-exact bytes).
 * Q6_K and Q8_0 block pointers need only 2-byte alignment (ggml rows of an
 * odd number of 210- or 34-byte blocks), Q5_K ones 16. Type Q4_K gives the
 * Q4_K entry points above. */
int spq4k_to_float(spq4k_ctx *ctx, int type, const void *vx, float *y, int64_t k);
int spq4k_quantize_chunk(spq4k_ctx *ctx, int type, const float *src, void *dst, int64_t nrow, int64_t n_per_row);
int spq4k_vec_dot_q8K(spq4k_ctx *ctx, int type, int n, float *s, const void *vx, const void *vy);
int spq4k_to_float_host(spq4k_ctx *ctx, int type, const void *vx, float *y, int64_t k);
int spq4k_quantize_chunk_host(spq4k_ctx *ctx, int type, const float *src, void *dst, int64_t nrow,
                              int64_t n_per_row);
int spq4k_vec_dot_q8K_host(spq4k_ctx *ctx, int type, int n, float *s, const void *vx, const void *vy);

/* Q8_0's CPU type traits (ggml-cpu.c:258-261), k and n multiples of 32:
 * spq4k_quantize_q8_0 : ggml_from_float_t for Q8_0 = quantize_row_q8_0 of the
 *                       CPU backend (arch/x86/quants.c:302-367: d = max|x| /
 *                       127 as fp16, q = round-half-even(x * 127 / max|x|));
 *                       bit-exact blocks. It differs from the model-file
 *                       encoder (spq4k_quantize_chunk) on rounding ties.
 * spq4k_vec_dot_q8_0  : ggml_vec_dot_q8_0_q8_0 with nrc = 1
 *                       (arch/x86/quants.c:1170-1204); vx Q8_0 weights, vy
 *                       Q8_0 activations; *s is a device float. */
int spq4k_quantize_q8_0(spq4k_ctx *ctx, const float *x, void *vy, int64_t k);
int spq4k_vec_dot_q8_0(spq4k_ctx *ctx, int n, float *s, const void *vx, const void *vy);
int spq4k_quantize_q8_0_host(spq4k_ctx *ctx, const float *x, void *vy, int64_t k);
int spq4k_vec_dot_q8_0_host(spq4k_ctx *ctx, int n, float *s, const void *vx, const void *vy);

int spq4k_dequant_host(spq4k_ctx *ctx, const void *vx, float *y, int64_t k);
int spq4k_quantize_q8K_host(spq4k_ctx *ctx, const float *x, void *vy, int64_t k);
int spq4k_quantize_q4K_host(spq4k_ctx *ctx, const float *src, void *dst, int64_t nrow, int64_t n_per_row);
int spq4k_vec_dot_host(spq4k_ctx *ctx, int n, float *s, const void *vx, const void *vy);

/* ---- matmul ------------------------------------------------------------
 * spq4k_gemv     : GGML_OP_MUL_MAT for 1 <= T <= 8 (ggml_mul_mat(W[K,M],
 *                  x[K,T]), ggml.h:1414-1420; CPU ggml-cpu.c:1241-1439; CUDA
 *                  mmvq.cu:1029). Fused on-chip Q8_K quantisation.
 * spq4k_gemv_multi: n <= 4 matrices with the same K and the same input x in
 *                  one launch (q/k/v, gate/up: forward.cpp:1100-1104,
 *                  1596-1600); y[i] is [T][M_i].
 * spq4k_gemm     : GGML_OP_MUL_MAT for any T (prefill; CUDA mmq.cuh:3478):
 *                  Q8_K activations and int8 MFMA on gfx950.
 * spq4k_gemm_multi: n <= 4 matrices with the same K and the same input X
 *                  (q/k/v, gate/up of a prefill batch: forward.cpp:1100-1104,
 *                  1596-1600): X is quantised once; Y[i] is [T][M_i].
 * spq4k_mul_mat  : dispatch by T, as ggml-cuda.cu:2366-2449 does
 *                  (T <= 8 -> gemv, otherwise gemm).
 * spq4k_moe      : GGML_OP_MUL_MAT_ID (ggml_mul_mat_id(as[K,M,E], b[K,ne11,T],
 *                  ids[n_used,T]), ggml.h:1434-1438; CPU ggml-cpu.c:1521-1690):
 *                  Y[t][s][r] = row r of expert ids[t][s] . Q8_K(X[t][s % ne11]),
 *                  ne11 in {1, n_used}; ids are device int32 [T][n_used].
 *                  Tokens are grouped per expert so each selected expert's
 *                  weights stream once per call.
 * For Q8_0 weights every matmul above quantises X to Q8_0 as
 * spq4k_quantize_q8_0 does (the vec_dot_type of Q8_0) in place of Q8_K. */
int spq4k_gemv(spq4k_ctx *ctx, const spq4k_weights *W, const float *x, float *y, int64_t T);
int spq4k_gemv_multi(spq4k_ctx *ctx, int n, const spq4k_weights *const *W, const float *x,
                     float *const *y, int64_t T);
int spq4k_gemm(spq4k_ctx *ctx, const spq4k_weights *W, const float *X, float *Y, int64_t T);
int spq4k_gemm_multi(spq4k_ctx *ctx, int n, const spq4k_weights *const *W, const float *X, float *const *Y,
                     int64_t T);
int spq4k_mul_mat(spq4k_ctx *ctx, const spq4k_weights *W, const float *X, float *Y, int64_t T);
/* spq4k_mul_mat_noalloc: spq4k_mul_mat (same kernels, same results) with
 * every intermediate (activation planes, K-split partial sums) in a fixed
 * device array of SPQ4K_NOALLOC_SCRATCH_BYTES that each GPU holds from the
 * library's first use on it until the process ends, in place of the
 * context's scratch: the call never allocates (no hipMalloc, hipFree or
 * allocating library routine). It has no counterpart in the reference; it is
 * for callers that cannot allocate: code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation. Limit: T rows of K inputs
 * whose activation planes (spq4k_reserve's sizes) exceed
 * SPQ4K_NOALLOC_PLANES_MAX are rejected with -EINVAL. Every call on one GPU
 * shares its array, from any context: calls that overlap on one GPU (two
 * streams, two threads, two contexts) race on it and must be ordered by the
 * caller. */
#define SPQ4K_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
#define SPQ4K_NOALLOC_PLANES_MAX ((size_t)24 << 20)
int spq4k_mul_mat_noalloc(spq4k_ctx *ctx, const spq4k_weights *W, const float *X, float *Y, int64_t T);
int spq4k_moe(spq4k_ctx *ctx, const spq4k_weights *bank, const int32_t *ids, int64_t n_used,
              int64_t ne11, int64_t T, const float *X, float *Y);
/* spq4k_moe_multi: the n (1 or 2) GGML_OP_MUL_MAT_ID nodes of one MoE layer
 * that share ids and input, the expert up and gate banks
 * (desktop/engine/src/forward.cpp:1100-1101: ggml_mul_mat_id(ffn_up_exps,
 * cur, selected) and ggml_mul_mat_id(ffn_gate_exps, cur, selected)). Banks
 * share type, K and E (M may differ); Y[i] is [T][n_used][M_i], each equal
 * to spq4k_moe(banks[i], ...). Small batches of K-quant banks sweep both
 * banks in one launch; batches whose experts get two pairs on average share
 * one routing and one matrix-core launch (banks of equal M, K a multiple of
 * 256); otherwise the banks run one after the other. */
int spq4k_moe_multi(spq4k_ctx *ctx, int n, const spq4k_weights *const *banks, const int32_t *ids,
                    int64_t n_used, int64_t ne11, int64_t T, const float *X, float *const *Y);
/* spq4k_dequant_matvec: the reference's scalar BurnHard matvec, beast_matvec
 * (desktop/beast_canyon/sp_beast_canyon.c:1122-1134, used by its MoE
 * forward, :455-562): Y[t][r] = sum_j dequant(W[r])[j] * X[t][j] with the fp32
 * activations as given -- no Q8_K quantisation, so its outputs differ from
 * spq4k_mul_mat's (the ggml CPU path's arithmetic) by about 0.75% normwise
 * at N(0, 0.02) weights and N(0, 1) activations. The dequantised weights
 * are the format's own dequantiser's bit for bit (dequantize_row_q4_K, _q5_K,
 * _q6_K, _q8_0; the reference's beast_dequant_q5_K / _q6_K, :1025-1085, read
 * other bits than those formats and are not followed); each product is
 * rounded to fp32 and the products are added in fp32 (per lane, then across
 * the lane group in a fixed order, where beast_matvec adds them serially).
 * Dense Q4_K, Q5_K, Q6_K or Q8_0 matrices, any T (tokens run in groups of up
 * to 8), K <= 32768; X [T][K] 16-byte aligned, Y [T][M], device pointers; the
 * _host twin copies in and out. */
int spq4k_dequant_matvec(spq4k_ctx *ctx, const spq4k_weights *W, const float *X, float *Y, int64_t T);
int spq4k_dequant_matvec_host(spq4k_ctx *ctx, const spq4k_weights *W, const float *X, float *Y, int64_t T);
/* spq4k_beast_moe_forward: the reference's BurnHard MoE forward for one
 * token (sp_beast_moe_forward, desktop/beast_canyon/sp_beast_canyon.c:455-562)
 * with its routing (sp_beast_route_experts, :385-443), on the GPU:
 *   score_e = softmax(router_logits)_e (fp32: the largest logit, expf of the
 *             differences, their sum in expert order);
 *   the top_k experts by score, the lowest index first among equal scores,
 *             their scores divided by the sum of the chosen ones;
 *   per chosen expert, in rank order: g = beast_matvec(gate_e, hidden),
 *             u = beast_matvec(up_e, hidden), h = (g / (1 + expf(-g))) * u
 *             (beast_silu_mul, :1168-1173), d = beast_matvec(down_e, h),
 *             output += score * d (fused multiply-add, as the reference's
 *             GCC build compiles it).
 * beast_matvec's arithmetic as in spq4k_dequant_matvec (fp32 activations,
 * no Q8_K; the dequantised weights bit for bit, the products summed per lane
 * and across the wave where the reference adds serially). top_k <= 0 means 2
 * (the reference's default) and is capped at E; at most 16. Banks of Q4_K,
 * Q5_K, Q6_K or Q8_0, each of its own type (a Q4_K_M file's Q6_K down bank
 * beside Q4_K gate / up ones): gate and up [n_ff x n_embd] x E, down
 * [n_embd x n_ff] x E, E <= 4096, rows of at most 32768 values. router_logits [E], hidden [n_embd] (16-byte aligned),
 * output [n_embd]; ids / scores [top_k] receive the routing when not NULL
 * (engine->routing's expert_ids / expert_scores). Device pointers; the _host
 * twin copies in and out. */
int spq4k_beast_moe_forward(spq4k_ctx *ctx, const spq4k_weights *gate, const spq4k_weights *up,
                            const spq4k_weights *down, const float *router_logits, int64_t top_k,
                            const float *hidden, float *output, int32_t *ids, float *scores);
int spq4k_beast_moe_forward_host(spq4k_ctx *ctx, const spq4k_weights *gate, const spq4k_weights *up,
                                 const spq4k_weights *down, const float *router_logits, int64_t top_k,
                                 const float *hidden, float *output, int32_t *ids, float *scores);
/* spq4k_moe_ffn: the routed-expert FFN block of a MoE layer, the unit the
 * reference's BURN_MOE custom op replaces (sp_build_burn_moe_op,
 * desktop/engine/src/burn_moe_op.cpp:377-430, computing burn_moe_compute,
 * :202-372: per token and slot, gate and up, silu(gate) * up, down, weighted
 * sum) with the arithmetic of the stock ggml graph it stands for
 * (forward.cpp:1098-1117):
 *   G, U = ggml_mul_mat_id(gate / up, X, ids)          [T][n_used][n_ff]
 *   H    = silu(G) * U                                  ggml_silu, ggml_mul
 *   D    = ggml_mul_mat_id(down, H, ids)   (input row t * n_used + s)
 *   Y[t] = sum_s D[t][s] * weights[t][s]   fp32 products added in double in
 *                                          slot order (ggml_mul, ggml_sum_rows)
 * gate and up banks [n_embd -> n_ff] x E share type and shape; down is
 * [n_ff -> n_embd] x E of any supported type. ids [T][n_used] int32 and
 * weights [T][n_used] fp32 (the router's top-k and its weights, the
 * op's `selected` and `weights` sources), X [T][n_embd] (16-byte aligned),
 * Y [T][n_embd]; device pointers. Equals spq4k_moe_multi(gate, up),
 * spq4k_swiglu, spq4k_moe(down, ne11 = n_used) and the weighted sum run one
 * after the other, bit for bit. The _host twin copies in and out. */
int spq4k_moe_ffn(spq4k_ctx *ctx, const spq4k_weights *gate, const spq4k_weights *up, const spq4k_weights *down,
                  const int32_t *ids, const float *weights, int64_t n_used, int64_t T, const float *X, float *Y);
int spq4k_moe_ffn_host(spq4k_ctx *ctx, const spq4k_weights *gate, const spq4k_weights *up,
                       const spq4k_weights *down, const int32_t *ids, const float *weights, int64_t n_used,
                       int64_t T, const float *X, float *Y);

/* ---- the operations either side of the matvec ---------------------------
 * spq4k_rms_norm         : ggml_mul(ggml_rms_norm(x, eps), w) over T rows of K
 *                          (ggml-cpu/ops.cpp:3724-3784): y = x * s * w with
 *                          s = 1 / sqrtf(mean + eps), mean = (float)(sum of
 *                          the fp32 squares in double / K). Bit-exact but for
 *                          the double sum's order (a different mean needs the
 *                          sum within ~2^-40 of a float rounding boundary).
 * spq4k_mul_mat_rms_norm : y_i = W_i . rms_norm(x) * norm_w for n <= 4
 *                          matrices sharing the input (the attention and FFN
 *                          pre-norms, forward.cpp:1693-1696): at T = 1 one
 *                          launch, the norm in the matvec's prologue;
 *                          otherwise the norm pass, then spq4k_mul_mat's path.
 * spq4k_mul_mat_swiglu   : y = silu(Wg . xb) * (Wu . xb), xb = x, or
 *                          rms_norm(x) * norm_w when norm_w is not NULL (the
 *                          dense SwiGLU front half, forward.cpp:1703-1706;
 *                          ggml-cuda fuses the same gate in mmvq.cu:437-470):
 *                          at T = 1 one launch (gate row and up row side by
 *                          side, SiLU and the product in the epilogue);
 *                          otherwise gate and up, then one element-wise pass.
 *                          Wg and Wu share type, K and M; y is [T][M].
 * Device pointers; x, norm_w 16-byte aligned; eps >= 0. */
int spq4k_rms_norm(spq4k_ctx *ctx, const float *x, const float *w, float eps, float *y, int64_t K, int64_t T);
/* y = silu(g) * u over n values (ggml_silu then ggml_mul; ggml_swiglu_split's
 * ggml_vec_swiglu_f32, ggml-cpu/vec.cpp:433): the unfused epilogue */
int spq4k_swiglu(spq4k_ctx *ctx, const float *g, const float *u, float *y, int64_t n);
int spq4k_mul_mat_rms_norm(spq4k_ctx *ctx, int n, const spq4k_weights *const *W, const float *x,
                           const float *norm_w, float eps, float *const *y, int64_t T);
int spq4k_mul_mat_swiglu(spq4k_ctx *ctx, const spq4k_weights *Wg, const spq4k_weights *Wu, const float *x,
                         const float *norm_w, float eps, float *y, int64_t T);

int spq4k_mul_mat_host(spq4k_ctx *ctx, const spq4k_weights *W, const float *X, float *Y, int64_t T);
int spq4k_moe_host(spq4k_ctx *ctx, const spq4k_weights *bank, const int32_t *ids, int64_t n_used,
                   int64_t ne11, int64_t T, const float *X, float *Y);

/* ---- decode chains: dependent T = 1 stages in one launch -----------------
 * Replaces, for a run of a dense decode graph's nodes, the per-node
 * execution of the reference's decode layer (build_block_decode,
 * desktop/engine/src/forward.cpp:2663-2856: rms_norm * attn_norm, the q/k/v
 * MUL_MATs, the o MUL_MAT, the residual add, rms_norm * ffn_norm, gate / up,
 * silu * up, down, the residual add; and the output head, :3411-3413) --
 * everything but the attention core, which stays with the engine. Each
 * stage is
 *     x    = in0 (+ in1)                    ggml_add, fp32
 *     x_out = x                             when x_out is set (the residual)
 *     x    = rms_norm(x, eps) * norm_w      when norm_w is set
 *     y[i] = W[i] . Q8_K(x), i < n          n <= 4 matrices sharing x
 *  or y[0] = silu(W[0] . Q8_K(x)) * (W[1] . Q8_K(x))   with glu (n = 2)
 * with the arithmetic of spq4k_mul_mat_rms_norm / spq4k_mul_mat_swiglu at
 * T = 1 (the norm bit-exact but for its double sum's order; Q8_K bit-exact;
 * the matvec's per-lane sums those of the decode kernel). The stages run
 * in order, each seeing every earlier stage's outputs, in one cooperative
 * launch that streams the next stages' weights while a stage waits for the
 * previous one. Q4_K weights, E = 1, K <= 12288; per stage
 * (1 + [in1] + [norm_w]) * K <= 12288; all pointers device pointers,
 * 16-byte aligned; a stage's outputs (y[i], x_out) must overlap neither its
 * inputs (in0, in1, norm_w) nor each other (-EINVAL). Stages may read what
 * any earlier stage wrote.
 *   spq4k_chain_create  validates and uploads the stage table;
 *   spq4k_chain_run     launches it on the context's stream (asynchronous);
 *   spq4k_chain_status  synchronises and returns 0, or -ETIMEDOUT if a
 *                       stage wait gave up (the outputs are then invalid;
 *                       the chain is reset for the next run);
 *   spq4k_chain_free    releases it.
 * A chain runs one launch at a time (its barrier counters are its own).
 * No reference entry point takes a whole chain; the per-node entry points
 * above remain the drop-in for single nodes. */
typedef struct spq4k_chain spq4k_chain;
typedef struct spq4k_chain_stage {
    int n;                             /* matrices sharing the input, 1..4 (2 with glu) */
    int glu;                           /* y[0] = silu(W[0] . x) * (W[1] . x) */
    const spq4k_weights *W[4];
    float *y[4];                       /* [M_i] each */
    const float *in0;                  /* [K] */
    const float *in1;                  /* [K] or NULL */
    float *x_out;                      /* [K] or NULL */
    const float *norm_w;               /* [K] or NULL */
} spq4k_chain_stage;
int spq4k_chain_create(spq4k_ctx *ctx, const spq4k_chain_stage *stages, int n_stages, float eps,
                       spq4k_chain **out);
int spq4k_chain_run(spq4k_ctx *ctx, spq4k_chain *chain);
int spq4k_chain_status(spq4k_ctx *ctx, spq4k_chain *chain);
void spq4k_chain_free(spq4k_chain *chain);

#ifdef __cplusplus
}
#endif

#endif /* SPQ4K_H */
