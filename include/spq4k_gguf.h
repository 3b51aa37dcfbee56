/*
 * spq4k_gguf.h — GGUF model files and GPU weight residency for libspq4k.
 *
 * The reference engine loads a model by memory-mapping the GGUF file, parsing
 * it with ggml's reader in no_alloc mode and either pointing each tensor into
 * the mapping (LlamaWeights::load_cpu_mmap_,
 * desktop/engine/src/llama_weights.cpp:441-480) or copying the weights into
 * one backend buffer (LlamaWeights::load_backend_offload_, :483-720: partial
 * offload of layers [0, n_gpu_layers), and the split of an MoE expert bank
 * whose first experts stay on the CPU). This header is the same two steps for
 * the weights libspq4k runs:
 *
 *   spq4k_gguf_*  : the file (gguf_init_from_file with no_alloc and the
 *                   engine's mmap; the gguf_get_* accessors of
 *                   vendor/ggml/include/gguf.h). Host only, no GPU needed.
 *   spq4k_model_* : uploads every Q4_K / Q5_K / Q6_K / Q8_0 matrix of the
 *                   file that the offload settings place on the GPU into one
 *                   device allocation, once, and hands out spq4k_weights for
 *                   them by tensor name.
 *
 * Functions return 0 or a negative errno value (-EINVAL for a malformed file
 * or bad argument, -ENOENT and the like from open, -ENOMEM, -EIO for a HIP
 * failure); spq4k_gguf_strerror() describes the last failure of the calling
 * thread. Accessors return -1 / NULL / 0 for a bad index.
 */
#ifndef SPQ4K_GGUF_H
#define SPQ4K_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "spq4k.h"

#ifdef __cplusplus
extern "C" {
#endif

/* value types of GGUF metadata (enum gguf_type, gguf.h:53-67) */
enum {
    SPQ4K_GGUF_UINT8 = 0,
    SPQ4K_GGUF_INT8 = 1,
    SPQ4K_GGUF_UINT16 = 2,
    SPQ4K_GGUF_INT16 = 3,
    SPQ4K_GGUF_UINT32 = 4,
    SPQ4K_GGUF_INT32 = 5,
    SPQ4K_GGUF_FLOAT32 = 6,
    SPQ4K_GGUF_BOOL = 7,
    SPQ4K_GGUF_STRING = 8,
    SPQ4K_GGUF_ARRAY = 9,
    SPQ4K_GGUF_UINT64 = 10,
    SPQ4K_GGUF_INT64 = 11,
    SPQ4K_GGUF_FLOAT64 = 12
};

typedef struct spq4k_gguf spq4k_gguf;
typedef struct spq4k_model spq4k_model;

/* ---- the file ------------------------------------------------------------
 * spq4k_gguf_open maps `path` read-only and validates it as
 * gguf_init_from_file does (gguf.cpp:395-740), and also that every tensor's
 * bytes lie inside the file. The mapping lives until spq4k_gguf_close. */
int         spq4k_gguf_open(const char *path, spq4k_gguf **out);
void        spq4k_gguf_close(spq4k_gguf *g);
const char *spq4k_gguf_strerror(void);

uint32_t spq4k_gguf_version(const spq4k_gguf *g);
size_t   spq4k_gguf_alignment(const spq4k_gguf *g);    /* gguf_get_alignment */
size_t   spq4k_gguf_data_offset(const spq4k_gguf *g);  /* gguf_get_data_offset: file offset of the data section */
size_t   spq4k_gguf_data_size(const spq4k_gguf *g);    /* padded size of the data section */
size_t   spq4k_gguf_file_size(const spq4k_gguf *g);

/* metadata (gguf_get_n_kv, gguf_find_key, gguf_get_key, gguf_get_kv_type,
 * gguf_get_arr_type, gguf_get_arr_n, gguf_get_val_data / gguf_get_arr_data,
 * gguf_get_val_str / gguf_get_arr_str). val_data: the little-endian values of
 * a non-string scalar or array (bools as bytes 0 / 1); val_str: string j of a
 * string value (j = 0 for a scalar). arr_n is 1 for a scalar. */
int64_t     spq4k_gguf_n_kv(const spq4k_gguf *g);
int64_t     spq4k_gguf_find_key(const spq4k_gguf *g, const char *key);
const char *spq4k_gguf_key(const spq4k_gguf *g, int64_t i);
int         spq4k_gguf_kv_type(const spq4k_gguf *g, int64_t i);
int         spq4k_gguf_arr_type(const spq4k_gguf *g, int64_t i);
int64_t     spq4k_gguf_arr_n(const spq4k_gguf *g, int64_t i);
const void *spq4k_gguf_val_data(const spq4k_gguf *g, int64_t i);
const char *spq4k_gguf_val_str(const spq4k_gguf *g, int64_t i, int64_t j);

/* tensors (gguf_get_n_tensors, gguf_find_tensor, gguf_get_tensor_name,
 * gguf_get_tensor_type, gguf_get_tensor_offset, gguf_get_tensor_size).
 * tensor_shape fills ne[4] (ggml order: ne[0] the row length) and returns
 * ggml_n_dims; tensor_data points into the mapping at
 * data_offset + tensor_offset, as the engine's loader computes it
 * (llama_weights.cpp:465). */
int64_t     spq4k_gguf_n_tensors(const spq4k_gguf *g);
int64_t     spq4k_gguf_find_tensor(const spq4k_gguf *g, const char *name);
const char *spq4k_gguf_tensor_name(const spq4k_gguf *g, int64_t i);
int         spq4k_gguf_tensor_type(const spq4k_gguf *g, int64_t i);
int         spq4k_gguf_tensor_shape(const spq4k_gguf *g, int64_t i, int64_t ne[4]);
size_t      spq4k_gguf_tensor_offset(const spq4k_gguf *g, int64_t i);
size_t      spq4k_gguf_tensor_nbytes(const spq4k_gguf *g, int64_t i);
const void *spq4k_gguf_tensor_data(const spq4k_gguf *g, int64_t i);

/* ---- GPU residency ---------------------------------------------------------
 * spq4k_model_load uploads, on ctx's device, every tensor of type Q4_K, Q5_K,
 * Q6_K or Q8_0 with at least two dimensions (a matrix ne = [K, M] or an
 * expert bank [K, M, E]; ne[3] = 1) that LlamaWeights::load_backend_offload_
 * would place on the GPU:
 *   - n_gpu_layers < 0, or at least the file's layer count (the largest N of
 *     the "blk.N." names, plus one): every such tensor (full offload);
 *   - otherwise only those of layers "blk.N." with N < n_gpu_layers; the
 *     other layers and the tensors outside layers stay in the file mapping
 *     (llama_weights.cpp:519-528);
 *   - experts_on_cpu > 0 splits each "blk.N.ffn_{gate,up,down}_exps.weight"
 *     bank of an offloaded layer at pivot = min(experts_on_cpu, E - 1): the
 *     GPU holds experts [pivot, E) as a bank of E - pivot experts under the
 *     tensor's own name; experts [0, pivot) stay in the mapping, as the
 *     reference's "*_exps_cpu.weight" sub-bank (llama_weights.cpp:617-660).
 * All of it goes into one device allocation (ggml_backend_alloc_ctx_tensors),
 * copied from the mapping through pinned staging buffers with the copies of
 * one buffer overlapping the filling of the other; the call returns when the
 * weights are resident. The device bytes are the file's bytes. The model does
 * not keep the file open: the gguf may be closed after the call. */
int            spq4k_model_load(spq4k_ctx *ctx, const spq4k_gguf *g, int n_gpu_layers, int experts_on_cpu,
                                spq4k_model **out);
void           spq4k_model_free(spq4k_model *m);
/* resident weights of tensor `name` (owned by the model), NULL if the tensor
 * is not on the GPU */
spq4k_weights *spq4k_model_weights(const spq4k_model *m, const char *name);
/* first expert of the resident bank `name` (the split pivot; 0 unsplit), -1 if not resident */
int            spq4k_model_expert_base(const spq4k_model *m, const char *name);
int64_t        spq4k_model_n_tensors(const spq4k_model *m);
const char    *spq4k_model_tensor_name(const spq4k_model *m, int64_t i);
size_t         spq4k_model_nbytes(const spq4k_model *m);   /* device bytes of the allocation */

#ifdef __cplusplus
}
#endif

#endif /* SPQ4K_GGUF_H */
