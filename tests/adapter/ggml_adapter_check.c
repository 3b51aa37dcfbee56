/* ggml_adapter_check.c — test driver for the ggml adapter (include/spq4k_ggml.h).
 *
 * Test infrastructure: builds the same ggml graph twice in one context of the
 * reference's own ggml (compiled from its sources into oracle/_ref) — once with
 * ggml's GGML_OP_MUL_MAT / GGML_OP_MUL_MAT_ID nodes, once with the adapter's
 * spq4k nodes — computes it on the CPU with ggml_graph_compute_with_ctx and
 * returns both outputs; the Python test compares them with close_enough.
 * Weights are seeded N(0, 0.02) quantised by ggml_quantize_chunk (of the type
 * the caller asks), activations seeded N(0, 1).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "ggml-alloc.h"
#include "ggml-backend-impl.h"   /* the reference's buffer interface: a device buffer type for the tests */
#include "ggml-cpu.h"
#include "ggml.h"
#include "spq4k_ggml.h"

static uint64_t splitmix(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static void normal_fill(float *p, int64_t n, uint64_t seed, float std) {
    uint64_t s = seed;
    for (int64_t i = 0; i < n; i += 2) {
        const double u1 = ((splitmix(&s) >> 11) + 1.0) * (1.0 / 9007199254740993.0);
        const double u2 = (splitmix(&s) >> 11) * (1.0 / 9007199254740992.0);
        const double r = sqrt(-2.0 * log(u1));
        p[i] = (float)(std * r * cos(6.283185307179586 * u2));
        if (i + 1 < n) p[i + 1] = (float)(std * r * sin(6.283185307179586 * u2));
    }
}

/* a weight [K, M, E] of ggml type `type` from seeded N(0, 0.02) values */
static struct ggml_tensor *q_weight(struct ggml_context *ctx, int type, int64_t K, int64_t M, int64_t E,
                                    uint64_t seed, float *scratch) {
    struct ggml_tensor *w = ggml_new_tensor_3d(ctx, (enum ggml_type)type, K, M, E);
    normal_fill(scratch, K * M * E, seed, 0.02f);
    ggml_quantize_chunk((enum ggml_type)type, scratch, w->data, 0, M * E, K, NULL);
    return w;
}

static struct ggml_tensor *f32_input(struct ggml_context *ctx, int64_t ne0, int64_t ne1, int64_t ne2, uint64_t seed) {
    struct ggml_tensor *x = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, ne0, ne1, ne2);
    normal_fill((float *)x->data, ne0 * ne1 * ne2, seed, 1.0f);
    return x;
}

static int finish(struct ggml_context *ctx, spq4k_ggml *b, struct ggml_tensor *yr, struct ggml_tensor *ya,
                  int nthreads, float *y_ref, float *y_ada, char *err, int errlen) {
    int rc = 0;
    if (!yr || !ya) {
        snprintf(err, errlen, "graph construction failed");
        rc = -1;
    } else {
        struct ggml_cgraph *gf = ggml_new_graph(ctx);
        ggml_build_forward_expand(gf, yr);
        ggml_build_forward_expand(gf, ya);
        if (ggml_graph_compute_with_ctx(ctx, gf, nthreads) != GGML_STATUS_SUCCESS) {
            snprintf(err, errlen, "ggml_graph_compute failed");
            rc = -1;
        } else if (spq4k_ggml_status(b) != 0) {
            snprintf(err, errlen, "%s", spq4k_ggml_last_error(b));
            rc = spq4k_ggml_status(b);
        } else {
            memcpy(y_ref, yr->data, ggml_nbytes(yr));
            memcpy(y_ada, ya->data, ggml_nbytes(ya));
        }
    }
    spq4k_ggml_free(b);
    ggml_free(ctx);
    return rc;
}

static struct ggml_context *new_ctx(size_t bytes) {
    struct ggml_init_params ip = {bytes, NULL, false};
    return ggml_init(ip);
}

/* y [M, T] = W [K, M] x x [K, T], W of ggml type `type` */
int check_mul_mat(int type, int64_t M, int64_t K, int64_t T, uint64_t seed, int nthreads, float *y_ref, float *y_ada,
                  char *err, int errlen) {
    spq4k_ggml *b;
    int rc = spq4k_ggml_init(0, &b);
    if (rc) {
        snprintf(err, errlen, "spq4k_ggml_init: %d", rc);
        return rc;
    }
    struct ggml_context *ctx = new_ctx((size_t)M * K * 4 + (size_t)K * T * 16 + (size_t)M * T * 16 + (64 << 20));
    float *tmp = (float *)malloc((size_t)M * K * sizeof(float));
    struct ggml_tensor *W = q_weight(ctx, type, K, M, 1, seed, tmp);
    free(tmp);
    struct ggml_tensor *x = f32_input(ctx, K, T, 1, seed + 1);
    return finish(ctx, b, ggml_mul_mat(ctx, W, x), spq4k_ggml_mul_mat(ctx, W, x, b), nthreads, y_ref, y_ada, err,
                  errlen);
}

/* a gated feed-forward block, gate and up Q4_K, down of type down_type (a
 * Q4_K_M model stores some ffn_down tensors as Q6_K):
 * y [D, T] = down [F, D] x (silu(gate [D, F] x x) * (up [D, F] x x)).
 * y_ref: all ggml; y_ada: all three matmuls through the adapter; y_chk:
 * ggml's down matmul applied to the adapter's own hidden activations (the
 * per-op comparison for the last node, free of upstream re-quantisation). */
int check_mlp(int down_type, int64_t D, int64_t F, int64_t T, uint64_t seed, int nthreads, float *y_ref,
              float *y_ada, float *y_chk, char *err, int errlen) {
    spq4k_ggml *b;
    int rc = spq4k_ggml_init(0, &b);
    if (rc) {
        snprintf(err, errlen, "spq4k_ggml_init: %d", rc);
        return rc;
    }
    struct ggml_context *ctx = new_ctx((size_t)3 * D * F * 4 + (size_t)(D + F) * T * 64 + (64 << 20));
    float *tmp = (float *)malloc((size_t)D * F * sizeof(float));
    struct ggml_tensor *gate = q_weight(ctx, GGML_TYPE_Q4_K, D, F, 1, seed, tmp);
    struct ggml_tensor *up = q_weight(ctx, GGML_TYPE_Q4_K, D, F, 1, seed + 1, tmp);
    struct ggml_tensor *down = q_weight(ctx, down_type, F, D, 1, seed + 2, tmp);
    free(tmp);
    struct ggml_tensor *x = f32_input(ctx, D, T, 1, seed + 3);
    struct ggml_tensor *hr = ggml_mul(ctx, ggml_silu(ctx, ggml_mul_mat(ctx, gate, x)), ggml_mul_mat(ctx, up, x));
    struct ggml_tensor *yr = ggml_mul_mat(ctx, down, hr);
    struct ggml_tensor *ga = spq4k_ggml_mul_mat(ctx, gate, x, b), *ua = spq4k_ggml_mul_mat(ctx, up, x, b);
    struct ggml_tensor *ya = NULL, *yc = NULL;
    if (ga && ua) {
        struct ggml_tensor *ha = ggml_mul(ctx, ggml_silu(ctx, ga), ua);
        ya = spq4k_ggml_mul_mat(ctx, down, ha, b);
        yc = ggml_mul_mat(ctx, down, ha);
    }
    if (yc) {
        struct ggml_cgraph *gf = ggml_new_graph(ctx);
        ggml_build_forward_expand(gf, yc);
        ggml_build_forward_expand(gf, ya);
        ggml_build_forward_expand(gf, yr);
        if (ggml_graph_compute_with_ctx(ctx, gf, nthreads) != GGML_STATUS_SUCCESS) yc = NULL;
        else memcpy(y_chk, yc->data, ggml_nbytes(yc));
    }
    return finish(ctx, b, yr, yc ? ya : NULL, nthreads, y_ref, y_ada, err, errlen);
}

/* y [M, n_used, T] = mul_mat_id(as [K, M, E], x [K, ne11, T], ids [n_used, T]), as of type `type` */
int check_mul_mat_id(int type, int64_t M, int64_t K, int64_t E, int64_t n_used, int64_t ne11, int64_t T,
                     const int32_t *ids_in, uint64_t seed, int nthreads, float *y_ref, float *y_ada, char *err,
                     int errlen) {
    spq4k_ggml *b;
    int rc = spq4k_ggml_init(0, &b);
    if (rc) {
        snprintf(err, errlen, "spq4k_ggml_init: %d", rc);
        return rc;
    }
    struct ggml_context *ctx =
        new_ctx((size_t)M * K * E * 4 + (size_t)K * ne11 * T * 16 + (size_t)M * n_used * T * 16 + (64 << 20));
    float *tmp = (float *)malloc((size_t)M * K * E * sizeof(float));
    struct ggml_tensor *as = q_weight(ctx, type, K, M, E, seed, tmp);
    free(tmp);
    struct ggml_tensor *x = f32_input(ctx, K, ne11, T, seed + 1);
    struct ggml_tensor *ids = ggml_new_tensor_2d(ctx, GGML_TYPE_I32, n_used, T);
    memcpy(ids->data, ids_in, (size_t)n_used * T * sizeof(int32_t));
    return finish(ctx, b, ggml_mul_mat_id(ctx, as, x, ids), spq4k_ggml_mul_mat_id(ctx, as, x, ids, b), nthreads,
                  y_ref, y_ada, err, errlen);
}

/* The routed-expert FFN block of a MoE layer: y_ref is the stock ggml graph
 * (desktop/engine/src/forward.cpp:1098-1117: up and gate MUL_MAT_ID, silu,
 * mul, down MUL_MAT_ID, mul by the router weights, permute, cont, sum_rows,
 * reshape), y_ada the adapter's single node (spq4k_ggml_moe_ffn, in place of
 * the reference's BURN_MOE op); gate and up Q4_K [D, F, E], down of
 * down_type [F, D, E]; ids_in / w_in [T][n_used]; cur [D, T] seeded N(0, 1). */
int check_moe_ffn(int down_type, int64_t D, int64_t F, int64_t E, int64_t n_used, int64_t T, const int32_t *ids_in,
                  const float *w_in, uint64_t seed, int nthreads, float *y_ref, float *y_ada, char *err, int errlen) {
    spq4k_ggml *b;
    int rc = spq4k_ggml_init(0, &b);
    if (rc) {
        snprintf(err, errlen, "spq4k_ggml_init: %d", rc);
        return rc;
    }
    struct ggml_context *ctx =
        new_ctx((size_t)3 * D * F * E * 2 + (size_t)(D + F) * n_used * T * 64 + (64 << 20));
    float *tmp = (float *)malloc((size_t)D * F * E * sizeof(float));
    struct ggml_tensor *gate = q_weight(ctx, GGML_TYPE_Q4_K, D, F, E, seed, tmp);
    struct ggml_tensor *up = q_weight(ctx, GGML_TYPE_Q4_K, D, F, E, seed + 1, tmp);
    struct ggml_tensor *down = q_weight(ctx, down_type, F, D, E, seed + 2, tmp);
    free(tmp);
    struct ggml_tensor *cur = f32_input(ctx, D, T, 1, seed + 3);
    cur = ggml_reshape_2d(ctx, cur, D, T);
    struct ggml_tensor *sel = ggml_new_tensor_2d(ctx, GGML_TYPE_I32, n_used, T);
    memcpy(sel->data, ids_in, (size_t)n_used * T * sizeof(int32_t));
    struct ggml_tensor *wts = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, 1, n_used, T);
    memcpy(wts->data, w_in, (size_t)n_used * T * sizeof(float));
    /* the stock routed-expert graph */
    struct ggml_tensor *cur3 = ggml_reshape_3d(ctx, cur, D, 1, T);
    struct ggml_tensor *up_e = ggml_mul_mat_id(ctx, up, cur3, sel);
    struct ggml_tensor *gate_e = ggml_silu(ctx, ggml_mul_mat_id(ctx, gate, cur3, sel));
    struct ggml_tensor *par = ggml_mul(ctx, gate_e, up_e);
    struct ggml_tensor *down_e = ggml_mul_mat_id(ctx, down, par, sel);
    struct ggml_tensor *weighted = ggml_mul(ctx, down_e, wts);
    struct ggml_tensor *kfirst = ggml_cont(ctx, ggml_permute(ctx, weighted, 1, 0, 2, 3));
    struct ggml_tensor *yr = ggml_reshape_2d(ctx, ggml_sum_rows(ctx, kfirst), D, T);
    struct ggml_tensor *ya = spq4k_ggml_moe_ffn(ctx, cur, sel, wts, gate, up, down, b);
    return finish(ctx, b, yr, ya, nthreads, y_ref, y_ada, err, errlen);
}

/* The resident-weight table: a node on a weight keeps one GPU copy across
 * graphs; a tensor whose type or shape changed at the same addresses is
 * uploaded again; spq4k_ggml_forget drops copies. Returns 0 when every step
 * behaves, else the failing step's number. */
int check_resident(char *err, int errlen) {
    spq4k_ggml *b;
    int rc = spq4k_ggml_init(0, &b);
    if (rc) {
        snprintf(err, errlen, "spq4k_ggml_init: %d", rc);
        return rc;
    }
    struct ggml_context *ctx = new_ctx((size_t)64 << 20);
    const int64_t K = 512, M = 64;
    float *tmp = (float *)malloc((size_t)M * K * sizeof(float));
    struct ggml_tensor *W = q_weight(ctx, GGML_TYPE_Q4_K, K, M, 1, 5, tmp);
    struct ggml_tensor *x = f32_input(ctx, K, 1, 1, 6);
    int step = 0;
    for (int it = 0; it < 2 && !step; ++it) {
        struct ggml_tensor *y = spq4k_ggml_mul_mat(ctx, W, x, b);
        struct ggml_cgraph *gf = ggml_new_graph(ctx);
        ggml_build_forward_expand(gf, y);
        if (ggml_graph_compute_with_ctx(ctx, gf, 1) != GGML_STATUS_SUCCESS || spq4k_ggml_status(b)) step = 1 + it;
    }
    /* same tensor, same data pointer, same byte count, another shape: K = 256, M = 128 */
    if (!step) {
        W->ne[0] = K / 2;
        W->ne[1] = 2 * M;
        W->nb[1] = 144;
        W->nb[2] = W->nb[3] = W->nb[1] * (size_t)(2 * M);
        normal_fill(tmp, M * K, 9, 0.02f);
        ggml_quantize_chunk(GGML_TYPE_Q4_K, tmp, W->data, 0, 2 * M, K / 2, NULL);
        struct ggml_tensor *x2 = f32_input(ctx, K / 2, 1, 1, 7);
        struct ggml_tensor *y = spq4k_ggml_mul_mat(ctx, W, x2, b);
        struct ggml_tensor *yr = ggml_mul_mat(ctx, W, x2);
        struct ggml_cgraph *gf = ggml_new_graph(ctx);
        ggml_build_forward_expand(gf, y);
        ggml_build_forward_expand(gf, yr);
        if (!y || ggml_graph_compute_with_ctx(ctx, gf, 1) != GGML_STATUS_SUCCESS || spq4k_ggml_status(b)) {
            step = 3;
        } else {
            const float *a = (const float *)y->data, *r = (const float *)yr->data;
            for (int64_t i = 0; i < 2 * M && !step; ++i)
                if (!(fabsf(a[i] - r[i]) <= 1e-5f || fabsf(a[i] - r[i]) <= 1e-4f * fabsf(r[i]))) step = 4;
        }
    }
    if (!step && spq4k_ggml_forget(b, W) != 2) step = 5;   /* the copies of both shapes */
    if (!step && spq4k_ggml_forget(b, NULL) != 0) step = 6;
    free(tmp);
    if (step) snprintf(err, errlen, "resident-table step %d failed: %s", step, spq4k_ggml_last_error(b));
    spq4k_ggml_free(b);
    ggml_free(ctx);
    return step;
}

/* ---- device-resident graphs -------------------------------------------------
 * A minimal ggml buffer type in GPU memory (hipMalloc, is_host false), the
 * stand-in for a HIP build of ggml's device buffers: tensors allocated in it
 * have device addresses in tensor->data, as on the engine's GPU backend. */
static void dv_free(ggml_backend_buffer_t buf) { (void)hipFree(buf->context); }
static void *dv_base(ggml_backend_buffer_t buf) { return buf->context; }
static void dv_memset(ggml_backend_buffer_t buf, struct ggml_tensor *t, uint8_t v, size_t off, size_t size) {
    (void)buf;
    (void)hipMemset((char *)t->data + off, v, size);
}
static void dv_set(ggml_backend_buffer_t buf, struct ggml_tensor *t, const void *d, size_t off, size_t size) {
    (void)buf;
    (void)hipMemcpy((char *)t->data + off, d, size, hipMemcpyHostToDevice);
}
static void dv_get(ggml_backend_buffer_t buf, const struct ggml_tensor *t, void *d, size_t off, size_t size) {
    (void)buf;
    (void)hipMemcpy(d, (const char *)t->data + off, size, hipMemcpyDeviceToHost);
}
static void dv_clear(ggml_backend_buffer_t buf, uint8_t v) { (void)hipMemset(buf->context, v, buf->size); }
static const struct ggml_backend_buffer_i dv_iface = {
    .free_buffer = dv_free, .get_base = dv_base, .memset_tensor = dv_memset, .set_tensor = dv_set,
    .get_tensor = dv_get, .clear = dv_clear,
};
static const char *dvt_name(ggml_backend_buffer_type_t t) {
    (void)t;
    return "spq4k-test-device";
}
static ggml_backend_buffer_t dvt_alloc(ggml_backend_buffer_type_t t, size_t size) {
    void *p = NULL;
    if (hipMalloc(&p, size ? size : 256) != hipSuccess) return NULL;
    return ggml_backend_buffer_init(t, dv_iface, p, size);
}
static size_t dvt_align(ggml_backend_buffer_type_t t) {
    (void)t;
    return 256;
}
static bool dvt_is_host(ggml_backend_buffer_type_t t) {
    (void)t;
    return false;
}
static struct ggml_backend_buffer_type dv_buft = {
    .iface = {.get_name = dvt_name, .alloc_buffer = dvt_alloc, .get_alignment = dvt_align, .is_host = dvt_is_host},
};

/* A buffer type in plain host memory (malloc) that reports is_host false, as
 * ggml's CPU extra buffer types (repack, AMX) and other backends' buffers do:
 * its tensors are not this GPU's memory and must take the adapter's copy
 * path. */
static void hm_free(ggml_backend_buffer_t buf) { free(buf->context); }
static void hm_memset(ggml_backend_buffer_t buf, struct ggml_tensor *t, uint8_t v, size_t off, size_t size) {
    (void)buf;
    memset((char *)t->data + off, v, size);
}
static void hm_set(ggml_backend_buffer_t buf, struct ggml_tensor *t, const void *d, size_t off, size_t size) {
    (void)buf;
    memcpy((char *)t->data + off, d, size);
}
static void hm_get(ggml_backend_buffer_t buf, const struct ggml_tensor *t, void *d, size_t off, size_t size) {
    (void)buf;
    memcpy(d, (const char *)t->data + off, size);
}
static void hm_clear(ggml_backend_buffer_t buf, uint8_t v) { memset(buf->context, v, buf->size); }
static const struct ggml_backend_buffer_i hm_iface = {
    .free_buffer = hm_free, .get_base = dv_base, .memset_tensor = hm_memset, .set_tensor = hm_set,
    .get_tensor = hm_get, .clear = hm_clear,
};
static const char *hmt_name(ggml_backend_buffer_type_t t) {
    (void)t;
    return "spq4k-test-hostmem-not-host";
}
static ggml_backend_buffer_t hmt_alloc(ggml_backend_buffer_type_t t, size_t size) {
    void *p = aligned_alloc(256, ((size ? size : 256) + 255) & ~(size_t)255);
    if (!p) return NULL;
    return ggml_backend_buffer_init(t, hm_iface, p, size);
}
static struct ggml_backend_buffer_type hm_buft = {
    .iface = {.get_name = hmt_name, .alloc_buffer = hmt_alloc, .get_alignment = dvt_align, .is_host = dvt_is_host},
};

static int compute_graph(struct ggml_tensor *out, int nthreads) {
    struct ggml_init_params ip = {(size_t)16 << 20, NULL, false};
    struct ggml_context *gctx = ggml_init(ip);
    struct ggml_cgraph *gf = ggml_new_graph(gctx);
    ggml_build_forward_expand(gf, out);
    struct ggml_cplan plan = ggml_graph_plan(gf, nthreads, NULL);
    void *work = plan.work_size ? malloc(plan.work_size) : NULL;
    plan.work_data = work;
    const int rc = ggml_graph_compute(gf, &plan) == GGML_STATUS_SUCCESS ? 0 : -1;
    free(work);
    ggml_free(gctx);
    return rc;
}

/* The same node on host tensors (ggml's own MUL_MAT / the stock routed-expert
 * graph, y_ref) and through the adapter (y_ada) on tensors in a backend
 * buffer that is not host memory: GPU memory (check_device) or host memory
 * behind is_host false (check_hostmem_not_host).
 * mode 0: y [M, T] = W [K, M] x x [K, T] of ggml type `type`; mode 1: the
 * routed-expert FFN block (gate / up Q4_K [K, M, E], down of `type`
 * [M, K, E], n_used of E experts, ids_in / w_in [T][n_used]). Returns 0, or
 * the step that failed; *wrapped is set when the binding adopted the device
 * weight in place (its resident copy is W->data). */
static int check_in(ggml_backend_buffer_type_t buft, int mode, int type, int64_t M, int64_t K, int64_t E,
                    int64_t n_used, int64_t T, const int32_t *ids_in, const float *w_in, uint64_t seed, int nthreads,
                    float *y_ref, float *y_ada, int *wrapped, char *err, int errlen) {
    spq4k_ggml *b;
    int rc = spq4k_ggml_init(0, &b);
    if (rc) {
        snprintf(err, errlen, "spq4k_ggml_init: %d", rc);
        return rc;
    }
    const int64_t Eh = mode ? E : 1;
    struct ggml_context *hctx = new_ctx((size_t)3 * M * K * Eh * 2 + (size_t)(M + K) * T * n_used * 32 + (64 << 20));
    struct ggml_init_params dp = {(size_t)64 << 10, NULL, true};
    struct ggml_context *dctx = ggml_init(dp);
    float *tmp = (float *)malloc((size_t)M * K * Eh * sizeof(float));
    struct ggml_tensor *yr, *ya;
    struct ggml_tensor *hsrc[6], *dsrc[6];
    int nsrc;
    if (mode == 0) {
        hsrc[0] = q_weight(hctx, type, K, M, 1, seed, tmp);
        hsrc[1] = f32_input(hctx, K, T, 1, seed + 1);
        nsrc = 2;
        dsrc[0] = ggml_new_tensor_2d(dctx, hsrc[0]->type, K, M);
        dsrc[1] = ggml_new_tensor_2d(dctx, GGML_TYPE_F32, K, T);
        yr = ggml_mul_mat(hctx, hsrc[0], hsrc[1]);
        ya = spq4k_ggml_mul_mat(dctx, dsrc[0], dsrc[1], b);
    } else {
        struct ggml_tensor *gate = q_weight(hctx, GGML_TYPE_Q4_K, K, M, E, seed, tmp);
        struct ggml_tensor *up = q_weight(hctx, GGML_TYPE_Q4_K, K, M, E, seed + 1, tmp);
        struct ggml_tensor *down = q_weight(hctx, type, M, K, E, seed + 2, tmp);
        struct ggml_tensor *cur = ggml_reshape_2d(hctx, f32_input(hctx, K, T, 1, seed + 3), K, T);
        struct ggml_tensor *sel = ggml_new_tensor_2d(hctx, GGML_TYPE_I32, n_used, T);
        memcpy(sel->data, ids_in, (size_t)n_used * T * sizeof(int32_t));
        struct ggml_tensor *wts = ggml_new_tensor_3d(hctx, GGML_TYPE_F32, 1, n_used, T);
        memcpy(wts->data, w_in, (size_t)n_used * T * sizeof(float));
        struct ggml_tensor *cur3 = ggml_reshape_3d(hctx, cur, K, 1, T);
        struct ggml_tensor *par = ggml_mul(hctx, ggml_silu(hctx, ggml_mul_mat_id(hctx, gate, cur3, sel)),
                                           ggml_mul_mat_id(hctx, up, cur3, sel));
        struct ggml_tensor *weighted = ggml_mul(hctx, ggml_mul_mat_id(hctx, down, par, sel), wts);
        yr = ggml_reshape_2d(hctx, ggml_sum_rows(hctx, ggml_cont(hctx, ggml_permute(hctx, weighted, 1, 0, 2, 3))), K, T);
        hsrc[0] = cur; hsrc[1] = sel; hsrc[2] = wts; hsrc[3] = gate; hsrc[4] = up; hsrc[5] = down;
        nsrc = 6;
        for (int i = 0; i < 6; ++i) {
            dsrc[i] = ggml_new_tensor(dctx, hsrc[i]->type, GGML_MAX_DIMS, hsrc[i]->ne);
        }
        ya = spq4k_ggml_moe_ffn(dctx, dsrc[0], dsrc[1], dsrc[2], dsrc[3], dsrc[4], dsrc[5], b);
    }
    free(tmp);
    int step = 0;
    ggml_backend_buffer_t dbuf = NULL;
    if (!ya) step = 1;
    if (!step && !(dbuf = ggml_backend_alloc_ctx_tensors_from_buft(dctx, buft))) step = 2;
    if (!step) {
        for (int i = 0; i < nsrc; ++i) ggml_backend_tensor_set(dsrc[i], hsrc[i]->data, 0, ggml_nbytes(hsrc[i]));
        if (compute_graph(yr, nthreads) || compute_graph(ya, 1)) step = 3;
        else if (spq4k_ggml_status(b)) step = 4;
    }
    if (!step) {
        memcpy(y_ref, yr->data, ggml_nbytes(yr));
        ggml_backend_tensor_get(ya, y_ada, 0, ggml_nbytes(ya));
        const struct ggml_tensor *W = mode ? dsrc[3] : dsrc[0];
        *wrapped = spq4k_ggml_resident_data(b, W) == W->data;
    }
    if (step) snprintf(err, errlen, "%s check step %d: %s", ggml_backend_buft_name(buft), step, spq4k_ggml_last_error(b));
    spq4k_ggml_free(b);
    if (dbuf) ggml_backend_buffer_free(dbuf);
    ggml_free(dctx);
    ggml_free(hctx);
    return step;
}

int check_device(int mode, int type, int64_t M, int64_t K, int64_t E, int64_t n_used, int64_t T,
                 const int32_t *ids_in, const float *w_in, uint64_t seed, int nthreads, float *y_ref, float *y_ada,
                 int *wrapped, char *err, int errlen) {
    return check_in(&dv_buft, mode, type, M, K, E, n_used, T, ids_in, w_in, seed, nthreads, y_ref, y_ada, wrapped,
                    err, errlen);
}

int check_hostmem_not_host(int mode, int type, int64_t M, int64_t K, int64_t E, int64_t n_used, int64_t T,
                           const int32_t *ids_in, const float *w_in, uint64_t seed, int nthreads, float *y_ref,
                           float *y_ada, int *wrapped, char *err, int errlen) {
    return check_in(&hm_buft, mode, type, M, K, E, n_used, T, ids_in, w_in, seed, nthreads, y_ref, y_ada, wrapped,
                    err, errlen);
}

/* A small dense decoder built twice in one graph of the reference's ggml --
 * the CPU's MUL_MAT nodes (y_ref) and the adapter's (y_ada) -- the node
 * sequence of the engine's dense layer around attention (build_block_decode,
 * desktop/engine/src/forward.cpp:2663-2856) and its output head (:3411-3413):
 * per layer x = x + o(q(xa)) with xa = rms_norm(x) * attn_norm (the
 * attention core, not on this path, is stood in for by q; k and v feed only
 * attention and are left out), then x = x + down(silu(gate(xb)) * up(xb)) with
 * xb = rms_norm(x) * ffn_norm; logits = out(rms_norm(x) * out_norm). All
 * matrices Q4_K; norms, residual adds, SiLU and the product are ggml CPU ops
 * in both graphs. y_* are the logits [n_vocab, T].
 * Per node: every adapter matmul of the second graph (q, o, gate, up, down of
 * each layer, then the head) has a shadow ggml MUL_MAT on the same weight and
 * the same input tensor, so the CPU node is fed the adapter path's own
 * intermediate activations. When nodes_ada / nodes_chk are not NULL, the
 * adapter outputs and their shadows are written there, node after node in
 * that order ([rows, T] each: T * (n_q + 2 n_embd + 2 n_ff) a layer, then
 * T * n_vocab). */
#define DEC_MAX_NODES 64
int check_decoder(int n_layers, int64_t n_embd, int64_t n_q, int64_t n_ff, int64_t n_vocab, int64_t T,
                  uint64_t seed, int nthreads, float *y_ref, float *y_ada, float *nodes_ada, float *nodes_chk,
                  char *err, int errlen) {
    if (5 * n_layers + 1 > DEC_MAX_NODES) {
        snprintf(err, errlen, "at most %d layers", (DEC_MAX_NODES - 1) / 5);
        return -1;
    }
    struct ggml_tensor *node_a[DEC_MAX_NODES], *node_c[DEC_MAX_NODES];
    int nn = 0;
    spq4k_ggml *b;
    int rc = spq4k_ggml_init(0, &b);
    if (rc) {
        snprintf(err, errlen, "spq4k_ggml_init: %d", rc);
        return rc;
    }
    const size_t wvals = (size_t)n_layers * (n_embd * n_q * 2 + n_embd * n_ff * 3) + n_embd * n_vocab;
    struct ggml_context *ctx = new_ctx(wvals + (size_t)(n_embd + n_ff + n_vocab) * T * 400 + (256 << 20));
    const int64_t mx = n_ff * n_embd > n_vocab * n_embd ? n_ff * n_embd : n_vocab * n_embd;
    float *tmp = (float *)malloc((size_t)mx * sizeof(float));
    struct ggml_tensor *x0 = f32_input(ctx, n_embd, T, 1, seed);
    x0 = ggml_reshape_2d(ctx, x0, n_embd, T);
    struct ggml_tensor *xr = x0, *xa = x0;
    uint64_t s = seed + 1;
    const float eps = 1e-6f;
    for (int l = 0; l < n_layers; ++l) {
        struct ggml_tensor *wq = q_weight(ctx, GGML_TYPE_Q4_K, n_embd, n_q, 1, s++, tmp);
        struct ggml_tensor *wo = q_weight(ctx, GGML_TYPE_Q4_K, n_q, n_embd, 1, s++, tmp);
        struct ggml_tensor *wg = q_weight(ctx, GGML_TYPE_Q4_K, n_embd, n_ff, 1, s++, tmp);
        struct ggml_tensor *wu = q_weight(ctx, GGML_TYPE_Q4_K, n_embd, n_ff, 1, s++, tmp);
        struct ggml_tensor *wd = q_weight(ctx, GGML_TYPE_Q4_K, n_ff, n_embd, 1, s++, tmp);
        struct ggml_tensor *an = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, n_embd);
        struct ggml_tensor *fn = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, n_embd);
        normal_fill((float *)an->data, n_embd, s++, 0.2f);
        normal_fill((float *)fn->data, n_embd, s++, 0.2f);
        for (int64_t i = 0; i < n_embd; ++i) {
            ((float *)an->data)[i] += 1.0f;
            ((float *)fn->data)[i] += 1.0f;
        }
        for (int g = 0; g < 2; ++g) {
            struct ggml_tensor **x = g ? &xa : &xr;
            /* the adapter's node for g = 1 (and its shadow), ggml's for g = 0 */
#define DEC_MM(W, IN) (g ? (node_c[nn] = ggml_mul_mat(ctx, W, IN), node_a[nn++] = spq4k_ggml_mul_mat(ctx, W, IN, b)) \
                         : ggml_mul_mat(ctx, W, IN))
            struct ggml_tensor *h = ggml_mul(ctx, ggml_rms_norm(ctx, *x, eps), an);
            struct ggml_tensor *q = DEC_MM(wq, h);
            struct ggml_tensor *o = DEC_MM(wo, q);
            struct ggml_tensor *x1 = ggml_add(ctx, *x, o);
            struct ggml_tensor *hb = ggml_mul(ctx, ggml_rms_norm(ctx, x1, eps), fn);
            struct ggml_tensor *gt = DEC_MM(wg, hb);
            struct ggml_tensor *ut = DEC_MM(wu, hb);
            struct ggml_tensor *par = ggml_mul(ctx, ggml_silu(ctx, gt), ut);
            struct ggml_tensor *dn = DEC_MM(wd, par);
#undef DEC_MM
            *x = ggml_add(ctx, x1, dn);
        }
    }
    struct ggml_tensor *wout = q_weight(ctx, GGML_TYPE_Q4_K, n_embd, n_vocab, 1, s++, tmp);
    struct ggml_tensor *on = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, n_embd);
    normal_fill((float *)on->data, n_embd, s++, 0.2f);
    for (int64_t i = 0; i < n_embd; ++i) ((float *)on->data)[i] += 1.0f;
    free(tmp);
    struct ggml_tensor *yr = ggml_mul_mat(ctx, wout, ggml_mul(ctx, ggml_rms_norm(ctx, xr, eps), on));
    struct ggml_tensor *ha = ggml_mul(ctx, ggml_rms_norm(ctx, xa, eps), on);
    struct ggml_tensor *ya = spq4k_ggml_mul_mat(ctx, wout, ha, b);
    node_c[nn] = ggml_mul_mat(ctx, wout, ha);
    node_a[nn++] = ya;
    for (int i = 0; i < nn; ++i)
        if (!node_a[i]) ya = NULL;   /* graph construction failed */
    if (ya && nodes_ada && nodes_chk) {
        /* the shadows in the graph first, then the logits (finish computes
         * the same graph again, with every node already evaluated once) */
        struct ggml_cgraph *gf = ggml_new_graph(ctx);
        for (int i = 0; i < nn; ++i) {
            ggml_build_forward_expand(gf, node_c[i]);
            ggml_build_forward_expand(gf, node_a[i]);
        }
        ggml_build_forward_expand(gf, yr);
        if (ggml_graph_compute_with_ctx(ctx, gf, nthreads) != GGML_STATUS_SUCCESS) {
            ya = NULL;
        } else {
            size_t off = 0;
            for (int i = 0; i < nn; ++i) {
                memcpy(nodes_ada + off, node_a[i]->data, ggml_nbytes(node_a[i]));
                memcpy(nodes_chk + off, node_c[i]->data, ggml_nbytes(node_c[i]));
                off += (size_t)ggml_nelements(node_a[i]);
            }
        }
    }
    return finish(ctx, b, yr, ya, nthreads, y_ref, y_ada, err, errlen);
}
