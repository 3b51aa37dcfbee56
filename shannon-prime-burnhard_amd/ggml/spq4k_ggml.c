/* spq4k_ggml.c — ggml custom-op nodes for Q4_K / Q5_K / Q6_K / Q8_0 GGML_OP_MUL_MAT /
 * GGML_OP_MUL_MAT_ID, run on the GPU through spq4k (include/spq4k_ggml.h).
 *
 * The node is ggml_custom_4d (ggml.h:2610-2623) with the weight, the
 * activations (and ids) as sources, one task, and the binding as userdata.
 * Its callback:
 *   - does all the work on ith == 0, as the engine's own custom ops do
 *     (desktop/engine/src/forward.cpp:1248, burn_moe_op.cpp:203);
 *   - finds the weight in the resident table, uploading it on first use
 *     (spq4k_weights_upload_type with the tensor's ggml type), keyed by
 *     tensor, data pointer, byte count, type and shape so that a buffer
 *     reused for another tensor is uploaded again (spq4k_ggml_forget drops
 *     entries);
 *   - when every tensor of the node lives in a device (non-host) backend
 *     buffer -- a HIP build of ggml on this GPU -- runs on those device
 *     pointers in place: the weight is wrapped (spq4k_weights_wrap_type, no
 *     copy) and the activations and output never cross PCIe; the call
 *     synchronises before returning, as the next node may read the output;
 *   - otherwise reads activations and ids, and writes the output, through
 *     ggml_backend_tensor_get / _set when the tensor has a backend buffer and
 *     through tensor->data otherwise;
 *   - runs spq4k_mul_mat_host / spq4k_moe_host (GGML_OP_MUL_MAT: y[t][m] =
 *     W[m] . x[t]; GGML_OP_MUL_MAT_ID with the CPU driver's semantics,
 *     ggml-cpu.c:1521-1690), or spq4k_moe_ffn_host for the routed-expert FFN
 *     block node (the BURN_MOE op's unit, burn_moe_op.cpp:202-372): one copy
 *     of the activations in and of the block's output out, where the stock
 *     graph's three MUL_MAT_ID nodes would each cross PCIe.
 * A failure is recorded in the binding and the node's output is NaN.
 */
#include "spq4k_ggml.h"

#include <errno.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ggml-backend.h"

struct resident {
    const struct ggml_tensor *t;
    const void *data;
    size_t nbytes;
    enum ggml_type type;
    int64_t ne[3];
    spq4k_weights *w;
};

struct spq4k_ggml {
    spq4k_ctx *ctx;
    struct resident *res;
    int nres, cap;
    int status;
    char err[256];
};

int spq4k_ggml_init(int device, spq4k_ggml **out) {
    if (!out) return -EINVAL;
    *out = NULL;
    spq4k_ggml *b = (spq4k_ggml *)calloc(1, sizeof *b);
    if (!b) return -ENOMEM;
    int rc = spq4k_init(device, &b->ctx);
    if (rc) {
        free(b);
        return rc;
    }
    *out = b;
    return 0;
}

void spq4k_ggml_free(spq4k_ggml *b) {
    if (!b) return;
    for (int i = 0; i < b->nres; ++i) spq4k_weights_free(b->res[i].w);
    free(b->res);
    spq4k_free(b->ctx);
    free(b);
}

int spq4k_ggml_status(const spq4k_ggml *b) { return b ? b->status : -EINVAL; }

int spq4k_ggml_forget(spq4k_ggml *b, const struct ggml_tensor *W) {
    if (!b) return 0;
    int n = 0;
    for (int i = 0; i < b->nres;) {
        if (!W || b->res[i].t == W) {
            spq4k_weights_free(b->res[i].w);
            b->res[i] = b->res[--b->nres];
            ++n;
        } else {
            ++i;
        }
    }
    return n;
}

const char *spq4k_ggml_last_error(const spq4k_ggml *b) { return b ? b->err : "null binding"; }

const void *spq4k_ggml_resident_data(const spq4k_ggml *b, const struct ggml_tensor *W) {
    if (!b || !W) return NULL;
    for (int i = 0; i < b->nres; ++i)
        if (b->res[i].t == W && b->res[i].data == W->data) return spq4k_weights_data(b->res[i].w);
    return NULL;
}

static void fail(spq4k_ggml *b, struct ggml_tensor *dst, int code, const char *what) {
    if (b->status == 0) {
        b->status = code;
        snprintf(b->err, sizeof b->err, "%s: %s", what, code == -EIO ? spq4k_last_error(b->ctx) : strerror(-code));
    }
    const size_t n = (size_t)ggml_nelements(dst);
    float *nan = (float *)malloc(n * sizeof(float));
    if (!nan) return;
    for (size_t i = 0; i < n; ++i) nan[i] = NAN;
    if (dst->buffer)
        ggml_backend_tensor_set(dst, nan, 0, n * sizeof(float));
    else
        memcpy(dst->data, nan, n * sizeof(float));
    free(nan);
}

/* whether t lives in device memory of the binding's GPU, which spq4k can use
 * in place: a buffer that is not host memory (is_host false, as a HIP build of
 * ggml's device buffers) whose data the HIP runtime confirms as this GPU's
 * device memory. ggml's CPU extra buffer types (repack, AMX) and other
 * backends' buffers report is_host false too; their tensors take the copy
 * path. */
static int on_device(const spq4k_ggml *b, const struct ggml_tensor *t) {
    const struct ggml_tensor *s = t->view_src ? t->view_src : t;
    return s->buffer && !ggml_backend_buffer_is_host(s->buffer) && t->data &&
           spq4k_ptr_on_device(b->ctx, t->data, ggml_nbytes(t)) == 1;
}

/* tensor bytes in host memory: the tensor's own when it has no backend
 * buffer (*owned = 0), else a copy (*owned = 1) */
static void *host_bytes(const struct ggml_tensor *t, int *owned) {
    const size_t n = ggml_nbytes(t);
    if (!t->buffer) {
        *owned = 0;
        return t->data;
    }
    void *p = malloc(n);
    if (p) ggml_backend_tensor_get(t, p, 0, n);
    *owned = 1;
    return p;
}

/* the resident copy of W: found by tensor, data pointer, byte count, type
 * and shape (a recycled context can put a tensor of another type or shape at
 * the same addresses), else uploaded */
static int resident_weight(spq4k_ggml *b, const struct ggml_tensor *W, int64_t M, int64_t K, int64_t E,
                           spq4k_weights **out) {
    const size_t nbytes = ggml_nbytes(W);
    for (int i = 0; i < b->nres; ++i) {
        const struct resident *r = &b->res[i];
        if (r->t == W && r->data == W->data && r->nbytes == nbytes && r->type == W->type && r->ne[0] == W->ne[0] &&
            r->ne[1] == W->ne[1] && r->ne[2] == W->ne[2]) {
            *out = r->w;
            return 0;
        }
    }
    if (b->nres == b->cap) {
        const int cap = b->cap ? 2 * b->cap : 64;
        struct resident *r = (struct resident *)realloc(b->res, (size_t)cap * sizeof *r);
        if (!r) return -ENOMEM;
        b->res = r;
        b->cap = cap;
    }
    spq4k_weights *w = NULL;
    int rc;
    if (on_device(b, W)) {
        /* already in device memory: adopt it in place, no copy */
        rc = spq4k_weights_wrap_type(b->ctx, (int)W->type, W->data, M, K, E, &w);
    } else {
        int owned;
        void *bytes = host_bytes(W, &owned);
        if (!bytes) return -ENOMEM;
        rc = spq4k_weights_upload_type(b->ctx, (int)W->type, bytes, M, K, E, &w);
        if (owned) free(bytes);
    }
    if (rc) return rc;
    b->res[b->nres++] = (struct resident){W, W->data, nbytes, W->type, {W->ne[0], W->ne[1], W->ne[2]}, w};
    *out = w;
    return 0;
}

static void run_mul_mat(struct ggml_tensor *dst, int ith, int nth, void *userdata) {
    (void)nth;
    if (ith != 0) return;
    spq4k_ggml *b = (spq4k_ggml *)userdata;
    const struct ggml_tensor *W = dst->src[0], *x = dst->src[1];
    const int64_t K = W->ne[0], M = W->ne[1], T = x->ne[1];
    spq4k_weights *w;
    int rc = resident_weight(b, W, M, K, 1, &w);
    if (rc) {
        fail(b, dst, rc, "spq4k_ggml_mul_mat: weight upload");
        return;
    }
    if (on_device(b, x) && on_device(b, dst)) {
        /* device-resident node: the activations and the output stay on the GPU */
        rc = spq4k_mul_mat(b->ctx, w, (const float *)x->data, (float *)dst->data, T);
        if (!rc) rc = spq4k_synchronize(b->ctx);
        if (rc) fail(b, dst, rc, "spq4k_ggml_mul_mat");
        return;
    }
    int ox, oy = 0;
    const float *X = (const float *)host_bytes(x, &ox);
    float *Y = dst->buffer ? (float *)malloc((size_t)M * T * sizeof(float)) : (float *)dst->data;
    if (dst->buffer) oy = 1;
    if (!X || !Y) {
        if (ox) free((void *)X);
        if (oy) free(Y);
        fail(b, dst, -ENOMEM, "spq4k_ggml_mul_mat");
        return;
    }
    rc = spq4k_mul_mat_host(b->ctx, w, X, Y, T);
    if (rc == 0 && oy) ggml_backend_tensor_set(dst, Y, 0, (size_t)M * T * sizeof(float));
    if (ox) free((void *)X);
    if (oy) free(Y);
    if (rc) fail(b, dst, rc, "spq4k_ggml_mul_mat");
}

static void run_mul_mat_id(struct ggml_tensor *dst, int ith, int nth, void *userdata) {
    (void)nth;
    if (ith != 0) return;
    spq4k_ggml *b = (spq4k_ggml *)userdata;
    const struct ggml_tensor *as = dst->src[0], *x = dst->src[1], *ids = dst->src[2];
    const int64_t K = as->ne[0], M = as->ne[1], E = as->ne[2];
    const int64_t ne11 = x->ne[1], T = x->ne[2], n_used = ids->ne[0];
    spq4k_weights *w;
    int rc = resident_weight(b, as, M, K, E, &w);
    if (rc) {
        fail(b, dst, rc, "spq4k_ggml_mul_mat_id: weight upload");
        return;
    }
    if (on_device(b, x) && on_device(b, ids) && on_device(b, dst)) {
        rc = spq4k_moe(b->ctx, w, (const int32_t *)ids->data, n_used, ne11, T, (const float *)x->data,
                       (float *)dst->data);
        if (!rc) rc = spq4k_synchronize(b->ctx);
        if (rc) fail(b, dst, rc, "spq4k_ggml_mul_mat_id");
        return;
    }
    int ox, oi, oy = 0;
    const float *X = (const float *)host_bytes(x, &ox);
    const int32_t *I = (const int32_t *)host_bytes(ids, &oi);
    float *Y = dst->buffer ? (float *)malloc((size_t)M * n_used * T * sizeof(float)) : (float *)dst->data;
    if (dst->buffer) oy = 1;
    if (X && I && Y) rc = spq4k_moe_host(b->ctx, w, I, n_used, ne11, T, X, Y);
    else rc = -ENOMEM;
    if (rc == 0 && oy) ggml_backend_tensor_set(dst, Y, 0, (size_t)M * n_used * T * sizeof(float));
    if (ox) free((void *)X);
    if (oi) free((void *)I);
    if (oy) free(Y);
    if (rc) fail(b, dst, rc, "spq4k_ggml_mul_mat_id");
}

static void run_moe_ffn(struct ggml_tensor *dst, int ith, int nth, void *userdata) {
    (void)nth;
    if (ith != 0) return;
    spq4k_ggml *b = (spq4k_ggml *)userdata;
    const struct ggml_tensor *cur = dst->src[0], *sel = dst->src[1], *wts = dst->src[2];
    const struct ggml_tensor *gate = dst->src[3], *up = dst->src[4], *down = dst->src[5];
    const int64_t n_embd = cur->ne[0], T = cur->ne[1], n_used = sel->ne[0];
    spq4k_weights *wg, *wu, *wd;
    int rc = resident_weight(b, gate, gate->ne[1], gate->ne[0], gate->ne[2], &wg);
    if (!rc) rc = resident_weight(b, up, up->ne[1], up->ne[0], up->ne[2], &wu);
    if (!rc) rc = resident_weight(b, down, down->ne[1], down->ne[0], down->ne[2], &wd);
    if (rc) {
        fail(b, dst, rc, "spq4k_ggml_moe_ffn: weight upload");
        return;
    }
    if (on_device(b, cur) && on_device(b, sel) && on_device(b, wts) && on_device(b, dst)) {
        rc = spq4k_moe_ffn(b->ctx, wg, wu, wd, (const int32_t *)sel->data, (const float *)wts->data, n_used, T,
                           (const float *)cur->data, (float *)dst->data);
        if (!rc) rc = spq4k_synchronize(b->ctx);
        if (rc) fail(b, dst, rc, "spq4k_ggml_moe_ffn");
        return;
    }
    int ox, oi, ow, oy = 0;
    const float *X = (const float *)host_bytes(cur, &ox);
    const int32_t *I = (const int32_t *)host_bytes(sel, &oi);
    const float *Wt = (const float *)host_bytes(wts, &ow);
    float *Y = dst->buffer ? (float *)malloc((size_t)n_embd * T * sizeof(float)) : (float *)dst->data;
    if (dst->buffer) oy = 1;
    if (X && I && Wt && Y) rc = spq4k_moe_ffn_host(b->ctx, wg, wu, wd, I, Wt, n_used, T, X, Y);
    else rc = -ENOMEM;
    if (rc == 0 && oy) ggml_backend_tensor_set(dst, Y, 0, (size_t)n_embd * T * sizeof(float));
    if (ox) free((void *)X);
    if (oi) free((void *)I);
    if (ow) free((void *)Wt);
    if (oy) free(Y);
    if (rc) fail(b, dst, rc, "spq4k_ggml_moe_ffn");
}

/* weight types the library runs (spq4k.h: SPQ4K_TYPE_Q4_K, _Q5_K, _Q6_K, _Q8_0) */
static int supported(enum ggml_type t) {
    return t == GGML_TYPE_Q4_K || t == GGML_TYPE_Q5_K || t == GGML_TYPE_Q6_K || t == GGML_TYPE_Q8_0;
}

struct ggml_tensor *spq4k_ggml_mul_mat(struct ggml_context *ctx, struct ggml_tensor *W, struct ggml_tensor *x,
                                       spq4k_ggml *b) {
    if (!ctx || !W || !x || !b || !supported(W->type) || x->type != GGML_TYPE_F32 || x->ne[0] != W->ne[0] ||
        W->ne[2] != 1 || W->ne[3] != 1 || x->ne[2] != 1 || x->ne[3] != 1 || !ggml_is_contiguous(W) ||
        !ggml_is_contiguous(x))
        return NULL;
    struct ggml_tensor *args[2] = {W, x};
    return ggml_custom_4d(ctx, GGML_TYPE_F32, W->ne[1], x->ne[1], 1, 1, args, 2, run_mul_mat, 1, b);
}

struct ggml_tensor *spq4k_ggml_mul_mat_id(struct ggml_context *ctx, struct ggml_tensor *as, struct ggml_tensor *x,
                                          struct ggml_tensor *ids, spq4k_ggml *b) {
    if (!ctx || !as || !x || !ids || !b || !supported(as->type) || x->type != GGML_TYPE_F32 ||
        ids->type != GGML_TYPE_I32 || x->ne[0] != as->ne[0] || ids->ne[1] != x->ne[2] ||
        (x->ne[1] != 1 && x->ne[1] != ids->ne[0]) || as->ne[3] != 1 || x->ne[3] != 1 || !ggml_is_contiguous(as) ||
        !ggml_is_contiguous(x) || !ggml_is_contiguous(ids))
        return NULL;
    struct ggml_tensor *args[3] = {as, x, ids};
    return ggml_custom_4d(ctx, GGML_TYPE_F32, as->ne[1], ids->ne[0], ids->ne[1], 1, args, 3, run_mul_mat_id, 1, b);
}

struct ggml_tensor *spq4k_ggml_moe_ffn(struct ggml_context *ctx, struct ggml_tensor *cur, struct ggml_tensor *selected,
                                       struct ggml_tensor *weights, struct ggml_tensor *gate_exps,
                                       struct ggml_tensor *up_exps, struct ggml_tensor *down_exps, spq4k_ggml *b) {
    if (!ctx || !cur || !selected || !weights || !gate_exps || !up_exps || !down_exps || !b) return NULL;
    const int64_t n_embd = cur->ne[0], T = cur->ne[1], k = selected->ne[0];
    const struct ggml_tensor *banks[3] = {gate_exps, up_exps, down_exps};
    for (int i = 0; i < 3; ++i)
        if (!supported(banks[i]->type) || banks[i]->ne[3] != 1 || !ggml_is_contiguous(banks[i])) return NULL;
    if (cur->type != GGML_TYPE_F32 || cur->ne[2] != 1 || cur->ne[3] != 1 || !ggml_is_contiguous(cur) ||
        selected->type != GGML_TYPE_I32 || selected->ne[1] != T || selected->ne[2] != 1 ||
        !ggml_is_contiguous(selected) || weights->type != GGML_TYPE_F32 || ggml_nelements(weights) != k * T ||
        !ggml_is_contiguous(weights) || gate_exps->type != up_exps->type || gate_exps->ne[0] != n_embd ||
        up_exps->ne[0] != n_embd || up_exps->ne[1] != gate_exps->ne[1] || up_exps->ne[2] != gate_exps->ne[2] ||
        down_exps->ne[0] != gate_exps->ne[1] || down_exps->ne[1] != n_embd || down_exps->ne[2] != gate_exps->ne[2] ||
        k > gate_exps->ne[2])
        return NULL;
    struct ggml_tensor *args[6] = {cur, selected, weights, gate_exps, up_exps, down_exps};
    return ggml_custom_4d(ctx, GGML_TYPE_F32, n_embd, T, 1, 1, args, 6, run_moe_ffn, 1, b);
}
