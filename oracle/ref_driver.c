/*
 * ref_driver.c — a thin harness around the reference's own ggml CPU library,
 * compiled from /root/reference/vendor/ggml by oracle/Makefile into
 * oracle/_ref/. TEST INFRASTRUCTURE ONLY: used by tests/golden/gen_golden.py
 * to write golden vectors, by tests to pin the oracle, and by bench.py's
 * cpu_baseline leg to time the reference's CPU path.
 *
 * Everything below calls the reference's public API (ggml.h, ggml-cpu.h);
 * no reference arithmetic is re-implemented here.
 *   - type traits (Q4_K, and Q5_K / Q6_K through the *_type forms):
 *     ggml_get_type_traits(Q4_K)->to_float (dequantize_row_q4_K),
 *     ggml_get_type_traits_cpu(Q8_K)->from_float (quantize_row_q8_K),
 *     ggml_get_type_traits_cpu(Q4_K)->vec_dot (ggml_vec_dot_q4_K_q8_K),
 *     ggml_quantize_chunk(Q4_K, ..., imatrix = NULL)
 *   - graphs: ggml_mul_mat / ggml_mul_mat_id nodes computed by
 *     ggml_graph_compute on a persistent ggml threadpool, i.e.
 *     ggml_compute_forward_mul_mat(_id) in ggml-cpu/ggml-cpu.c:1241 / :1521,
 *     with weights wrapped in place like llama_weights.cpp:701 does.
 */
#include "ggml.h"
#include "ggml-cpu.h"

#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* declared in ggml-cpu/quants.h (internal); exported by the library */
void ggml_vec_dot_q4_K_q8_K_generic(int n, float *s, size_t bs, const void *vx, size_t bx,
                                    const void *vy, size_t by, int nrc);
void ggml_vec_dot_q6_K_q8_K_generic(int n, float *s, size_t bs, const void *vx, size_t bx,
                                    const void *vy, size_t by, int nrc);
void ggml_vec_dot_q5_K_q8_K_generic(int n, float *s, size_t bs, const void *vx, size_t bx,
                                    const void *vy, size_t by, int nrc);
void ggml_vec_dot_q8_0_q8_0_generic(int n, float *s, size_t bs, const void *vx, size_t bx,
                                    const void *vy, size_t by, int nrc);

static int g_inited = 0;
static void ensure_init(void) {
    if (!g_inited) { ggml_cpu_init(); g_inited = 1; }
}

size_t ref_quantize_q4K(const float *src, void *dst, int64_t nrow, int64_t n_per_row) {
    ensure_init();
    return ggml_quantize_chunk(GGML_TYPE_Q4_K, src, dst, 0, nrow, n_per_row, NULL);
}

void ref_dequant_q4K(const void *x, float *y, int64_t k) {
    ensure_init();
    ggml_get_type_traits(GGML_TYPE_Q4_K)->to_float(x, y, k);
}

void ref_quantize_q8K(const float *x, void *y, int64_t k) {
    ensure_init();
    ggml_get_type_traits_cpu(GGML_TYPE_Q8_K)->from_float(x, y, k);
}

float ref_vec_dot(int n, const void *vx, const void *vy) {
    ensure_init();
    float s = 0;
    ggml_get_type_traits_cpu(GGML_TYPE_Q4_K)->vec_dot(n, &s, 0, vx, 0, vy, 0, 1);
    return s;
}

float ref_vec_dot_generic(int n, const void *vx, const void *vy) {
    ensure_init();
    float s = 0;
    ggml_vec_dot_q4_K_q8_K_generic(n, &s, 0, vx, 0, vy, 0, 1);
    return s;
}

/* the same traits for any weight type (GGML_TYPE_Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14) */
size_t ref_quantize_type(int type, const float *src, void *dst, int64_t nrow, int64_t n_per_row) {
    ensure_init();
    return ggml_quantize_chunk((enum ggml_type)type, src, dst, 0, nrow, n_per_row, NULL);
}

void ref_dequant_type(int type, const void *x, float *y, int64_t k) {
    ensure_init();
    ggml_get_type_traits((enum ggml_type)type)->to_float(x, y, k);
}

float ref_vec_dot_type(int type, int n, const void *vx, const void *vy, int generic) {
    ensure_init();
    float s = 0;
    if (generic && type == GGML_TYPE_Q6_K) ggml_vec_dot_q6_K_q8_K_generic(n, &s, 0, vx, 0, vy, 0, 1);
    else if (generic && type == GGML_TYPE_Q5_K) ggml_vec_dot_q5_K_q8_K_generic(n, &s, 0, vx, 0, vy, 0, 1);
    else if (generic && type == GGML_TYPE_Q8_0) ggml_vec_dot_q8_0_q8_0_generic(n, &s, 0, vx, 0, vy, 0, 1);
    else if (generic) ggml_vec_dot_q4_K_q8_K_generic(n, &s, 0, vx, 0, vy, 0, 1);
    else ggml_get_type_traits_cpu((enum ggml_type)type)->vec_dot(n, &s, 0, vx, 0, vy, 0, 1);
    return s;
}

/* the CPU backend's activation quantiser for a weight type's vec_dot_type
 * (Q8_K for the K-quants, Q8_0 for Q8_0): ggml_get_type_traits_cpu(vdt)->from_float */
void ref_quantize_vec_dot_type(int type, const float *x, void *y, int64_t k) {
    ensure_init();
    const enum ggml_type vdt = ggml_get_type_traits_cpu((enum ggml_type)type)->vec_dot_type;
    ggml_get_type_traits_cpu(vdt)->from_float(x, y, k);
}

int ref_has_avx512(void) { return ggml_cpu_has_avx512(); }
int ref_has_avx2(void) { return ggml_cpu_has_avx2(); }

/* ---- graphs ------------------------------------------------------------ */
typedef struct {
    struct ggml_context *ctx;
    struct ggml_cgraph *gf;
    struct ggml_threadpool *tp;
    struct ggml_cplan plan;
    void *work;
} ref_graph;

static ref_graph *graph_begin(int n_nodes) {
    ensure_init();
    ref_graph *g = (ref_graph *)calloc(1, sizeof(ref_graph));
    size_t meta = ggml_tensor_overhead() * (size_t)(4 * n_nodes + 8)
                + ggml_graph_overhead_custom((size_t)(4 * n_nodes + 8), false) + 4096;
    struct ggml_init_params ip = { meta, NULL, true };
    g->ctx = ggml_init(ip);
    g->gf = ggml_new_graph_custom(g->ctx, (size_t)(4 * n_nodes + 8), false);
    return g;
}

static int graph_finish(ref_graph *g, int nthreads) {
    struct ggml_threadpool_params tpp = ggml_threadpool_params_default(nthreads);
    g->tp = ggml_threadpool_new(&tpp);
    if (!g->tp) return -1;
    g->plan = ggml_graph_plan(g->gf, nthreads, g->tp);
    if (g->plan.work_size > 0) {
        g->work = malloc(g->plan.work_size);
        if (!g->work) return -1;
        g->plan.work_data = (uint8_t *)g->work;
    }
    return 0;
}

void ref_graph_destroy(void *h) {
    ref_graph *g = (ref_graph *)h;
    if (!g) return;
    if (g->tp) ggml_threadpool_free(g->tp);
    free(g->work);
    ggml_free(g->ctx);
    free(g);
}

/* n dense matmuls dst_i[T][M_i] = W_i[M_i x K_i] * X_i[T][K_i], all in one
 * graph (computed node after node, as ggml's CPU backend does for a layer).
 * Buffers are the caller's and are used in place. */
void *ref_mm_create_type(int type, int n, const void *const *W, const int64_t *M, const int64_t *K,
                         const float *const *X, float *const *Y, int64_t T, int nthreads) {
    ref_graph *g = graph_begin(n);
    for (int i = 0; i < n; ++i) {
        struct ggml_tensor *w = ggml_new_tensor_2d(g->ctx, (enum ggml_type)type, K[i], M[i]);
        struct ggml_tensor *x = ggml_new_tensor_2d(g->ctx, GGML_TYPE_F32, K[i], T);
        w->data = (void *)W[i];
        x->data = (void *)X[i];
        struct ggml_tensor *y = ggml_mul_mat(g->ctx, w, x);
        y->data = Y[i];
        ggml_build_forward_expand(g->gf, y);
    }
    if (graph_finish(g, nthreads) != 0) { ref_graph_destroy(g); return NULL; }
    return g;
}

void *ref_mm_create(int n, const void *const *W, const int64_t *M, const int64_t *K,
                    const float *const *X, float *const *Y, int64_t T, int nthreads) {
    return ref_mm_create_type(GGML_TYPE_Q4_K, n, W, M, K, X, Y, T, nthreads);
}

/* dst[T][k][M] = mul_mat_id(as[E][M][K], X[T][ne11][K], ids[T][k]) */
void *ref_mmid_create_type(int type, const void *as, int64_t M, int64_t K, int64_t E, const float *X,
                           int64_t ne11, const int32_t *ids, int64_t k, int64_t T, float *Y,
                           int nthreads) {
    ref_graph *g = graph_begin(1);
    struct ggml_tensor *a = ggml_new_tensor_3d(g->ctx, (enum ggml_type)type, K, M, E);
    struct ggml_tensor *b = ggml_new_tensor_3d(g->ctx, GGML_TYPE_F32, K, ne11, T);
    struct ggml_tensor *id = ggml_new_tensor_2d(g->ctx, GGML_TYPE_I32, k, T);
    a->data = (void *)as;
    b->data = (void *)X;
    id->data = (void *)ids;
    struct ggml_tensor *y = ggml_mul_mat_id(g->ctx, a, b, id);
    y->data = Y;
    ggml_build_forward_expand(g->gf, y);
    if (graph_finish(g, nthreads) != 0) { ref_graph_destroy(g); return NULL; }
    return g;
}

void *ref_mmid_create(const void *as, int64_t M, int64_t K, int64_t E, const float *X,
                      int64_t ne11, const int32_t *ids, int64_t k, int64_t T, float *Y,
                      int nthreads) {
    return ref_mmid_create_type(GGML_TYPE_Q4_K, as, M, K, E, X, ne11, ids, k, T, Y, nthreads);
}

/* Runs the graph iters times; returns the wall seconds of each run in secs. */
int ref_graph_run(void *h, int iters, double *secs) {
    ref_graph *g = (ref_graph *)h;
    for (int it = 0; it < iters; ++it) {
        struct timespec t0, t1;
        clock_gettime(CLOCK_MONOTONIC, &t0);
        enum ggml_status st = ggml_graph_compute(g->gf, &g->plan);
        clock_gettime(CLOCK_MONOTONIC, &t1);
        if (st != GGML_STATUS_SUCCESS) return -1;
        if (secs) secs[it] = (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
    }
    return 0;
}

/* ---- the operations fused around the matvec ------------------------------ */
/* owned intermediate buffers of a graph (freed with it) */
typedef struct {
    ref_graph g;
    void *bufs[8];
    int nbufs;
} ref_graph_b;

static float *graph_buf(ref_graph_b *gb, size_t n) {
    float *p = (float *)malloc(n * sizeof(float));
    gb->bufs[gb->nbufs++] = p;
    return p;
}

void ref_graph_b_destroy(void *h) {
    ref_graph_b *gb = (ref_graph_b *)h;
    if (!gb) return;
    for (int i = 0; i < gb->nbufs; ++i) free(gb->bufs[i]);
    if (gb->g.tp) ggml_threadpool_free(gb->g.tp);
    free(gb->g.work);
    ggml_free(gb->g.ctx);
    free(gb);
}

static ref_graph_b *graph_b_begin(int n_nodes) {
    ref_graph *g = graph_begin(n_nodes);
    ref_graph_b *gb = (ref_graph_b *)calloc(1, sizeof(ref_graph_b));
    gb->g = *g;
    free(g);
    return gb;
}

/* Xn[T][K] = ggml_mul(ggml_rms_norm(X, eps), w) */
void *ref_rms_norm_create(const float *X, int64_t K, int64_t T, const float *w, float eps, float *Xn,
                          int nthreads) {
    ref_graph_b *gb = graph_b_begin(2);
    struct ggml_context *c = gb->g.ctx;
    struct ggml_tensor *x = ggml_new_tensor_2d(c, GGML_TYPE_F32, K, T);
    struct ggml_tensor *wt = ggml_new_tensor_1d(c, GGML_TYPE_F32, K);
    x->data = (void *)X;
    wt->data = (void *)w;
    struct ggml_tensor *n = ggml_rms_norm(c, x, eps);
    n->data = graph_buf(gb, (size_t)K * T);
    struct ggml_tensor *m = ggml_mul(c, n, wt);
    m->data = Xn;
    ggml_build_forward_expand(gb->g.gf, m);
    if (graph_finish(&gb->g, nthreads) != 0) { ref_graph_b_destroy(gb); return NULL; }
    return gb;
}

/* The dense SwiGLU front half of forward.cpp:1693-1706: xb = x, or
 * ggml_mul(ggml_rms_norm(x, eps), w) when w is given; Y[T][M] =
 * ggml_mul(ggml_silu(mul_mat(Wg, xb)), mul_mat(Wu, xb)). */
void *ref_swiglu_create(int type, const void *Wg, const void *Wu, int64_t M, int64_t K, const float *X, int64_t T,
                        const float *w, float eps, float *Y, int nthreads) {
    ref_graph_b *gb = graph_b_begin(6);
    struct ggml_context *c = gb->g.ctx;
    struct ggml_tensor *x = ggml_new_tensor_2d(c, GGML_TYPE_F32, K, T);
    x->data = (void *)X;
    struct ggml_tensor *xb = x;
    if (w) {
        struct ggml_tensor *wt = ggml_new_tensor_1d(c, GGML_TYPE_F32, K);
        wt->data = (void *)w;
        struct ggml_tensor *n = ggml_rms_norm(c, x, eps);
        n->data = graph_buf(gb, (size_t)K * T);
        xb = ggml_mul(c, n, wt);
        xb->data = graph_buf(gb, (size_t)K * T);
    }
    struct ggml_tensor *wg = ggml_new_tensor_2d(c, (enum ggml_type)type, K, M);
    struct ggml_tensor *wu = ggml_new_tensor_2d(c, (enum ggml_type)type, K, M);
    wg->data = (void *)Wg;
    wu->data = (void *)Wu;
    struct ggml_tensor *g = ggml_mul_mat(c, wg, xb);
    g->data = graph_buf(gb, (size_t)M * T);
    struct ggml_tensor *u = ggml_mul_mat(c, wu, xb);
    u->data = graph_buf(gb, (size_t)M * T);
    struct ggml_tensor *s = ggml_silu(c, g);
    s->data = graph_buf(gb, (size_t)M * T);
    struct ggml_tensor *y = ggml_mul(c, s, u);
    y->data = Y;
    ggml_build_forward_expand(gb->g.gf, y);
    if (graph_finish(&gb->g, nthreads) != 0) { ref_graph_b_destroy(gb); return NULL; }
    return gb;
}

int ref_graph_b_run(void *h) {
    ref_graph_b *gb = (ref_graph_b *)h;
    return ggml_graph_compute(gb->g.gf, &gb->g.plan) == GGML_STATUS_SUCCESS ? 0 : -1;
}
