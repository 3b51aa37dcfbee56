/*
 * beast_driver.c — test infrastructure only (never linked into libspq4k).
 *
 * Exposes the reference's own beast_matvec (a static function of
 * desktop/beast_canyon/sp_beast_canyon.c:1122-1134, the BurnHard scalar
 * dequant-then-dot matvec), its expert routing (sp_beast_route_experts,
 * :385-443) and the MoE forward built on them (:455-562) to the tests: this
 * file includes that source file where it lies under /root/reference and adds
 * exported wrappers. `make -C
 * oracle ref` compiles it with the flags the reference's CMake gives that file
 * under GCC (desktop/beast_canyon/CMakeLists.txt:52-54: -O3 -mfma -mf16c and
 * GCC's default fp contraction), with -march=native narrowed to x86-64-v3 so
 * the library loads on any AVX2 host (the loops it runs are element-wise or
 * serial, so the vector width does not change a result). Everything else in
 * the file is unreferenced and dropped by --gc-sections; the result links
 * with -z defs, against libc and libm only.
 */
#include "sp_beast_canyon.c"

__attribute__((visibility("default")))
int ref_beast_matvec(const void *W, unsigned type, const float *x, float *y, int n_out, int n_in) {
    float *scratch = (float *)malloc((size_t)n_in * sizeof(float));
    if (!scratch) return -1;
    sp_optane_tensor_t t;
    memset(&t, 0, sizeof t);
    t.ptr = (void *)W;
    t.type = type;
    beast_matvec(&t, x, y, scratch, n_out, n_in);
    free(scratch);
    return 0;
}

/* sp_beast_route_experts (sp_beast_canyon.c:385-443) on a zeroed engine whose
 * only settings are the top-k (config.n_experts_per_token) and no GPUs: the
 * reference's own softmax, top-k and renormalisation. */
__attribute__((visibility("default")))
int ref_beast_route(const float *logits, int n_experts, int top_k, int *ids, float *scores) {
    sp_beast_engine_t *engine = (sp_beast_engine_t *)calloc(1, sizeof *engine);
    if (!engine) return -1;
    engine->config.n_experts_per_token = top_k;
    sp_beast_route_experts(engine, logits, n_experts);
    const sp_expert_routing_t *r = &engine->routing;
    for (int k = 0; k < r->n_selected; ++k) {
        ids[k] = r->expert_ids[k];
        scores[k] = r->expert_scores[k];
    }
    const int n = r->n_selected;
    free(engine);
    return n;
}

/* sp_beast_moe_forward (sp_beast_canyon.c:455-562) for one token over expert
 * banks held contiguously in memory (E experts of gate / up [n_ff x n_embd]
 * and down [n_embd x n_ff]), each bank of its own type as the reference's
 * tensors are: the reference's routing, beast_matvec and beast_silu_mul, and
 * its per-expert loop restated (:486-545: gate, up, silu(gate) * up, down,
 * output += score * down_out, output zeroed first); the engine's reservoir
 * lookup, prefetch, CRT telemetry and barrier, which do not touch the
 * numbers, are left out. Returns the number of experts. */
__attribute__((visibility("default")))
int ref_beast_moe_types(const void *gate, unsigned tg, const void *up, unsigned tu, const void *down, unsigned td,
                        int n_experts, int n_embd, int n_ff, const float *logits, int top_k, const float *hidden,
                        float *output, int *ids, float *scores) {
    int k_sel = ref_beast_route(logits, n_experts, top_k, ids, scores);
    if (k_sel < 0) return -1;
    const size_t gb = beast_row_bytes(tg, n_embd) * (size_t)n_ff;      /* one expert of gate */
    const size_t ub = beast_row_bytes(tu, n_embd) * (size_t)n_ff;      /* one expert of up */
    const size_t db = beast_row_bytes(td, n_ff) * (size_t)n_embd;      /* one expert of down */
    float *gate_buf = (float *)malloc((size_t)n_ff * sizeof(float));
    float *up_buf = (float *)malloc((size_t)n_ff * sizeof(float));
    float *down_out = (float *)malloc((size_t)n_embd * sizeof(float));
    float *scratch = (float *)malloc((size_t)(n_embd > n_ff ? n_embd : n_ff) * sizeof(float));
    if (!gate_buf || !up_buf || !down_out || !scratch) return -1;
    memset(output, 0, (size_t)n_embd * sizeof(float));
    sp_optane_tensor_t t_g, t_u, t_d;
    memset(&t_g, 0, sizeof t_g);
    memset(&t_u, 0, sizeof t_u);
    memset(&t_d, 0, sizeof t_d);
    t_g.type = tg;
    t_u.type = tu;
    t_d.type = td;
    for (int k = 0; k < k_sel; ++k) {
        const int eid = ids[k];
        const float score = scores[k];
        t_g.ptr = (void *)((const uint8_t *)gate + (size_t)eid * gb);
        t_u.ptr = (void *)((const uint8_t *)up + (size_t)eid * ub);
        t_d.ptr = (void *)((const uint8_t *)down + (size_t)eid * db);
        beast_matvec(&t_g, hidden, gate_buf, scratch, n_ff, n_embd);
        beast_matvec(&t_u, hidden, up_buf, scratch, n_ff, n_embd);
        beast_silu_mul(gate_buf, up_buf, n_ff);
        beast_matvec(&t_d, gate_buf, down_out, scratch, n_embd, n_ff);
        for (int i = 0; i < n_embd; i++) {
            output[i] += score * down_out[i];
        }
    }
    free(gate_buf);
    free(up_buf);
    free(down_out);
    free(scratch);
    return k_sel;
}

/* the forward with one type for all three banks */
__attribute__((visibility("default")))
int ref_beast_moe(const void *gate, const void *up, const void *down, unsigned type, int n_experts, int n_embd,
                  int n_ff, const float *logits, int top_k, const float *hidden, float *output, int *ids,
                  float *scores) {
    return ref_beast_moe_types(gate, type, up, type, down, type, n_experts, n_embd, n_ff, logits, top_k, hidden,
                               output, ids, scores);
}
