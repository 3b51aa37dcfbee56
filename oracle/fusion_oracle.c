/*
 * fusion_oracle.c — CPU restatement of the operations fused around the
 * matvec (test oracle).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the fused GPU paths, never a
 * product path. Built into liboracle_q4k.so (gcc -O2 -ffp-contract=off).
 * Paths relative to /root/reference/vendor/ggml/src/.
 */
#include "q4k_oracle.h"

#include <math.h>

/* ggml_rms_norm followed by ggml_mul by w, per row of K values. Follows
 * ggml-cpu/ops.cpp:3752-3779 (ggml_compute_forward_rms_norm_f32, and its
 * fused RMS_NORM + MUL form): the squares rounded to fp32 and summed in
 * double in index order; mean = (float)(sum / K); scale = 1.0f / sqrtf(mean
 * + eps); y = x * scale * w evaluated left to right. */
void or_rms_norm(const float *x, int64_t K, int64_t T, const float *w, float eps, float *y) {
    for (int64_t t = 0; t < T; ++t) {
        const float *xr = x + t * K;
        double sum = 0.0;
        for (int64_t i = 0; i < K; ++i) sum += (double)(xr[i] * xr[i]);
        const float mean = (float)(sum / (double)K);
        const float scale = 1.0f / sqrtf(mean + eps);
        float *yr = y + t * K;
        for (int64_t i = 0; i < K; ++i) yr[i] = xr[i] * scale * (w ? w[i] : 1.0f);
    }
}

/* y = silu(g) * u element-wise: ggml_silu (ggml_silu_f32, ggml-cpu/vec.h:1064-1066,
 * x / (1 + expf(-x)); the x86 kernels use their own vector exp, within an ulp
 * of it) then ggml_mul. */
void or_swiglu(const float *g, const float *u, int64_t n, float *y) {
    for (int64_t i = 0; i < n; ++i) {
        const float s = g[i] / (1.0f + expf(-g[i]));
        y[i] = s * u[i];
    }
}
