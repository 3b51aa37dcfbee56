/*
 * q8_0_oracle.c — CPU restatement of the reference's Q8_0 path (test oracle).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the Q8_0 HIP kernels, never a
 * product path. Built into liboracle_q4k.so (gcc -O2 -ffp-contract=off). Each
 * function cites the reference function it restates, relative to
 * /root/reference/vendor/ggml/src/.
 *
 * Q8_0 block (ggml-common.h:241-245), 34 bytes per 32 values: fp16 d @0,
 * int8 qs[32] @2; value = qs * d. Q8_0 weights take Q8_0 activations
 * (vec_dot_type, ggml-cpu/ggml-cpu.c:258-261), quantised by the CPU
 * backend's quantize_row_q8_0 (arch/x86/quants.c:302-397), which rounds
 * differently from the file-format encoder quantize_row_q8_0_ref
 * (ggml-quants.c:234-257); both are restated.
 */
#include "q4k_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* Round half to even of a float holding |v| < 2^23, as _mm256_round_ps with
 * _MM_ROUND_NEAREST does; written with the 1.5 * 2^23 addition (the same
 * trick as nearest_int), then subtracted back. */
static float rint_even(float v) {
    if (!(fabsf(v) < 8388608.0f)) return v;
    const float big = v < 0 ? -8388608.0f : 8388608.0f;
    return (v + big) - big;
}

/* Activations fp32 -> Q8_0 in the CPU backend's order. Follows
 * ggml-cpu/arch/x86/quants.c:302-367 (quantize_row_q8_0, AVX2): max |x| of
 * the 32 values; d = max / 127 stored as fp16; id = 127 / max (0 for max 0);
 * q = round-half-even(x * id) as int8. */
void or_quantize_row_q8_0(const float *x, void *vy, int64_t k) {
    or_block_q8_0 *y = (or_block_q8_0 *)vy;
    const int64_t nb = k / OR_QK8_0;
    for (int64_t i = 0; i < nb; ++i, x += OR_QK8_0) {
        float amax = 0;
        for (int j = 0; j < OR_QK8_0; ++j) {
            const float a = fabsf(x[j]);
            amax = a > amax ? a : amax;
        }
        const float d = amax / 127.f;
        y[i].d = or_fp32_to_fp16(d);
        const float id = amax != 0.0f ? 127.f / amax : 0.0f;
        for (int j = 0; j < OR_QK8_0; ++j) {
            const float r = rint_even(x[j] * id);
            y[i].qs[j] = (int8_t)(r > 127.f ? 127 : (r < -128.f ? -128 : (int)r));
        }
    }
}

/* Weights fp32 -> Q8_0 as the model-file encoder makes them. Follows
 * ggml-quants.c:234-257 (quantize_row_q8_0_ref), reached by
 * ggml_quantize_chunk(GGML_TYPE_Q8_0, ..., imatrix = NULL): d = amax / 127,
 * id = 1 / d, q = roundf(x * id) (half away from zero). */
void or_quantize_row_q8_0_ref(const float *x, void *vy, int64_t k) {
    or_block_q8_0 *y = (or_block_q8_0 *)vy;
    const int64_t nb = k / OR_QK8_0;
    for (int64_t i = 0; i < nb; ++i, x += OR_QK8_0) {
        float amax = 0.0f;
        for (int j = 0; j < OR_QK8_0; ++j) amax = fmaxf(amax, fabsf(x[j]));
        const float d = amax / 127;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = or_fp32_to_fp16(d);
        for (int j = 0; j < OR_QK8_0; ++j) y[i].qs[j] = (int8_t)roundf(x[j] * id);
    }
}

/* Q8_0 -> fp32. Follows ggml-quants.c:491-505 (dequantize_row_q8_0). */
void or_dequantize_row_q8_0(const void *vx, float *y, int64_t k) {
    const or_block_q8_0 *x = (const or_block_q8_0 *)vx;
    const int64_t nb = k / OR_QK8_0;
    for (int64_t i = 0; i < nb; ++i) {
        const float d = or_fp16_to_fp32(x[i].d);
        for (int j = 0; j < OR_QK8_0; ++j) y[i * OR_QK8_0 + j] = (float)x[i].qs[j] * d;
    }
}

/* S[b] = sum of qx * qy over block b: the integer core of both dots. */
void or_block_sums_q8_0(int n, const void *vx, const void *vy, int32_t *S) {
    const or_block_q8_0 *x = (const or_block_q8_0 *)vx;
    const or_block_q8_0 *y = (const or_block_q8_0 *)vy;
    for (int b = 0; b < n / OR_QK8_0; ++b) {
        int32_t s = 0;
        for (int j = 0; j < OR_QK8_0; ++j) s += (int32_t)x[b].qs[j] * y[b].qs[j];
        S[b] = s;
    }
}

/* Q8_0 . Q8_0 in the portable order. Follows ggml-cpu/quants.c:400-428
 * (ggml_vec_dot_q8_0_q8_0_generic): sumf += sumi * (dx * dy). */
float or_vec_dot_q8_0_generic(int n, const void *vx, const void *vy) {
    const or_block_q8_0 *x = (const or_block_q8_0 *)vx;
    const or_block_q8_0 *y = (const or_block_q8_0 *)vy;
    float sumf = 0;
    for (int b = 0; b < n / OR_QK8_0; ++b) {
        int32_t s = 0;
        for (int j = 0; j < OR_QK8_0; ++j) s += (int32_t)x[b].qs[j] * y[b].qs[j];
        sumf += (float)s * (or_fp16_to_fp32(x[b].d) * or_fp16_to_fp32(y[b].d));
    }
    return sumf;
}

/* Q8_0 . Q8_0 in the x86 kernel's order. Follows
 * ggml-cpu/arch/x86/quants.c:1187-1204 (AVX2 branch): lane m (0..7) of a block
 * is the int32 sum over values 4m .. 4m+3 (mul_sum_i8_pairs_float, :122-134);
 * acc[m] = fma(dx * dy, float(lane m), acc[m]); hsum_float_8. */
float or_vec_dot_q8_0_avx2order(int n, const void *vx, const void *vy) {
    const or_block_q8_0 *x = (const or_block_q8_0 *)vx;
    const or_block_q8_0 *y = (const or_block_q8_0 *)vy;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = 0; b < n / OR_QK8_0; ++b) {
        const float d = or_fp16_to_fp32(x[b].d) * or_fp16_to_fp32(y[b].d);
        for (int m = 0; m < 8; ++m) {
            int32_t s = 0;
            for (int e = 0; e < 4; ++e) s += (int32_t)x[b].qs[4 * m + e] * y[b].qs[4 * m + e];
            acc[m] = fmaf(d, (float)s, acc[m]);
        }
    }
    const float r0 = acc[4] + acc[0], r1 = acc[5] + acc[1], r2 = acc[6] + acc[2], r3 = acc[7] + acc[3];
    return (r0 + r2) + (r1 + r3);
}

double or_vec_dot_q8_0_exact(int n, const void *vx, const void *vy) {
    const or_block_q8_0 *x = (const or_block_q8_0 *)vx;
    const or_block_q8_0 *y = (const or_block_q8_0 *)vy;
    double acc = 0;
    for (int b = 0; b < n / OR_QK8_0; ++b) {
        int32_t s = 0;
        for (int j = 0; j < OR_QK8_0; ++j) s += (int32_t)x[b].qs[j] * y[b].qs[j];
        acc += (double)or_fp16_to_fp32(x[b].d) * (double)or_fp16_to_fp32(y[b].d) * (double)s;
    }
    return acc;
}

/* GGML_OP_MUL_MAT for Q8_0 weights: each activation row is converted with
 * the CPU backend's quantize_row_q8_0, then dst[t][r] = vec_dot (order 1 =
 * x86, 0 = generic). Follows ggml-cpu/ggml-cpu.c:1241-1439 as the Q4_K driver. */
int or_mul_mat_q8_0(const void *W, int64_t M, int64_t K, const float *X, int64_t T, float *Y, int order) {
    if (K % OR_QK8_0) return -22;
    const int64_t nb = K / OR_QK8_0;
    const size_t row_bytes = (size_t)nb * OR_Q8_0_BLOCK_BYTES;
    or_block_q8_0 *q8 = (or_block_q8_0 *)malloc((size_t)nb * sizeof(or_block_q8_0));
    for (int64_t t = 0; t < T; ++t) {
        or_quantize_row_q8_0(X + t * K, q8, K);
        for (int64_t r = 0; r < M; ++r) {
            const void *wr = (const uint8_t *)W + (size_t)r * row_bytes;
            Y[t * M + r] = order ? or_vec_dot_q8_0_avx2order((int)K, wr, q8) : or_vec_dot_q8_0_generic((int)K, wr, q8);
        }
    }
    free(q8);
    return 0;
}

/* GGML_OP_MUL_MAT_ID for a Q8_0 bank (ggml-cpu/ggml-cpu.c:1521-1690). */
int or_mul_mat_id_q8_0(const void *as, int64_t M, int64_t K, int64_t E, const float *X, int64_t ne11,
                       const int32_t *ids, int64_t k, int64_t T, float *Y, int order) {
    if (K % OR_QK8_0) return -22;
    const int64_t nb = K / OR_QK8_0;
    const size_t row_bytes = (size_t)nb * OR_Q8_0_BLOCK_BYTES;
    or_block_q8_0 *q8 = (or_block_q8_0 *)malloc((size_t)nb * sizeof(or_block_q8_0));
    for (int64_t t = 0; t < T; ++t) {
        for (int64_t s = 0; s < k; ++s) {
            const int32_t e = ids[t * k + s];
            if (e < 0 || e >= E) { free(q8); return -22; }
            or_quantize_row_q8_0(X + (t * ne11 + (s % ne11)) * K, q8, K);
            const uint8_t *base = (const uint8_t *)as + (size_t)e * row_bytes * (size_t)M;
            for (int64_t r = 0; r < M; ++r) {
                const void *wr = base + (size_t)r * row_bytes;
                Y[(t * k + s) * M + r] =
                    order ? or_vec_dot_q8_0_avx2order((int)K, wr, q8) : or_vec_dot_q8_0_generic((int)K, wr, q8);
            }
        }
    }
    free(q8);
    return 0;
}
