/*
 * q6k_oracle.c — CPU restatement of the reference's Q6_K path (test oracle).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the Q6_K HIP kernels, never a
 * product path. Built into liboracle_q4k.so with q4k_oracle.c (gcc -O2
 * -ffp-contract=off). Each function cites the reference function it restates,
 * relative to /root/reference/vendor/ggml/src/.
 *
 * Q6_K block (ggml-common.h:348-357), 210 bytes per 256 weights:
 *   ql[128] @0    low 4 bits, qh[64] @128  high 2 bits,
 *   scales[16] @192  int8 per 16-weight sub-block,  d @208  fp16.
 * Weight e = 128 n + 32 h + l (n < 2, h < 4, l < 32) is
 *   q = (nibble h>>1 of ql[64 n + 32 (h & 1) + l]) | (bits 2h..2h+1 of qh[32 n + l]) << 4
 * and dequantises to d * scales[8 n + 2 h + l / 16] * (q - 32).
 */
#include "q4k_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* 6-bit value (0..63) of element e of a block. */
static inline int q6_at(const or_block_q6K *b, int e) {
    const int n = e >> 7, h = (e >> 5) & 3, l = e & 31;
    const uint8_t lo = b->ql[64 * n + 32 * (h & 1) + l];
    const int nib = (h >> 1) ? (lo >> 4) : (lo & 0x0F);
    const int hi = (b->qh[32 * n + l] >> (2 * h)) & 3;
    return nib | (hi << 4);
}

/* ------------------------------------------------------------------------ */
/* Symmetric fit of n values to L in [0, 2 nmax) (stored as l + nmax).
 * Follows ggml-quants.c:566-635 (make_qx_quants) for the call the Q6_K
 * encoder makes: rmse_type = 1 (weights x^2), no importance weights. The
 * signed value of largest magnitude sets iscale = -nmax / max; the first
 * rounding gives the least-squares scale sumlx / suml2; then 18 perturbed
 * inverse scales -(nmax + 0.1 is) / max, is = -9..9 without 0, replace it when
 * sumlx^2 > best * suml2. Operation order as in the reference, so the returned
 * scale and L are bit-identical. */
static float qx_fit(int n, int nmax, const float *x, int8_t *L) {
    float max = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = (float)(-nmax) / max;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = or_nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (int8_t)(l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    float scale = suml2 != 0.f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -((float)nmax + 0.1f * (float)is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = or_nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * (float)l;
            suml2 += w * (float)l * (float)l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = or_nearest_int(iscale * x[i]);
                l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
                L[i] = (int8_t)(l + nmax);
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

/* Q6_K encoder. Follows ggml-quants.c:1807-1875 (quantize_row_q6_K_ref):
 * sixteen 16-value fits (qx_fit with nmax 32); the fit scale of largest
 * magnitude (first one on ties) sets iscale = -128 / max_scale, d =
 * fp16(1 / iscale) and the int8 sub-block scales min(127, nearest_int(iscale *
 * scale_j)); a block whose largest fit scale is below 1e-15 is all zero.
 * The 6-bit values are recomputed from the stored d * scale_j as
 * clamp(nearest_int(x / (d * scale_j)), -32, 31) + 32, keeping the fit's L
 * where d * scale_j == 0, and packed per the layout in the file header. */
void or_quantize_row_q6K(const float *x, void *vy, int64_t k) {
    or_block_q6K *y = (or_block_q6K *)vy;
    const int64_t nb = k / OR_QK_K;
    int8_t L[OR_QK_K];
    float scales[16];
    for (int64_t i = 0; i < nb; ++i, x += OR_QK_K) {
        float max_scale = 0, max_abs_scale = 0;
        for (int ib = 0; ib < 16; ++ib) {
            const float s = qx_fit(16, 32, x + 16 * ib, L + 16 * ib);
            scales[ib] = s;
            const float as = fabsf(s);
            if (as > max_abs_scale) { max_abs_scale = as; max_scale = s; }
        }
        if (max_abs_scale < 1e-15f) {
            memset(&y[i], 0, sizeof y[i]);
            continue;
        }
        const float iscale = -128.f / max_scale;
        y[i].d = or_fp32_to_fp16(1 / iscale);
        for (int ib = 0; ib < 16; ++ib) {
            const int v = or_nearest_int(iscale * scales[ib]);
            y[i].scales[ib] = (int8_t)(v < 127 ? v : 127);
        }
        const float dd = or_fp16_to_fp32(y[i].d);
        for (int j = 0; j < 16; ++j) {
            const float d = dd * (float)y[i].scales[j];
            if (d == 0.0f) continue;
            for (int ii = 0; ii < 16; ++ii) {
                int l = or_nearest_int(x[16 * j + ii] / d);
                l = l < -32 ? -32 : (l > 31 ? 31 : l);
                L[16 * j + ii] = (int8_t)(l + 32);
            }
        }
        for (int n = 0; n < 2; ++n) {
            const int8_t *Ln = L + 128 * n;
            uint8_t *ql = y[i].ql + 64 * n;
            uint8_t *qh = y[i].qh + 32 * n;
            for (int l = 0; l < 32; ++l) {
                ql[l] = (uint8_t)((Ln[l] & 0x0F) | ((Ln[l + 64] & 0x0F) << 4));
                ql[l + 32] = (uint8_t)((Ln[l + 32] & 0x0F) | ((Ln[l + 96] & 0x0F) << 4));
                qh[l] = (uint8_t)((Ln[l] >> 4) | ((Ln[l + 32] >> 4) << 2) | ((Ln[l + 64] >> 4) << 4) |
                                  ((Ln[l + 96] >> 4) << 6));
            }
        }
    }
}

/* ggml_quantize_chunk for Q6_K without an importance matrix.
 * Follows ggml-quants.c:1992-1996 (quantize_q6_K, quant_weights == NULL):
 * the whole nrow x n_per_row array is encoded as one row. */
size_t or_quantize_q6K(const float *src, void *dst, int64_t nrow, int64_t n_per_row) {
    or_quantize_row_q6K(src, dst, nrow * n_per_row);
    return (size_t)(nrow * (n_per_row / OR_QK_K)) * OR_Q6K_BLOCK_BYTES;
}

/* Q6_K -> fp32. Follows ggml-quants.c:1877-1906 (dequantize_row_q6_K):
 * y = (d * scale) * (q - 32), each product rounded once. */
void or_dequantize_row_q6K(const void *vx, float *y, int64_t k) {
    const or_block_q6K *x = (const or_block_q6K *)vx;
    const int64_t nb = k / OR_QK_K;
    for (int64_t i = 0; i < nb; ++i) {
        const float d = or_fp16_to_fp32(x[i].d);
        for (int e = 0; e < OR_QK_K; ++e) {
            const int j = e >> 4;   /* 8 n + 2 h + l / 16 */
            const float ds = d * (float)x[i].scales[j];
            y[i * OR_QK_K + e] = ds * (float)(q6_at(&x[i], e) - 32);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Exact integer sub-block sums S[16 b + j] = sum over the 16 weights of
 * sub-block j of block b of (q - 32) * q8. No reference function returns them;
 * they are the integer core of ggml-cpu/quants.c:800-852 and
 * arch/x86/quants.c:2306-2366. */
void or_subblock_sums_q6K(int n, const void *vx, const void *vy, int32_t *S) {
    const or_block_q6K *x = (const or_block_q6K *)vx;
    const or_block_q8K *y = (const or_block_q8K *)vy;
    const int nb = n / OR_QK_K;
    for (int b = 0; b < nb; ++b) {
        for (int j = 0; j < 16; ++j) {
            int32_t s = 0;
            for (int l = 0; l < 16; ++l) s += (q6_at(&x[b], 16 * j + l) - 32) * (int32_t)y[b].qs[16 * j + l];
            S[16 * b + j] = s;
        }
    }
}

/* Q6_K . Q8_K in the float order of the portable kernel.
 * Follows ggml-cpu/quants.c:800-852 (ggml_vec_dot_q6_K_q8_K_generic): eight
 * int32 lanes aux32[l] = sum_j scale_j * (q - 32) * q8 over elements 8 g + l;
 * per block sums[l] += (fp16(d) * d8) * aux32[l]; then sumf += sums[0..7]. */
float or_vec_dot_q6K_generic(int n, const void *vx, const void *vy) {
    const or_block_q6K *x = (const or_block_q6K *)vx;
    const or_block_q8K *y = (const or_block_q8K *)vy;
    const int nb = n / OR_QK_K;
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = 0; b < nb; ++b) {
        int32_t aux32[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int e = 0; e < OR_QK_K; ++e) {
            const int16_t p = (int16_t)((q6_at(&x[b], e) - 32) * y[b].qs[e]);
            aux32[e & 7] += (int32_t)x[b].scales[e >> 4] * p;
        }
        const float d = or_fp16_to_fp32(x[b].d) * y[b].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
    }
    float sumf = 0;
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* Q6_K . Q8_K in the float order of the x86 kernel that the reference's CPU
 * backend runs. Follows ggml-cpu/arch/x86/quants.c:2300-2366 (AVX2 branch of
 * ggml_vec_dot_q6_K_q8_K) lane by lane: int32 lane m (0..7) holds, over both
 * 128-value halves and the four 32-value quarters h, scale_{8n+2h+m/4} times
 * the sum of q * q8 (q unsigned, 0..63) over elements 128 n + 32 h + 4 m .. + 3,
 * minus 32 (bsums[2m] scale_{2m} + bsums[2m+1] scale_{2m+1}); then
 * acc[m] = fma(d8 * fp16(d), float(lane m), acc[m]) and hsum_float_8
 * (arch/x86/quants.c:43-49). */
float or_vec_dot_q6K_avx2order(int n, const void *vx, const void *vy) {
    const or_block_q6K *x = (const or_block_q6K *)vx;
    const or_block_q8K *y = (const or_block_q8K *)vy;
    const int nb = n / OR_QK_K;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = 0; b < nb; ++b) {
        const float d = y[b].d * or_fp16_to_fp32(x[b].d);
        int32_t lane[8];
        for (int m = 0; m < 8; ++m) {
            int32_t s = 0;
            for (int nn = 0; nn < 2; ++nn) {
                for (int h = 0; h < 4; ++h) {
                    int32_t p = 0;
                    for (int e = 0; e < 4; ++e) {
                        const int el = 128 * nn + 32 * h + 4 * m + e;
                        p += q6_at(&x[b], el) * (int32_t)y[b].qs[el];
                    }
                    s += (int32_t)x[b].scales[8 * nn + 2 * h + m / 4] * p;
                }
            }
            const int32_t sub = (int32_t)y[b].bsums[2 * m] * x[b].scales[2 * m] +
                                (int32_t)y[b].bsums[2 * m + 1] * x[b].scales[2 * m + 1];
            lane[m] = s - sub * 32;
        }
        for (int m = 0; m < 8; ++m) acc[m] = fmaf(d, (float)lane[m], acc[m]);
    }
    const float r0 = acc[4] + acc[0], r1 = acc[5] + acc[1], r2 = acc[6] + acc[2], r3 = acc[7] + acc[3];
    return (r0 + r2) + (r1 + r3);
}

/* The same dot product with the integer part exact and the float combine in
 * double: sum_b fp16(d) * d8 * sum_j scale_j * S_bj. */
double or_vec_dot_q6K_exact(int n, const void *vx, const void *vy) {
    const or_block_q6K *x = (const or_block_q6K *)vx;
    const or_block_q8K *y = (const or_block_q8K *)vy;
    const int nb = n / OR_QK_K;
    double acc = 0;
    int32_t S[16];
    for (int b = 0; b < nb; ++b) {
        or_subblock_sums_q6K(OR_QK_K, &x[b], &y[b], S);
        int64_t I = 0;
        for (int j = 0; j < 16; ++j) I += (int64_t)x[b].scales[j] * S[j];
        acc += (double)or_fp16_to_fp32(x[b].d) * (double)y[b].d * (double)I;
    }
    return acc;
}
