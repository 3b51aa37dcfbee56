/*
 * q5k_oracle.c — CPU restatement of the reference's Q5_K path (test oracle).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the Q5_K HIP kernels, never a
 * product path. Built into liboracle_q4k.so with q4k_oracle.c (gcc -O2
 * -ffp-contract=off). Each function cites the reference function it restates,
 * relative to /root/reference/vendor/ggml/src/.
 *
 * Q5_K block (ggml-common.h:334-346), 176 bytes per 256 weights:
 *   d @0, dmin @2 (fp16), scales[12] @4 (the Q4_K 6-bit packing),
 *   qh[32] @16 (high bits), qs[128] @48 (low 4 bits).
 * Weight e = 64 g + 32 h + l (g < 4, h < 2, l < 32) is
 *   q = nibble h of qs[32 g + l] + 16 * bit (2 g + h) of qh[l]   (0..31)
 * in sub-block j = 2 g + h and dequantises to d * sc_j * q - dmin * m_j.
 */
#include "q4k_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline int q5_at(const or_block_q5K *b, int e) {
    const int g = e >> 6, h = (e >> 5) & 1, l = e & 31;
    const uint8_t q = b->qs[32 * g + l];
    const int nib = h ? (q >> 4) : (q & 0x0F);
    return nib + (((b->qh[l] >> (2 * g + h)) & 1) << 4);
}

/* Q5_K encoder. Follows ggml-quants.c:1582-1667 (quantize_row_q5_K_ref): the
 * Q4_K encoder's steps with 5-bit values — per sub-block weights av_x + |x|,
 * make_qkx2_quants(32, 31, ..., rmin = -0.5, rdelta = 0.1, nstep = 15); the
 * 6-bit scale/min packing and fp16 d, dmin of Q4_K; values recomputed as
 * clamp(nearest_int((x + dm) / d), 0, 31) where d * sc != 0; low nibbles
 * packed as Q4_K packs them and bit 4 of value 64 g + 32 h + l set as bit
 * 2 g + h of qh[l]. */
void or_quantize_row_q5K(const float *x, void *vy, int64_t k) {
    or_block_q5K *y = (or_block_q5K *)vy;
    const int64_t nb = k / OR_QK_K;
    uint8_t L[OR_QK_K];
    uint8_t Laux[32];
    float wts[32];
    float mins[8];
    float scales[8];

    for (int64_t i = 0; i < nb; ++i, x += OR_QK_K) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; ++j) {
            const float *xs = x + 32 * j;
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += xs[l] * xs[l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) wts[l] = av_x + fabsf(xs[l]);
            scales[j] = or_qkx2_fit(32, 31, xs, wts, L + 32 * j, &mins[j], Laux, -0.5f, 0.1f, 15);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        uint8_t *s = y[i].scales;
        memset(s, 0, 12);
        for (int j = 0; j < 8; ++j) {
            uint8_t ls = (uint8_t)or_nearest_int(inv_scale * scales[j]);
            uint8_t lm = (uint8_t)or_nearest_int(inv_min * mins[j]);
            if (ls > 63) ls = 63;
            if (lm > 63) lm = 63;
            if (j < 4) {
                s[j] = ls;
                s[j + 4] = lm;
            } else {
                s[j + 4] = (uint8_t)((ls & 0x0F) | ((lm & 0x0F) << 4));
                s[j - 4] |= (uint8_t)((ls >> 4) << 6);
                s[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        y[i].d = or_fp32_to_fp16(max_scale / 63.f);
        y[i].dmin = or_fp32_to_fp16(max_min / 63.f);

        const float dd = or_fp16_to_fp32(y[i].d);
        const float dm0 = or_fp16_to_fp32(y[i].dmin);
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, m;
            or_scale_min_k4(j, s, &sc, &m);
            const float d = dd * (float)sc;
            if (d == 0.0f) continue;
            const float dm = dm0 * (float)m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = or_nearest_int((x[32 * j + ii] + dm) / d);
                l = l < 0 ? 0 : (l > 31 ? 31 : l);
                L[32 * j + ii] = (uint8_t)l;
            }
        }
        memset(y[i].qh, 0, 32);
        for (int g = 0; g < 4; ++g) {
            for (int l = 0; l < 32; ++l) {
                const int l1 = L[64 * g + l], l2 = L[64 * g + 32 + l];
                y[i].qs[32 * g + l] = (uint8_t)((l1 & 0x0F) | ((l2 & 0x0F) << 4));
                y[i].qh[l] |= (uint8_t)(((l1 >> 4) << (2 * g)) | ((l2 >> 4) << (2 * g + 1)));
            }
        }
    }
}

/* ggml_quantize_chunk for Q5_K without an importance matrix.
 * Follows ggml-quants.c:1789-1793 (quantize_q5_K, quant_weights == NULL). */
size_t or_quantize_q5K(const float *src, void *dst, int64_t nrow, int64_t n_per_row) {
    or_quantize_row_q5K(src, dst, nrow * n_per_row);
    return (size_t)(nrow * (n_per_row / OR_QK_K)) * OR_Q5K_BLOCK_BYTES;
}

/* Q5_K -> fp32. Follows ggml-quants.c:1669-1694 (dequantize_row_q5_K):
 * y = (d * sc) * q - (dmin * m), each product and the difference rounded once. */
void or_dequantize_row_q5K(const void *vx, float *y, int64_t k) {
    const or_block_q5K *x = (const or_block_q5K *)vx;
    const int64_t nb = k / OR_QK_K;
    for (int64_t i = 0; i < nb; ++i) {
        const float d = or_fp16_to_fp32(x[i].d);
        const float dmin = or_fp16_to_fp32(x[i].dmin);
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, m;
            or_scale_min_k4(j, x[i].scales, &sc, &m);
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            for (int l = 0; l < 32; ++l)
                y[i * OR_QK_K + 32 * j + l] = d1 * (float)q5_at(&x[i], 32 * j + l) - m1;
        }
    }
}

/* Exact integer sub-block sums S[8 b + j] = sum over the 32 weights of
 * sub-block j of q5 * q8: the integer core of ggml-cpu/quants.c:720-798 and
 * arch/x86/quants.c:2078-2174. */
void or_subblock_sums_q5K(int n, const void *vx, const void *vy, int32_t *S) {
    const or_block_q5K *x = (const or_block_q5K *)vx;
    const or_block_q8K *y = (const or_block_q8K *)vy;
    const int nb = n / OR_QK_K;
    for (int b = 0; b < nb; ++b) {
        for (int j = 0; j < 8; ++j) {
            int32_t s = 0;
            for (int l = 0; l < 32; ++l) s += q5_at(&x[b], 32 * j + l) * (int32_t)y[b].qs[32 * j + l];
            S[8 * b + j] = s;
        }
    }
}

/* Q5_K . Q8_K in the float order of the portable kernel.
 * Follows ggml-cpu/quants.c:720-798 (ggml_vec_dot_q5_K_q8_K_generic): lanes
 * aux32[l] = sum_j sc_j * q5 * q8 over elements 32 j + 8 g + l; per block
 * sums[l] += (fp16(d) * d8) * aux32[l] and sumf -= (fp16(dmin) * d8) *
 * sum_k bsums[k] m_{k/2}; finally sumf += sums[0..7]. */
float or_vec_dot_q5K_generic(int n, const void *vx, const void *vy) {
    const or_block_q5K *x = (const or_block_q5K *)vx;
    const or_block_q8K *y = (const or_block_q8K *)vy;
    const int nb = n / OR_QK_K;
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float sumf = 0;
    for (int b = 0; b < nb; ++b) {
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; ++j) or_scale_min_k4(j, x[b].scales, &sc[j], &mn[j]);
        int32_t aux32[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int e = 0; e < OR_QK_K; ++e) {
            const int16_t p = (int16_t)(q5_at(&x[b], e) * y[b].qs[e]);
            aux32[e & 7] += (int32_t)sc[e >> 5] * p;
        }
        int32_t sumi = 0;
        for (int k = 0; k < 16; ++k) sumi += (int32_t)y[b].bsums[k] * (int32_t)mn[k / 2];
        const float d = or_fp16_to_fp32(x[b].d) * y[b].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
        const float dmin = or_fp16_to_fp32(x[b].dmin) * y[b].d;
        sumf -= dmin * (float)sumi;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* Q5_K . Q8_K in the float order of the x86 kernel.
 * Follows ggml-cpu/arch/x86/quants.c:2078-2174 (AVX2 branch of
 * ggml_vec_dot_q5_K_q8_K) lane by lane: int32 lane m (0..7) holds
 * sum_g sc_{2g} sum_{e<4} q5 q8 (elements 64 g + 4 m + e) + sc_{2g+1} (same at
 * + 32); acc[m] = fma(d8 * fp16(d), float(lane m), acc[m]); the min term is
 * one scalar summs += (-d8 * fp16(dmin)) * sum_j m_j (bsums[2j] + bsums[2j+1]);
 * the result is hsum_float_8(acc) + summs. */
float or_vec_dot_q5K_avx2order(int n, const void *vx, const void *vy) {
    const or_block_q5K *x = (const or_block_q5K *)vx;
    const or_block_q8K *y = (const or_block_q8K *)vy;
    const int nb = n / OR_QK_K;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float summs = 0;
    for (int b = 0; b < nb; ++b) {
        const float d = y[b].d * or_fp16_to_fp32(x[b].d);
        const float dmin = -y[b].d * or_fp16_to_fp32(x[b].dmin);
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; ++j) or_scale_min_k4(j, x[b].scales, &sc[j], &mn[j]);
        int32_t tm = 0;
        for (int j = 0; j < 8; ++j) tm += (int32_t)mn[j] * ((int32_t)y[b].bsums[2 * j] + y[b].bsums[2 * j + 1]);
        summs += dmin * (float)tm;
        int32_t lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int g = 0; g < 4; ++g) {
            for (int m = 0; m < 8; ++m) {
                int32_t lo = 0, hi = 0;
                for (int e = 0; e < 4; ++e) {
                    const int el = 64 * g + 4 * m + e;
                    lo += q5_at(&x[b], el) * (int32_t)y[b].qs[el];
                    hi += q5_at(&x[b], el + 32) * (int32_t)y[b].qs[el + 32];
                }
                lane[m] += (int32_t)sc[2 * g] * lo + (int32_t)sc[2 * g + 1] * hi;
            }
        }
        for (int m = 0; m < 8; ++m) acc[m] = fmaf(d, (float)lane[m], acc[m]);
    }
    const float r0 = acc[4] + acc[0], r1 = acc[5] + acc[1], r2 = acc[6] + acc[2], r3 = acc[7] + acc[3];
    return ((r0 + r2) + (r1 + r3)) + summs;
}

/* The same dot product with the integer parts exact and the combine in
 * double: sum_b fp16(d) d8 I_b - fp16(dmin) d8 M_b. */
double or_vec_dot_q5K_exact(int n, const void *vx, const void *vy) {
    const or_block_q5K *x = (const or_block_q5K *)vx;
    const or_block_q8K *y = (const or_block_q8K *)vy;
    const int nb = n / OR_QK_K;
    double acc = 0;
    int32_t S[8];
    for (int b = 0; b < nb; ++b) {
        or_subblock_sums_q5K(OR_QK_K, &x[b], &y[b], S);
        int64_t I = 0, Mt = 0;
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, m;
            or_scale_min_k4(j, x[b].scales, &sc, &m);
            I += (int64_t)sc * S[j];
            Mt += (int64_t)m * ((int64_t)y[b].bsums[2 * j] + y[b].bsums[2 * j + 1]);
        }
        acc += (double)or_fp16_to_fp32(x[b].d) * (double)y[b].d * (double)I -
               (double)or_fp16_to_fp32(x[b].dmin) * (double)y[b].d * (double)Mt;
    }
    return acc;
}
