/*
 * q4k_oracle.c — CPU restatement of the reference's Q4_K path (test oracle).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never a product
 * path. Build: oracle/Makefile (gcc -O2 -ffp-contract=off). Each function
 * cites the reference function it restates, relative to
 * /root/reference/vendor/ggml/src/.
 */
#include "q4k_oracle.h"
#include "synth_math.h"

#include <math.h>
#include <string.h>
#include <stdlib.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32. Follows ggml-impl.h:384-430 (ggml_compute_fp16_to_fp32 /
 * ggml_compute_fp32_to_fp16): an exact widening and a round-to-nearest-even
 * narrowing with NaN -> 0x7E00|sign. Written here from the IEEE-754 binary16
 * definition; pinned against numpy's float16 over every half value and a
 * sweep of floats (tests/test_oracle_math.py). */
float or_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24, exact in fp32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return u2f(f2u(v) | sign);
    }
    if (exp == 31) {
        return u2f(sign | 0x7F800000u | (man << 13));
    }
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t or_fp32_to_fp16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return sign | 0x7E00u;            /* NaN */
    if (ax >= 0x477FF000u) return sign | 0x7C00u;           /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                 /* below 2^-14: subnormal half */
        float v = u2f(ax) * 16777216.0f;                    /* |f| * 2^24, exact */
        float r = (v + 8388608.0f) - 8388608.0f;            /* RNE to integer (v < 2^10) */
        return sign | (uint16_t)r;
    }
    uint32_t e = (ax >> 23) - 112u;                         /* rebias 127 -> 15 */
    uint32_t man = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return sign | (uint16_t)h;
}

/* ------------------------------------------------------------------------ */
/* Round to nearest, ties to even, valid for |v| <= 2^22 - 1.
 * Follows ggml-quants.c:559-564 (nearest_int): adding 1.5 * 2^23 places the
 * rounded integer in the low mantissa bits. Outside the valid range the same
 * bit pattern is returned as the reference would return, so that clamped
 * call sites stay bit-identical. */
int or_nearest_int(float v) {
    float biased = v + 12582912.0f;
    return (int)(f2u(biased) & 0x007FFFFFu) - 0x00400000;
}

/* ------------------------------------------------------------------------ */
/* Sub-block j (0..7) scale and min from the 12 packed bytes.
 * Follows ggml-quants.c:818-825 (get_scale_min_k4): bytes 0-3 hold the low
 * 6 bits of scales 0-3 (top 2 bits: high bits of scales 4-7), bytes 4-7 the
 * same for mins, bytes 8-11 the low nibbles of scale/min 4-7. */
void or_scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 0x3F;
        *m  = s[j + 4] & 0x3F;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *m  = (uint8_t)((s[j + 4] >> 4)   | ((s[j] >> 6) << 4));
    }
}

/* ------------------------------------------------------------------------ */
/* Weighted min/max fit of one 32-value sub-block to L in [0, nmax].
 * Follows ggml-quants.c:737-816 (make_qkx2_quants) with use_mad = false:
 * an initial fit from (min, max), then nstep+1 candidate inverse scales
 * (rmin + rdelta*is + nmax)/(max - min), each refined by the weighted
 * least-squares (scale, min) for its rounding; the lowest weighted squared
 * error wins. The operation order matches the reference so that the chosen
 * L, scale and min are bit-identical. Returns scale, writes -min. */
float or_qkx2_fit(int n, int nmax, const float *x, const float *w, uint8_t *L,
                 float *neg_min, uint8_t *Laux, float rmin, float rdelta, int nstep) {
    float lo = x[0], hi = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (lo > 0) lo = 0;
    if (hi == lo) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *neg_min = -lo;
        return 0.0f;
    }
    float inv = (float)nmax / (hi - lo);
    float scale = 1.0f / inv;
    float best = 0.0f;
    for (int i = 0; i < n; ++i) {
        int l = or_nearest_int(inv * (x[i] - lo));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        L[i] = (uint8_t)l;
        float diff = scale * (float)L[i] + lo - x[i];
        diff = diff * diff;
        best += w[i] * diff;
    }
    if (nstep < 1) {
        *neg_min = -lo;
        return scale;
    }
    for (int is = 0; is <= nstep; ++is) {
        inv = (rmin + rdelta * (float)is + (float)nmax) / (hi - lo);
        float sl = 0, sl2 = 0, sxl = 0;
        for (int i = 0; i < n; ++i) {
            int l = or_nearest_int(inv * (x[i] - lo));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t)l;
            float fl = (float)l;
            sl  += w[i] * fl;
            sl2 += w[i] * fl * fl;
            sxl += w[i] * fl * x[i];
        }
        float D = sum_w * sl2 - sl * sl;
        if (D > 0) {
            float cs = (sum_w * sxl - sum_x * sl) / D;
            float cm = (sl2 * sum_x - sl * sxl) / D;
            if (cm > 0) {
                cm = 0;
                cs = sxl / sl2;
            }
            float err = 0;
            for (int i = 0; i < n; ++i) {
                float diff = cs * (float)Laux[i] + cm - x[i];
                diff = diff * diff;
                err += w[i] * diff;
            }
            if (err < best) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best = err;
                scale = cs;
                lo = cm;
            }
        }
    }
    *neg_min = -lo;
    return scale;
}

/* Q4_K encoder. Follows ggml-quants.c:1395-1465 (quantize_row_q4_K_ref):
 * per sub-block weights av_x + |x| with av_x = sqrt(mean x^2); qkx2_fit with
 * (rmin, rdelta, nstep) = (-1, 0.1, 20); scales and mins requantised to 6 bits
 * against max/63 and packed per or_scale_min_k4; d, dmin stored as fp16; the
 * 4-bit values recomputed from the stored (d*sc, dmin*m) as
 * clamp(nearest_int((x + dm)/d), 0, 15), keeping the fit's L where d*sc == 0;
 * nibble packing q[l] = L[l] | L[l+32] << 4 per 64 values. */
void or_quantize_row_q4K(const float *x, void *vy, int64_t k) {
    or_block_q4K *y = (or_block_q4K *)vy;
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
            float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) wts[l] = av_x + fabsf(xs[l]);
            scales[j] = or_qkx2_fit(32, 15, xs, wts, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        float inv_min   = max_min   > 0 ? 63.f / max_min   : 0.f;
        uint8_t *s = y[i].scales;
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
                s[j]     |= (uint8_t)((lm >> 4) << 6);
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
                l = l < 0 ? 0 : (l > 15 ? 15 : l);
                L[32 * j + ii] = (uint8_t)l;
            }
        }
        uint8_t *q = y[i].qs;
        for (int g = 0; g < 4; ++g) {
            for (int l = 0; l < 32; ++l) {
                q[32 * g + l] = (uint8_t)(L[64 * g + l] | (L[64 * g + 32 + l] << 4));
            }
        }
    }
}

/* ggml_quantize_chunk for Q4_K without an importance matrix.
 * Follows ggml-quants.c:1564-1568 (quantize_q4_K, quant_weights == NULL):
 * the whole nrow x n_per_row array is encoded as one row. */
size_t or_quantize_q4K(const float *src, void *dst, int64_t nrow, int64_t n_per_row) {
    or_quantize_row_q4K(src, dst, nrow * n_per_row);
    return (size_t)(nrow * (n_per_row / OR_QK_K)) * OR_Q4K_BLOCK_BYTES;
}

/* Q4_K -> fp32. Follows ggml-quants.c:1467-1489 (dequantize_row_q4_K):
 * y = (d*sc) * q - (dmin*m), each product and the difference rounded once. */
void or_dequantize_row_q4K(const void *vx, float *y, int64_t k) {
    const or_block_q4K *x = (const or_block_q4K *)vx;
    const int64_t nb = k / OR_QK_K;
    for (int64_t i = 0; i < nb; ++i) {
        const float d = or_fp16_to_fp32(x[i].d);
        const float dmin = or_fp16_to_fp32(x[i].dmin);
        for (int g = 0; g < 4; ++g) {
            uint8_t sc0, m0, sc1, m1;
            or_scale_min_k4(2 * g, x[i].scales, &sc0, &m0);
            or_scale_min_k4(2 * g + 1, x[i].scales, &sc1, &m1);
            const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
            const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
            const uint8_t *q = x[i].qs + 32 * g;
            float *yo = y + i * OR_QK_K + 64 * g;
            for (int l = 0; l < 32; ++l) yo[l]      = d1 * (float)(q[l] & 0x0F) - mm1;
            for (int l = 0; l < 32; ++l) yo[32 + l] = d2 * (float)(q[l] >> 4) - mm2;
        }
    }
}

/* fp32 -> Q8_K. Follows ggml-quants.c:2692-2729 (quantize_row_q8_K_ref):
 * the first element of largest |x| sets max (with its sign);
 * iscale = -127/max; q = min(127, nearest_int(iscale * x)); bsums are sums of
 * 16 consecutive q; d = 1/iscale. An all-zero block gives d = 0 and q = 0;
 * the reference leaves that block's bsums unwritten, this restatement writes
 * zeros (their dot-product contribution is multiplied by d = 0 either way). */
void or_quantize_row_q8K(const float *x, void *vy, int64_t k) {
    or_block_q8K *y = (or_block_q8K *)vy;
    const int64_t nb = k / OR_QK_K;
    for (int64_t i = 0; i < nb; ++i, x += OR_QK_K) {
        float amax = 0, vmax = 0;
        for (int j = 0; j < OR_QK_K; ++j) {
            float ax = fabsf(x[j]);
            if (ax > amax) { amax = ax; vmax = x[j]; }
        }
        if (amax == 0.0f) {
            y[i].d = 0;
            memset(y[i].qs, 0, sizeof y[i].qs);
            memset(y[i].bsums, 0, sizeof y[i].bsums);
            continue;
        }
        const float iscale = -127.f / vmax;
        for (int j = 0; j < OR_QK_K; ++j) {
            int v = or_nearest_int(iscale * x[j]);
            y[i].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int g = 0; g < 16; ++g) {
            int s = 0;
            for (int l = 0; l < 16; ++l) s += y[i].qs[16 * g + l];
            y[i].bsums[g] = (int16_t)s;
        }
        y[i].d = 1 / iscale;
    }
}

/* ------------------------------------------------------------------------ */
/* 4-bit value of element e (0..255) of a block: element 64g + 32h + l is the
 * low (h = 0) or high (h = 1) nibble of qs[32g + l]. */
static inline int q4_at(const or_block_q4K *b, int e) {
    const int g = e >> 6, h = (e >> 5) & 1, l = e & 31;
    const uint8_t q = b->qs[32 * g + l];
    return h ? (q >> 4) : (q & 0x0F);
}

/* Exact integer sub-block sums (Appendix A of the path: S_bj). No reference
 * function returns them; they are the integer core of
 * ggml-cpu/quants.c:645-718 and arch/x86/quants.c:1919-1982. Pinned by a
 * brute-force int64 evaluation in the tests. */
void or_subblock_sums(int n, const void *vx, const void *vy, int32_t *S) {
    const or_block_q4K *x = (const or_block_q4K *)vx;
    const or_block_q8K *y = (const or_block_q8K *)vy;
    const int nb = n / OR_QK_K;
    for (int b = 0; b < nb; ++b) {
        for (int j = 0; j < 8; ++j) {
            int32_t s = 0;
            for (int l = 0; l < 32; ++l) s += q4_at(&x[b], 32 * j + l) * (int32_t)y[b].qs[32 * j + l];
            S[8 * b + j] = s;
        }
    }
}

/* Q4_K . Q8_K in the float order of the portable kernel.
 * Follows ggml-cpu/quants.c:645-718 (ggml_vec_dot_q4_K_q8_K_generic): eight
 * int32 lane sums aux32[l] = sum_j sc_j * sum_{g<4} q4*q8 at 32j + 8g + l; per
 * block sums[l] += (fp16(d) * d8) * aux32[l] and
 * sumf -= (fp16(dmin) * d8) * sum_k bsums[k] * m_{k/2}; finally
 * sumf += sums[0..7] in lane order. Uncontracted (-ffp-contract=off). */
float or_vec_dot_generic(int n, const void *vx, const void *vy) {
    const or_block_q4K *x = (const or_block_q4K *)vx;
    const or_block_q8K *y = (const or_block_q8K *)vy;
    const int nb = n / OR_QK_K;
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float sumf = 0;
    for (int b = 0; b < nb; ++b) {
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; ++j) or_scale_min_k4(j, x[b].scales, &sc[j], &mn[j]);
        int32_t aux32[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < 8; ++j) {
            for (int g = 0; g < 4; ++g) {
                for (int l = 0; l < 8; ++l) {
                    const int e = 32 * j + 8 * g + l;
                    const int16_t p = (int16_t)(q4_at(&x[b], e) * y[b].qs[e]);
                    aux32[l] += (int32_t)sc[j] * p;
                }
            }
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

/* Q4_K . Q8_K in the float order of the x86 kernel that the reference's CPU
 * backend runs. Follows ggml-cpu/arch/x86/quants.c:1919-1982 (AVX2 branch of
 * ggml_vec_dot_q4_K_q8_K) lane by lane: eight int32 lanes, lane q holding
 * bytes 4q..4q+3 of each 32-byte chunk (sc_{2j} on low nibbles, sc_{2j+1} on
 * high nibbles); acc[q] = fma(d8*fp16(d), float(lane q), acc[q]); four min
 * lanes acc_m[p] = fma(-d8*fp16(dmin), float(m_{2p} s_{2p} + m_{2p+1} s_{2p+1}),
 * acc_m[p]) with s_k = bsums[2k] + bsums[2k+1]; then the horizontal sums of
 * hsum_float_8 (arch/x86/quants.c:43-49) and of acc_m. */
float or_vec_dot_avx2order(int n, const void *vx, const void *vy) {
    const or_block_q4K *x = (const or_block_q4K *)vx;
    const or_block_q8K *y = (const or_block_q8K *)vy;
    const int nb = n / OR_QK_K;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float accm[4] = {0, 0, 0, 0};
    for (int b = 0; b < nb; ++b) {
        const float d = y[b].d * or_fp16_to_fp32(x[b].d);
        const float dmin = -y[b].d * or_fp16_to_fp32(x[b].dmin);
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; ++j) or_scale_min_k4(j, x[b].scales, &sc[j], &mn[j]);
        int32_t s2[8];
        for (int k = 0; k < 8; ++k) s2[k] = (int32_t)y[b].bsums[2 * k] + (int32_t)y[b].bsums[2 * k + 1];
        for (int p = 0; p < 4; ++p) {
            const int32_t prod = (int32_t)mn[2 * p] * s2[2 * p] + (int32_t)mn[2 * p + 1] * s2[2 * p + 1];
            accm[p] = fmaf(dmin, (float)prod, accm[p]);
        }
        int32_t lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < 4; ++j) {
            const uint8_t *q4 = x[b].qs + 32 * j;
            const int8_t *q8 = y[b].qs + 64 * j;
            for (int q = 0; q < 8; ++q) {
                int32_t lo = 0, hi = 0;
                for (int e = 0; e < 4; ++e) {
                    lo += (int32_t)(q4[4 * q + e] & 0x0F) * q8[4 * q + e];
                    hi += (int32_t)(q4[4 * q + e] >> 4) * q8[32 + 4 * q + e];
                }
                lane[q] += (int32_t)sc[2 * j] * lo + (int32_t)sc[2 * j + 1] * hi;
            }
        }
        for (int q = 0; q < 8; ++q) acc[q] = fmaf(d, (float)lane[q], acc[q]);
    }
    float r0 = acc[4] + acc[0], r1 = acc[5] + acc[1], r2 = acc[6] + acc[2], r3 = acc[7] + acc[3];
    float h = (r0 + r2) + (r1 + r3);
    float m = (accm[0] + accm[2]) + (accm[1] + accm[3]);
    return h + m;
}

/* The same dot product with the integer parts exact and the float combine in
 * double: sum_b fp16(d)*d8*I_b - fp16(dmin)*d8*M_b. */
double or_vec_dot_exact(int n, const void *vx, const void *vy) {
    const or_block_q4K *x = (const or_block_q4K *)vx;
    const or_block_q8K *y = (const or_block_q8K *)vy;
    const int nb = n / OR_QK_K;
    double acc = 0;
    int32_t S[8];
    for (int b = 0; b < nb; ++b) {
        or_subblock_sums(OR_QK_K, &x[b], &y[b], S);
        int64_t I = 0, Mt = 0;
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, m;
            or_scale_min_k4(j, x[b].scales, &sc, &m);
            I += (int64_t)sc * S[j];
            Mt += (int64_t)m * ((int64_t)y[b].bsums[2 * j] + y[b].bsums[2 * j + 1]);
        }
        const double dd = (double)or_fp16_to_fp32(x[b].d) * (double)y[b].d;
        const double dm = (double)or_fp16_to_fp32(x[b].dmin) * (double)y[b].d;
        acc += dd * (double)I - dm * (double)Mt;
    }
    return acc;
}

/* ------------------------------------------------------------------------ */
/* Row geometry and vec_dot of a weight type (ggml-cpu/ggml-cpu.c:297-316:
 * both types take Q8_K activations). */
static size_t block_bytes(int type) {
    return type == OR_TYPE_Q4_K ? OR_Q4K_BLOCK_BYTES
         : type == OR_TYPE_Q5_K ? OR_Q5K_BLOCK_BYTES
         : type == OR_TYPE_Q6_K ? OR_Q6K_BLOCK_BYTES : 0;
}

static float type_dot(int type, int order, int n, const void *wr, const void *q8) {
    if (type == OR_TYPE_Q6_K)
        return order ? or_vec_dot_q6K_avx2order(n, wr, q8) : or_vec_dot_q6K_generic(n, wr, q8);
    if (type == OR_TYPE_Q5_K)
        return order ? or_vec_dot_q5K_avx2order(n, wr, q8) : or_vec_dot_q5K_generic(n, wr, q8);
    return order ? or_vec_dot_avx2order(n, wr, q8) : or_vec_dot_generic(n, wr, q8);
}

/* Dense driver. Follows ggml-cpu/ggml-cpu.c:1241-1439
 * (ggml_compute_forward_mul_mat): each activation row is converted to Q8_K
 * (the vec_dot_type of Q4_K and Q6_K, ggml-cpu.c:297-316), then dst[t][r] =
 * vec_dot(K, W row r, Q8_K row t). Thread chunking does not change any value. */
int or_mul_mat_type(int type, const void *W, int64_t M, int64_t K, const float *X, int64_t T,
                    float *Y, int order) {
    const int64_t nb = K / OR_QK_K;
    const size_t row_bytes = (size_t)nb * block_bytes(type);
    if (!row_bytes) return -22;
    or_block_q8K *q8 = (or_block_q8K *)malloc((size_t)nb * sizeof(or_block_q8K));
    for (int64_t t = 0; t < T; ++t) {
        or_quantize_row_q8K(X + t * K, q8, K);
        for (int64_t r = 0; r < M; ++r)
            Y[t * M + r] = type_dot(type, order, (int)K, (const uint8_t *)W + (size_t)r * row_bytes, q8);
    }
    free(q8);
    return 0;
}

void or_mul_mat(const void *W, int64_t M, int64_t K, const float *X, int64_t T,
                float *Y, int order) {
    (void)or_mul_mat_type(OR_TYPE_Q4_K, W, M, K, X, T, Y, order);
}

/* Expert-gathered driver. Follows ggml-cpu/ggml-cpu.c:1441-1511 and
 * 1521-1690 (ggml_compute_forward_mul_mat_id): for token t and slot s the
 * expert is ids[t][s]; its input row is X[t][s % ne11] (ne11 == 1 broadcasts
 * one row to every slot); dst[t][s][r] = vec_dot(expert row r, Q8_K(input)). */
int or_mul_mat_id_type(int type, const void *as, int64_t M, int64_t K, int64_t E,
                       const float *X, int64_t ne11, const int32_t *ids, int64_t k,
                       int64_t T, float *Y, int order) {
    const int64_t nb = K / OR_QK_K;
    const size_t row_bytes = (size_t)nb * block_bytes(type);
    if (!row_bytes) return -22;
    const size_t expert_bytes = row_bytes * (size_t)M;
    or_block_q8K *q8 = (or_block_q8K *)malloc((size_t)nb * sizeof(or_block_q8K));
    for (int64_t t = 0; t < T; ++t) {
        for (int64_t s = 0; s < k; ++s) {
            const int32_t e = ids[t * k + s];
            if (e < 0 || e >= E) { free(q8); return -22; }
            or_quantize_row_q8K(X + (t * ne11 + (s % ne11)) * K, q8, K);
            const uint8_t *base = (const uint8_t *)as + (size_t)e * expert_bytes;
            for (int64_t r = 0; r < M; ++r)
                Y[(t * k + s) * M + r] = type_dot(type, order, (int)K, base + (size_t)r * row_bytes, q8);
        }
    }
    free(q8);
    return 0;
}

int or_mul_mat_id(const void *as, int64_t M, int64_t K, int64_t E,
                  const float *X, int64_t ne11, const int32_t *ids, int64_t k,
                  int64_t T, float *Y, int order) {
    return or_mul_mat_id_type(OR_TYPE_Q4_K, as, M, K, E, X, ne11, ids, k, T, Y, order);
}

/* Q8_K -> fp32. Follows ggml-quants.c:2731-2740 (dequantize_row_q8_K):
 * y = d * q, one fp32 product per value. */
void or_dequantize_row_q8K(const void *vx, float *y, int64_t k) {
    const or_block_q8K *x = (const or_block_q8K *)vx;
    const int64_t nb = k / OR_QK_K;
    for (int64_t i = 0; i < nb; ++i)
        for (int j = 0; j < OR_QK_K; ++j) y[i * OR_QK_K + j] = x[i].d * (float)x[i].qs[j];
}

/* fp32 weights of one row of a weight type (its to_float), 0 or -22 */
static int dequant_row_type(int type, const void *src, float *w, int64_t K) {
    if (type == OR_TYPE_Q4_K) or_dequantize_row_q4K(src, w, K);
    else if (type == OR_TYPE_Q5_K) or_dequantize_row_q5K(src, w, K);
    else if (type == OR_TYPE_Q6_K) or_dequantize_row_q6K(src, w, K);
    else if (type == OR_TYPE_Q8_0) or_dequantize_row_q8_0(src, w, K);
    else return -22;
    return 0;
}

static size_t row_bytes_type(int type, int64_t K) {
    if (type == OR_TYPE_Q8_0) return (size_t)(K / 32) * 34;
    return (size_t)(K / OR_QK_K) * block_bytes(type);
}

/* Dequant-then-dot in double with the fp32 activations as given: the exact
 * value of sum_c dequant(W)[r][c] * x[t][c] for the type's to_float weights.
 * It is what an fp32-activation dequant-then-dot computes in exact
 * arithmetic (the reference's scalar path: beast_matvec,
 * desktop/beast_canyon/sp_beast_canyon.c:1122-1134, which rounds its sum in
 * fp32); Q8_K-activation kernels differ from it by the quantisation of x. */
int or_mul_mat_dequant_f64_type(int type, const void *W, int64_t M, int64_t K, const float *X,
                                int64_t T, double *Y) {
    const size_t rb = row_bytes_type(type, K);
    if (!rb) return -22;
    float *wrow = (float *)malloc((size_t)K * sizeof(float));
    for (int64_t r = 0; r < M; ++r) {
        if (dequant_row_type(type, (const uint8_t *)W + (size_t)r * rb, wrow, K)) { free(wrow); return -22; }
        for (int64_t t = 0; t < T; ++t) {
            double acc = 0;
            const float *xt = X + t * K;
            for (int64_t c = 0; c < K; ++c) acc += (double)wrow[c] * (double)xt[c];
            Y[t * M + r] = acc;
        }
    }
    free(wrow);
    return 0;
}

void or_mul_mat_dequant_f64(const void *W, int64_t M, int64_t K, const float *X,
                            int64_t T, double *Y) {
    (void)or_mul_mat_dequant_f64_type(OR_TYPE_Q4_K, W, M, K, X, T, Y);
}

/* The second form of the parity bar for the Q8_K / Q8_0 matmuls: the exact
 * value of sum_c dequant(W)[r][c] * dequant(Q(x[t]))[c] in double, where Q is
 * the CPU backend's activation quantiser of the type's vec_dot_type
 * (quantize_row_q8_K, ggml-quants.c:2692-2729; for Q8_0 weights
 * quantize_row_q8_0, ggml-cpu/arch/x86/quants.c:302-367) and dequant its
 * to_float (dequantize_row_q8_K, ggml-quants.c:2731-2740; dequantize_row_q8_0,
 * :491-505). ggml_vec_dot_q4_K_q8_K computes the same sum with integer
 * sub-block sums and an fp32 combine, so its outputs sit within fp32
 * rounding of this one. */
int or_mul_mat_dq_f64_type(int type, const void *W, int64_t M, int64_t K, const float *X,
                           int64_t T, double *Y) {
    const size_t rb = row_bytes_type(type, K);
    if (!rb) return -22;
    const int q80 = type == OR_TYPE_Q8_0;
    float *wrow = (float *)malloc((size_t)K * sizeof(float));
    float *xq = (float *)malloc((size_t)(T * K) * sizeof(float));
    void *qb = malloc(q80 ? (size_t)(K / 32) * 34 : (size_t)(K / OR_QK_K) * sizeof(or_block_q8K));
    for (int64_t t = 0; t < T; ++t) {
        if (q80) {
            or_quantize_row_q8_0(X + t * K, qb, K);
            or_dequantize_row_q8_0(qb, xq + t * K, K);
        } else {
            or_quantize_row_q8K(X + t * K, qb, K);
            or_dequantize_row_q8K(qb, xq + t * K, K);
        }
    }
    int rc = 0;
    for (int64_t r = 0; r < M && !rc; ++r) {
        rc = dequant_row_type(type, (const uint8_t *)W + (size_t)r * rb, wrow, K);
        for (int64_t t = 0; t < T && !rc; ++t) {
            double acc = 0;
            const float *xt = xq + t * K;
            for (int64_t c = 0; c < K; ++c) acc += (double)wrow[c] * (double)xt[c];
            Y[t * M + r] = acc;
        }
    }
    free(wrow);
    free(xq);
    free(qb);
    return rc;
}

/* beast_matvec (desktop/beast_canyon/sp_beast_canyon.c:1122-1134) for Q4_K
 * and Q8_0 rows, as the reference's own build of that file evaluates it
 * (desktop/beast_canyon/CMakeLists.txt:52-54, GCC -O3 -mfma):
 *   Q4_K (beast_dequant_q4_K, :1000-1021): w = d*sc * q - dmin*m. The
 *     compiler fuses the multiply-subtract, but d*sc (an fp16 times a 6-bit
 *     integer) times a 4-bit q is exact in fp32, so w equals
 *     dequantize_row_q4_K's value bit for bit;
 *   Q8_0 (beast_dequant_q8_0, :976-984): w = q * d;
 *   y = y + w[c]*x[c] over c = 0 .. K-1 in index order, each product and
 *     each sum rounded to fp32 (the vectorised loop multiplies eight at a
 *     time and adds them one by one; its fused tail serves only K not a
 *     multiple of 8, which no K-quant row has).
 * beast_dequant_q5_K (:1056-1085) and beast_dequant_q6_K (:1025-1053) read
 * other bits than ggml's dequantize_row_q5_K / _q6_K (Q5_K: the qh bit of
 * the 64-value group where the format has one per 32-value sub-block; Q6_K:
 * one scale per 32 values where the format has one per 16, and the high
 * nibbles of ql[l] and the low ones of ql[l + 32] in each other's place), so
 * they are not restated: for Q5_K and Q6_K rows the loop above runs over the
 * format's own dequantiser (dequantize_row_q5_K / _q6_K, ggml-quants.c:
 * 1669-1696 / 1877-1905, restated here as or_dequantize_row_q5K / _q6K). */
int or_beast_matvec_type(int type, const void *W, int64_t M, int64_t K, const float *x, float *y) {
    if (type != OR_TYPE_Q4_K && type != OR_TYPE_Q8_0 && type != OR_TYPE_Q5_K && type != OR_TYPE_Q6_K) return -22;
    const size_t rb = row_bytes_type(type, K);
    if (!rb) return -22;
    float *w = (float *)malloc((size_t)K * sizeof(float));
    for (int64_t r = 0; r < M; ++r) {
        const uint8_t *src = (const uint8_t *)W + (size_t)r * rb;
        if (type == OR_TYPE_Q5_K || type == OR_TYPE_Q6_K) {
            (void)dequant_row_type(type, src, w, K);
        } else if (type == OR_TYPE_Q4_K) {
            const or_block_q4K *b = (const or_block_q4K *)src;
            for (int64_t i = 0; i < K / OR_QK_K; ++i) {
                const float d = or_fp16_to_fp32(b[i].d), dmin = or_fp16_to_fp32(b[i].dmin);
                for (int g = 0; g < 4; ++g) {
                    uint8_t sc0, m0, sc1, m1;
                    or_scale_min_k4(2 * g, b[i].scales, &sc0, &m0);
                    or_scale_min_k4(2 * g + 1, b[i].scales, &sc1, &m1);
                    const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
                    const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
                    const uint8_t *q = b[i].qs + 32 * g;
                    float *wo = w + i * OR_QK_K + 64 * g;
                    for (int l = 0; l < 32; ++l) wo[l] = d1 * (float)(q[l] & 0x0F) - mm1;
                    for (int l = 0; l < 32; ++l) wo[32 + l] = d2 * (float)(q[l] >> 4) - mm2;
                }
            }
        } else {
            for (int64_t i = 0; i < K / 32; ++i) {
                const float d = or_fp16_to_fp32((uint16_t)(src[34 * i] | (src[34 * i + 1] << 8)));
                for (int j = 0; j < 32; ++j) w[32 * i + j] = (float)(int8_t)src[34 * i + 2 + j] * d;
            }
        }
        float sum = 0.0f;
        for (int64_t c = 0; c < K; ++c) sum += w[c] * x[c];
        y[r] = sum;
    }
    free(w);
    return 0;
}

/* sp_beast_moe_forward's per-expert loop (desktop/beast_canyon/
 * sp_beast_canyon.c:486-545) over a given routing: output zeroed, then for
 * each selected expert in rank order g = beast_matvec(gate_e, hidden),
 * u = beast_matvec(up_e, hidden), h = (g / (1 + expf(-g))) * u
 * (beast_silu_mul, :1168-1173), d = beast_matvec(down_e, h),
 * output = fmaf(score, d, output) (:541-543 as the reference's GCC build
 * contracts it). Each bank has its own type (the reference's tensors carry
 * theirs; beast_matvec dispatches per tensor): gate / up [n_ff x n_embd] x E,
 * down [n_embd x n_ff] x E, contiguous experts. An id outside 0 .. E-1 is
 * skipped. */
int or_beast_moe_routed(int tg, const void *gate, int tu, const void *up, int td, const void *down, int64_t E,
                        int64_t n_embd, int64_t n_ff, const int32_t *ids, const float *scores, int64_t k,
                        const float *hidden, float *out) {
    const size_t rg = row_bytes_type(tg, n_embd), ru = row_bytes_type(tu, n_embd), rd = row_bytes_type(td, n_ff);
    if (!rg || !ru || !rd) return -22;
    float *g = (float *)malloc((size_t)n_ff * sizeof(float));
    float *u = (float *)malloc((size_t)n_ff * sizeof(float));
    float *d = (float *)malloc((size_t)n_embd * sizeof(float));
    int rc = (g && u && d) ? 0 : -12;
    for (int64_t i = 0; i < n_embd; ++i) out[i] = 0.0f;
    for (int64_t s = 0; s < k && !rc; ++s) {
        const int64_t e = ids[s];
        if (e < 0 || e >= E) continue;
        rc = or_beast_matvec_type(tg, (const uint8_t *)gate + (size_t)e * n_ff * rg, n_ff, n_embd, hidden, g);
        if (!rc) rc = or_beast_matvec_type(tu, (const uint8_t *)up + (size_t)e * n_ff * ru, n_ff, n_embd, hidden, u);
        if (rc) break;
        for (int64_t i = 0; i < n_ff; ++i) g[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
        rc = or_beast_matvec_type(td, (const uint8_t *)down + (size_t)e * n_embd * rd, n_embd, n_ff, g, d);
        if (rc) break;
        for (int64_t i = 0; i < n_embd; ++i) out[i] = fmaf(scores[s], d[i], out[i]);
    }
    free(g);
    free(u);
    free(d);
    return rc;
}

/* ------------------------------------------------------------------------ */
void or_synth_fill(float *out, int64_t n, uint64_t seed, int dist, int64_t cols,
                   float mean, float std, float outlier_mult, int64_t offset) {
    for (int64_t i = 0; i < n; ++i) {
        out[i] = spq_synth_value(seed, dist, (uint64_t)(offset + i), (uint64_t)cols,
                                 mean, std, outlier_mult);
    }
}
