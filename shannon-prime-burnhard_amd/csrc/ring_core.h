// ring_core.h — one Q4_K super-block x Q8_K activations on gfx950 matrix
// cores, read from an LDS stage (device code shared by the ring kernels of
// k_gemm.hip and k_moe.hip).
//
// Numerics are those of the reference CPU path (ggml_vec_dot_q4_K_q8_K,
// ggml-cpu/arch/x86/quants.c:1900-1982), with the integer sums exact:
//   acc[row][t] += d8_t (d_row I - dmin_row M),  I = sum_j sc_j S_j,  M = sum_j m_j BS_j
//   - a 6-bit scale sc = 8*sh + sl (sh, sl in 0..7) is folded into two int8
//     operands sh*q4 and sl*q4 (both <= 105): v_mfma_i32_16x16x64_i8 gives
//     H = sum sh q4 q8 and L = sum sl q4 q8 over the super-block, I = 8H + L;
//   - M comes from one v_mfma_f32_16x16x16_f16 per tile: BS_j = 32 hi_j + lo_j
//     (hi_j in -127..127, lo_j in 0..31) and the k slots hold (32 m_j, hi_j)
//     and (m_j, lo_j); every operand, product (<= 2016 * 127) and partial sum
//     (< 2^22) is an integer that fp16 / fp32 represent exactly.
//
// Stage layout (bytes): rows of 144-byte super-blocks (the wave's RT*16 rows
// start at `wt`); per token a 272-byte row of Q8_K values in the permuted
// order of quantize_q8k_planes (`qreg`: values 64q + 8s .. +7, 64q + 32 + 8s
// .. +7 at 64q + 16s); per token the 48-byte min operand of Q8Planes::mn
// (`mreg`). Lane (c16, q) holds output rows 4q .. 4q+3 of each 16-row tile and
// token c16 of each 16-token tile; k-slot group q of step s is the low and the
// high nibbles of bytes 8s .. 8s+7 of the 32-byte nibble group q, so a lane's
// sub-blocks 2q, 2q + 1 keep one scale pair for the whole super-block.
#pragma once

#include "gemv_core.h"

namespace spq4k {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

constexpr int RING_QS = 272;   // LDS bytes per token row of Q8_K values (256 + one spare 16-byte slot)

__device__ __forceinline__ uint32_t pk_mul_u16(uint32_t a, uint32_t b) {
    // two 16-bit products (v_pk_mul_lo_u16); each byte of `a` is < 16 and each
    // 16-bit half of `b` is < 8, so no product carries across a byte
    u16x2 x, y;
    __builtin_memcpy(&x, &a, 4);
    __builtin_memcpy(&y, &b, 4);
    const u16x2 z = x * y;
    uint32_t r;
    __builtin_memcpy(&r, &z, 4);
    return r;
}

template <int RT, int CT>
__device__ __forceinline__ void ring_block(const uint8_t* wt, const uint8_t* qreg, const uint8_t* mreg, int c16, int q,
                                           v4f (&acc)[RT][CT]) {
    v4i ch[RT][CT], cl[RT][CT];
    uint32_t SH0[RT], SL0[RT], SH1[RT], SL1[RT];
    v4i wq[RT][2];
    h4 am[RT];
    float dr[RT][4], dmr[RT][4];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const uint8_t* wr = wt + (r * 16 + c16) * Q4K_BYTES;
        const v4i hdr = *reinterpret_cast<const v4i*>(wr);
        wq[r][0] = *reinterpret_cast<const v4i*>(wr + 16 + 32 * q);
        wq[r][1] = *reinterpret_cast<const v4i*>(wr + 32 + 32 * q);
        // d, dmin of output rows 4q .. 4q+3 of this row tile
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t h = *reinterpret_cast<const uint32_t*>(wt + (r * 16 + 4 * q + i) * Q4K_BYTES);
            dr[r][i] = half_bits_to_float(h & 0xFFFFu);
            dmr[r][i] = half_bits_to_float(h >> 16);
        }
        const ScaleMin sm = unpack_scale_min((uint32_t)hdr.y, (uint32_t)hdr.z, (uint32_t)hdr.w);
        // this lane's sub-blocks 2q (low nibbles) and 2q + 1 (high nibbles)
        const uint32_t sc01 = (q < 2 ? sm.sc_lo : sm.sc_hi) >> (16 * (q & 1));
        SH0[r] = ((sc01 >> 3) & 7u) * 0x10001u;
        SL0[r] = (sc01 & 7u) * 0x10001u;
        SH1[r] = ((sc01 >> 11) & 7u) * 0x10001u;
        SL1[r] = ((sc01 >> 8) & 7u) * 0x10001u;
        // min operand of row c16: 32 m_j in k slots 0..7, m_j in slots
        // 8..15 (0x6400 | m is the fp16 1024 + m, rescaled exactly)
        const uint32_t mw = (q & 1) ? sm.m_hi : sm.m_lo;
        const uint32_t x01 = __builtin_amdgcn_perm(0x64646464u, mw, 0x04010400u);
        const uint32_t x23 = __builtin_amdgcn_perm(0x64646464u, mw, 0x04030402u);
        h2 a01, a23;
        __builtin_memcpy(&a01, &x01, 4);
        __builtin_memcpy(&a23, &x23, 4);
        const _Float16 f = q < 2 ? (_Float16)32.0f : (_Float16)1.0f;
        const _Float16 o = q < 2 ? (_Float16)-32768.0f : (_Float16)-1024.0f;
        const h2 fv = {f, f}, ov = {o, o};
        const h2 b01 = a01 * fv + ov, b23 = a23 * fv + ov;
        am[r] = h4{b01.x, b01.y, b23.x, b23.y};
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            ch[r][ct] = v4i{0, 0, 0, 0};
            cl[r][ct] = v4i{0, 0, 0, 0};
        }
    }
    // activation fragment of token c16, step s: values 64q + 8s .. +7 and
    // 64q + 32 + 8s .. +7, stored contiguously by the permuted Q8_K planes
    const uint8_t* qb = qreg + c16 * RING_QS + 64 * q;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        v4i bq[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) bq[ct] = *reinterpret_cast<const v4i*>(qb + ct * 16 * RING_QS + 16 * s);
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const uint32_t w0 = (uint32_t)wq[r][s >> 1][2 * (s & 1)];
            const uint32_t w1 = (uint32_t)wq[r][s >> 1][2 * (s & 1) + 1];
            const uint32_t l0 = w0 & 0x0F0F0F0Fu, l1 = w1 & 0x0F0F0F0Fu;
            const uint32_t u0 = (w0 >> 4) & 0x0F0F0F0Fu, u1 = (w1 >> 4) & 0x0F0F0F0Fu;
            const v4i ah = {(int)pk_mul_u16(l0, SH0[r]), (int)pk_mul_u16(l1, SH0[r]),
                            (int)pk_mul_u16(u0, SH1[r]), (int)pk_mul_u16(u1, SH1[r])};
            const v4i al = {(int)pk_mul_u16(l0, SL0[r]), (int)pk_mul_u16(l1, SL0[r]),
                            (int)pk_mul_u16(u0, SL1[r]), (int)pk_mul_u16(u1, SL1[r])};
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                ch[r][ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah, bq[ct], ch[r][ct], 0, 0, 0);
                cl[r][ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al, bq[ct], cl[r][ct], 0, 0, 0);
            }
        }
    }
    const uint8_t* mb = mreg + c16 * Q8MN_BYTES;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
        const h4 bm = *reinterpret_cast<const h4*>(mb + ct * 16 * Q8MN_BYTES + 8 * q);
        const float d8 = *reinterpret_cast<const float*>(mb + ct * 16 * Q8MN_BYTES + 32);
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const v4f cm = __builtin_amdgcn_mfma_f32_16x16x16f16(am[r], bm, v4f{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int I = (ch[r][ct][i] << 3) + cl[r][ct][i];
                acc[r][ct][i] = fmaf(d8, fmaf(-dmr[r][i], cm[i], dr[r][i] * (float)I), acc[r][ct][i]);
            }
        }
    }
}

}  // namespace spq4k
