// ring_core.h — one Q4_K super-block (or one Q6_K block, ring_block_q6 below)
// x Q8_K activations on gfx950 matrix cores, read from an LDS stage (device
// code shared by the ring kernels of k_gemm.hip and k_moe.hip).
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
#include "q5k_core.h"

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
    }
    // activation fragment of token c16, step s: values 64q + 8s .. +7 and
    // 64q + 32 + 8s .. +7, stored contiguously by the permuted Q8_K planes
    // folded weight operands of every step, made once for all token tiles
    v4i ah[RT][4], al[RT][4];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t w0 = (uint32_t)wq[r][s >> 1][2 * (s & 1)];
            const uint32_t w1 = (uint32_t)wq[r][s >> 1][2 * (s & 1) + 1];
            const uint32_t l0 = w0 & 0x0F0F0F0Fu, l1 = w1 & 0x0F0F0F0Fu;
            const uint32_t u0 = (w0 >> 4) & 0x0F0F0F0Fu, u1 = (w1 >> 4) & 0x0F0F0F0Fu;
            ah[r][s] = v4i{(int)pk_mul_u16(l0, SH0[r]), (int)pk_mul_u16(l1, SH0[r]), (int)pk_mul_u16(u0, SH1[r]),
                           (int)pk_mul_u16(u1, SH1[r])};
            al[r][s] = v4i{(int)pk_mul_u16(l0, SL0[r]), (int)pk_mul_u16(l1, SL0[r]), (int)pk_mul_u16(u0, SL1[r]),
                           (int)pk_mul_u16(u1, SL1[r])};
        }
    // tile by tile: a tile's eight-MFMA chain is followed by its combine, so
    // the combine's VALU work overlaps the next tile's MFMAs and only a few
    // tiles' integer sums are live at a time
    const uint8_t* qb = qreg + c16 * RING_QS + 64 * q;
    const uint8_t* mb = mreg + c16 * Q8MN_BYTES;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
        v4i bq[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) bq[s] = *reinterpret_cast<const v4i*>(qb + ct * 16 * RING_QS + 16 * s);
        const h4 bm = *reinterpret_cast<const h4*>(mb + ct * 16 * Q8MN_BYTES + 8 * q);
        const float d8 = *reinterpret_cast<const float*>(mb + ct * 16 * Q8MN_BYTES + 32);
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            v4i ch = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[r][0], bq[0], v4i{0, 0, 0, 0}, 0, 0, 0);
            v4i cl = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[r][0], bq[0], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int s = 1; s < 4; ++s) {
                ch = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[r][s], bq[s], ch, 0, 0, 0);
                cl = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[r][s], bq[s], cl, 0, 0, 0);
            }
            const v4f cm = __builtin_amdgcn_mfma_f32_16x16x16f16(am[r], bm, v4f{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int I = (ch[i] << 3) + cl[i];
                acc[r][ct][i] = fmaf(d8, fmaf(-dmr[r][i], cm[i], dr[r][i] * (float)I), acc[r][ct][i]);
            }
        }
    }
}


// ---------------------------------------------------------------------------
// The same super-block on 32x32 tiles: v_mfma_i32_32x32x32_i8, which sustains
// 1.7x the int8 rate of the 16x16x64 form on gfx950 (4.7 against 2.8 POP/s
// measured), and v_mfma_f32_32x32x16_f16 for the min term.
// Lane (c32, h) = (lane & 31, lane >> 5). Operand k slots: step s (0..7) of
// lane half h holds the low and the high nibbles of bytes 8*(s&3) .. +7 of
// nibble group 2h + (s >> 2) (sub-blocks 4h + 2(s>>2) and +1), i.e. values
// 64g + 8(s&3) .. +7 and 64g + 32 + 8(s&3) .. +7 of group g = 2h + (s>>2),
// which the permuted Q8_K row stores at 64g + 16(s&3) (one 16-byte read).
// Min-term slots: half 0 holds (32 m_j, hi_j), half 1 (m_j, lo_j), j = 0..7.
// Output element i of lane (c32, h): row 8(i/4) + 4h + (i%4) of the 32-row
// tile, token c32 of the 32-token tile.
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

template <int RT, int CT>
__device__ __forceinline__ void ring_block32(const uint8_t* wt, const uint8_t* qreg, const uint8_t* mreg, int lane,
                                             v16f (&acc)[RT][CT]) {
    const int c32 = lane & 31, h = lane >> 5;
    v4i ah[RT][8], al[RT][8];
    h8 am[RT];
    float dr[RT][16], dmr[RT][16];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const uint8_t* wr = wt + (r * 32 + c32) * Q4K_BYTES;
        const v4i hdr = *reinterpret_cast<const v4i*>(wr);
        v4i wq[4];   // groups 2h, 2h + 1 of qs
#pragma unroll
        for (int k = 0; k < 4; ++k) wq[k] = *reinterpret_cast<const v4i*>(wr + 16 + 64 * h + 16 * k);
        // d, dmin of output rows 8(i/4) + 4h + (i%4)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t hd =
                *reinterpret_cast<const uint32_t*>(wt + (r * 32 + 8 * (i >> 2) + 4 * h + (i & 3)) * Q4K_BYTES);
            dr[r][i] = half_bits_to_float(hd & 0xFFFFu);
            dmr[r][i] = half_bits_to_float(hd >> 16);
        }
        const ScaleMin sm = unpack_scale_min((uint32_t)hdr.y, (uint32_t)hdr.z, (uint32_t)hdr.w);
        const uint32_t scw = h ? sm.sc_hi : sm.sc_lo;   // sub-blocks 4h .. 4h+3
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int gl = s >> 2;
            const uint32_t sc01 = scw >> (16 * gl);      // sub-blocks 4h + 2gl (low nibbles), +1 (high)
            const uint32_t SH0 = ((sc01 >> 3) & 7u) * 0x10001u, SL0 = (sc01 & 7u) * 0x10001u;
            const uint32_t SH1 = ((sc01 >> 11) & 7u) * 0x10001u, SL1 = ((sc01 >> 8) & 7u) * 0x10001u;
            const v4i& g = wq[2 * gl + ((s & 3) >> 1)];
            const uint32_t w0 = (uint32_t)g[2 * (s & 1)], w1 = (uint32_t)g[2 * (s & 1) + 1];
            const uint32_t l0 = w0 & 0x0F0F0F0Fu, l1 = w1 & 0x0F0F0F0Fu;
            const uint32_t u0 = (w0 >> 4) & 0x0F0F0F0Fu, u1 = (w1 >> 4) & 0x0F0F0F0Fu;
            ah[r][s] = v4i{(int)pk_mul_u16(l0, SH0), (int)pk_mul_u16(l1, SH0), (int)pk_mul_u16(u0, SH1),
                           (int)pk_mul_u16(u1, SH1)};
            al[r][s] = v4i{(int)pk_mul_u16(l0, SL0), (int)pk_mul_u16(l1, SL0), (int)pk_mul_u16(u0, SL1),
                           (int)pk_mul_u16(u1, SL1)};
        }
        // min operand of row c32: 32 m_j (half 0) or m_j (half 1), j = 0..7;
        // 0x6400 | m is the fp16 1024 + m, rescaled exactly
        const _Float16 f = h == 0 ? (_Float16)32.0f : (_Float16)1.0f;
        const _Float16 o = h == 0 ? (_Float16)-32768.0f : (_Float16)-1024.0f;
        const h2 fv = {f, f}, ov = {o, o};
        h2 mh[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t mw = k < 2 ? sm.m_lo : sm.m_hi;
            const uint32_t x = __builtin_amdgcn_perm(0x64646464u, mw, (k & 1) ? 0x04030402u : 0x04010400u);
            h2 a;
            __builtin_memcpy(&a, &x, 4);
            mh[k] = a * fv + ov;
        }
        am[r] = h8{mh[0].x, mh[0].y, mh[1].x, mh[1].y, mh[2].x, mh[2].y, mh[3].x, mh[3].y};
    }
    const uint8_t* qb = qreg + c32 * RING_QS + 128 * h;
    const uint8_t* mb = mreg + c32 * Q8MN_BYTES + 16 * h;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
        v4i bq[8];
#pragma unroll
        for (int s = 0; s < 8; ++s)
            bq[s] = *reinterpret_cast<const v4i*>(qb + ct * 32 * RING_QS + 64 * (s >> 2) + 16 * (s & 3));
        const h8 bm = *reinterpret_cast<const h8*>(mb + ct * 32 * Q8MN_BYTES);
        const float d8 = *reinterpret_cast<const float*>(mb - 16 * h + ct * 32 * Q8MN_BYTES + 32);
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            v16i ch = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah[r][0], bq[0], v16i{}, 0, 0, 0);
            v16i cl = __builtin_amdgcn_mfma_i32_32x32x32_i8(al[r][0], bq[0], v16i{}, 0, 0, 0);
#pragma unroll
            for (int s = 1; s < 8; ++s) {
                ch = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah[r][s], bq[s], ch, 0, 0, 0);
                cl = __builtin_amdgcn_mfma_i32_32x32x32_i8(al[r][s], bq[s], cl, 0, 0, 0);
            }
            const v16f cm = __builtin_amdgcn_mfma_f32_32x32x16_f16(am[r], bm, v16f{}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int I = (ch[i] << 3) + cl[i];
                acc[r][ct][i] = fmaf(d8, fmaf(-dmr[r][i], cm[i], dr[r][i] * (float)I), acc[r][ct][i]);
            }
        }
    }
}


// ---------------------------------------------------------------------------
// One Q6_K block (ggml-common.h:348-357) on 16x16 tiles, for the ring kernel
// with F = 1. Numerics of ggml_vec_dot_q6_K_q8_K
// (ggml-cpu/arch/x86/quants.c:2288-2366) with the integer sums exact:
//   acc[row][t] += (d_row d8_t) I,   I = sum_j scale_j sum_{k in j} (q_k - 32) q8_k
// The int8 scale (-128..127) is folded into the weight operand:
// w = scale * (q - 32) lies in -4096..4096, written w = 256 a + b with
// b = w - 256 round(w / 256) in -128..127 and a in -16..16, two int8
// operands; v_mfma_i32_16x16x64_i8 gives A = sum a q8 and B = sum b q8 over
// the block and I = 256 A + B exactly (|256 A| < 2^27).
// Lane (c16, q), step s: the k slots are those of the Q4_K ring (values
// 64q + 8s .. +7 and 64q + 32 + 8s .. +7, the permuted Q8_K order), which in
// Q6_K are quarters h0 = 2 (q & 1) and h0 + 1 of half n = q >> 1 at
// l = 8s .. 8s+7: nibble q & 1 of ql[64n + l] and ql[64n + 32 + l] and bits
// 4 (q & 1) .. +3 of qh[32n + l]; their sub-blocks 8n + 2 h0 + s / 2 and
// 8n + 2 h0 + 2 + s / 2.
// Stage rows are Q6K_LDS = 224 bytes: block bytes 0..207, then 194..209 (the
// last 16-byte load of a block reads its final 16 bytes), so d is at 222.
constexpr int Q6K_LDS = 224;

// u16 lanes w0 = v0 * sc + c, w1 = v2 * sc + c of bytes v0..v3 (v_pk_mad_u16)
__device__ __forceinline__ uint32_t pk_mad_u16(uint32_t a, uint32_t b, uint32_t c) {
    u16x2 x, y, z;
    __builtin_memcpy(&x, &a, 4);
    __builtin_memcpy(&y, &b, 4);
    __builtin_memcpy(&z, &c, 4);
    const u16x2 r = x * y + z;
    uint32_t o;
    __builtin_memcpy(&o, &r, 4);
    return o;
}

// Four 6-bit values (bytes of v) times a scale, split into the two int8
// operands: sc2 = scale in both u16 halves, c2 = 128 - 32 scale in both.
// u = w + 128 = 256 a + (b + 128) with b + 128 in 0..255: a is the high byte
// of u, b its low byte minus 128.
__device__ __forceinline__ void q6_fold(uint32_t v, uint32_t sc2, uint32_t c2, uint32_t& ahi, uint32_t& blo) {
    const uint32_t ev = __builtin_amdgcn_perm(0u, v, 0x0C020C00u);   // bytes 0, 2 -> u16 lanes
    const uint32_t od = __builtin_amdgcn_perm(0u, v, 0x0C030C01u);   // bytes 1, 3
    const uint32_t ue = pk_mad_u16(ev, sc2, c2), uo = pk_mad_u16(od, sc2, c2);
    blo = __builtin_amdgcn_perm(uo, ue, 0x06020400u) ^ 0x80808080u;   // low bytes: e0 o0 e1 o1
    ahi = __builtin_amdgcn_perm(uo, ue, 0x07030501u);                 // high bytes
}

template <int RT, int CT>
__device__ __forceinline__ void ring_block_q6(const uint8_t* wt, const uint8_t* qreg, const uint8_t* mreg, int c16,
                                              int q, v4f (&acc)[RT][CT]) {
    const int n = q >> 1, ns = 4 * (q & 1);
    v4i aa[RT][4], ab[RT][4];
    float dr[RT][4];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const uint8_t* wr = wt + (r * 16 + c16) * Q6K_LDS;
        v4i ql[4], qh[2];
#pragma unroll
        for (int k = 0; k < 4; ++k) ql[k] = *reinterpret_cast<const v4i*>(wr + 64 * n + 16 * k);
#pragma unroll
        for (int k = 0; k < 2; ++k) qh[k] = *reinterpret_cast<const v4i*>(wr + 128 + 32 * n + 16 * k);
        // scales 8n + 2h0 + {0, 1, 2, 3}: (h0, l < 16), (h0, l >= 16), (h0 + 1, l < 16), (h0 + 1, l >= 16)
        const uint32_t scw = *reinterpret_cast<const uint32_t*>(wr + 192 + 8 * n + 4 * (q & 1));
        uint32_t sc2[4], c2[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int sv = (int)(int8_t)((scw >> (8 * k)) & 0xFFu);
            sc2[k] = ((uint32_t)sv & 0xFFFFu) * 0x10001u;
            c2[k] = ((uint32_t)(128 - 32 * sv) & 0xFFFFu) * 0x10001u;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint16_t hd = *reinterpret_cast<const uint16_t*>(wt + (r * 16 + 4 * q + i) * Q6K_LDS + 222);
            dr[r][i] = half_bits_to_float(hd);
        }
        // dword position p (l = 4p .. 4p+3): quarter h0 from ql[p], h0 + 1 from ql[8 + p]
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            uint32_t av[4], bv[4];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int pp = 2 * s + e;
                const uint32_t lo = (uint32_t)ql[pp >> 2][pp & 3], hi = (uint32_t)ql[2 + (pp >> 2)][pp & 3];
                const uint32_t hb = (uint32_t)qh[pp >> 2][pp & 3] >> ns;
                const uint32_t v0 = ((lo >> ns) & 0x0F0F0F0Fu) | ((hb & 0x03030303u) << 4);
                const uint32_t v1 = ((hi >> ns) & 0x0F0F0F0Fu) | (((hb >> 2) & 0x03030303u) << 4);
                q6_fold(v0, sc2[s >> 1], c2[s >> 1], av[e], bv[e]);
                q6_fold(v1, sc2[2 + (s >> 1)], c2[2 + (s >> 1)], av[2 + e], bv[2 + e]);
            }
            aa[r][s] = v4i{(int)av[0], (int)av[1], (int)av[2], (int)av[3]};
            ab[r][s] = v4i{(int)bv[0], (int)bv[1], (int)bv[2], (int)bv[3]};
        }
    }
    const uint8_t* qb = qreg + c16 * RING_QS + 64 * q;
    const uint8_t* mb = mreg + c16 * Q8MN_BYTES;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
        v4i bq[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) bq[s] = *reinterpret_cast<const v4i*>(qb + ct * 16 * RING_QS + 16 * s);
        const float d8 = *reinterpret_cast<const float*>(mb + ct * 16 * Q8MN_BYTES + 32);
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            v4i ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(aa[r][0], bq[0], v4i{0, 0, 0, 0}, 0, 0, 0);
            v4i cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(ab[r][0], bq[0], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int s = 1; s < 4; ++s) {
                ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(aa[r][s], bq[s], ca, 0, 0, 0);
                cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(ab[r][s], bq[s], cb, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int I = (ca[i] << 8) + cb[i];
                acc[r][ct][i] = fmaf(dr[r][i] * d8, (float)I, acc[r][ct][i]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// One Q5_K super-block (176 bytes: d, dmin, the Q4_K scale/min packing,
// qh[32] at 16, qs[128] at 48) x Q8_K activations on 16x16 tiles, with the
// Q4_K lane mapping and the same permuted Q8_K stage. A weight value is
// q5 = nibble + 16 * bit of qh (ggml_vec_dot_q5_K_q8_K,
// ggml-cpu/arch/x86/quants.c:2078-2174): lane (c16, q) takes nibble group q
// and bits 2q (low nibbles) and 2q + 1 (high nibbles) of the 32 qh bytes.
// q5 reaches 31, so the 6-bit scale is split in three, sc = 16a + 4b + c with
// a, b, c in 0..3: the int8 operands a*q5, b*q5, c*q5 (<= 93) feed three MFMA
// chains A, B, C and I = sum_j sc_j S_j = 16A + 4B + C exactly; the min term
// is Q4_K's (one f16 MFMA, exact).
template <int RT, int CT>
__device__ __forceinline__ void ring_block_q5(const uint8_t* wt, const uint8_t* qreg, const uint8_t* mreg, int c16,
                                              int q, v4f (&acc)[RT][CT]) {
    v4i aa[RT][4], ab[RT][4], ac[RT][4];
    h4 am[RT];
    float dr[RT][4], dmr[RT][4];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const uint8_t* wr = wt + (r * 16 + c16) * Q5K_BYTES;
        const v4i hdr = *reinterpret_cast<const v4i*>(wr);
        const v4i qh0 = *reinterpret_cast<const v4i*>(wr + 16);
        const v4i qh1 = *reinterpret_cast<const v4i*>(wr + 32);
        v4i wq[2];
        wq[0] = *reinterpret_cast<const v4i*>(wr + 48 + 32 * q);
        wq[1] = *reinterpret_cast<const v4i*>(wr + 64 + 32 * q);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t h = *reinterpret_cast<const uint32_t*>(wt + (r * 16 + 4 * q + i) * Q5K_BYTES);
            dr[r][i] = half_bits_to_float(h & 0xFFFFu);
            dmr[r][i] = half_bits_to_float(h >> 16);
        }
        const ScaleMin sm = unpack_scale_min((uint32_t)hdr.y, (uint32_t)hdr.z, (uint32_t)hdr.w);
        const uint32_t sc01 = (q < 2 ? sm.sc_lo : sm.sc_hi) >> (16 * (q & 1));
        const uint32_t s0 = sc01 & 63u, s1 = (sc01 >> 8) & 63u;
        const uint32_t A0 = (s0 >> 4) * 0x10001u, B0 = ((s0 >> 2) & 3u) * 0x10001u, C0 = (s0 & 3u) * 0x10001u;
        const uint32_t A1 = (s1 >> 4) * 0x10001u, B1 = ((s1 >> 2) & 3u) * 0x10001u, C1 = (s1 & 3u) * 0x10001u;
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
        const uint32_t qh[8] = {(uint32_t)qh0.x, (uint32_t)qh0.y, (uint32_t)qh0.z, (uint32_t)qh0.w,
                                (uint32_t)qh1.x, (uint32_t)qh1.y, (uint32_t)qh1.z, (uint32_t)qh1.w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t w0 = (uint32_t)wq[s >> 1][2 * (s & 1)];
            const uint32_t w1 = (uint32_t)wq[s >> 1][2 * (s & 1) + 1];
            const uint32_t h0 = qh[2 * s], h1 = qh[2 * s + 1];
            const uint32_t l0 = (w0 & 0x0F0F0F0Fu) | (((h0 >> (2 * q)) & 0x01010101u) << 4);
            const uint32_t l1 = (w1 & 0x0F0F0F0Fu) | (((h1 >> (2 * q)) & 0x01010101u) << 4);
            const uint32_t u0 = ((w0 >> 4) & 0x0F0F0F0Fu) | (((h0 >> (2 * q + 1)) & 0x01010101u) << 4);
            const uint32_t u1 = ((w1 >> 4) & 0x0F0F0F0Fu) | (((h1 >> (2 * q + 1)) & 0x01010101u) << 4);
            aa[r][s] = v4i{(int)pk_mul_u16(l0, A0), (int)pk_mul_u16(l1, A0), (int)pk_mul_u16(u0, A1),
                           (int)pk_mul_u16(u1, A1)};
            ab[r][s] = v4i{(int)pk_mul_u16(l0, B0), (int)pk_mul_u16(l1, B0), (int)pk_mul_u16(u0, B1),
                           (int)pk_mul_u16(u1, B1)};
            ac[r][s] = v4i{(int)pk_mul_u16(l0, C0), (int)pk_mul_u16(l1, C0), (int)pk_mul_u16(u0, C1),
                           (int)pk_mul_u16(u1, C1)};
        }
    }
    const uint8_t* qb = qreg + c16 * RING_QS + 64 * q;
    const uint8_t* mb = mreg + c16 * Q8MN_BYTES;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
        v4i bq[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) bq[s] = *reinterpret_cast<const v4i*>(qb + ct * 16 * RING_QS + 16 * s);
        const h4 bm = *reinterpret_cast<const h4*>(mb + ct * 16 * Q8MN_BYTES + 8 * q);
        const float d8 = *reinterpret_cast<const float*>(mb + ct * 16 * Q8MN_BYTES + 32);
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            v4i ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(aa[r][0], bq[0], v4i{0, 0, 0, 0}, 0, 0, 0);
            v4i cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(ab[r][0], bq[0], v4i{0, 0, 0, 0}, 0, 0, 0);
            v4i cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(ac[r][0], bq[0], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int s = 1; s < 4; ++s) {
                ca = __builtin_amdgcn_mfma_i32_16x16x64_i8(aa[r][s], bq[s], ca, 0, 0, 0);
                cb = __builtin_amdgcn_mfma_i32_16x16x64_i8(ab[r][s], bq[s], cb, 0, 0, 0);
                cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(ac[r][s], bq[s], cc, 0, 0, 0);
            }
            const v4f cm = __builtin_amdgcn_mfma_f32_16x16x16f16(am[r], bm, v4f{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int I = (ca[i] << 4) + (cb[i] << 2) + cc[i];
                acc[r][ct][i] = fmaf(d8, fmaf(-dmr[r][i], cm[i], dr[r][i] * (float)I), acc[r][ct][i]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// One 256-value chunk of Q8_0 rows (eight 34-byte blocks, fp16 d then 32
// int8 values: 272 bytes a row, 17 stage slots) x Q8_0 activations (the
// token's int8 values in natural order, RING_QS bytes a token row; its eight
// fp32 block scales at the start of its Q8MN_BYTES of mreg) on 16x16 tiles.
// Block j is one v_mfma_i32_16x16x32_i8 (lane (c16, q) holds values 8q .. 8q+7
// of row c16 and of token c16) giving the exact integer dot of every (row,
// token) pair, then y += (d_w * d_x) * (float)sum: the per-block combine of
// ggml_vec_dot_q8_0_q8_0 (ggml-cpu/arch/x86/quants.c). A row's values start 2
// bytes into its block: the 8-byte LDS reads are 2-byte aligned (gfx950 LDS
// takes unaligned addresses).
constexpr int Q80_RING_ROW = 272;
template <int RT, int CT>
__device__ __forceinline__ void ring_block_q80(const uint8_t* wt, const uint8_t* qreg, const uint8_t* mreg, int c16,
                                               int q, v4f (&acc)[RT][CT]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        long a[RT];
        float dw[RT][4];
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            __builtin_memcpy(&a[r], wt + (r * 16 + c16) * Q80_RING_ROW + 34 * j + 2 + 8 * q, 8);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint16_t h;
                __builtin_memcpy(&h, wt + (r * 16 + 4 * q + i) * Q80_RING_ROW + 34 * j, 2);
                dw[r][i] = half_bits_to_float(h);
            }
        }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            long b;
            __builtin_memcpy(&b, qreg + (ct * 16 + c16) * RING_QS + 32 * j + 8 * q, 8);
            const float dx = *reinterpret_cast<const float*>(mreg + (ct * 16 + c16) * Q8MN_BYTES + 4 * j);
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const v4i s = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[r], b, v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[r][ct][i] = fmaf(dw[r][i] * dx, (float)s[i], acc[r][ct][i]);
            }
        }
    }
}

}  // namespace spq4k
