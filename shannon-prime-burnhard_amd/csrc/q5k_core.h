// q5k_core.h — the Q5_K x Q8_K matvec building blocks (FmtQ5K policy of the
// format-templated GEMV and expert kernels).
//
// Block format (ggml, vendor/ggml/src/ggml-common.h:334-346), 176 B per 256
// weights: fp16 d @0, fp16 dmin @2, scales[12] @4 (the Q4_K 6-bit scale/min
// packing), qh[32] @16 (high bits), qs[128] @48 (low 4 bits). Weight
// e = 64 g + 32 h + l is nibble h of qs[32 g + l] plus 16 * bit (2 g + h) of
// qh[l] (0..31), in sub-block j = 2 g + h: d * sc_j * q - dmin * m_j.
//
// Lane mapping: the Q4_K one (gemv_core.h). Lane l4 of a quad takes nibble
// group g = l4 (sub-blocks 2 l4 and 2 l4 + 1) and reads, besides the 16-byte
// header and its 32 qs bytes, all 32 qh bytes, of which it uses bits 2 l4
// and 2 l4 + 1. Its two integer sub-block sums and the min term are then
// formed exactly as for Q4_K: ggml_vec_dot_q5_K_q8_K
// (ggml-cpu/quants.c:720-798, arch/x86/quants.c:2078-2174) with the integer
// parts exact and only the fp32 summation order changed.
#pragma once

#include "gemv_core.h"

namespace spq4k {

constexpr int Q5K_BYTES = 176;

struct W5 {
    uint4 hdr;        // d | dmin << 16, scale bytes 0-3, 4-7, 8-11
    uint4 qa, qb;     // qs[32 l4 .. +31]
    uint4 ha, hb;     // qh[0 .. 31]
};

__device__ __forceinline__ W5 load_w5(const uint8_t* __restrict__ blk, int l4) {
    W5 w;
    w.hdr = *reinterpret_cast<const uint4*>(blk);
    const uint4* h = reinterpret_cast<const uint4*>(blk + 16);
    w.ha = h[0];
    w.hb = h[1];
    const uint4* q = reinterpret_cast<const uint4*>(blk + 48 + 32 * l4);
    w.qa = q[0];
    w.qb = q[1];
    return w;
}

// 5-bit planes of the lane's 64 values: lo[i] = elements 64 l4 + 4i .. +3
// (sub-block 2 l4), hi[i] = elements 64 l4 + 32 + 4i .. +3 (sub-block 2 l4 + 1).
__device__ __forceinline__ Nib split_q5(const W5& w, int l4) {
    Nib n;
    const uint32_t q[8] = {w.qa.x, w.qa.y, w.qa.z, w.qa.w, w.qb.x, w.qb.y, w.qb.z, w.qb.w};
    const uint32_t h[8] = {w.ha.x, w.ha.y, w.ha.z, w.ha.w, w.hb.x, w.hb.y, w.hb.z, w.hb.w};
    const int b0 = 2 * l4;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        n.lo[i] = (int)((q[i] & 0x0F0F0F0Fu) | (((h[i] >> b0) & 0x01010101u) << 4));
        n.hi[i] = (int)(((q[i] >> 4) & 0x0F0F0F0Fu) | (((h[i] >> (b0 + 1)) & 0x01010101u) << 4));
    }
    return n;
}

// acc + this lane's share of the block against register activations (the
// Q4_K decode layout of Q8Reg).
__device__ __forceinline__ float block_dot5_reg(const W5& w, int l4, const Q8Reg& q, float acc) {
    const float d = half_bits_to_float(w.hdr.x & 0xFFFFu);
    const float dmin = half_bits_to_float(w.hdr.x >> 16);
    int sc0, sc1, m0, m1;
    scales_of_quarter(w.hdr, l4, sc0, sc1, m0, m1);
    const Nib n = split_q5(w, l4);
    int S0 = 0, S1 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        S0 = dot4(n.lo[i], q.a[i], S0);
        S1 = dot4(n.hi[i], q.a[8 + i], S1);
    }
    // |S| <= 32 * 31 * 127 and sc <= 63: exact in 24-bit multiplies (full rate)
    const int A = __mul24(sc0, S0) + __mul24(sc1, S1);
    const int B = m0 * q.bsA + m1 * q.bsB;
    acc = fmaf(d * q.d8, (float)A, acc);
    acc = fmaf(-(dmin * q.d8), (float)B, acc);
    return acc;
}

// One block of one row against T staged activation rows (LDS planes).
template <int T>
__device__ __forceinline__ void block_dot5(const W5& w, int l4, const Q8Lds& L, int bb, int CB, bool live,
                                           float (&acc)[T]) {
    const BlkC k = block_consts(w.hdr, l4);
    const Nib n = split_q5(w, l4);
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int slot = t * CB + bb;
        int S0, S1;
        subblock_pair(n, L.q8 + slot * 256, l4, S0, S1);
        int A = k.sc0 * S0 + k.sc1 * S1;
        int B = min_term(L.bs + slot * 16, l4, k.m0, k.m1);
        A = live ? A : 0;
        B = live ? B : 0;
        const float d8 = L.d8[slot];
        acc[t] = fmaf(k.d * d8, (float)A, acc[t]);
        acc[t] = fmaf(-(k.dmin * d8), (float)B, acc[t]);
    }
}

struct FmtQ5K {
    static constexpr int BYTES = Q5K_BYTES;
    using W = W5;
    using R = Q8Reg;
    static __device__ __forceinline__ W load(const uint8_t* blk, int l4) { return load_w5(blk, l4); }
    static __device__ __forceinline__ void load_reg(const Q8Lds& L, int b, int l4, R& q) { load_q8reg(L, b, l4, q); }
    static __device__ __forceinline__ float dot_reg(const W& w, int l4, const R& q, float acc) {
        return block_dot5_reg(w, l4, q, acc);
    }
    template <int T>
    static __device__ __forceinline__ void dot(const W& w, int l4, const Q8Lds& L, int bb, int CB, bool live,
                                               float (&acc)[T]) {
        block_dot5<T>(w, l4, L, bb, CB, live, acc);
    }
};

}  // namespace spq4k
