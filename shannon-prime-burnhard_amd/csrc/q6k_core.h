// q6k_core.h — the Q6_K x Q8_K matvec building blocks (decode and small-batch
// GEMV, expert-gathered matvec, the reference-shaped vec_dot).
//
// Block format (ggml, vendor/ggml/src/ggml-common.h:348-357), 210 B per 256
// weights: ql[128] @0 (low 4 bits), qh[64] @128 (high 2 bits), int8
// scales[16] @192 (one per 16 weights), fp16 d @208. Weight
// e = 128 n + 32 h + l (n < 2, h < 4, l < 32) is
//     q = nibble (h >> 1) of ql[64 n + 32 (h & 1) + l] | bits 2h..2h+1 of qh[32 n + l] << 4
// in 0..63, belongs to sub-block j = 8 n + 2 h + l / 16 and stands for
// d * scales[j] * (q - 32).
//
// Lane mapping (quads on a block, as for Q4_K): lane l4 = 2 n + s of a quad
// takes half n and the l range 16 s .. 16 s + 15 of all four quarters h, i.e.
// the 48 bytes ql[64 n + 16 s ..+15], ql[64 n + 32 + 16 s ..+15],
// qh[32 n + 16 s ..+15], and the scales 8 n + 2 h + s. Each lane forms four
// exact integer sub-block sums with the -32 offset folded into the
// accumulator's start value (-32 * bsums[j], the x86 kernel's q8sclsub,
// ggml-cpu/arch/x86/quants.c:2316-2318):
//     S_j = sum q * q8 - 32 * bsums[j],   I = sum_h scales[j_h] * S_{j_h}
//     acc += (fp16(d) * d8) * I
// This is ggml_vec_dot_q6_K_q8_K (ggml-cpu/quants.c:800-852,
// arch/x86/quants.c:2300-2366) with the integer parts exact and only the fp32
// summation order changed.
//
// Blocks are 210 bytes, so block starts are only 2-byte aligned; the loads
// below declare that alignment (global loads on gfx950 take unaligned
// addresses; the declaration keeps the compiler from picking scalar loads,
// which need 4-byte alignment).
#pragma once

#include "gemv_core.h"

namespace spq4k {

constexpr int Q6K_BYTES = 210;

typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32x2_a2 __attribute__((ext_vector_type(2), aligned(2)));
typedef uint16_t u16_a2 __attribute__((aligned(2)));

__device__ __forceinline__ uint4 load16_a2(const uint8_t* p) {
    const u32x4_a2 v = *reinterpret_cast<const u32x4_a2*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 load8_a2(const uint8_t* p) {
    const u32x2_a2 v = *reinterpret_cast<const u32x2_a2*>(p);
    return make_uint2(v.x, v.y);
}

// Registers of one lane for one block.
struct W6 {
    uint4 lo;    // ql[64 n + 16 s .. +15]       quarters h = 0 (low nibbles), 2 (high nibbles)
    uint4 hi;    // ql[64 n + 32 + 16 s .. +15]  quarters h = 1, 3
    uint4 qh;    // qh[32 n + 16 s .. +15]
    uint2 sc;    // scales[8 n .. 8 n + 7]
    uint32_t d;  // fp16 d in the low half
};

__device__ __forceinline__ W6 load_w6(const uint8_t* __restrict__ blk, int l4) {
    const int n = l4 >> 1, s = l4 & 1;
    W6 w;
    w.lo = load16_a2(blk + 64 * n + 16 * s);
    w.hi = load16_a2(blk + 64 * n + 32 + 16 * s);
    w.qh = load16_a2(blk + 128 + 32 * n + 16 * s);
    w.sc = load8_a2(blk + 192 + 8 * n);
    w.d = *reinterpret_cast<const u16_a2*>(blk + 208);
    return w;
}

// The 6-bit values of one dword position i of the four quarters: q[h] holds
// elements 128 n + 32 h + 16 s + 4 i .. + 3 as unsigned bytes 0..63.
__device__ __forceinline__ void q6_dword(uint32_t a, uint32_t b, uint32_t c, uint32_t (&q)[4]) {
    q[0] = (a & 0x0F0F0F0Fu) | ((c & 0x03030303u) << 4);
    q[1] = (b & 0x0F0F0F0Fu) | ((c & 0x0C0C0C0Cu) << 2);
    q[2] = ((a >> 4) & 0x0F0F0F0Fu) | (c & 0x30303030u);
    q[3] = ((b >> 4) & 0x0F0F0F0Fu) | ((c >> 2) & 0x30303030u);
}

// Signed scale of quarter h for this lane: scales[8 n + 2 h + s].
__device__ __forceinline__ int q6_scale(const uint2& sc, int h, int s) {
    const uint32_t w = h < 2 ? sc.x : sc.y;
    return (int)(int8_t)((w >> (16 * (h & 1) + 8 * s)) & 0xFFu);
}

// Activation registers of one lane for one block (decode kernels):
//   a[4 h + i] = q8[128 n + 32 h + 16 s + 4 i .. + 3],   o[h] = -32 * bsums[8 n + 2 h + s]
struct Q8Reg6 {
    int a[16];
    int o[4];
    float d8;
};

__device__ __forceinline__ void load_q8reg6(const Q8Lds& L, int b, int l4, Q8Reg6& q) {
    const int n = l4 >> 1, s = l4 & 1;
    const int8_t* base = L.q8 + b * 256 + 128 * n + 16 * s;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const int4 v = *reinterpret_cast<const int4*>(base + 32 * h);
        q.a[4 * h] = v.x; q.a[4 * h + 1] = v.y; q.a[4 * h + 2] = v.z; q.a[4 * h + 3] = v.w;
        q.o[h] = -32 * (int)L.bs[b * 16 + 8 * n + 2 * h + s];
    }
    q.d8 = L.d8[b];
}

// The lane's 64 six-bit values: q[4 h + i] = elements 128 n + 32 h + 16 s + 4 i .. + 3.
__device__ __forceinline__ void q6_extract(const W6& w, uint32_t (&q)[16]) {
    const uint32_t A[4] = {w.lo.x, w.lo.y, w.lo.z, w.lo.w};
    const uint32_t B[4] = {w.hi.x, w.hi.y, w.hi.z, w.hi.w};
    const uint32_t Cq[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t v[4];
        q6_dword(A[i], B[i], Cq[i], v);
#pragma unroll
        for (int h = 0; h < 4; ++h) q[4 * h + i] = v[h];
    }
}

// sum_h scale_h * (sum q * q8 - 32 bsum_h) for one lane: exact (|S_h| < 2^17,
// |scale| <= 128).
__device__ __forceinline__ int q6_lane_int(const uint32_t (&q)[16], const int (&sc)[4], const int (&a)[16],
                                           const int (&o)[4]) {
    int I = 0;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        int S = o[h];
#pragma unroll
        for (int i = 0; i < 4; ++i) S = dot4((int)q[4 * h + i], a[4 * h + i], S);
        I += sc[h] * S;
    }
    return I;
}

__device__ __forceinline__ void q6_scales(const W6& w, int l4, int (&sc)[4]) {
#pragma unroll
    for (int h = 0; h < 4; ++h) sc[h] = q6_scale(w.sc, h, l4 & 1);
}

__device__ __forceinline__ float block_dot6_reg(const W6& w, int l4, const Q8Reg6& r, float acc) {
    uint32_t q[16];
    int sc[4];
    q6_extract(w, q);
    q6_scales(w, l4, sc);
    const int I = q6_lane_int(q, sc, r.a, r.o);
    return fmaf(half_bits_to_float(w.d) * r.d8, (float)I, acc);
}

// One block of one row against T staged activation rows (LDS planes).
template <int T>
__device__ __forceinline__ void block_dot6(const W6& w, int l4, const Q8Lds& L, int bb, int CB, bool live,
                                           float (&acc)[T]) {
    const float d = half_bits_to_float(w.d);
    uint32_t q[16];
    int sc[4];
    q6_extract(w, q);
    q6_scales(w, l4, sc);
#pragma unroll
    for (int t = 0; t < T; ++t) {
        Q8Reg6 r;
        load_q8reg6(L, t * CB + bb, l4, r);
        int I = q6_lane_int(q, sc, r.a, r.o);
        I = live ? I : 0;
        acc[t] = fmaf(d * r.d8, (float)I, acc[t]);
    }
}

// ---------------------------------------------------------------------------
// Weight-format policy of Q6_K (the Q4_K one, FmtQ4K, is in gemv_core.h).
struct FmtQ6K {
    static constexpr int BYTES = Q6K_BYTES;
    using W = W6;
    using R = Q8Reg6;
    static __device__ __forceinline__ W load(const uint8_t* blk, int l4) { return load_w6(blk, l4); }
    static __device__ __forceinline__ void load_reg(const Q8Lds& L, int b, int l4, R& q) {
        load_q8reg6(L, b, l4, q);
    }
    static __device__ __forceinline__ float dot_reg(const W& w, int l4, const R& q, float acc) {
        return block_dot6_reg(w, l4, q, acc);
    }
    template <int T>
    static __device__ __forceinline__ void dot(const W& w, int l4, const Q8Lds& L, int bb, int CB, bool live,
                                               float (&acc)[T]) {
        block_dot6<T>(w, l4, L, bb, CB, live, acc);
    }
};

}  // namespace spq4k
