// q4k_device.h — device-side building blocks for the gfx950 Q4_K kernels.
//
// Block formats (ggml, vendor/ggml/src/ggml-common.h:317-328 and :361-365):
//   Q4_K super-block, 144 B: fp16 d @0, fp16 dmin @2, scales[12] @4, qs[128] @16;
//        weight e = 64g + 32h + l (g<4, h<2, l<32) is nibble h of qs[32g + l] and
//        belongs to sub-block j = 2g + h with 6-bit scale sc_j and min m_j.
//   Q8_K block, 292 B: f32 d @0, int8 qs[256] @4, int16 bsums[16] @260.
//
// All code here is compiled with -ffp-contract=off; where a fused multiply-add
// is wanted it is written as fmaf.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace spq4k {

constexpr int QK = 256;
constexpr int Q4K_BYTES = 144;
constexpr int Q8K_BYTES = 292;

__device__ __forceinline__ float half_bits_to_float(uint32_t h16) {
    // v_cvt_f32_f16: exact widening, identical to the reference's
    // ggml_compute_fp16_to_fp32 (ggml-impl.h:384) for every non-NaN input.
    _Float16 h;
    uint16_t b = (uint16_t)h16;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// Round to nearest, ties to even, for |v| < 2^22: the value v + 1.5*2^23 has
// bit pattern 0x4B400000 + round(v). Same result as the reference's
// nearest_int (ggml-quants.c:559-564) over its valid range.
__device__ __forceinline__ int nearest_int_small(float v) {
    float r = v + 12582912.0f;
    return (int)__float_as_uint(r) - 0x4B400000;
}

// The reference's nearest_int bit for bit, also outside the valid range
// (used by the Q4_K encoder, whose call sites clamp the result).
__device__ __forceinline__ int nearest_int_ref(float v) {
    float r = v + 12582912.0f;
    return (int)(__float_as_uint(r) & 0x007FFFFFu) - 0x00400000;
}

// All 8 scales and 8 mins of a block as bytes, from the 12 packed scale bytes
// s0 = bytes 0-3, s1 = bytes 4-7, s2 = bytes 8-11 (get_scale_min_k4,
// ggml-quants.c:818-825, evaluated four sub-blocks at a time):
//   sc[0..3] = lo6(s0)                      m[0..3] = lo6(s1)
//   sc[4..7] = lo4(s2) | hi2(s0) << 4       m[4..7] = hi4(s2) | hi2(s1) << 4
struct ScaleMin {
    uint32_t sc_lo, sc_hi, m_lo, m_hi;  // byte i of *_lo -> j = i, of *_hi -> j = 4 + i
};

__device__ __forceinline__ ScaleMin unpack_scale_min(uint32_t s0, uint32_t s1, uint32_t s2) {
    ScaleMin r;
    r.sc_lo = s0 & 0x3F3F3F3Fu;
    r.m_lo  = s1 & 0x3F3F3F3Fu;
    r.sc_hi = (s2 & 0x0F0F0F0Fu) | (((s0 >> 6) & 0x03030303u) << 4);
    r.m_hi  = ((s2 >> 4) & 0x0F0F0F0Fu) | (((s1 >> 6) & 0x03030303u) << 4);
    return r;
}

__device__ __forceinline__ int byte_of(uint32_t w, int i) {
    return (int)((w >> (8 * i)) & 0xFFu);
}

// Signed 4-way int8 dot product with accumulate (v_dot4_i32_i8).
__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// -------------------------------------------------------------------------
// Q8_K quantisation of one 256-value block by 16 lanes (lane e of the 16 owns
// values 16e .. 16e+15), following quantize_row_q8_K_ref
// (ggml-quants.c:2692-2729):
//   the first value of largest |x| (ties -> lowest index) gives max, with sign;
//   iscale = -127/max; q = min(127, nearest_int(iscale*x)); d = 1/iscale;
//   bsums[e] = sum of the 16 q of lane e. An all-zero (or all-NaN) block gives
//   d = 0, q = 0 and bsums = 0.
// The 16 lanes must be an aligned 16-lane slice of the wave.
struct Q8Lane {
    uint32_t q[4];   // 16 int8 values, little-endian
    int bsum;
    float d;         // the block's d (same in all 16 lanes)
};

__device__ __forceinline__ Q8Lane quantize_q8k_16(const float (&x)[16], int e) {
    // key = |x| bits (non-negative floats order as integers) : (255 - idx) : sign
    uint32_t best_hi = 0, best_lo = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t bits = __float_as_uint(x[i]);
        uint32_t ab = bits & 0x7FFFFFFFu;
        if (ab > 0x7F800000u) ab = 0;  // NaN never wins (its |x| > amax is false)
        const uint32_t lo = ((uint32_t)(255 - (16 * e + i)) << 1) | (bits >> 31);
        // strict '>' on |x| keeps the first index on ties; lo breaks ties the same way
        if (ab > best_hi || (ab == best_hi && lo > best_lo)) { best_hi = ab; best_lo = lo; }
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
        const uint32_t oh = __shfl_xor(best_hi, off, 16);
        const uint32_t ol = __shfl_xor(best_lo, off, 16);
        if (oh > best_hi || (oh == best_hi && ol > best_lo)) { best_hi = oh; best_lo = ol; }
    }
    Q8Lane r;
    if (best_hi == 0) {
        r.q[0] = r.q[1] = r.q[2] = r.q[3] = 0;
        r.bsum = 0;
        r.d = 0.0f;
        return r;
    }
    const float amax = __uint_as_float(best_hi);
    const float vmax = (best_lo & 1u) ? -amax : amax;
    const float iscale = -127.0f / vmax;
    int s = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t packed = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // the exact reference rounding and int8 store, so that even
            // degenerate blocks (subnormal max, infinities) match bit for bit
            int v = nearest_int_ref(iscale * x[4 * w + i]);
            v = v < 127 ? v : 127;
            const int q8 = (int)(int8_t)(v & 0xFF);
            s += q8;
            packed |= ((uint32_t)q8 & 0xFFu) << (8 * i);
        }
        r.q[w] = packed;
    }
    r.bsum = s;
    r.d = 1.0f / iscale;
    return r;
}

// -------------------------------------------------------------------------
// Wave-level helpers
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace spq4k
