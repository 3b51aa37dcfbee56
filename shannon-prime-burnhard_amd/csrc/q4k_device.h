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

// The reference's nearest_int (ggml-quants.c:559-564) bit for bit: adding
// 1.5*2^23 leaves round-to-nearest-even(v) in the low mantissa bits for
// |v| < 2^22; outside that range the same bit pattern is returned as the
// reference returns (callers clamp).
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

// Signed 4-way int8 dot product with accumulate (v_dot4_i32_i8).
__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// -------------------------------------------------------------------------
// DPP lane exchange within rows of 16 lanes (gfx9 DPP controls).
enum : int {
    DPP_XOR1 = 0xB1,      // quad_perm [1,0,3,2]
    DPP_XOR2 = 0x4E,      // quad_perm [2,3,0,1]
    DPP_ROR4 = 0x124,     // row_ror:4
    DPP_ROR8 = 0x128,     // row_ror:8
    DPP_SHR4 = 0x114,     // row_shr:4 (lanes 0-3 of a row read 0)
    DPP_SHR8 = 0x118,     // row_shr:8 (lanes 0-7 of a row read 0)
    DPP_BCAST15 = 0x142,  // row_bcast:15 (lane 15 of row r -> row r+1)
    DPP_BCAST31 = 0x143,  // row_bcast:31 (lane 31 -> rows 2 and 3)
};

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over each aligned group of N lanes (N = 1, 2, 4, 8, 16, 32, 64); the sum
// is exact in the LAST lane of each group (lane N-1 mod N), other lanes hold
// partial sums. Fixed combination order: deterministic.
template <int N>
__device__ __forceinline__ float group_sum_last(float v) {
    if (N >= 2) v += dpp_f32<DPP_XOR1>(v);
    if (N >= 4) v += dpp_f32<DPP_XOR2>(v);
    if (N >= 8) v += dpp_f32<DPP_SHR4>(v);     // lanes 4-7 (12-15) += lanes 0-3 (8-11)
    if (N >= 16) v += dpp_f32<DPP_SHR8>(v);    // lane 15 += lane 7
    // rows 1 and 3 add lane 15 of rows 0 and 2: lanes 31 and 63 hold 32-lane sums
    if (N >= 32) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_BCAST15, 0xA, 0xF, false));
    // rows 2 and 3 add lane 31: lane 63 holds the wave sum
    if (N >= 64) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_BCAST31, 0xC, 0xF, false));
    return v;
}

// -------------------------------------------------------------------------
// Q8_K quantisation of one 256-value block by an aligned 16-lane row of the
// wave (lane e of the 16 owns values 16e .. 16e+15), following
// quantize_row_q8_K_ref (ggml-quants.c:2692-2729):
//   the first value of largest |x| (ties -> lowest index) gives max, with sign;
//   iscale = -127/max; q = min(127, nearest_int(iscale*x)) stored as int8;
//   d = 1/iscale; bsums[e] = sum of the 16 stored q of lane e.
// An all-zero (or all-NaN) block gives d = 0, q = 0 and bsums = 0.
struct Q8Lane {
    uint32_t q[4];   // 16 int8 values, little-endian
    int bsum;
    float d;         // the block's d (same in all 16 lanes)
};

// Signed value of the first element of largest |x| over the 16-lane row,
// found with an exact (|x|, index) key search; NaN never wins, as in the
// reference's `ax > amax` test. Returns +-0 when every |x| is 0 or NaN.
__device__ __forceinline__ float first_absmax_16(const float (&x)[16], int e) {
    // key = |x| bits (non-negative floats order as integers) : (255 - idx) : sign
    uint32_t best_hi = 0, best_lo = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t bits = __float_as_uint(x[i]);
        uint32_t ab = bits & 0x7FFFFFFFu;
        ab = ab > 0x7F800000u ? 0u : ab;
        // within a lane later indices only replace on a strictly larger |x|
        const bool take = ab > best_hi;
        best_hi = take ? ab : best_hi;
        best_lo = take ? (((uint32_t)(255 - (16 * e + i)) << 1) | (bits >> 31)) : best_lo;
    }
    // lexicographic max of (hi, lo) over the 16 lanes
#define SPQ_KEYMAX(CTRL)                                                  \
    {                                                                     \
        const uint32_t oh = dpp_u32<CTRL>(best_hi);                       \
        const uint32_t ol = dpp_u32<CTRL>(best_lo);                       \
        const bool t = (oh > best_hi) || (oh == best_hi && ol > best_lo); \
        best_hi = t ? oh : best_hi;                                       \
        best_lo = t ? ol : best_lo;                                       \
    }
    SPQ_KEYMAX(DPP_XOR1)
    SPQ_KEYMAX(DPP_XOR2)
    SPQ_KEYMAX(DPP_ROR4)
    SPQ_KEYMAX(DPP_ROR8)
#undef SPQ_KEYMAX
    const float amax = __uint_as_float(best_hi);
    return (best_lo & 1u) ? -amax : amax;
}

__device__ __forceinline__ Q8Lane quantize_q8k_16(const float (&x)[16], int e) {
    // Largest and smallest value of the row (fmaxf/fminf skip NaN, as the
    // reference's comparison does). When the largest |x| occurs with one sign
    // only, that sign is the max's; when +a and -a both occur (or the row is
    // all zero / NaN) the first index decides, by the exact key search.
    float mx = x[0], mn = x[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) {
        mx = fmaxf(mx, x[i]);
        mn = fminf(mn, x[i]);
    }
    mx = fmaxf(mx, dpp_f32<DPP_XOR1>(mx)); mn = fminf(mn, dpp_f32<DPP_XOR1>(mn));
    mx = fmaxf(mx, dpp_f32<DPP_XOR2>(mx)); mn = fminf(mn, dpp_f32<DPP_XOR2>(mn));
    mx = fmaxf(mx, dpp_f32<DPP_ROR4>(mx)); mn = fminf(mn, dpp_f32<DPP_ROR4>(mn));
    mx = fmaxf(mx, dpp_f32<DPP_ROR8>(mx)); mn = fminf(mn, dpp_f32<DPP_ROR8>(mn));
    const float neg = -mn;
    float vmax;
    if (mx > neg) {
        vmax = mx;
    } else if (neg > mx) {
        vmax = mn;
    } else {
        vmax = first_absmax_16(x, e);
    }
    Q8Lane r;
    if (!(fabsf(vmax) > 0.0f)) {
        r.q[0] = r.q[1] = r.q[2] = r.q[3] = 0;
        r.bsum = 0;
        r.d = 0.0f;
        return r;
    }
    const float iscale = -127.0f / vmax;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // the exact reference rounding and int8 store, so that even
            // degenerate blocks (subnormal max, infinities) match bit for bit
            const int t = nearest_int_ref(iscale * x[4 * w + i]);
            v[i] = (uint32_t)(t < 127 ? t : 127);
        }
        // low bytes packed little-endian: v0 | v1 << 8 | v2 << 16 | v3 << 24
        const uint32_t p01 = __builtin_amdgcn_perm(v[1], v[0], 0x0C0C0400u);
        const uint32_t p23 = __builtin_amdgcn_perm(v[3], v[2], 0x04000C0Cu);
        r.q[w] = p01 | p23;
    }
    // sum of the 16 stored int8 values
    int s = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) s = __builtin_amdgcn_sdot4((int)r.q[w], 0x01010101, s, false);
    r.bsum = s;
    r.d = 1.0f / iscale;
    return r;
}

}  // namespace spq4k
