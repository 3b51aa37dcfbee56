// k_dqdot_x.hip — fp32-activation dequant-then-dot for rows of every library
// weight type (Q4_K, Q5_K, Q6_K, Q8_0) on gfx950: the arithmetic of the
// reference's scalar BurnHard matvec, beast_matvec
// (desktop/beast_canyon/sp_beast_canyon.c:1122-1134), which dispatches each
// row to a per-type dequantiser (beast_dequant_row, :1087-1106) and dots it
// with the activations as given (no Q8_K):
//     for each row r: w = dequant(W[r]);  y[r] = sum_j w[j] * x[j]
// and the parts of the BurnHard MoE forward (:455-562) built on it for banks
// of any of those types (k_dqdot.hip keeps the tuned all-Q4_K forward).
//
// Weights are the format's own dequantiser's, bit for bit (ggml's to_float):
//   Q8_0 dequantize_row_q8_0 (ggml-quants.c:491-505): w = q * d, exact;
//   Q6_K dequantize_row_q6_K (:1877-1905): w = (d * sc_j) * (q - 32), sc_j
//        the int8 scale of the value's 16-value sub-block; d * sc_j (fp16 by
//        int8) is exact, so w is one rounding of the exact product;
//   Q5_K dequantize_row_q5_K (:1669-1696) and Q4_K dequantize_row_q4_K
//        (:1467-1489): w = (d * sc) * q - dmin * m; (d * sc) * q is exact (at
//        most 22 significant bits), so the fused multiply-subtract used here
//        rounds once, as the separate product and difference do.
// The reference's own beast_dequant_q6_K (:1025-1052) and beast_dequant_q5_K
// (:1056-1085) read other bits than those formats (a scale per 32 values and
// swapped nibbles for Q6_K, the qh bit of the 64-value group for Q5_K), so for
// those two types the format's dequantiser is the one followed.
// Every product w * x is rounded to fp32 and added in fp32, per lane and then
// across the lane group in a fixed DPP order, where the reference adds
// serially (fp32 reassociation only).
//
// Mapping: a group of 256 weights (a K-quant block, eight Q8_0 blocks) is
// split among a quad of lanes, 64 weights a lane as 16 float4 slots, the
// split each format's byte layout favours (DqxQ6K::slot below; the others
// take 64 consecutive weights a lane). A row is taken by LPR lanes (4 x its
// group count rounded up to a power of two, at most 64: LPR / 4 groups a
// pass), 64 / LPR rows side by side in a wave. The activations are staged in
// LDS lane-major (slot j of lane ll of pass it at (it * 16 + j) * LPR + ll):
// a group's lanes read consecutive 16-byte words, the groups of a wave the
// same ones. Each lane keeps the next piece's loads in flight while it
// computes the current one.
#include "launch.h"
#include "q5k_core.h"
#include "q6k_core.h"
#include "spq4k.h"

namespace spq4k {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) f32x4 lf32x4;

// ---- per-format policies -----------------------------------------------------
// load(row, g, l4, nunit): lane l4's bytes of group g of a row (g clamped to
//   the row, so every load is in bounds);
// live(g, l4, half, nunit): whether slots 8 half .. 8 half + 7 of that lane
//   hold weights of the row (nunit: the row's groups; for Q8_0 its blocks);
// prep / deq: the lane's scale terms, and slot j's four weights;
// lane_of / slot_of: where float4 w4 (weights 4 w4 .. 4 w4 + 3) of a group
//   sits.

struct DqxQ8_0 {
    static constexpr int UNIT = 32;           // weights a block
    static constexpr int UNIT_BYTES = 34;
    static constexpr int GROUP_UNITS = 8;
    struct W {
        uint4 a0, a1, b0, b1;                 // qs of blocks 2 l4 and 2 l4 + 1 of the group
        uint32_t d;                           // their fp16 d, low and high half
    };
    struct Pre {
        float d[2];
    };
    __device__ static W load(const uint8_t* __restrict__ row, int g, int l4, int nunit) {
        const int b = 8 * g + 2 * l4;
        const int b0 = b < nunit ? b : nunit - 1, b1 = b + 1 < nunit ? b + 1 : nunit - 1;
        const uint8_t* p0 = row + (size_t)b0 * UNIT_BYTES;
        const uint8_t* p1 = row + (size_t)b1 * UNIT_BYTES;
        W w;
        w.a0 = load16_a2(p0 + 2);
        w.a1 = load16_a2(p0 + 18);
        w.b0 = load16_a2(p1 + 2);
        w.b1 = load16_a2(p1 + 18);
        w.d = (uint32_t)*reinterpret_cast<const u16_a2*>(p0) | ((uint32_t)*reinterpret_cast<const u16_a2*>(p1) << 16);
        return w;
    }
    __device__ static bool live(int g, int l4, int half, int nunit) { return 8 * g + 2 * l4 + half < nunit; }
    __device__ static Pre prep(const W& w, int) {
        Pre p;
        p.d[0] = half_bits_to_float(w.d & 0xFFFFu);
        p.d[1] = half_bits_to_float(w.d >> 16);
        return p;
    }
    __device__ static void deq(const W& w, const Pre& p, int, int j, float (&o)[4]) {
        const uint4& v = j < 4 ? w.a0 : j < 8 ? w.a1 : j < 12 ? w.b0 : w.b1;
        const uint32_t q = (j & 3) == 0 ? v.x : (j & 3) == 1 ? v.y : (j & 3) == 2 ? v.z : v.w;
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = (float)(int)(int8_t)((q >> (8 * k)) & 0xFFu) * p.d[j >> 3];
    }
    __device__ static int lane_of(int w4) { return w4 >> 4; }
    __device__ static int slot_of(int w4) { return w4 & 15; }
};

// Q6_K: the lane split of q6k_core.h -- lane l4 = 2 n + s takes half n and
// the 16-weight runs s of all four quarters h: slot j = 4 h + i holds weights
// 128 n + 32 h + 16 s + 4 i .. + 3
struct DqxQ6K {
    static constexpr int UNIT = 256;
    static constexpr int UNIT_BYTES = Q6K_BYTES;
    static constexpr int GROUP_UNITS = 1;
    typedef W6 W;
    struct Pre {
        float ds[4];                          // d * scale of quarter h (exact)
    };
    __device__ static W load(const uint8_t* __restrict__ row, int g, int l4, int nunit) {
        return load_w6(row + (size_t)(g < nunit ? g : nunit - 1) * Q6K_BYTES, l4);
    }
    __device__ static bool live(int g, int, int, int nunit) { return g < nunit; }
    __device__ static Pre prep(const W& w, int l4) {
        Pre p;
        const float d = half_bits_to_float(w.d & 0xFFFFu);
#pragma unroll
        for (int h = 0; h < 4; ++h) p.ds[h] = d * (float)q6_scale(w.sc, h, l4 & 1);
        return p;
    }
    __device__ static void deq(const W& w, const Pre& p, int, int j, float (&o)[4]) {
        const int h = j >> 2, i = j & 3;
        const uint32_t a = i == 0 ? w.lo.x : i == 1 ? w.lo.y : i == 2 ? w.lo.z : w.lo.w;
        const uint32_t b = i == 0 ? w.hi.x : i == 1 ? w.hi.y : i == 2 ? w.hi.z : w.hi.w;
        const uint32_t c = i == 0 ? w.qh.x : i == 1 ? w.qh.y : i == 2 ? w.qh.z : w.qh.w;
        uint32_t q[4];
        q6_dword(a, b, c, q);
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = p.ds[h] * (float)((int)((q[h] >> (8 * k)) & 0xFFu) - 32);
    }
    __device__ static int lane_of(int w4) { return 2 * (w4 >> 5) + ((w4 >> 2) & 1); }
    __device__ static int slot_of(int w4) { return 4 * ((w4 >> 3) & 3) + (w4 & 3); }
};

// the sub-block scale terms of lane l4 (sub-blocks 2 l4 and 2 l4 + 1) from a
// K-quant header word set (fp16 d | dmin << 16, scale bytes 0-3, 4-7, 8-11)
struct DqxKPre {
    float d1, m1, d2, m2;
};
__device__ __forceinline__ DqxKPre dqx_kpre(const uint4& h, int l4) {
    const float d = half_bits_to_float(h.x & 0xFFFFu);
    const float dmin = half_bits_to_float(h.x >> 16);
    const ScaleMin sm = unpack_scale_min(h.y, h.z, h.w);
    const uint32_t scw = l4 < 2 ? sm.sc_lo : sm.sc_hi;
    const uint32_t mw = l4 < 2 ? sm.m_lo : sm.m_hi;
    const int sh = 16 * (l4 & 1);
    DqxKPre p;
    p.d1 = d * (float)((scw >> sh) & 0xFFu);
    p.m1 = dmin * (float)((mw >> sh) & 0xFFu);
    p.d2 = d * (float)((scw >> (sh + 8)) & 0xFFu);
    p.m2 = dmin * (float)((mw >> (sh + 8)) & 0xFFu);
    return p;
}

__device__ __forceinline__ uint32_t u4_at(const uint4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

struct DqxQ5K {
    static constexpr int UNIT = 256;
    static constexpr int UNIT_BYTES = Q5K_BYTES;
    static constexpr int GROUP_UNITS = 1;
    typedef W5 W;
    typedef DqxKPre Pre;
    __device__ static W load(const uint8_t* __restrict__ row, int g, int l4, int nunit) {
        return load_w5(row + (size_t)(g < nunit ? g : nunit - 1) * Q5K_BYTES, l4);
    }
    __device__ static bool live(int g, int, int, int nunit) { return g < nunit; }
    __device__ static Pre prep(const W& w, int l4) { return dqx_kpre(w.hdr, l4); }
    __device__ static void deq(const W& w, const Pre& p, int l4, int j, float (&o)[4]) {
        const int half = j >> 3, i = j & 7;
        const uint32_t q = i < 4 ? u4_at(w.qa, i) : u4_at(w.qb, i - 4);
        const uint32_t hb = i < 4 ? u4_at(w.ha, i) : u4_at(w.hb, i - 4);
        const uint32_t v = ((half ? q >> 4 : q) & 0x0F0F0F0Fu) | (((hb >> (2 * l4 + half)) & 0x01010101u) << 4);
        const float dd = half ? p.d2 : p.d1, mm = half ? p.m2 : p.m1;
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = __builtin_fmaf(dd, (float)((v >> (8 * k)) & 0xFFu), -mm);
    }
    __device__ static int lane_of(int w4) { return w4 >> 4; }
    __device__ static int slot_of(int w4) { return w4 & 15; }
};

struct DqxQ4K {
    static constexpr int UNIT = 256;
    static constexpr int UNIT_BYTES = Q4K_BYTES;
    static constexpr int GROUP_UNITS = 1;
    struct W {
        uint4 h, qa, qb;
    };
    typedef DqxKPre Pre;
    __device__ static W load(const uint8_t* __restrict__ row, int g, int l4, int nunit) {
        const uint8_t* blk = row + (size_t)(g < nunit ? g : nunit - 1) * Q4K_BYTES;
        W w;
        w.h = *reinterpret_cast<const uint4*>(blk);
        w.qa = *reinterpret_cast<const uint4*>(blk + 16 + 32 * l4);
        w.qb = *reinterpret_cast<const uint4*>(blk + 32 + 32 * l4);
        return w;
    }
    __device__ static bool live(int g, int, int, int nunit) { return g < nunit; }
    __device__ static Pre prep(const W& w, int l4) { return dqx_kpre(w.h, l4); }
    __device__ static void deq(const W& w, const Pre& p, int, int j, float (&o)[4]) {
        const int half = j >> 3, i = j & 7;
        const uint32_t q = i < 4 ? u4_at(w.qa, i) : u4_at(w.qb, i - 4);
        const uint32_t v = (half ? q >> 4 : q) & 0x0F0F0F0Fu;
        const float dd = half ? p.d2 : p.d1, mm = half ? p.m2 : p.m1;
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = __builtin_fmaf(dd, (float)((v >> (8 * k)) & 0xFFu), -mm);
    }
    __device__ static int lane_of(int w4) { return w4 >> 4; }
    __device__ static int slot_of(int w4) { return w4 & 15; }
};

// ---- shared pieces -----------------------------------------------------------

// x (K values) into the staging layout of LPR-lane rows at xs, eight loads a
// thread in flight at a time (unconditional: past the end they read the last
// float4, which is not stored)
template <class P, int LPR>
__device__ __forceinline__ void dqx_stage(const float* __restrict__ x, int K, f32x4* xs) {
    constexpr int GPP = LPR / 4;              // groups a pass
    const f32x4* xr = reinterpret_cast<const f32x4*>(x);
    const int n4 = K >> 2;
    for (int base = threadIdx.x; base < n4; base += 8 * (int)blockDim.x) {
        f32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e4 = base + u * (int)blockDim.x;
            v[u] = xr[e4 < n4 ? e4 : n4 - 1];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e4 = base + u * (int)blockDim.x;
            if (e4 < n4) {
                const int g = e4 >> 6, w4 = e4 & 63, it = g / GPP;
                xs[(it * 16 + P::slot_of(w4)) * LPR + 4 * (g - it * GPP) + P::lane_of(w4)] = v[u];
            }
        }
    }
}

// acc[t] += this lane's products of one piece (group g of the row); xl points
// at token 0's slot 0 of the piece's pass for this lane, tstride float4 apart
template <class P, int LPR, int T>
__device__ __forceinline__ void dqx_piece(const typename P::W& w, int l4, int g, int nunit, const lf32x4* xl,
                                          int tstride, float (&acc)[T]) {
    const typename P::Pre pre = P::prep(w, l4);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        if (!P::live(g, l4, half, nunit)) continue;
#pragma unroll
        for (int i4 = 0; i4 < 8; ++i4) {
            const int j = 8 * half + i4;
            float wv[4];
            P::deq(w, pre, l4, j, wv);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const f32x4 x = xl[t * tstride + j * LPR];
                float a = acc[t];
                a = a + wv[0] * x.x;
                a = a + wv[1] * x.y;
                a = a + wv[2] * x.z;
                a = a + wv[3] * x.w;
                acc[t] = a;
            }
        }
    }
}

// the dot of the row at `row` (one per lane group) for T tokens: every pass,
// the next pass's loads in flight while the current one is computed
template <class P, int LPR, int T>
__device__ __forceinline__ void dqx_row(const uint8_t* __restrict__ row, int npass, int nunit, int l4, int gl,
                                        const lf32x4* xl, int tstride, float (&acc)[T]) {
    constexpr int GPP = LPR / 4;
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.0f;
    typename P::W cur = P::load(row, gl, l4, nunit);
    for (int it = 0; it < npass; ++it) {
        const int g = gl + GPP * it;
        const typename P::W nxt = P::load(row, g + GPP, l4, nunit);   // past the end: a clamped, unused load
        dqx_piece<P, LPR, T>(cur, l4, g, nunit, xl + it * 16 * LPR, tstride, acc);
        cur = nxt;
    }
}

template <class P>
__host__ __device__ constexpr int dqx_groups(int64_t K) {
    return (int)((K + 255) / 256);
}

template <class P>
__host__ __device__ constexpr int dqx_units(int64_t K) {
    return (int)(K / P::UNIT);
}

// ---- kernels -----------------------------------------------------------------
// Each lane group walks the pieces of its rows (a piece: a pass of LPR / 4
// groups of a row) with the next piece's loads in flight while it computes
// the current one, across row boundaries too; the first piece's loads go out
// before the activations are staged. Every load is unconditional (a row past
// the end is clamped to a valid one and dropped), so the wait before a
// piece's use counts exactly the loads issued after it.

// dense rows: Y[t * y_ts + r] for r < M, t < nt <= T (tokens past nt are
// neither staged nor stored; their products, of unstaged LDS, are dropped);
// rows_per_wg consecutive rows a workgroup of 4 waves
template <class P, int LPR, int T>
__global__ __launch_bounds__(256) void dqx_matvec_kernel(const uint8_t* __restrict__ W, size_t row_bytes, int M, int K,
                                                         const float* __restrict__ X, int64_t x_ts, int nt,
                                                         float* __restrict__ Y, int64_t y_ts, int rows_per_wg) {
    extern __shared__ __align__(16) f32x4 dqx_x[];
    constexpr int GPP = LPR / 4, RW = 64 / LPR;
    const int ngroup = dqx_groups<P>(K), nunit = dqx_units<P>(K);
    const int npass = (ngroup + GPP - 1) / GPP;
    const int tstride = npass * 16 * LPR;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane / LPR, ll = lane % LPR;
    const int l4 = ll & 3, gl = ll >> 2;
    const int r0 = blockIdx.x * rows_per_wg;
    const int r1 = r0 + rows_per_wg < M ? r0 + rows_per_wg : M;
    // the wave's rows rb + grp, rb = r0 + wave RW, + 4 RW, ...
    auto row_at = [&](int rb) {
        const int r = rb + grp;
        return W + (size_t)(r < r1 ? r : r1 - 1) * row_bytes;
    };
    int rb = r0 + wave * RW;
    typename P::W cur = P::load(row_at(rb < r1 ? rb : r0), gl, l4, nunit);
    for (int t = 0; t < nt; ++t) dqx_stage<P, LPR>(X + t * x_ts, K, dqx_x + (size_t)t * tstride);
    __syncthreads();
    const lf32x4* xl = (const lf32x4*)dqx_x + ll;
    for (; rb < r1; rb += 4 * RW) {                                // uniform over the wave
        const uint8_t* row = row_at(rb);
        const uint8_t* nrow = row_at(rb + 4 * RW < r1 ? rb + 4 * RW : rb);
        float acc[T];
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = 0.0f;
        for (int it = 0; it < npass; ++it) {
            const int g = gl + GPP * it;
            const bool same = it + 1 < npass;                        // the next piece: this row's next pass,
            const typename P::W nxt = P::load(same ? row : nrow, same ? g + GPP : gl, l4, nunit);   // else the next row's first
            dqx_piece<P, LPR, T>(cur, l4, g, nunit, xl + it * 16 * LPR, tstride, acc);
            cur = nxt;
        }
        const int r = rb + grp;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float sm = group_sum_last<LPR>(acc[t]);
            if (ll == LPR - 1 && r < r1 && t < nt) Y[(int64_t)t * y_ts + r] = sm;
        }
    }
}

// the selected experts' rows against the hidden row: sweep row q = s rows + r
// (s < top_k) is row r of expert ids[s]. MODE 0: H[q] = the dot of `bank`'s
// row; MODE 1: H[q] = silu(H[q]) * the dot (beast_silu_mul, :1168-1173, with
// the gate's dot stored by a MODE 0 launch); MODE 2: gate (`bank`) and up
// (`bank1`, the same type) in one launch, H[q] = silu(gate . x) * (up . x).
// 0 where ids[s] names no expert.
template <class P, int LPR, int MODE>
__global__ __launch_bounds__(256) void dqx_experts_kernel(const uint8_t* __restrict__ bank,
                                                          const uint8_t* __restrict__ bank1, size_t expert_bytes,
                                                          size_t row_bytes, int rows, int K,
                                                          const int32_t* __restrict__ ids, int E, int top_k,
                                                          const float* __restrict__ hidden, float* __restrict__ H,
                                                          int rows_per_wg) {
    extern __shared__ __align__(16) f32x4 dqx_x[];
    constexpr int GPP = LPR / 4, RW = 64 / LPR;
    const int ngroup = dqx_groups<P>(K), nunit = dqx_units<P>(K);
    const int npass = (ngroup + GPP - 1) / GPP;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane / LPR, ll = lane % LPR;
    const int l4 = ll & 3, gl = ll >> 2;
    const int total = top_k * rows;
    const int q0 = blockIdx.x * rows_per_wg;
    const int q1 = q0 + rows_per_wg < total ? q0 + rows_per_wg : total;
    struct Src {
        const uint8_t* w;
        const uint8_t* w1;
        bool live;
    };
    auto src_at = [&](int qb) {
        Src o;
        const int q = qb + grp < q1 ? qb + grp : q1 - 1;
        const int s = q / rows, r = q - s * rows;
        const int e = ids[s];
        o.live = e >= 0 && e < E;
        const size_t off = (size_t)(o.live ? e : 0) * expert_bytes + (size_t)r * row_bytes;
        o.w = bank + off;
        o.w1 = (MODE == 2 ? bank1 : bank) + off;
        return o;
    };
    int qb = q0 + wave * RW;
    Src cs = src_at(qb < q1 ? qb : q0);
    typename P::W cur = P::load(cs.w, gl, l4, nunit);
    typename P::W cur1 = cur;
    if (MODE == 2) cur1 = P::load(cs.w1, gl, l4, nunit);
    dqx_stage<P, LPR>(hidden, K, dqx_x);
    __syncthreads();
    const lf32x4* xl = (const lf32x4*)dqx_x + ll;
    for (; qb < q1; qb += 4 * RW) {                                // uniform over the wave
        const Src ns = src_at(qb + 4 * RW < q1 ? qb + 4 * RW : qb);
        float acc[1] = {0.0f}, acc1[1] = {0.0f};
        for (int it = 0; it < npass; ++it) {
            const int g = gl + GPP * it;
            const bool same = it + 1 < npass;
            const typename P::W nxt = P::load(same ? cs.w : ns.w, same ? g + GPP : gl, l4, nunit);
            typename P::W nxt1 = nxt;
            if (MODE == 2) nxt1 = P::load(same ? cs.w1 : ns.w1, same ? g + GPP : gl, l4, nunit);
            dqx_piece<P, LPR, 1>(cur, l4, g, nunit, xl + it * 16 * LPR, 0, acc);
            if (MODE == 2) dqx_piece<P, LPR, 1>(cur1, l4, g, nunit, xl + it * 16 * LPR, 0, acc1);
            cur = nxt;
            cur1 = nxt1;
        }
        const float d = group_sum_last<LPR>(acc[0]);
        const float d1 = MODE == 2 ? group_sum_last<LPR>(acc1[0]) : 0.0f;
        const int q = qb + grp;
        if (ll == LPR - 1 && q < q1) {
            if (MODE == 0) {
                H[q] = cs.live ? d : 0.0f;
            } else if (MODE == 1) {
                const float gt = H[q];
                H[q] = cs.live ? (gt / (1.0f + expf(-gt))) * d : 0.0f;
            } else {
                H[q] = cs.live ? (d / (1.0f + expf(-d))) * d1 : 0.0f;
            }
        }
        cs = ns;
    }
}

// down rows of the selected experts against their H rows, summed in rank
// order as out[i] += score * down (:541-543, fused multiply-add as the
// reference's GCC build contracts it), one wave a row: the valid selected
// experts, compacted in rank order, are dealt to the lane groups (slot v to
// group v % GPW), each group walking the pieces of its slots' rows with the
// next piece in flight; the wave then adds the slots' products in rank order.
// Every selected expert's H row is staged once a workgroup (top_k rows in
// LDS); an id outside [0, E) is skipped.
constexpr int DQX_DOWN_WAVES = 8;

template <class P, int LPR>
__global__ __launch_bounds__(DQX_DOWN_WAVES * 64) void dqx_down_rows_kernel(
    const uint8_t* __restrict__ down, size_t expert_bytes, size_t row_bytes, int n_embd, int n_ff,
    const int32_t* __restrict__ ids, int E, const float* __restrict__ scores, int top_k, const float* __restrict__ H,
    float* __restrict__ out) {
    extern __shared__ __align__(16) f32x4 dqx_x[];
    __shared__ int v_e[BEAST_MAX_TOPK], v_s[BEAST_MAX_TOPK];
    __shared__ float v_sc[BEAST_MAX_TOPK];
    __shared__ float v_d[DQX_DOWN_WAVES * BEAST_MAX_TOPK];
    __shared__ int v_n;
    constexpr int GPP = LPR / 4, GPW = 64 / LPR;
    const int ngroup = dqx_groups<P>(n_ff), nunit = dqx_units<P>(n_ff);
    const int npass = (ngroup + GPP - 1) / GPP;
    const int tstride = npass * 16 * LPR;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane / LPR, ll = lane % LPR;
    const int l4 = ll & 3, gl = ll >> 2;
    const int row = blockIdx.x * DQX_DOWN_WAVES + wave;
    const size_t roff = (size_t)(row < n_embd ? row : n_embd - 1) * row_bytes;
    // this group's first slot (the grp-th valid one, rank order), found by
    // every lane from the ids so that its loads go out before the staging
    int fe = 0, cnt = 0;
    for (int s = 0; s < top_k; ++s) {
        const int e = ids[s];
        const bool ok = e >= 0 && e < E;
        if (ok && cnt == grp) fe = e;
        cnt += ok ? 1 : 0;
    }
    typename P::W cur = P::load(down + (size_t)fe * expert_bytes + roff, gl, l4, nunit);
    if (threadIdx.x == 0) {
        int n = 0;
        for (int s = 0; s < top_k; ++s) {
            const int e = ids[s];
            if (e >= 0 && e < E) {
                v_e[n] = e;
                v_s[n] = s;
                v_sc[n] = scores[s];
                ++n;
            }
        }
        v_n = n;
    }
    for (int s = 0; s < top_k; ++s) dqx_stage<P, LPR>(H + (size_t)s * n_ff, n_ff, dqx_x + (size_t)s * tstride);
    __syncthreads();
    const int nv = v_n;
    const int per = (nv + GPW - 1) / GPW;                             // slots a group (uniform)
    const int pieces = per * npass;
    // piece c of the group: its slot k = c / npass (the valid slot grp + GPW k),
    // pass c % npass; nv >= 1 whenever a piece runs, so v_e[0] is set
    int k = 0, it = 0;
    float acc[1] = {0.0f};
    for (int c = 0; c < pieces; ++c) {
        const int nk = it + 1 < npass ? k : k + 1;
        const int nit = it + 1 < npass ? it + 1 : 0;
        const int nvi = grp + GPW * nk;
        const int ne = v_e[nvi < nv ? nvi : (grp < nv ? grp : 0)];
        const typename P::W nxt = P::load(down + (size_t)ne * expert_bytes + roff, gl + GPP * nit, l4, nunit);
        const int vi = grp + GPW * k;
        const bool live = vi < nv;
        const lf32x4* xl = (const lf32x4*)dqx_x + (size_t)v_s[live ? vi : 0] * tstride + it * 16 * LPR + ll;
        if (live) dqx_piece<P, LPR, 1>(cur, l4, gl + GPP * it, nunit, xl, 0, acc);
        if (it == npass - 1) {                                        // uniform: the slot's last pass
            const float d = group_sum_last<LPR>(acc[0]);
            if (ll == LPR - 1 && live) v_d[wave * BEAST_MAX_TOPK + vi] = d;
            acc[0] = 0.0f;
        }
        cur = nxt;
        k = nk;
        it = nit;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if (lane == 0 && row < n_embd) {
        float o = 0.0f;
        for (int v = 0; v < nv; ++v) o = fmaf(v_sc[v], v_d[wave * BEAST_MAX_TOPK + v], o);
        out[row] = o;
    }
}

// The same sum for rows whose selected experts' H rows do not all fit the
// staging area: a lane group holds up to DQX_DOWN_RPW rows, its workgroup
// rows_per_wg consecutive rows; the H rows are staged one expert at a time.
constexpr int DQX_DOWN_RPW = 8;

template <class P, int LPR>
__global__ __launch_bounds__(256) void dqx_down_kernel(const uint8_t* __restrict__ down, size_t expert_bytes,
                                                       size_t row_bytes, int n_embd, int n_ff,
                                                       const int32_t* __restrict__ ids, int E,
                                                       const float* __restrict__ scores, int top_k,
                                                       const float* __restrict__ H, float* __restrict__ out,
                                                       int rows_per_wg) {
    extern __shared__ __align__(16) f32x4 dqx_x[];
    constexpr int GPP = LPR / 4, RW = 64 / LPR;
    const int ngroup = dqx_groups<P>(n_ff), nunit = dqx_units<P>(n_ff);
    const int npass = (ngroup + GPP - 1) / GPP;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane / LPR, ll = lane % LPR;
    const int l4 = ll & 3, gl = ll >> 2;
    const lf32x4* xl = (const lf32x4*)dqx_x + ll;
    const int r0 = blockIdx.x * rows_per_wg;
    const int r1 = r0 + rows_per_wg < n_embd ? r0 + rows_per_wg : n_embd;
    float acc[DQX_DOWN_RPW];
#pragma unroll
    for (int j = 0; j < DQX_DOWN_RPW; ++j) acc[j] = 0.0f;
    for (int s = 0; s < top_k; ++s) {
        const int e = ids[s];
        if (e < 0 || e >= E) continue;         // uniform over the workgroup
        __syncthreads();                       // the previous expert's readers are done
        dqx_stage<P, LPR>(H + (size_t)s * n_ff, n_ff, dqx_x);
        __syncthreads();
        const float sc = scores[s];
        const uint8_t* base = down + (size_t)e * expert_bytes;
#pragma unroll
        for (int j = 0; j < DQX_DOWN_RPW; ++j) {
            const int rb = r0 + (wave + 4 * j) * RW;
            if (rb >= r1) break;               // uniform over the wave
            const int r = rb + grp;
            float d[1];
            dqx_row<P, LPR, 1>(base + (size_t)(r < r1 ? r : r1 - 1) * row_bytes, npass, nunit, l4, gl, xl, 0, d);
            acc[j] = fmaf(sc, group_sum_last<LPR>(d[0]), acc[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < DQX_DOWN_RPW; ++j) {
        const int r = r0 + (wave + 4 * j) * RW + grp;
        if (ll == LPR - 1 && r < r1) out[r] = acc[j];
    }
}

// ---- launches ------------------------------------------------------------------

int dqx_lpr(int ngroup) {
    int l = 4;
    while (l < 64 && l < 4 * ngroup) l *= 2;
    return l;
}

// LDS bytes of one staged row of K values for LPR-lane rows
template <class P>
size_t dqx_row_lds(int64_t K, int lpr) {
    const int gpp = lpr / 4;
    const int64_t npass = (dqx_groups<P>(K) + gpp - 1) / gpp;
    return (size_t)npass * 16 * lpr * sizeof(f32x4);
}

template <class Kern>
hipError_t dqx_lds_attr(Kern k, size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    return hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

// about two workgroups a CU, each a contiguous run of rows (a multiple of the
// rows its four waves take side by side): every workgroup stages the whole
// activation row, so fewer, longer runs read less of it again
int64_t dqx_rows_per_wg(int64_t total, int rw, int num_cus) {
    const int64_t want = (int64_t)num_cus * 2, unit = 4LL * rw;
    int64_t per = (total + want - 1) / want;
    return (per + unit - 1) / unit * unit;
}

template <class P, int LPR, int T>
hipError_t dqx_matvec_lt(const uint8_t* W, int M, int K, const float* X, int64_t x_ts, int nt, float* Y, int64_t y_ts,
                         int num_cus, hipStream_t st) {
    const size_t row_bytes = (size_t)(K / P::UNIT) * P::UNIT_BYTES;
    const size_t lds = (size_t)T * dqx_row_lds<P>(K, LPR);
    hipError_t e = dqx_lds_attr(dqx_matvec_kernel<P, LPR, T>, lds);
    if (e != hipSuccess) return e;
    const int64_t rpw = dqx_rows_per_wg(M, 64 / LPR, num_cus);
    hipLaunchKernelGGL((dqx_matvec_kernel<P, LPR, T>), dim3((unsigned)((M + rpw - 1) / rpw)), dim3(256), lds, st, W,
                       row_bytes, M, K, X, x_ts, nt, Y, y_ts, (int)rpw);
    return hipGetLastError();
}

// T = 1 at every row width; more tokens (2, 4 or 8 a launch) with 64-lane rows
template <class P>
hipError_t dqx_matvec_p(const uint8_t* W, int M, int K, const float* X, int64_t x_ts, float* Y, int64_t y_ts, int T,
                        int num_cus, hipStream_t st) {
    if (T == 1) {
        switch (dqx_lpr(dqx_groups<P>(K))) {
            case 4: return dqx_matvec_lt<P, 4, 1>(W, M, K, X, x_ts, T, Y, y_ts, num_cus, st);
            case 8: return dqx_matvec_lt<P, 8, 1>(W, M, K, X, x_ts, T, Y, y_ts, num_cus, st);
            case 16: return dqx_matvec_lt<P, 16, 1>(W, M, K, X, x_ts, T, Y, y_ts, num_cus, st);
            case 32: return dqx_matvec_lt<P, 32, 1>(W, M, K, X, x_ts, T, Y, y_ts, num_cus, st);
            default: return dqx_matvec_lt<P, 64, 1>(W, M, K, X, x_ts, T, Y, y_ts, num_cus, st);
        }
    }
    if (T == 2) return dqx_matvec_lt<P, 64, 2>(W, M, K, X, x_ts, T, Y, y_ts, num_cus, st);
    if (T <= 4) return dqx_matvec_lt<P, 64, 4>(W, M, K, X, x_ts, T, Y, y_ts, num_cus, st);
    return dqx_matvec_lt<P, 64, 8>(W, M, K, X, x_ts, T, Y, y_ts, num_cus, st);
}

template <class P, int LPR, int MODE>
hipError_t dqx_experts_m(const uint8_t* bank, const uint8_t* bank1, int E, int rows, int K, const int32_t* ids,
                         int top_k, const float* hidden, float* H, int num_cus, hipStream_t st) {
    const size_t row_bytes = (size_t)(K / P::UNIT) * P::UNIT_BYTES;
    const size_t expert_bytes = row_bytes * rows;
    const size_t lds = dqx_row_lds<P>(K, LPR);
    const int64_t total = (int64_t)top_k * rows;
    const int64_t rpw = dqx_rows_per_wg(total, 64 / LPR, num_cus);
    hipError_t e = dqx_lds_attr(dqx_experts_kernel<P, LPR, MODE>, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((dqx_experts_kernel<P, LPR, MODE>), dim3((unsigned)((total + rpw - 1) / rpw)), dim3(256), lds,
                       st, bank, bank1, expert_bytes, row_bytes, rows, K, ids, E, top_k, hidden, H, (int)rpw);
    return hipGetLastError();
}

template <class P, int LPR>
hipError_t dqx_experts_l(int mode, const uint8_t* bank, const uint8_t* bank1, int E, int rows, int K,
                         const int32_t* ids, int top_k, const float* hidden, float* H, int num_cus, hipStream_t st) {
    if (mode == 2) return dqx_experts_m<P, LPR, 2>(bank, bank1, E, rows, K, ids, top_k, hidden, H, num_cus, st);
    if (mode == 1) return dqx_experts_m<P, LPR, 1>(bank, bank1, E, rows, K, ids, top_k, hidden, H, num_cus, st);
    return dqx_experts_m<P, LPR, 0>(bank, bank1, E, rows, K, ids, top_k, hidden, H, num_cus, st);
}

template <class P>
hipError_t dqx_experts_p(int mode, const uint8_t* bank, const uint8_t* bank1, int E, int rows, int K,
                         const int32_t* ids, int top_k, const float* hidden, float* H, int num_cus, hipStream_t st) {
    switch (dqx_lpr(dqx_groups<P>(K))) {
        case 4: return dqx_experts_l<P, 4>(mode, bank, bank1, E, rows, K, ids, top_k, hidden, H, num_cus, st);
        case 8: return dqx_experts_l<P, 8>(mode, bank, bank1, E, rows, K, ids, top_k, hidden, H, num_cus, st);
        case 16: return dqx_experts_l<P, 16>(mode, bank, bank1, E, rows, K, ids, top_k, hidden, H, num_cus, st);
        case 32: return dqx_experts_l<P, 32>(mode, bank, bank1, E, rows, K, ids, top_k, hidden, H, num_cus, st);
        default: return dqx_experts_l<P, 64>(mode, bank, bank1, E, rows, K, ids, top_k, hidden, H, num_cus, st);
    }
}

template <class P, int LPR>
hipError_t dqx_down_l(const uint8_t* down, int E, int n_embd, int n_ff, const int32_t* ids, const float* scores,
                      int top_k, const float* H, float* out, int num_cus, hipStream_t st) {
    const size_t row_bytes = (size_t)(n_ff / P::UNIT) * P::UNIT_BYTES;
    const size_t expert_bytes = row_bytes * n_embd;
    const size_t lds = dqx_row_lds<P>(n_ff, LPR);
    hipError_t e;
    if ((size_t)top_k * lds <= DQ_MATVEC_LDS_MAX) {
        // every selected expert's H row staged at once: a wave a row
        e = dqx_lds_attr(dqx_down_rows_kernel<P, LPR>, (size_t)top_k * lds);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((dqx_down_rows_kernel<P, LPR>), dim3((unsigned)((n_embd + DQX_DOWN_WAVES - 1) / DQX_DOWN_WAVES)),
                           dim3(DQX_DOWN_WAVES * 64), (size_t)top_k * lds, st, down, expert_bytes, row_bytes, n_embd,
                           n_ff, ids, E, scores, top_k, H, out);
        return hipGetLastError();
    }
    e = dqx_lds_attr(dqx_down_kernel<P, LPR>, lds);
    if (e != hipSuccess) return e;
    // rows in runs of a multiple of the workgroup's side-by-side rows, at most
    // DQX_DOWN_RPW a lane group, about two workgroups a CU: each workgroup
    // stages every selected expert's H row, so longer runs read less of it again
    constexpr int RW = 64 / LPR;
    const int64_t want = 2LL * num_cus, unit = 4LL * RW;
    int64_t rpw = ((int64_t)n_embd + want - 1) / want;
    rpw = (rpw + unit - 1) / unit * unit;
    if (rpw > unit * DQX_DOWN_RPW) rpw = unit * DQX_DOWN_RPW;
    hipLaunchKernelGGL((dqx_down_kernel<P, LPR>), dim3((unsigned)((n_embd + rpw - 1) / rpw)), dim3(256), lds, st, down,
                       expert_bytes, row_bytes, n_embd, n_ff, ids, E, scores, top_k, H, out, (int)rpw);
    return hipGetLastError();
}

template <class P>
hipError_t dqx_down_p(const uint8_t* down, int E, int n_embd, int n_ff, const int32_t* ids, const float* scores,
                      int top_k, const float* H, float* out, int num_cus, hipStream_t st) {
    switch (dqx_lpr(dqx_groups<P>(n_ff))) {
        case 4: return dqx_down_l<P, 4>(down, E, n_embd, n_ff, ids, scores, top_k, H, out, num_cus, st);
        case 8: return dqx_down_l<P, 8>(down, E, n_embd, n_ff, ids, scores, top_k, H, out, num_cus, st);
        case 16: return dqx_down_l<P, 16>(down, E, n_embd, n_ff, ids, scores, top_k, H, out, num_cus, st);
        case 32: return dqx_down_l<P, 32>(down, E, n_embd, n_ff, ids, scores, top_k, H, out, num_cus, st);
        default: return dqx_down_l<P, 64>(down, E, n_embd, n_ff, ids, scores, top_k, H, out, num_cus, st);
    }
}

// the type's block size in values, or 0 for a type these kernels do not take
int dqx_unit(int type) {
    switch (type) {
        case SPQ4K_TYPE_Q8_0: return 32;
        case SPQ4K_TYPE_Q4_K:
        case SPQ4K_TYPE_Q5_K:
        case SPQ4K_TYPE_Q6_K: return 256;
        default: return 0;
    }
}

template <class P>
size_t dqx_lds_p(int64_t K, int T) {
    return (size_t)T * dqx_row_lds<P>(K, T == 1 ? dqx_lpr(dqx_groups<P>(K)) : 64);
}

}  // namespace

size_t dqx_lds_bytes(int type, int64_t K, int T) {
    const int t = T == 1 ? 1 : T == 2 ? 2 : T <= 4 ? 4 : 8;    // the token count the launch stages
    switch (type) {
        case SPQ4K_TYPE_Q8_0: return dqx_lds_p<DqxQ8_0>(K, t);
        case SPQ4K_TYPE_Q6_K: return dqx_lds_p<DqxQ6K>(K, t);
        case SPQ4K_TYPE_Q5_K: return dqx_lds_p<DqxQ5K>(K, t);
        case SPQ4K_TYPE_Q4_K: return dqx_lds_p<DqxQ4K>(K, t);
        default: return SIZE_MAX;
    }
}

hipError_t launch_dqx_matvec(int type, const uint8_t* W, int M, int64_t K, const float* X, int64_t x_tstride,
                             float* Y, int64_t y_tstride, int T, int num_cus, hipStream_t st) {
    const int unit = dqx_unit(type);
    if (!unit || M <= 0 || K <= 0 || K % unit || K > INT32_MAX || T < 1 || T > DQ_MATVEC_MAX_T ||
        dqx_lds_bytes(type, K, T) > DQ_MATVEC_LDS_MAX)
        return hipErrorInvalidValue;
    switch (type) {
        case SPQ4K_TYPE_Q8_0: return dqx_matvec_p<DqxQ8_0>(W, M, (int)K, X, x_tstride, Y, y_tstride, T, num_cus, st);
        case SPQ4K_TYPE_Q6_K: return dqx_matvec_p<DqxQ6K>(W, M, (int)K, X, x_tstride, Y, y_tstride, T, num_cus, st);
        case SPQ4K_TYPE_Q5_K: return dqx_matvec_p<DqxQ5K>(W, M, (int)K, X, x_tstride, Y, y_tstride, T, num_cus, st);
        default: return dqx_matvec_p<DqxQ4K>(W, M, (int)K, X, x_tstride, Y, y_tstride, T, num_cus, st);
    }
}

hipError_t launch_dqx_experts(int type, int mode, const uint8_t* bank, const uint8_t* bank1, int E, int rows,
                              int64_t K, const int32_t* ids, int top_k, const float* hidden, float* H, int num_cus,
                              hipStream_t st) {
    const int unit = dqx_unit(type);
    if (!unit || mode < 0 || mode > 2 || (mode == 2 && !bank1) || E < 1 || rows <= 0 || K <= 0 || K % unit ||
        K > INT32_MAX || top_k < 1 || top_k > BEAST_MAX_TOPK || (int64_t)top_k * rows > INT32_MAX ||
        dqx_lds_bytes(type, K, 1) > DQ_MATVEC_LDS_MAX)
        return hipErrorInvalidValue;
    switch (type) {
        case SPQ4K_TYPE_Q8_0:
            return dqx_experts_p<DqxQ8_0>(mode, bank, bank1, E, rows, (int)K, ids, top_k, hidden, H, num_cus, st);
        case SPQ4K_TYPE_Q6_K:
            return dqx_experts_p<DqxQ6K>(mode, bank, bank1, E, rows, (int)K, ids, top_k, hidden, H, num_cus, st);
        case SPQ4K_TYPE_Q5_K:
            return dqx_experts_p<DqxQ5K>(mode, bank, bank1, E, rows, (int)K, ids, top_k, hidden, H, num_cus, st);
        default:
            return dqx_experts_p<DqxQ4K>(mode, bank, bank1, E, rows, (int)K, ids, top_k, hidden, H, num_cus, st);
    }
}

hipError_t launch_dqx_down(int type, const uint8_t* down, int E, int n_embd, int64_t n_ff, const int32_t* ids,
                           const float* scores, int top_k, const float* H, float* out, int num_cus, hipStream_t st) {
    const int unit = dqx_unit(type);
    if (!unit || E < 1 || n_embd <= 0 || n_ff <= 0 || n_ff % unit || n_ff > INT32_MAX || top_k < 1 ||
        top_k > BEAST_MAX_TOPK || dqx_lds_bytes(type, n_ff, 1) > DQ_MATVEC_LDS_MAX)
        return hipErrorInvalidValue;
    switch (type) {
        case SPQ4K_TYPE_Q8_0:
            return dqx_down_p<DqxQ8_0>(down, E, n_embd, (int)n_ff, ids, scores, top_k, H, out, num_cus, st);
        case SPQ4K_TYPE_Q6_K:
            return dqx_down_p<DqxQ6K>(down, E, n_embd, (int)n_ff, ids, scores, top_k, H, out, num_cus, st);
        case SPQ4K_TYPE_Q5_K:
            return dqx_down_p<DqxQ5K>(down, E, n_embd, (int)n_ff, ids, scores, top_k, H, out, num_cus, st);
        default: return dqx_down_p<DqxQ4K>(down, E, n_embd, (int)n_ff, ids, scores, top_k, H, out, num_cus, st);
    }
}

}  // namespace spq4k
