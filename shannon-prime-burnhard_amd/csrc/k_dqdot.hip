// k_dqdot.hip — Q4_K dequant-then-dot with fp32 activations on gfx950: the
// arithmetic of the reference's scalar BurnHard matvec, beast_matvec
// (desktop/beast_canyon/sp_beast_canyon.c:1122-1134):
//     for each row r: w = dequantize_row_q4_K(W[r]);  y[r] = sum_j w[j] * x[j]
// with x used as given (no Q8_K quantisation). The dequantised weights are
// ggml's bit for bit (d * sc -> * q -> - dmin * m, each rounded, as
// dequantize_row_q4_K, ggml-quants.c:1467-1489); every product w * x is
// rounded to fp32 and added in fp32 -- the reference adds them serially in
// index order, this kernel per lane and then across the wave in a fixed
// order, so the sums agree to fp32 reassociation (well inside 1e-4).
//
// Mapping: one wave per row at a time, lane (bsub, l4) = (lane >> 2, lane & 3)
// takes quarter l4 of blocks bsub, bsub + 16, ... (the 32 qs bytes of group
// g = l4: sub-blocks 2 l4 and 2 l4 + 1), three 16-byte loads a block. Each
// wave keeps the next row's loads in flight while it computes the current
// one. x is staged in LDS lane-major -- for pass it (blocks 16 it .. 16 it +
// 15), float4 i4 of lane L sits at ((it * 16 + i4) * 64 + L) -- so the 64
// lanes read 64 consecutive float4 per instruction (no bank conflicts).
#include "gemv_core.h"
#include "launch.h"

namespace spq4k {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) f32x4 lf32x4;

struct DqRow {
    uint4 h, qa, qb;
};

__device__ __forceinline__ DqRow dq_load(const uint8_t* __restrict__ row, int nb, int bsub, int l4, int it) {
    DqRow w;
    int b = bsub + 16 * it;
    b = b < nb ? b : nb - 1;   // lanes past the row's end load a valid block, their products are dropped
    const uint8_t* blk = row + (size_t)b * Q4K_BYTES;
    w.h = *reinterpret_cast<const uint4*>(blk);
    w.qa = *reinterpret_cast<const uint4*>(blk + 16 + 32 * l4);
    w.qb = *reinterpret_cast<const uint4*>(blk + 32 + 32 * l4);
    return w;
}

__device__ __forceinline__ uint32_t qw_hi(uint32_t v) { return v >> 4; }

// acc[t] += this lane's 64 products of its block (lane l4 of the block's four:
// values 64 l4 .. 64 l4 + 63) for each token; xf(t, j) is float4 j of those
// 64 values of token t
template <int T, class XF>
__device__ __forceinline__ void dq_block_x(const DqRow& w, int l4, XF xf, float (&acc)[T]) {
    const float d = half_bits_to_float(w.h.x & 0xFFFFu);
    const float dmin = half_bits_to_float(w.h.x >> 16);
    const ScaleMin sm = unpack_scale_min(w.h.y, w.h.z, w.h.w);
    const uint32_t scw = l4 < 2 ? sm.sc_lo : sm.sc_hi;
    const uint32_t mw = l4 < 2 ? sm.m_lo : sm.m_hi;
    const int sh = 16 * (l4 & 1);
    const float d1 = d * (float)((scw >> sh) & 0xFFu);
    const float m1 = dmin * (float)((mw >> sh) & 0xFFu);
    const float d2 = d * (float)((scw >> (sh + 8)) & 0xFFu);
    const float m2 = dmin * (float)((mw >> (sh + 8)) & 0xFFu);
    const uint32_t q[8] = {w.qa.x, w.qa.y, w.qa.z, w.qa.w, w.qb.x, w.qb.y, w.qb.z, w.qb.w};
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const float dd = half ? d2 : d1, mm = half ? m2 : m1;
#pragma unroll
        for (int i4 = 0; i4 < 8; ++i4) {
            // the four nibbles of this half as bytes (one byte convert each);
            // w = dd q - mm in one rounding: dd q is exact in fp32 (an fp16
            // times a 6-bit scale times a 4-bit q, at most 21 significant
            // bits), so the fused form equals the multiply-then-subtract
            uint32_t qn = (half ? qw_hi(q[i4]) : q[i4]) & 0x0F0F0F0Fu;
            asm volatile("" : "+v"(qn));   // keep the masked word: byte converts, not a field extract each
            float wv[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) wv[k] = __builtin_fmaf(dd, (float)((qn >> (8 * k)) & 0xFFu), -mm);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const f32x4 x = xf(t, 8 * half + i4);
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

// the block (bsub + 16 it) against x staged lane-major in LDS
template <int T>
__device__ __forceinline__ void dq_block(const DqRow& w, int l4, const lf32x4* xl, int npass, int it, int lane,
                                         float (&acc)[T]) {
    dq_block_x<T>(w, l4, [&](int t, int j) { return xl[(((size_t)t * npass + it) * 16 + j) * 64 + lane]; }, acc);
}

template <int T>
__global__ __launch_bounds__(256) void dequant_matvec_kernel(const uint8_t* __restrict__ W, int M, int nb,
                                                             const float* __restrict__ X, int64_t x_tstride,
                                                             float* __restrict__ Y, int64_t y_tstride,
                                                             int rows_per_wg) {
    extern __shared__ __align__(16) f32x4 dq_x[];
    const int npass = (nb + 15) >> 4;
    // stage x: token t, float4 e4 of the row (value 4 e4): block b = e4 >> 6,
    // group g = (e4 >> 4) & 3, float4 i4 = e4 & 15 -> pass b >> 4, lane 4 (b & 15) + g
    for (int t = 0; t < T; ++t) {
        const f32x4* xr = reinterpret_cast<const f32x4*>(X + (int64_t)t * x_tstride);
        for (int e4 = threadIdx.x; e4 < nb * 64; e4 += 256) {
            const int b = e4 >> 6, g = (e4 >> 4) & 3, i4 = e4 & 15;
            dq_x[(((size_t)t * npass + (b >> 4)) * 16 + i4) * 64 + 4 * (b & 15) + g] = xr[e4];
        }
    }
    __syncthreads();
    const lf32x4* xl = (const lf32x4*)dq_x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int l4 = lane & 3, bsub = lane >> 2;
    const int r0 = blockIdx.x * rows_per_wg;
    const int r1 = r0 + rows_per_wg < M ? r0 + rows_per_wg : M;
    int r = r0 + wave;
    if (r >= r1) return;
    const size_t row_bytes = (size_t)nb * Q4K_BYTES;
    DqRow cur = dq_load(W + (size_t)r * row_bytes, nb, bsub, l4, 0);
    while (r < r1) {
        float acc[T];
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = 0.0f;
        for (int it = 0; it < npass; ++it) {
            // the next piece: this row's next pass, else the first pass of the
            // wave's next row (clamped to a valid row so the load is in bounds)
            const int nit = it + 1 < npass ? it + 1 : 0;
            int nr = it + 1 < npass ? r : r + 4;
            nr = nr < r1 ? nr : r;
            const DqRow nxt = dq_load(W + (size_t)nr * row_bytes, nb, bsub, l4, nit);
            if (bsub + 16 * it < nb) dq_block<T>(cur, l4, xl, npass, it, lane, acc);
            cur = nxt;
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float s = group_sum_last<64>(acc[t]);
            if (lane == 63) Y[(int64_t)t * y_tstride + r] = s;
        }
        r += 4;
    }
}

// Rows of at most 16 blocks (K, n_embd or n_ff up to 4096): LPR lanes a
// weight row (4 a block, rounded up to a power of two), 64 / LPR rows side by
// side in a wave. The activations are staged in LDS, float4 j of lane ll of a row at
// j * LPR + ll (a row's lanes read consecutive 16-byte words, the rows of a
// wave the same ones), with their loads issued ahead of the weights' and each
// wave's weight loads all in flight before its first product. Products and
// sums per lane are dq_block's.

// x of nb blocks into the staging layout, from values a thread loaded:
// float4 e4 of x (value 4 e4) is float4 (e4 & 15) of lane 4 (e4 >> 6) + ((e4 >> 4) & 3)
template <int LPR>
__device__ __forceinline__ void dq_stage_put(f32x4* xs, int e4, const f32x4& v) {
    xs[(e4 & 15) * LPR + 4 * (e4 >> 6) + ((e4 >> 4) & 3)] = v;
}

// N rows' products at once, each against its own staged x (xl[n]), their
// sums interleaved so that a lone wave on its SIMD has N independent chains;
// each row's products and sum are dq_block's. Returns each row's sum in the
// last lane of its group.
template <int LPR, int N>
__device__ __forceinline__ void dq_dots_lds(const DqRow (&w)[N], int l4, int bsub, int nb, const lf32x4* const (&xl)[N],
                                            int ll, float (&out)[N]) {
    float acc[N];
#pragma unroll
    for (int n = 0; n < N; ++n) acc[n] = 0.0f;
    if (bsub < nb) {
        float dd[N][2], mm[N][2];
#pragma unroll
        for (int n = 0; n < N; ++n) {
            const float d = half_bits_to_float(w[n].h.x & 0xFFFFu);
            const float dmin = half_bits_to_float(w[n].h.x >> 16);
            const ScaleMin sm = unpack_scale_min(w[n].h.y, w[n].h.z, w[n].h.w);
            const uint32_t scw = l4 < 2 ? sm.sc_lo : sm.sc_hi;
            const uint32_t mw = l4 < 2 ? sm.m_lo : sm.m_hi;
            const int sh = 16 * (l4 & 1);
            dd[n][0] = d * (float)((scw >> sh) & 0xFFu);
            mm[n][0] = dmin * (float)((mw >> sh) & 0xFFu);
            dd[n][1] = d * (float)((scw >> (sh + 8)) & 0xFFu);
            mm[n][1] = dmin * (float)((mw >> (sh + 8)) & 0xFFu);
        }
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
            for (int i4 = 0; i4 < 8; ++i4) {
#pragma unroll
                for (int n = 0; n < N; ++n) {
                    const uint32_t qw = i4 < 4 ? (&w[n].qa.x)[i4] : (&w[n].qb.x)[i4 - 4];
                    uint32_t qn = (half ? qw_hi(qw) : qw) & 0x0F0F0F0Fu;
                    asm volatile("" : "+v"(qn));
                    const f32x4 x = xl[n][(8 * half + i4) * LPR + ll];
                    float wv[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        wv[k] = __builtin_fmaf(dd[n][half], (float)((qn >> (8 * k)) & 0xFFu), -mm[n][half]);
                    float a = acc[n];
                    a = a + wv[0] * x.x;
                    a = a + wv[1] * x.y;
                    a = a + wv[2] * x.z;
                    a = a + wv[3] * x.w;
                    acc[n] = a;
                }
            }
        }
    }
#pragma unroll
    for (int n = 0; n < N; ++n) out[n] = group_sum_last<LPR>(acc[n]);
}

// One token, rows of at most 16 blocks (K <= 4096): LPR = 4 nb rounded up to
// a power of two lanes a row, 64 / LPR rows side by side in a wave, R steps a
// wave; x staged once a workgroup (float4 j of lane ll at j * LPR + ll), every
// weight load of a wave issued before its first product and the R rows' sums
// interleaved. The lane arithmetic and the reduction are
// dequant_matvec_kernel's, so the outputs are the same bit for bit.
template <int LPR, int R>
__global__ __launch_bounds__(256) void dequant_matvec_short_kernel(const uint8_t* __restrict__ W, int M, int nb,
                                                                   const float* __restrict__ X,
                                                                   float* __restrict__ Y) {
    constexpr int RW = 64 / LPR;
    __shared__ f32x4 xs[16 * LPR];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane / LPR, ll = lane % LPR;
    const int l4 = ll & 3, bsub = ll >> 2;
    const int row0 = (blockIdx.x * 4 + wave) * RW * R + grp;   // this lane group's first row; then + RW each step
    const size_t row_bytes = (size_t)nb * Q4K_BYTES;
    // x loads first (unconditional: past the row's end they read its last float4)
    const f32x4* x4 = reinterpret_cast<const f32x4*>(X);
    f32x4 xr[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int e4 = threadIdx.x + 256 * k;
        xr[k] = x4[e4 < nb * 64 ? e4 : nb * 64 - 1];
    }
    DqRow w[R];
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const int r = row0 + u * RW;
        w[u] = dq_load(W + (size_t)(r < M ? r : M - 1) * row_bytes, nb, bsub, l4, 0);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int e4 = threadIdx.x + 256 * k;
        if (e4 < nb * 64) dq_stage_put<LPR>(xs, e4, xr[k]);
    }
    __syncthreads();
    const lf32x4* xl[R];
#pragma unroll
    for (int u = 0; u < R; ++u) xl[u] = (const lf32x4*)xs;
    float d[R];
    dq_dots_lds<LPR, R>(w, l4, bsub, nb, xl, ll, d);
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const int r = row0 + u * RW;
        if (ll == LPR - 1 && r < M) Y[r] = d[u];
    }
}

template <int LPR, int R>
hipError_t launch_dq_short(const uint8_t* W, int M, int nb, const float* X, float* Y, hipStream_t st) {
    constexpr int per_wg = 4 * (64 / LPR) * R;
    hipLaunchKernelGGL((dequant_matvec_short_kernel<LPR, R>), dim3((unsigned)((M + per_wg - 1) / per_wg)), dim3(256), 0,
                       st, W, M, nb, X, Y);
    return hipGetLastError();
}

// R (rows a lane group takes) in {1, 2, 4}: the largest that still leaves at
// least two workgroups a CU (the launch is a latency chain: a lone wave on its
// SIMD waits out its loads however many rows it interleaves; measured on
// 4096 x 4096: 5.9 us with R = 1 or 2, 7.5 us with R = 4)
template <int LPR>
hipError_t launch_dq_short_r(const uint8_t* W, int M, int nb, const float* X, float* Y, int num_cus,
                             hipStream_t st) {
    int best = 1;
    for (int r = 2; r <= 4; r *= 2) {
        const int64_t per = 4LL * (64 / LPR) * r;
        if ((M + per - 1) / per >= 2LL * num_cus) best = r;
    }
    if (best == 4) return launch_dq_short<LPR, 4>(W, M, nb, X, Y, st);
    if (best == 2) return launch_dq_short<LPR, 2>(W, M, nb, X, Y, st);
    return launch_dq_short<LPR, 1>(W, M, nb, X, Y, st);
}

template <int T>
hipError_t launch_dq_t(const uint8_t* W, int M, int nb, const float* X, int64_t x_tstride, float* Y,
                       int64_t y_tstride, int grid, int rows_per_wg, size_t lds, hipStream_t st) {
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)dequant_matvec_kernel<T>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(dequant_matvec_kernel<T>, dim3((unsigned)grid), dim3(256), lds, st, W, M, nb, X, x_tstride, Y,
                       y_tstride, rows_per_wg);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The BurnHard MoE forward for one token (sp_beast_moe_forward,
// desktop/beast_canyon/sp_beast_canyon.c:455-562): routing, then per selected
// expert gate / up / down matvecs of beast_matvec's arithmetic and the
// score-weighted sum.

// x (one row of nb blocks) into the lane-major staging of dequant_matvec_kernel,
// eight loads a thread in flight at a time (unconditional: past the row's end
// they read its last float4, which is not stored)
__device__ __forceinline__ void dq_stage_row(const float* __restrict__ x, int nb, f32x4* dq_x) {
    const f32x4* xr = reinterpret_cast<const f32x4*>(x);
    const int n4 = nb * 64;
    for (int base = threadIdx.x; base < n4; base += 8 * blockDim.x) {
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
                const int b = e4 >> 6, g = (e4 >> 4) & 3, i4 = e4 & 15;
                dq_x[((size_t)(b >> 4) * 16 + i4) * 64 + 4 * (b & 15) + g] = v[u];
            }
        }
    }
}

// A candidate (score, index) as one 64-bit key that orders as the selection
// does: a score is >= +0 (an exp over a positive sum), whose bits order as
// its value, in the high word; 0xFFFFFFFF - index in the low word, so that of
// equal scores the lower index is the larger key. Key 0 is no candidate (an
// entry taken, past E, or a NaN score, which the reference's strictly-greater
// scan never picks).
__device__ __forceinline__ uint64_t route_key(float sc, int i) {
    return sc >= 0.0f ? ((uint64_t)__float_as_uint(sc) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i) : 0ull;
}

template <int CTRL, int ROWS>
__device__ __forceinline__ uint64_t route_max_dpp(uint64_t k) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)k, CTRL, ROWS, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(k >> 32), CTRL, ROWS, 0xF, false);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    return o > k ? o : k;
}

// sp_beast_route_experts (:385-443) in one wave: the largest logit (NaNs
// skipped, -1e30 when none), exp_i = expf(l_i - max), their fp32 sum in index
// order, score_i = exp_i / sum; top_k rounds, each taking the unselected
// expert of the largest score (the lowest index among equal ones, as the
// reference's strictly-greater scan); the chosen scores renormalised by
// 1 / (their fp32 sum in rank order) when that sum is positive.
__global__ __launch_bounds__(64) void beast_route_kernel(const float* __restrict__ logits, int E, int top_k,
                                                         int32_t* __restrict__ ids, float* __restrict__ scores) {
    // E exps for lane 0's sum in index order, then (E > 256) the keys of
    // entries 256 and on, lane + 64 (j - 4) for entry lane + 64 j
    extern __shared__ __align__(16) float rt_score[];
    const int lane = threadIdx.x;
    const int per = (E + 63) >> 6;                 // entries a lane: i = lane + 64 j
    // the logits into LDS, eight loads a lane in flight at a time (indices
    // past E read the last logit and are not kept)
    float m = -1e30f;
    for (int j0 = 0; j0 < per; j0 += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = lane + 64 * (j0 + u);
            v[u] = logits[i < E ? i : E - 1];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = lane + 64 * (j0 + u);
            if (i < E) {
                rt_score[i] = v[u];
                if (v[u] > m) m = v[u];
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        if (o > m) m = o;
    }
    for (int j = 0; j < per; ++j) {
        const int i = lane + 64 * j;
        if (i < E) rt_score[i] = expf(rt_score[i] - m);
    }
    __syncthreads();
    float sum = 0.0f;
    if (lane == 0) {
        // serial in index order, four values a read
        int i = 0;
        for (; i + 4 <= E; i += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(rt_score + i);
            sum += v.x;
            sum += v.y;
            sum += v.z;
            sum += v.w;
        }
        for (; i < E; ++i) sum += rt_score[i];
    }
    sum = __shfl(sum, 0, 64);
    // each lane's candidates, score_i = exp_i / sum: the first four keys in
    // registers, the rest in LDS (each read back only by the lane that wrote it)
    uint64_t key[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = lane + 64 * j;
        key[j] = i < E ? route_key(rt_score[i] / sum, i) : 0ull;
    }
    uint64_t* const lkey = reinterpret_cast<uint64_t*>(rt_score + ((E + 3) & ~3));
    for (int j = 4; j < per; ++j) {
        const int i = lane + 64 * j;
        lkey[lane + 64 * (j - 4)] = i < E ? route_key(rt_score[i] / sum, i) : 0ull;
    }
    float chosen = 0.0f, ssum = 0.0f;
    int mine = -1;
    for (int k = 0; k < top_k; ++k) {
        uint64_t b = key[0] > key[1] ? key[0] : key[1];
        const uint64_t b2 = key[2] > key[3] ? key[2] : key[3];
        b = b2 > b ? b2 : b;
        for (int j = 4; j < per; ++j) {
            const uint64_t kk = lkey[lane + 64 * (j - 4)];
            b = kk > b ? kk : b;
        }
        // the wave's largest key: within rows of 16 lanes, then lane 15 of
        // each row into the next, lane 31 into rows 2 and 3: lane 63 ends
        // with it
        b = route_max_dpp<DPP_XOR1, 0xF>(b);
        b = route_max_dpp<DPP_XOR2, 0xF>(b);
        b = route_max_dpp<0x141, 0xF>(b);          // row_half_mirror
        b = route_max_dpp<0x140, 0xF>(b);          // row_mirror
        b = route_max_dpp<DPP_BCAST15, 0xA>(b);
        b = route_max_dpp<DPP_BCAST31, 0xC>(b);
        const uint32_t wlo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, 63);
        const uint32_t whi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), 63);
        const uint64_t wk = ((uint64_t)whi << 32) | wlo;
        const int wi = wk ? (int)(0xFFFFFFFFu - wlo) : -1;
        const float wv = wk ? __uint_as_float(whi) : -1e30f;
        // the chosen entry leaves its lane's candidates (keys are unique)
#pragma unroll
        for (int j = 0; j < 4; ++j) key[j] = key[j] == wk ? 0ull : key[j];
        if (wi >= 0 && (wi & 63) == lane && (wi >> 6) >= 4) lkey[lane + 64 * ((wi >> 6) - 4)] = 0ull;
        if (lane == k) {
            chosen = wv;
            mine = wi;
        }
        ssum += wv;                                // rank order, the same on every lane
    }
    if (lane < top_k) {
        const float inv = ssum > 0.0f ? 1.0f / ssum : 1.0f;
        ids[lane] = mine;
        scores[lane] = ssum > 0.0f ? chosen * inv : chosen;
    }
}

// Rows of more than 16 blocks: every pass of a row's loads issued at once (NP
// passes, the row's count rounded up to 2, 4 or 8; a pass past the row's end
// loads its last block and its products are dropped), then its passes'
// products as dq_block's and the fixed wave reduction.
template <int NP>
__device__ __forceinline__ void dq_load_passes(const uint8_t* __restrict__ row, int nb, int bsub, int l4,
                                               DqRow (&w)[NP]) {
#pragma unroll
    for (int it = 0; it < NP; ++it) w[it] = dq_load(row, nb, bsub, l4, it);
}

template <int NP>
__device__ __forceinline__ float dq_dot_passes(const DqRow (&w)[NP], int nb, const lf32x4* xl, int lane) {
    const int l4 = lane & 3, bsub = lane >> 2;
    float acc[1] = {0.0f};
#pragma unroll
    for (int it = 0; it < NP; ++it)
        if (bsub + 16 * it < nb) dq_block<1>(w[it], l4, xl, 1, it, lane, acc);
    return __shfl(group_sum_last<64>(acc[0]), 63, 64);
}

// gate and up rows of every selected expert against the hidden state, and
// silu(gate) * up (beast_silu_mul, :1168-1173): H[s][r], s < top_k, r < n_ff;
// a wave per sweep row (s, r) at a time, its gate and up rows' loads issued
// together; rows_per_wg consecutive sweep rows a workgroup of 4 waves.
template <int NP>
__global__ __launch_bounds__(256) void beast_gate_up_kernel(const uint8_t* __restrict__ gate,
                                                            const uint8_t* __restrict__ up, size_t expert_bytes,
                                                            int n_ff, int nb, const int32_t* __restrict__ ids,
                                                            int E, int top_k, const float* __restrict__ hidden,
                                                            float* __restrict__ H, int rows_per_wg) {
    extern __shared__ __align__(16) f32x4 dq_x[];
    dq_stage_row(hidden, nb, dq_x);
    __syncthreads();
    const lf32x4* xl = (const lf32x4*)dq_x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int l4 = lane & 3, bsub = lane >> 2;
    const int total = top_k * n_ff;
    const int q0 = blockIdx.x * rows_per_wg;
    const int q1 = q0 + rows_per_wg < total ? q0 + rows_per_wg : total;
    const size_t row_bytes = (size_t)nb * Q4K_BYTES;
    for (int q = q0 + wave; q < q1; q += 4) {
        const int s = q / n_ff, r = q - s * n_ff;
        const int e = ids[s];
        const bool live = e >= 0 && e < E;    // no expert (a routing with no candidate): nothing
        const size_t off = (size_t)(live ? e : 0) * expert_bytes + (size_t)r * row_bytes;
        DqRow wg[NP], wu[NP];
        dq_load_passes<NP>(gate + off, nb, bsub, l4, wg);
        dq_load_passes<NP>(up + off, nb, bsub, l4, wu);
        const float g = dq_dot_passes<NP>(wg, nb, xl, lane);
        const float u = dq_dot_passes<NP>(wu, nb, xl, lane);
        if (lane == 0) H[q] = live ? (g / (1.0f + expf(-g))) * u : 0.0f;
    }
}

// down rows of every selected expert against that expert's H row, summed in
// rank order as output += score * down (:541-543, fused multiply-add as the
// reference's GCC build contracts it): out[i], rows_per_wg consecutive rows
// a workgroup of 4 waves, at most BEAST_DOWN_RPW a wave, each row's loads
// issued while the previous row is computed; the H rows are staged one expert
// at a time.
template <int NP>
__global__ __launch_bounds__(256) void beast_down_sum_kernel(const uint8_t* __restrict__ down, size_t expert_bytes,
                                                             int n_embd, int nb, const int32_t* __restrict__ ids,
                                                             int E, const float* __restrict__ scores, int top_k,
                                                             const float* __restrict__ H, int n_ff,
                                                             float* __restrict__ out, int rows_per_wg) {
    extern __shared__ __align__(16) f32x4 dq_x[];
    const lf32x4* xl = (const lf32x4*)dq_x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int l4 = lane & 3, bsub = lane >> 2;
    const int r0 = blockIdx.x * rows_per_wg;
    const int r1 = r0 + rows_per_wg < n_embd ? r0 + rows_per_wg : n_embd;
    const size_t row_bytes = (size_t)nb * Q4K_BYTES;
    static_assert(BEAST_DOWN_RPW % 2 == 0, "rows are taken in pairs");
    float acc[BEAST_DOWN_RPW];
#pragma unroll
    for (int j = 0; j < BEAST_DOWN_RPW; ++j) acc[j] = 0.0f;
    // the wave's rows: nrow of them (uniform over the wave; the second of a
    // pair past r1 reads row r1 - 1 and is dropped)
    const int nrow = r0 + wave < r1 ? (r1 - r0 - wave + 3) / 4 : 0;
    auto row_of = [&](int j) {
        const int i = r0 + wave + 4 * j;
        return i < r1 ? i : r1 - 1;
    };
    for (int s = 0; s < top_k; ++s) {
        const int e = ids[s];
        if (e < 0 || e >= E) continue;         // uniform over the workgroup
        const uint8_t* base = down + (size_t)e * expert_bytes;
        DqRow wa[NP], wb[NP];
        if (nrow > 0) dq_load_passes<NP>(base + (size_t)row_of(0) * row_bytes, nb, bsub, l4, wa);
        __syncthreads();                       // the previous expert's readers are done
        dq_stage_row(H + (size_t)s * n_ff, nb, dq_x);
        __syncthreads();
        const float sc = scores[s];
#pragma unroll
        for (int j = 0; j < BEAST_DOWN_RPW; j += 2) {
            if (j >= nrow) break;              // uniform over the wave
            if (j + 1 < nrow) dq_load_passes<NP>(base + (size_t)row_of(j + 1) * row_bytes, nb, bsub, l4, wb);
            const float da = dq_dot_passes<NP>(wa, nb, xl, lane);
            acc[j] = fmaf(sc, da, acc[j]);
            if (j + 2 < nrow) dq_load_passes<NP>(base + (size_t)row_of(j + 2) * row_bytes, nb, bsub, l4, wa);
            if (j + 1 < nrow) {
                const float db = dq_dot_passes<NP>(wb, nb, xl, lane);
                acc[j + 1] = fmaf(sc, db, acc[j + 1]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < BEAST_DOWN_RPW; ++j) {
        const int i = r0 + wave + 4 * j;
        if (i < r1 && lane == 0) out[i] = acc[j];
    }
}

// The routing of sp_beast_route_experts (:385-443) by a workgroup of 256
// threads, entries i = t + 256 m to thread t: the largest logit (NaNs skipped,
// -1e30 when none), exp_i = expf(l_i - max) and their fp32 sum in index order
// (one thread), score_i = exp_i / sum; then, in place of top_k rounds of
// "the unselected expert of the largest score, the lowest index among equal
// ones", each candidate's rank among all of them by its key (route_key: the
// same order), rank < top_k taking slot rank; slots left (fewer candidates
// than top_k) hold expert -1 and score -1e30, as a round that finds none.
// Every thread returns with sel_id / sel_v (the chosen scores before the
// renormalisation) in LDS; the renormalised scores go to sel_sc.
struct RouteLds {
    uint64_t* key;     // E keys
    float* ex;         // E logits, then exps
    int* sel_id;       // BEAST_MAX_TOPK
    float* sel_v;      // BEAST_MAX_TOPK
    float* sel_sc;     // BEAST_MAX_TOPK
    float* red;        // 8: the waves' maxima, the sum
};

template <int CTRL, int ROWS>
__device__ __forceinline__ float route_fmax_dpp(float v) {
    const float o = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-1e30f), __float_as_int(v), CTRL, ROWS,
                                                               0xF, false));
    return o > v ? o : v;
}

// lg0: logits[min(t, E - 1)], loaded by the caller ahead of its other loads
__device__ __forceinline__ void beast_route_wg(const float* __restrict__ logits, float lg0, int E, int top_k,
                                               const RouteLds& L) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    float m = -1e30f;
    if (t < E) {
        L.ex[t] = lg0;
        if (lg0 > m) m = lg0;
    }
    for (int i = t + 256; i < E; i += 256) {
        const float v = logits[i];
        L.ex[i] = v;
        if (v > m) m = v;
    }
    if (t < BEAST_MAX_TOPK) {
        L.sel_id[t] = -1;
        L.sel_v[t] = -1e30f;
    }
    // the wave's largest (lane 63), then the workgroup's
    m = route_fmax_dpp<DPP_XOR1, 0xF>(m);
    m = route_fmax_dpp<DPP_XOR2, 0xF>(m);
    m = route_fmax_dpp<0x141, 0xF>(m);
    m = route_fmax_dpp<0x140, 0xF>(m);
    m = route_fmax_dpp<DPP_BCAST15, 0xA>(m);
    m = route_fmax_dpp<DPP_BCAST31, 0xC>(m);
    if (lane == 63) L.red[wave] = m;
    __syncthreads();
    m = L.red[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) m = L.red[w] > m ? L.red[w] : m;
    for (int i = t; i < E; i += 256) L.ex[i] = expf(L.ex[i] - m);
    __syncthreads();
    if (t == 0) {
        // serial in index order, 32 values read ahead of their adds
        float sum = 0.0f;
        int i = 0;
        for (; i + 32 <= E; i += 32) {
            f32x4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const f32x4*>(L.ex + i + 4 * u);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                sum += v[u].x;
                sum += v[u].y;
                sum += v[u].z;
                sum += v[u].w;
            }
        }
        for (; i < E; ++i) sum += L.ex[i];
        L.red[4] = sum;
    }
    __syncthreads();
    const float sum = L.red[4];
    for (int i = t; i < E; i += 256) L.key[i] = route_key(L.ex[i] / sum, i);
    __syncthreads();
    for (int i = t; i < E; i += 256) {
        const uint64_t ki = L.key[i];
        if (ki == 0) continue;                     // no candidate
        // 16 keys read ahead of their compares (every thread reads the same
        // words: broadcasts)
        int rank = 0;
        int j = 0;
        for (; j + 16 <= E; j += 16) {
            uint64_t kj[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) kj[u] = L.key[j + u];
#pragma unroll
            for (int u = 0; u < 16; ++u) rank += kj[u] > ki;
        }
        for (; j < E; ++j) rank += L.key[j] > ki;
        if (rank < top_k) {
            L.sel_id[rank] = i;
            L.sel_v[rank] = __uint_as_float((uint32_t)(ki >> 32));
        }
    }
    __syncthreads();
    if (t < top_k) {
        float ssum = 0.0f;                         // rank order
        for (int k = 0; k < top_k; ++k) ssum += L.sel_v[k];
        const float inv = ssum > 0.0f ? 1.0f / ssum : 1.0f;
        L.sel_sc[t] = ssum > 0.0f ? L.sel_v[t] * inv : L.sel_v[t];
    }
    __syncthreads();
}

// bytes of dynamic LDS the routing takes for E experts (16-byte aligned parts)
__host__ __device__ inline size_t beast_route_lds_bytes(int E) {
    const size_t e4 = (size_t)((E + 3) & ~3);
    return e4 * 8 + e4 * 4 + 3 * BEAST_MAX_TOPK * 4 + 8 * 4;
}

__device__ __forceinline__ RouteLds route_lds_at(unsigned char* base, int E) {
    const size_t e4 = (size_t)((E + 3) & ~3);
    RouteLds L;
    L.key = reinterpret_cast<uint64_t*>(base);
    L.ex = reinterpret_cast<float*>(base + e4 * 8);
    L.sel_id = reinterpret_cast<int*>(base + e4 * 12);
    L.sel_v = reinterpret_cast<float*>(base + e4 * 12 + BEAST_MAX_TOPK * 4);
    L.sel_sc = reinterpret_cast<float*>(base + e4 * 12 + 2 * BEAST_MAX_TOPK * 4);
    L.red = reinterpret_cast<float*>(base + e4 * 12 + 3 * BEAST_MAX_TOPK * 4);
    return L;
}

// The routing and gate / up in one launch (rows of at most 16 blocks): every
// workgroup routes the token itself (its x loads in flight meanwhile), so the
// experts come from LDS rather than from a previous launch; workgroup 0
// stores the ids and renormalised scores for the down launch. Sweep row
// q = (s, r) is the pair of half rows 2q (gate) and 2q + 1 (up); a workgroup
// takes 4 RW U consecutive half rows (RW = 64 / LPR), a wave RW U of them in
// U steps, every weight load in flight before the first product, and the
// gate half's last lane writes H[q] = silu(g) * u (beast_silu_mul,
// :1168-1173).
template <int LPR, int U>
__global__ __launch_bounds__(256) void beast_route_gate_up_kernel(const uint8_t* __restrict__ gate,
                                                                 const uint8_t* __restrict__ up, size_t expert_bytes,
                                                                 int n_ff, int nb, const float* __restrict__ logits,
                                                                 int E, int top_k, int32_t* __restrict__ ids,
                                                                 float* __restrict__ scores,
                                                                 const float* __restrict__ hidden,
                                                                 float* __restrict__ H) {
    constexpr int RW = 64 / LPR, HPW = 4 * RW * U;
    static_assert(RW * U % 2 == 0, "a wave takes whole gate / up pairs");
    static_assert(HPW <= 512, "a workgroup's sweep rows span at most two slots (n_ff >= 256)");
    extern __shared__ __align__(16) unsigned char rg_lds[];
    f32x4* xs = reinterpret_cast<f32x4*>(rg_lds);                     // 16 LPR float4
    const RouteLds L = route_lds_at(rg_lds + 16 * LPR * 16, E);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane / LPR, ll = lane % LPR;
    const int l4 = ll & 3, bsub = ll >> 2;
    const int total2 = 2 * top_k * n_ff;
    const int h0 = blockIdx.x * HPW;
    const size_t row_bytes = (size_t)nb * Q4K_BYTES;
    // the logits first (the routing waits on them), then x: it lands while
    // the routing runs
    const float lg0 = logits[(int)threadIdx.x < E ? (int)threadIdx.x : E - 1];
    const f32x4* x4 = reinterpret_cast<const f32x4*>(hidden);
    f32x4 xr[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int e4 = threadIdx.x + 256 * k;
        xr[k] = x4[e4 < nb * 64 ? e4 : nb * 64 - 1];
    }
    beast_route_wg(logits, lg0, E, top_k, L);
    if (blockIdx.x == 0 && (int)threadIdx.x < top_k) {
        ids[threadIdx.x] = L.sel_id[threadIdx.x];
        scores[threadIdx.x] = L.sel_sc[threadIdx.x];
    }
    DqRow w[U];
    bool live[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        int hr = h0 + (wave * U + u) * RW + grp;
        hr = hr < total2 ? hr : total2 - 1;
        const int q = hr >> 1, s = q / n_ff, r = q - s * n_ff;
        const int e = L.sel_id[s];
        live[u] = e >= 0 && e < E;
        const uint8_t* base = (hr & 1) ? up : gate;
        w[u] = dq_load(base + (size_t)(live[u] ? e : 0) * expert_bytes + (size_t)r * row_bytes, nb, bsub, l4, 0);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int e4 = threadIdx.x + 256 * k;
        if (e4 < nb * 64) dq_stage_put<LPR>(xs, e4, xr[k]);
    }
    __syncthreads();
    const lf32x4* xl[U];
#pragma unroll
    for (int u = 0; u < U; ++u) xl[u] = (const lf32x4*)xs;
    float d[U];
    dq_dots_lds<LPR, U>(w, l4, bsub, nb, xl, ll, d);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int hr = h0 + (wave * U + u) * RW + grp;
        float g, uv;
        bool mine;
        if (RW >= 2) {
            uv = __shfl(d[u], (lane + LPR) & 63, 64);
            g = d[u];
            mine = (grp & 1) == 0 && ll == LPR - 1;
        } else {
            if (u & 1) continue;
            uv = d[u + 1 < U ? u + 1 : u];
            g = d[u];
            mine = lane == 63;
        }
        if (mine && hr < total2) H[hr >> 1] = live[u] ? (g / (1.0f + expf(-g))) * uv : 0.0f;
    }
}

// down and the weighted sum: a workgroup takes 4 R consecutive output rows, a
// wave R of them, and sweeps the selected experts in rounds of GPW = 64 / LPR
// consecutive slots (group g takes slot GPW k + g in round k); two rounds'
// hidden rows are staged in LDS at a time and their weight loads issued
// together. After each round the row sums are folded in slot order,
// o = fmaf(score_s, d_s, o), the rank order of the reference's accumulation.
template <int LPR, int R>
__global__ __launch_bounds__(256) void beast_down_short_kernel(const uint8_t* __restrict__ down, size_t expert_bytes,
                                                              int n_embd, int nb, const int32_t* __restrict__ ids,
                                                              int E, const float* __restrict__ scores, int top_k,
                                                              const float* __restrict__ H, int n_ff,
                                                              float* __restrict__ out) {
    constexpr int GPW = 64 / LPR, CH = 2 * GPW;
    constexpr int SS = 16 * LPR + 4;          // a slot's staging stride in float4 (64 bytes of padding)
    __shared__ f32x4 hs[CH * SS];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane / LPR, ll = lane % LPR;
    const int l4 = ll & 3, bsub = ll >> 2;
    const int i0 = (blockIdx.x * 4 + wave) * R;
    const size_t row_bytes = (size_t)nb * Q4K_BYTES;
    const int nb64 = nb * 64;
    // slot s's expert and score in lane s (top_k <= 16)
    const int my_e = lane < top_k ? ids[lane] : -1;
    const float my_sc = lane < top_k ? scores[lane] : 0.0f;
    float o[R];
#pragma unroll
    for (int j = 0; j < R; ++j) o[j] = 0.0f;
    const int rounds = (top_k + GPW - 1) / GPW;
    for (int k = 0; k < rounds; k += 2) {
        const int s0 = GPW * k;
        const int nv = (top_k - s0 < CH ? top_k - s0 : CH) * nb64;   // float4 of the chunk's hidden rows
        // the chunk's hidden rows (CH nb 64 <= 2048 float4: at most 8 a thread)
        f32x4 hr[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int e4r = (int)threadIdx.x + 256 * m;
            const int e4 = e4r < nv ? e4r : nv - 1;   // unconditional
            const int sl = e4 / nb64;
            hr[m] = reinterpret_cast<const f32x4*>(H + (size_t)(s0 + sl) * n_ff)[e4 - sl * nb64];
        }
        DqRow w[2][R] = {};                    // a dead slot's rows: zero blocks, never folded
        bool live[2];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int s = GPW * (k + p) + grp;
            const int e = __shfl(my_e, s & 63, 64);
            live[p] = s < top_k && e >= 0 && e < E;
            if (live[p]) {
#pragma unroll
                for (int j = 0; j < R; ++j) {
                    const int i = i0 + j < n_embd ? i0 + j : n_embd - 1;
                    w[p][j] = dq_load(down + (size_t)e * expert_bytes + (size_t)i * row_bytes, nb, bsub, l4, 0);
                }
            }
        }
        if (k > 0) __syncthreads();            // the previous chunk's readers are done
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int e4 = threadIdx.x + 256 * m;
            if (e4 < nv) {
                const int sl = e4 / nb64;
                dq_stage_put<LPR>(hs + sl * SS, e4 - sl * nb64, hr[m]);
            }
        }
        __syncthreads();
        // both rounds' rows at once
        DqRow wf[2 * R];
        const lf32x4* xl[2 * R];
        float df[2 * R];
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int j = 0; j < R; ++j) {
                wf[p * R + j] = w[p][j];
                xl[p * R + j] = (const lf32x4*)(hs + (GPW * p + grp) * SS);
            }
        dq_dots_lds<LPR, 2 * R>(wf, l4, bsub, nb, xl, ll, df);
#pragma unroll
        for (int p = 0; p < 2; ++p) {
#pragma unroll
            for (int g = 0; g < GPW; ++g) {
                const int sg = GPW * (k + p) + g;
                if (sg >= top_k) break;
                const int eg = __builtin_amdgcn_readlane(my_e, sg);
                if (eg < 0 || eg >= E) continue;   // no expert: nothing
                const float sc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_sc), sg));
#pragma unroll
                for (int j = 0; j < R; ++j)
                    o[j] = fmaf(sc, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(df[p * R + j]),
                                                                             g * LPR + LPR - 1)),
                                o[j]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < R; ++j)
        if (lane == j && i0 + j < n_embd) out[i0 + j] = o[j];
}

// the half-row steps U a gate / up wave takes: 2 or 4, whichever leaves the
// busiest CU the fewer rows
inline int beast_gu_steps(int64_t total2, int rw, int num_cus) {
    int best = 2;
    int64_t best_load = -1;
    for (int u = 2; u <= 4; u += 2) {
        const int64_t hpw = 4LL * rw * u, wgs = (total2 + hpw - 1) / hpw;
        const int64_t load = (wgs + num_cus - 1) / num_cus * hpw;
        if (best_load < 0 || load <= best_load) {
            best = u;
            best_load = load;
        }
    }
    return best;
}

template <int LPR, int U>
hipError_t launch_route_gate_up(const uint8_t* gate, const uint8_t* up, size_t gu_bytes, int n_ff, int nb_e,
                                const float* logits, int E, int top_k, int32_t* ids, float* scores,
                                const float* hidden, float* H, hipStream_t st) {
    constexpr int HPW = 4 * (64 / LPR) * U;
    const int64_t total2 = 2 * (int64_t)top_k * n_ff;
    const size_t lds = (size_t)16 * LPR * 16 + beast_route_lds_bytes(E);
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute((const void*)beast_route_gate_up_kernel<LPR, U>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((beast_route_gate_up_kernel<LPR, U>), dim3((unsigned)((total2 + HPW - 1) / HPW)), dim3(256), lds,
                       st, gate, up, gu_bytes, n_ff, nb_e, logits, E, top_k, ids, scores, hidden, H);
    return hipGetLastError();
}

template <int LPR>
hipError_t launch_beast_short(const uint8_t* gate, const uint8_t* up, const uint8_t* down, size_t gu_bytes,
                              size_t dn_bytes, int n_embd, int n_ff, int nb_e, int nb_f, const float* logits, int E,
                              int top_k, int32_t* ids, float* scores, const float* hidden, float* H, float* out,
                              bool do_gate_up, int num_cus, hipStream_t st) {
    constexpr int RW = 64 / LPR;
    if (do_gate_up) {
        const int64_t total2 = 2 * (int64_t)top_k * n_ff;
        if (beast_gu_steps(total2, RW, num_cus) == 4)
            return launch_route_gate_up<LPR, 4>(gate, up, gu_bytes, n_ff, nb_e, logits, E, top_k, ids, scores, hidden,
                                                H, st);
        return launch_route_gate_up<LPR, 2>(gate, up, gu_bytes, n_ff, nb_e, logits, E, top_k, ids, scores, hidden, H,
                                            st);
    }
    // down: a row a wave while that leaves at most four workgroups a CU
    if ((int64_t)(n_embd + 3) / 4 > 4LL * num_cus) {
        hipLaunchKernelGGL((beast_down_short_kernel<LPR, 2>), dim3((unsigned)((n_embd + 7) / 8)), dim3(256), 0, st, down,
                           dn_bytes, n_embd, nb_f, ids, E, scores, top_k, H, n_ff, out);
    } else {
        hipLaunchKernelGGL((beast_down_short_kernel<LPR, 1>), dim3((unsigned)((n_embd + 3) / 4)), dim3(256), 0, st, down,
                           dn_bytes, n_embd, nb_f, ids, E, scores, top_k, H, n_ff, out);
    }
    return hipGetLastError();
}

// lanes a row for rows of nb blocks (nb <= 16): 4 nb rounded up to a power of two
hipError_t launch_beast_short_nb(int nb, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                                 size_t gu_bytes, size_t dn_bytes, int n_embd, int n_ff, int nb_e, int nb_f,
                                 const float* logits, int E, int top_k, int32_t* ids, float* scores,
                                 const float* hidden, float* H, float* out, bool do_gate_up, int num_cus,
                                 hipStream_t st) {
#define BEAST_SHORT(L)                                                                                             \
    launch_beast_short<L>(gate, up, down, gu_bytes, dn_bytes, n_embd, n_ff, nb_e, nb_f, logits, E, top_k, ids, scores, \
                          hidden, H, out, do_gate_up, num_cus, st)
    if (nb <= 1) return BEAST_SHORT(4);
    if (nb <= 2) return BEAST_SHORT(8);
    if (nb <= 4) return BEAST_SHORT(16);
    if (nb <= 8) return BEAST_SHORT(32);
    return BEAST_SHORT(64);
#undef BEAST_SHORT
}

}  // namespace

size_t dequant_matvec_lds_bytes(int T, int nb) { return (size_t)T * ((nb + 15) / 16) * 16 * 64 * 16; }

template <int NP>
hipError_t launch_beast_gate_up_np(const uint8_t* gate, const uint8_t* up, size_t gu_bytes, int n_ff, int nb,
                                   const int32_t* ids, int E, int top_k, const float* hidden, float* H, int rpw,
                                   int grid, size_t lds, hipStream_t st) {
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute((const void*)beast_gate_up_kernel<NP>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(beast_gate_up_kernel<NP>, dim3((unsigned)grid), dim3(256), lds, st, gate, up, gu_bytes, n_ff,
                       nb, ids, E, top_k, hidden, H, rpw);
    return hipGetLastError();
}

template <int NP>
hipError_t launch_beast_down_np(const uint8_t* down, size_t dn_bytes, int n_embd, int nb, const int32_t* ids, int E,
                                const float* scores, int top_k, const float* H, int n_ff, float* out, int drw,
                                int grid, size_t lds, hipStream_t st) {
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute((const void*)beast_down_sum_kernel<NP>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(beast_down_sum_kernel<NP>, dim3((unsigned)grid), dim3(256), lds, st, down, dn_bytes, n_embd,
                       nb, ids, E, scores, top_k, H, n_ff, out, drw);
    return hipGetLastError();
}

hipError_t launch_beast_route(const float* logits, int E, int top_k, int32_t* ids, float* scores, hipStream_t st) {
    if (E < 1 || E > BEAST_MAX_EXPERTS || top_k < 1 || top_k > BEAST_MAX_TOPK) return hipErrorInvalidValue;
    const size_t lds_rt = (size_t)((E + 3) & ~3) * sizeof(float) + (E > 256 ? (size_t)(E - 256 + 63) / 64 * 64 * 8 : 0);
    hipLaunchKernelGGL(beast_route_kernel, dim3(1), dim3(64), lds_rt, st, logits, E, top_k, ids, scores);
    return hipGetLastError();
}

hipError_t launch_beast_route_gate_up(const uint8_t* gate, const uint8_t* up, int E, int n_embd, int n_ff,
                                      const float* logits, int top_k, const float* hidden, int32_t* ids,
                                      float* scores, float* H, int num_cus, hipStream_t st) {
    if (E < 1 || E > BEAST_MAX_EXPERTS || top_k < 1 || top_k > BEAST_MAX_TOPK || n_embd % 256 || n_ff % 256)
        return hipErrorInvalidValue;
    const int nb_e = n_embd / 256;
    const size_t lds_e = dequant_matvec_lds_bytes(1, nb_e);
    if (lds_e > DQ_MATVEC_LDS_MAX) return hipErrorInvalidValue;
    const size_t gu_bytes = (size_t)n_ff * nb_e * Q4K_BYTES;
    const int64_t want = (int64_t)num_cus * 4;
    hipError_t e;
    if (nb_e <= 16) {
        // the routing inside the gate / up launch
        e = launch_beast_short_nb(nb_e, gate, up, nullptr, gu_bytes, 0, n_embd, n_ff, nb_e, 0, logits, E, top_k, ids,
                                  scores, hidden, H, nullptr, true, num_cus, st);
    } else {
        e = launch_beast_route(logits, E, top_k, ids, scores, st);
        if (e != hipSuccess) return e;
        // about four workgroups a CU over top_k * n_ff sweep rows
        const int64_t total = (int64_t)top_k * n_ff;
        int64_t rpw = (total + want - 1) / want;
        rpw = (rpw + 3) & ~(int64_t)3;
        const int np = (nb_e + 15) / 16;
        e = np <= 2 ? launch_beast_gate_up_np<2>(gate, up, gu_bytes, n_ff, nb_e, ids, E, top_k, hidden, H, (int)rpw,
                                                 (int)((total + rpw - 1) / rpw), lds_e, st)
            : np <= 4 ? launch_beast_gate_up_np<4>(gate, up, gu_bytes, n_ff, nb_e, ids, E, top_k, hidden, H, (int)rpw,
                                                   (int)((total + rpw - 1) / rpw), lds_e, st)
                      : launch_beast_gate_up_np<8>(gate, up, gu_bytes, n_ff, nb_e, ids, E, top_k, hidden, H, (int)rpw,
                                                   (int)((total + rpw - 1) / rpw), lds_e, st);
    }
    return e;
}

hipError_t launch_beast_down(const uint8_t* down, int E, int n_embd, int n_ff, const int32_t* ids,
                             const float* scores, int top_k, const float* H, float* out, int num_cus,
                             hipStream_t st) {
    if (E < 1 || E > BEAST_MAX_EXPERTS || top_k < 1 || top_k > BEAST_MAX_TOPK || n_embd % 256 || n_ff % 256)
        return hipErrorInvalidValue;
    const int nb_f = n_ff / 256;
    const size_t lds_f = dequant_matvec_lds_bytes(1, nb_f);
    if (lds_f > DQ_MATVEC_LDS_MAX) return hipErrorInvalidValue;
    const size_t dn_bytes = (size_t)n_embd * nb_f * Q4K_BYTES;
    // down and the weighted sum
    if (nb_f <= 16)
        return launch_beast_short_nb(nb_f, nullptr, nullptr, down, 0, dn_bytes, n_embd, n_ff, 0, nb_f, nullptr, E,
                                     top_k, const_cast<int32_t*>(ids), const_cast<float*>(scores), nullptr,
                                     const_cast<float*>(H), out, false, num_cus, st);
    // rows in runs of a multiple of 4, at most BEAST_DOWN_RPW a wave, about two
    // workgroups a CU: each workgroup stages every selected expert's whole
    // hidden row, so longer runs read less of it again (4096 x 14336, top-2:
    // 79.5 us a forward with two workgroups a CU, 88.1 with four, 88.4 with one)
    const int64_t want_d = 2 * (int64_t)num_cus;
    int64_t drw = ((int64_t)n_embd + want_d - 1) / want_d;
    drw = (drw + 3) & ~(int64_t)3;
    if (drw > 4 * BEAST_DOWN_RPW) drw = 4 * BEAST_DOWN_RPW;
    const int np = (nb_f + 15) / 16;
    const int grid = (int)((n_embd + drw - 1) / drw);
    if (np <= 2)
        return launch_beast_down_np<2>(down, dn_bytes, n_embd, nb_f, ids, E, scores, top_k, H, n_ff, out, (int)drw,
                                       grid, lds_f, st);
    if (np <= 4)
        return launch_beast_down_np<4>(down, dn_bytes, n_embd, nb_f, ids, E, scores, top_k, H, n_ff, out, (int)drw,
                                       grid, lds_f, st);
    return launch_beast_down_np<8>(down, dn_bytes, n_embd, nb_f, ids, E, scores, top_k, H, n_ff, out, (int)drw, grid,
                                   lds_f, st);
}

hipError_t launch_dequant_matvec(const uint8_t* W, int M, int nb, const float* X, int64_t x_tstride, float* Y,
                                 int64_t y_tstride, int T, int num_cus, hipStream_t st) {
    if (M <= 0 || nb <= 0 || T < 1 || T > DQ_MATVEC_MAX_T) return hipErrorInvalidValue;
    const size_t lds = dequant_matvec_lds_bytes(T, nb);
    if (lds > DQ_MATVEC_LDS_MAX) return hipErrorInvalidValue;
    if (T == 1 && nb <= 16) {
        if (nb <= 1) return launch_dq_short_r<4>(W, M, nb, X, Y, num_cus, st);
        if (nb <= 2) return launch_dq_short_r<8>(W, M, nb, X, Y, num_cus, st);
        if (nb <= 4) return launch_dq_short_r<16>(W, M, nb, X, Y, num_cus, st);
        if (nb <= 8) return launch_dq_short_r<32>(W, M, nb, X, Y, num_cus, st);
        return launch_dq_short_r<64>(W, M, nb, X, Y, num_cus, st);
    }
    // about four workgroups a CU, each a contiguous range of rows (a multiple of its four waves)
    int64_t want = (int64_t)num_cus * 4;
    int64_t rows_per_wg = ((int64_t)M + want - 1) / want;
    rows_per_wg = (rows_per_wg + 3) & ~(int64_t)3;
    const int64_t grid = ((int64_t)M + rows_per_wg - 1) / rows_per_wg;
    switch (T) {
        case 1: return launch_dq_t<1>(W, M, nb, X, x_tstride, Y, y_tstride, (int)grid, (int)rows_per_wg, lds, st);
        case 2: return launch_dq_t<2>(W, M, nb, X, x_tstride, Y, y_tstride, (int)grid, (int)rows_per_wg, lds, st);
        case 3: return launch_dq_t<3>(W, M, nb, X, x_tstride, Y, y_tstride, (int)grid, (int)rows_per_wg, lds, st);
        case 4: return launch_dq_t<4>(W, M, nb, X, x_tstride, Y, y_tstride, (int)grid, (int)rows_per_wg, lds, st);
        case 5: return launch_dq_t<5>(W, M, nb, X, x_tstride, Y, y_tstride, (int)grid, (int)rows_per_wg, lds, st);
        case 6: return launch_dq_t<6>(W, M, nb, X, x_tstride, Y, y_tstride, (int)grid, (int)rows_per_wg, lds, st);
        case 7: return launch_dq_t<7>(W, M, nb, X, x_tstride, Y, y_tstride, (int)grid, (int)rows_per_wg, lds, st);
        default: return launch_dq_t<8>(W, M, nb, X, x_tstride, Y, y_tstride, (int)grid, (int)rows_per_wg, lds, st);
    }
}

}  // namespace spq4k
