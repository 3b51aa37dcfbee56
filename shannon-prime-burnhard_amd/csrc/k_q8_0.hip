// k_q8_0.hip — GGML_TYPE_Q8_0 weights on gfx950: conversions and the
// matvecs (dense with T <= 8 tokens, expert-gathered).
//
// Q8_0 block (ggml-common.h:241-245): fp16 d, int8 qs[32]; 34 bytes per 32
// values, so block starts are only 2-byte aligned (loads declare it, as the
// Q6_K ones do). Q8_0 weights take Q8_0 activations (vec_dot_type,
// ggml-cpu.c:258-261), made by the CPU backend's quantize_row_q8_0
// (arch/x86/quants.c:302-367):
//   d = max|x| / 127 (stored as fp16), id = 127 / max|x|, q = round-half-even(x id).
// The model-file encoder quantize_row_q8_0_ref (ggml-quants.c:234-257) rounds
// half away from zero with id = 1 / d; spq4k_quantize_chunk follows it.
// The dot is ggml_vec_dot_q8_0_q8_0 (arch/x86/quants.c:1170-1204): per block
// the exact integer sum of 32 products times fp16(dw) * fp16(dx).
//
// Matvec mapping: a group of LPR lanes (8, 16, 32 or 64, chosen from K so
// that a lane holds 2 to 8 blocks) takes one weight row; lane g of the group
// takes blocks g, g + LPR, ... (34 contiguous bytes each, so a group reads
// its row as one stream), up to NITC blocks in registers at a time. The
// activations are Q8_0 planes: int8 values [row][K] and fp32 scales
// [row][K/32] (the fp16 d widened), either quantised by every workgroup into
// LDS or, when they do not fit, written once by quantize_q8_0_planes_kernel.
// Per block and token: eight sdot4, one fma. The group's lane sums are
// combined in a fixed DPP order.
#include "launch.h"
#include "q6k_core.h"

namespace spq4k {

constexpr int QK80 = 32;
constexpr int Q80_BYTES = 34;
constexpr int Q80_WAVES = 8;

__device__ __forceinline__ float f16_at(const uint8_t* p) {
    return half_bits_to_float(*reinterpret_cast<const u16_a2*>(p));
}

__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
    const _Float16 h = (_Float16)f;
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

// One 32-value block held by an aligned group of 8 lanes (4 values each),
// quantised with the CPU backend's activation rounding: returns the lane's
// four int8 values packed and the block's fp16 d.
__device__ __forceinline__ uint32_t q80_lane(const float4 v, uint16_t& d16) {
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 8));
    d16 = f32_to_f16_rne(amax / 127.f);
    const float id = amax != 0.0f ? 127.f / amax : 0.0f;
    const float x[4] = {v.x, v.y, v.z, v.w};
    uint32_t r = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float t = __builtin_rintf(x[i] * id);
        t = fminf(fmaxf(t, -128.f), 127.f);
        r |= ((uint32_t)(int)t & 0xFFu) << (8 * i);
    }
    return r;
}

// ---- element-wise conversions --------------------------------------------------------

// fp32 -> Q8_0 blocks (ggml layout), activation rounding (quantize_row_q8_0).
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float* __restrict__ x, uint8_t* __restrict__ y,
                                                            int64_t nblocks) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t blk0 = gid >> 3;
    const bool valid = blk0 < nblocks;
    const int64_t blk = valid ? blk0 : nblocks - 1;   // whole 8-lane groups stay in the shuffles
    const int e = (int)(gid & 7);
    const float4 v = *reinterpret_cast<const float4*>(x + blk * QK80 + 4 * e);
    uint16_t d16;
    const uint32_t q = q80_lane(v, d16);
    if (!valid) return;
    uint16_t* o = reinterpret_cast<uint16_t*>(y + blk * Q80_BYTES);
    if (e == 0) o[0] = d16;
    o[1 + 2 * e] = (uint16_t)(q & 0xFFFFu);
    o[2 + 2 * e] = (uint16_t)(q >> 16);
}

// fp32 -> Q8_0 blocks as the model-file encoder makes them
// (quantize_row_q8_0_ref): d = max / 127, id = 1 / d, roundf.
__global__ __launch_bounds__(256) void quantize_q8_0_ref_kernel(const float* __restrict__ x, uint8_t* __restrict__ y,
                                                                int64_t nblocks) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t blk0 = gid >> 3;
    const bool valid = blk0 < nblocks;
    const int64_t blk = valid ? blk0 : nblocks - 1;
    const int e = (int)(gid & 7);
    const float4 v = *reinterpret_cast<const float4*>(x + blk * QK80 + 4 * e);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 8));
    const float d = amax / 127;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const float xs[4] = {v.x, v.y, v.z, v.w};
    uint32_t q = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) q |= ((uint32_t)(int)roundf(xs[i] * id) & 0xFFu) << (8 * i);
    if (!valid) return;
    uint16_t* o = reinterpret_cast<uint16_t*>(y + blk * Q80_BYTES);
    if (e == 0) o[0] = f32_to_f16_rne(d);
    o[1 + 2 * e] = (uint16_t)(q & 0xFFFFu);
    o[2 + 2 * e] = (uint16_t)(q >> 16);
}

// Q8_0 -> fp32 (dequantize_row_q8_0, ggml-quants.c:491-505): y = q * d.
__global__ __launch_bounds__(256) void dequant_q8_0_kernel(const uint8_t* __restrict__ x, float* __restrict__ y,
                                                           int64_t nblocks) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t blk = gid >> 3;
    if (blk >= nblocks) return;
    const int e = (int)(gid & 7);
    const uint8_t* b = x + blk * Q80_BYTES;
    const float d = f16_at(b);
    const u16_a2* q16 = reinterpret_cast<const u16_a2*>(b + 2 + 4 * e);
    const uint32_t q = (uint32_t)q16[0] | ((uint32_t)q16[1] << 16);
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (float)(int8_t)((q >> (8 * i)) & 0xFFu) * d;
    *reinterpret_cast<float4*>(y + blk * QK80 + 4 * e) = make_float4(o[0], o[1], o[2], o[3]);
}

// fp32 rows x[r * x_tstride + k] -> Q8_0 planes: q [rows][K] int8, d
// [rows][K/32] fp32 (the fp16 d widened); activation rounding.
__global__ __launch_bounds__(256) void quantize_q8_0_planes_kernel(const float* __restrict__ x, int64_t x_tstride,
                                                                   int rows, int nb, int8_t* __restrict__ q,
                                                                   float* __restrict__ d) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t item0 = gid >> 3, nitems = (int64_t)rows * nb;
    const bool valid = item0 < nitems;
    const int64_t item = valid ? item0 : nitems - 1;
    const int64_t t = item / nb, b = item - t * nb;
    const int e = (int)(gid & 7);
    const float4 v = *reinterpret_cast<const float4*>(x + t * x_tstride + b * QK80 + 4 * e);
    uint16_t d16;
    const uint32_t qq = q80_lane(v, d16);
    if (!valid) return;
    *reinterpret_cast<uint32_t*>(q + item * QK80 + 4 * e) = qq;
    if (e == 0) d[item] = half_bits_to_float(d16);
}

// Exact block sums S[r][b] = sum of qw * qa over block b of row r against the
// activation quantisation of x (the integer core of ggml_vec_dot_q8_0_q8_0).
__global__ __launch_bounds__(256) void block_sums_q8_0_kernel(const uint8_t* __restrict__ W, int M, int nb,
                                                              const float* __restrict__ x, int32_t* __restrict__ S) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t item0 = gid >> 3, nitems = (int64_t)M * nb;
    const bool valid = item0 < nitems;
    const int64_t item = valid ? item0 : nitems - 1;
    const int64_t r = item / nb, b = item - r * nb;
    const int e = (int)(gid & 7);
    const float4 v = *reinterpret_cast<const float4*>(x + b * QK80 + 4 * e);
    uint16_t d16;
    const int a = (int)q80_lane(v, d16);
    const u16_a2* w16 = reinterpret_cast<const u16_a2*>(W + (r * nb + b) * Q80_BYTES + 2 + 4 * e);
    const int w = (int)((uint32_t)w16[0] | ((uint32_t)w16[1] << 16));
    int s = dot4(w, a, 0);
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) s += __shfl_xor(s, off, 8);
    if (valid && e == 0) S[item] = s;
}

// One Q8_0 row . one Q8_0 activation row (ggml layouts), one wave.
__global__ __launch_bounds__(64) void vec_dot_q8_0_kernel(const uint8_t* __restrict__ wx,
                                                          const uint8_t* __restrict__ a, int nb,
                                                          float* __restrict__ out) {
    const int lane = threadIdx.x;
    float acc = 0.0f;
    for (int b = lane; b < nb; b += 64) {
        const uint8_t* pw = wx + (size_t)b * Q80_BYTES;
        const uint8_t* pa = a + (size_t)b * Q80_BYTES;
        const uint4 w0 = load16_a2(pw + 2), w1 = load16_a2(pw + 18);
        const uint4 x0 = load16_a2(pa + 2), x1 = load16_a2(pa + 18);
        int s = dot4((int)w0.x, (int)x0.x, 0);
        s = dot4((int)w0.y, (int)x0.y, s);
        s = dot4((int)w0.z, (int)x0.z, s);
        s = dot4((int)w0.w, (int)x0.w, s);
        s = dot4((int)w1.x, (int)x1.x, s);
        s = dot4((int)w1.y, (int)x1.y, s);
        s = dot4((int)w1.z, (int)x1.z, s);
        s = dot4((int)w1.w, (int)x1.w, s);
        acc = fmaf(f16_at(pw) * f16_at(pa), (float)s, acc);
    }
    acc = group_sum_last<64>(acc);
    if (lane == 63) *out = acc;
}

// ---- matvec core ------------------------------------------------------------------------

// The blocks of one row a lane holds: block base + LPR * it for it < NITC.
template <int NITC>
struct Q80W {
    uint4 lo[NITC], hi[NITC];
    float dw[NITC];
};

template <int LPR, int NITC>
__device__ __forceinline__ void q80_load(Q80W<NITC>& w, const uint8_t* __restrict__ wrow, int nb, int base) {
#pragma unroll
    for (int it = 0; it < NITC; ++it) {
        const int b = base + LPR * it;
        w.lo[it] = w.hi[it] = make_uint4(0, 0, 0, 0);
        w.dw[it] = 0.0f;
        if (b < nb) {
            const uint8_t* q = wrow + (size_t)b * Q80_BYTES;
            w.dw[it] = f16_at(q);
            w.lo[it] = load16_a2(q + 2);
            w.hi[it] = load16_a2(q + 18);
        }
    }
}

// acc[t] += the held blocks . activation row xr[t], t < cnt.
template <int LPR, int NITC, int T>
__device__ __forceinline__ void q80_mac(const Q80W<NITC>& w, int nb, int base, const int8_t* __restrict__ aq,
                                        const float* __restrict__ ad, const int (&xr)[T], int cnt,
                                        float (&acc)[T]) {
    const int64_t K = (int64_t)nb * QK80;
#pragma unroll
    for (int it = 0; it < NITC; ++it) {
        const int b = base + LPR * it;
        if (b < nb) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                if (t < cnt) {
                    const int4* a = reinterpret_cast<const int4*>(aq + xr[t] * K + (int64_t)b * QK80);
                    const int4 a0 = a[0], a1 = a[1];
                    int s = dot4((int)w.lo[it].x, a0.x, 0);
                    s = dot4((int)w.lo[it].y, a0.y, s);
                    s = dot4((int)w.lo[it].z, a0.z, s);
                    s = dot4((int)w.lo[it].w, a0.w, s);
                    s = dot4((int)w.hi[it].x, a1.x, s);
                    s = dot4((int)w.hi[it].y, a1.y, s);
                    s = dot4((int)w.hi[it].z, a1.z, s);
                    s = dot4((int)w.hi[it].w, a1.w, s);
                    acc[t] = fmaf(w.dw[it] * ad[xr[t] * (int64_t)nb + b], (float)s, acc[t]);
                }
            }
        }
    }
}

// acc[t] += row . activation row xr[t] over all nb blocks, NITC a lane at a time.
template <int LPR, int NITC, int T>
__device__ __forceinline__ void q80_dot(const uint8_t* __restrict__ wrow, int nb, int g,
                                        const int8_t* __restrict__ aq, const float* __restrict__ ad,
                                        const int (&xr)[T], int cnt, float (&acc)[T]) {
    for (int base = g; base < nb; base += LPR * NITC) {
        Q80W<NITC> w;
        q80_load<LPR, NITC>(w, wrow, nb, base);
        q80_mac<LPR, NITC, T>(w, nb, base, aq, ad, xr, cnt, acc);
    }
}

// Staging of the n_xrows activation rows in LDS: Q8_0 values [row][K] then
// scales [row][K/32] (q80_lds_bytes). Copied from the caller's planes (p.Aq)
// or quantised from p.X, 8 lanes a block.
__device__ __forceinline__ void q80_quant_item(const Q80Params& p, int item0, int nitems, float4 v, char* smem) {
    const int nb = p.nb;
    int8_t* lq = reinterpret_cast<int8_t*>(smem);
    float* ld = reinterpret_cast<float*>(smem + (size_t)p.n_xrows * nb * QK80);
    const int e = threadIdx.x & 7;
    uint16_t d16;
    const uint32_t qq = q80_lane(v, d16);
    if (item0 < nitems) {
        *reinterpret_cast<uint32_t*>(lq + (size_t)item0 * QK80 + 4 * e) = qq;
        if (e == 0) ld[item0] = half_bits_to_float(d16);
    }
}

__device__ __forceinline__ float4 q80_x_at(const Q80Params& p, int item0, int nitems) {
    const int item = item0 < nitems ? item0 : nitems - 1;   // whole 8-lane groups stay in the shuffles
    const int t = item / p.nb, b = item - t * p.nb;
    return *reinterpret_cast<const float4*>(p.X + t * p.x_tstride + b * QK80 + 4 * (threadIdx.x & 7));
}

__device__ __forceinline__ void q80_stage(const Q80Params& p, char* smem) {
    const int nb = p.nb;
    const int nitems = p.n_xrows * nb;
    if (p.Aq) {
        int8_t* lq = reinterpret_cast<int8_t*>(smem);
        float* ld = reinterpret_cast<float*>(smem + (size_t)p.n_xrows * nb * QK80);
        for (int i = threadIdx.x; i < nitems * 2; i += Q80_WAVES * 64)
            reinterpret_cast<int4*>(lq)[i] = reinterpret_cast<const int4*>(p.Aq)[i];
        for (int i = threadIdx.x; i < nitems; i += Q80_WAVES * 64) ld[i] = p.Ad[i];
    } else {
        for (int base = 0; base < nitems; base += Q80_WAVES * 8) {
            const int item0 = base + (threadIdx.x >> 3);
            q80_quant_item(p, item0, nitems, q80_x_at(p, item0, nitems), smem);
        }
    }
    __syncthreads();
}

// Input rows of at most Q80_XPASS * 64 blocks are quantised "x first": every
// thread loads its x values, the first weight row is put in flight, then the
// values are quantised into LDS and the barrier waits for LDS stores only, so
// the weight loads stay outstanding across it (memory loads complete in order).
constexpr int Q80_XPASS = 4;

// row pointer of the lane's group in the dense kernel (row rr < total_rows)
__device__ __forceinline__ const uint8_t* q80_dense_row(const Q80Params& p, int rr, size_t row_bytes) {
    const uint8_t* W = p.seg[0].W;
    int rb = 0;
#pragma unroll
    for (int k = 1; k < GEMV_MAX_SEG; ++k)
        if (rr >= p.seg[k].row_begin) {   // unused segments start at INT32_MAX
            W = p.seg[k].W;
            rb = p.seg[k].row_begin;
        }
    return W + (size_t)(rr - rb) * row_bytes;
}

template <int LPR, int T>
__device__ __forceinline__ void q80_dense_store(const Q80Params& p, int r, int total, int g, float (&acc)[T]) {
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = group_sum_last<LPR>(acc[t]);
    if (g == LPR - 1 && r < total) {
        float* Y = p.seg[0].Y;
        int64_t ys = p.seg[0].y_tstride;
        int rb = 0;
#pragma unroll
        for (int k = 1; k < GEMV_MAX_SEG; ++k)
            if (r >= p.seg[k].row_begin) {
                Y = p.seg[k].Y;
                ys = p.seg[k].y_tstride;
                rb = p.seg[k].row_begin;
            }
#pragma unroll
        for (int t = 0; t < T; ++t) Y[(int64_t)t * ys + (r - rb)] = acc[t];
    }
}

// Dense, K a multiple of 256 (eight-block chunks of a row start 16-byte
// aligned): the weights stream through a double buffer of each wave in LDS,
// Q80S_CB blocks (2176 bytes) at a time, by contiguous 16-byte
// global_load_lds, and are read back with unaligned LDS reads. The 34-byte
// block stride of direct loads keeps the texture addresser busy (each
// wave-wide 16-byte load spans 2 KB); contiguous lanes do not. A wave takes
// one row at a time, lane g block g of each chunk; its (row, chunk) items
// form one stream with the next item always in flight, across rows too.
// Activations in LDS as in gemv_q8_0_kernel; the per-block combine is its.
constexpr int Q80S_CB = 64;
constexpr int Q80S_SLOTS = Q80S_CB * Q80_BYTES / 16;          // 136
constexpr int Q80S_LOADS = (Q80S_SLOTS + 63) / 64;             // 3 wave-wide loads a chunk
constexpr int Q80S_BUF = Q80S_LOADS * 1024;
size_t q80s_weight_lds() { return (size_t)Q80_WAVES * 2 * Q80S_BUF; }

template <int T>
__global__ __launch_bounds__(Q80_WAVES * 64) void gemv_q8_0_staged_kernel(Q80Params p) {
    extern __shared__ __align__(1024) char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = p.nb;
    const size_t row_bytes = (size_t)nb * Q80_BYTES;
    const int total = p.total_rows;
    const int S = gridDim.x * Q80_WAVES;
    const int rw0 = blockIdx.x * Q80_WAVES + wave;
    const int nch = (nb + Q80S_CB - 1) / Q80S_CB;
    const int nrow = rw0 < total ? (total - 1 - rw0) / S + 1 : 0;
    const int nitem = nrow * nch;
    // the weight buffers sit behind the activations, at a 1 KB boundary
    const size_t act = ((size_t)p.n_xrows * nb * (QK80 + 4) + 1023) & ~(size_t)1023;   // q80_lds_bytes
    uint8_t* wbuf = reinterpret_cast<uint8_t*>(smem) + act + (size_t)wave * 2 * Q80S_BUF;
    auto issue = [&](int i) {
        const int ri = i / nch, c = i - ri * nch;
        const uint8_t* wr = q80_dense_row(p, rw0 + ri * S, row_bytes);
        const size_t lim = row_bytes - 16;
#pragma unroll
        for (int k = 0; k < Q80S_LOADS; ++k) {
            size_t o = (size_t)c * (Q80S_CB * Q80_BYTES) + (size_t)(k * 64 + lane) * 16;
            o = o < lim ? o : lim;                 // past the row's end: a valid address, never read back
            __builtin_amdgcn_global_load_lds((const void*)(wr + o),
                                             (__attribute__((address_space(3))) void*)(wbuf + (i & 1) * Q80S_BUF + k * 1024),
                                             16, 0, 0);
        }
    };
    q80_stage(p, smem);
    const int8_t* aq = reinterpret_cast<const int8_t*>(smem);
    const float* ad = reinterpret_cast<const float*>(smem + (size_t)p.n_xrows * nb * QK80);
    const int64_t K = (int64_t)nb * QK80;
    if (nitem > 0) issue(0);
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.0f;
    for (int i = 0; i < nitem; ++i) {
        // the buffer refilled next was read in the previous item (its LDS
        // reads have returned: their values were used)
        if (i + 1 < nitem) {
            issue(i + 1);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(Q80S_LOADS) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        const int ri = i / nch, c = i - ri * nch;
        const int b = c * Q80S_CB + lane;
        if (b < nb) {
            const uint8_t* q = wbuf + (i & 1) * Q80S_BUF + lane * Q80_BYTES;
            uint16_t h;
            uint4 lo, hi;
            __builtin_memcpy(&h, q, 2);
            __builtin_memcpy(&lo, q + 2, 16);
            __builtin_memcpy(&hi, q + 18, 16);
            const float dw = half_bits_to_float(h);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int4* a = reinterpret_cast<const int4*>(aq + t * K + (int64_t)b * QK80);
                const int4 a0 = a[0], a1 = a[1];
                int sm = dot4((int)lo.x, a0.x, 0);
                sm = dot4((int)lo.y, a0.y, sm);
                sm = dot4((int)lo.z, a0.z, sm);
                sm = dot4((int)lo.w, a0.w, sm);
                sm = dot4((int)hi.x, a1.x, sm);
                sm = dot4((int)hi.y, a1.y, sm);
                sm = dot4((int)hi.z, a1.z, sm);
                sm = dot4((int)hi.w, a1.w, sm);
                acc[t] = fmaf(dw * ad[t * (int64_t)nb + b], (float)sm, acc[t]);
            }
        }
        if (c == nch - 1) {
            q80_dense_store<64, T>(p, rw0 + ri * S, total, lane, acc);
#pragma unroll
            for (int t = 0; t < T; ++t) acc[t] = 0.0f;
        }
    }
}

// Dense: the rows of up to four matrices sharing the input (segments), T
// tokens, activation row t for token t; y[t * y_tstride + r]. GX: the
// activations are read from the global planes p.Aq / p.Ad (rows too long
// for LDS), otherwise staged in LDS. PIPE (rows of one pass, NITC blocks a
// lane): the next row's blocks are loaded while the current one is used.
template <int LPR, int NITC, int T, bool GX, bool PIPE>
__global__ __launch_bounds__(Q80_WAVES * 64) void gemv_q8_0_kernel(Q80Params p) {
    extern __shared__ __align__(16) char smem[];
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane & (LPR - 1);
    const int sub = lane / LPR;
    const int nb = p.nb;
    const size_t row_bytes = (size_t)nb * Q80_BYTES;
    const int total = p.total_rows;
    const int S = gridDim.x * Q80_WAVES * RPW;
    int r0 = (blockIdx.x * Q80_WAVES + wave) * RPW;
    auto row_of = [&](int rw) { return q80_dense_row(p, min(rw + sub, total - 1), row_bytes); };
    const int8_t* aq = p.Aq;
    const float* ad = p.Ad;
    Q80W<NITC> wa, wb;
    if (!GX) {
        const int nitems = p.n_xrows * nb;
        if (PIPE && !p.Aq && nitems <= Q80_XPASS * Q80_WAVES * 8) {
            float4 xv[Q80_XPASS];
#pragma unroll
            for (int ps = 0; ps < Q80_XPASS; ++ps) {
                const int item0 = ps * Q80_WAVES * 8 + (threadIdx.x >> 3);
                if (ps * Q80_WAVES * 8 < nitems) xv[ps] = q80_x_at(p, item0, nitems);
            }
            if (r0 < total) q80_load<LPR, NITC>(wa, row_of(r0), nb, g);
#pragma unroll
            for (int ps = 0; ps < Q80_XPASS; ++ps) {
                const int item0 = ps * Q80_WAVES * 8 + (threadIdx.x >> 3);
                if (ps * Q80_WAVES * 8 < nitems) q80_quant_item(p, item0, nitems, xv[ps], smem);
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): LDS stores only
            __builtin_amdgcn_s_barrier();
        } else {
            q80_stage(p, smem);
            if (PIPE && r0 < total) q80_load<LPR, NITC>(wa, row_of(r0), nb, g);
        }
        aq = reinterpret_cast<const int8_t*>(smem);
        ad = reinterpret_cast<const float*>(smem + (size_t)p.n_xrows * nb * QK80);
    } else if (PIPE && r0 < total) {
        q80_load<LPR, NITC>(wa, row_of(r0), nb, g);
    }
    int xr[T];
#pragma unroll
    for (int t = 0; t < T; ++t) xr[t] = t;
    if (PIPE) {
        while (r0 < total) {
            if (r0 + S < total) q80_load<LPR, NITC>(wb, row_of(r0 + S), nb, g);
            {
                float acc[T];
#pragma unroll
                for (int t = 0; t < T; ++t) acc[t] = 0.0f;
                q80_mac<LPR, NITC, T>(wa, nb, g, aq, ad, xr, T, acc);
                q80_dense_store<LPR, T>(p, r0 + sub, total, g, acc);
            }
            r0 += S;
            if (r0 >= total) break;
            if (r0 + S < total) q80_load<LPR, NITC>(wa, row_of(r0 + S), nb, g);
            {
                float acc[T];
#pragma unroll
                for (int t = 0; t < T; ++t) acc[t] = 0.0f;
                q80_mac<LPR, NITC, T>(wb, nb, g, aq, ad, xr, T, acc);
                q80_dense_store<LPR, T>(p, r0 + sub, total, g, acc);
            }
            r0 += S;
        }
    } else {
        for (; r0 < total; r0 += S) {
            float acc[T];
#pragma unroll
            for (int t = 0; t < T; ++t) acc[t] = 0.0f;
            q80_dot<LPR, NITC, T>(row_of(r0), nb, g, aq, ad, xr, T, acc);
            q80_dense_store<LPR, T>(p, r0 + sub, total, g, acc);
        }
    }
}

// Expert-gathered, one sweep: row r = pair * M + lr of expert ids[pair] on
// input row (pair / n_used) * ne11 + (pair % n_used) % ne11, for every
// routed pair (an expert chosen twice is streamed twice: small batches).
// The next row's blocks are loaded while the current one is used (rows of
// one pass).
__device__ __forceinline__ const uint8_t* q80_sweep_row(const Q80Params& p, int rr, size_t row_bytes, int& xrow,
                                                        bool& ok) {
    const int pair = rr / p.M, lr = rr - pair * p.M;
    const int e = p.ids[pair];
    ok = e >= 0 && e < p.E;
    const int t = pair / p.n_used, s = pair - t * p.n_used;
    xrow = t * p.ne11 + s % p.ne11;
    return p.bank + (size_t)(ok ? e : 0) * p.expert_bytes + (size_t)lr * row_bytes;
}

template <int LPR, int NITC, bool PIPE>
__global__ __launch_bounds__(Q80_WAVES * 64) void moe_q8_0_sweep_kernel(Q80Params p) {
    extern __shared__ __align__(16) char smem[];
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane & (LPR - 1);
    const int sub = lane / LPR;
    const int nb = p.nb;
    const size_t row_bytes = (size_t)nb * Q80_BYTES;
    const int total = p.total_rows;
    const int S = gridDim.x * Q80_WAVES * RPW;
    int r0 = (blockIdx.x * Q80_WAVES + wave) * RPW;
    int xa = 0, xb = 0;
    bool oka = false, okb = false;
    Q80W<NITC> wa, wb;
    if (PIPE && r0 < total) q80_load<LPR, NITC>(wa, q80_sweep_row(p, min(r0 + sub, total - 1), row_bytes, xa, oka), nb, g);
    q80_stage(p, smem);
    const int8_t* aq = reinterpret_cast<const int8_t*>(smem);
    const float* ad = reinterpret_cast<const float*>(smem + (size_t)p.n_xrows * nb * QK80);
    auto finish = [&](float acc, int r, bool ok) {
        acc = group_sum_last<LPR>(acc);
        if (g == LPR - 1 && r < total && ok) p.Y[r] = acc;   // row r of the sweep is Y[pair][lr]
    };
    if (PIPE) {
        while (r0 < total) {
            if (r0 + S < total)
                q80_load<LPR, NITC>(wb, q80_sweep_row(p, min(r0 + S + sub, total - 1), row_bytes, xb, okb), nb, g);
            {
                int xr[1] = {xa};
                float acc[1] = {0.0f};
                q80_mac<LPR, NITC, 1>(wa, nb, g, aq, ad, xr, 1, acc);
                finish(acc[0], r0 + sub, oka);
            }
            r0 += S;
            if (r0 >= total) break;
            if (r0 + S < total)
                q80_load<LPR, NITC>(wa, q80_sweep_row(p, min(r0 + S + sub, total - 1), row_bytes, xa, oka), nb, g);
            {
                int xr[1] = {xb};
                float acc[1] = {0.0f};
                q80_mac<LPR, NITC, 1>(wb, nb, g, aq, ad, xr, 1, acc);
                finish(acc[0], r0 + sub, okb);
            }
            r0 += S;
        }
    } else {
        for (; r0 < total; r0 += S) {
            const uint8_t* w = q80_sweep_row(p, min(r0 + sub, total - 1), row_bytes, xa, oka);
            int xr[1] = {xa};
            float acc[1] = {0.0f};
            q80_dot<LPR, NITC, 1>(w, nb, g, aq, ad, xr, 1, acc);
            finish(acc[0], r0 + sub, oka);
        }
    }
}

// Expert-gathered, grouped: workgroup (a, grp) takes active expert a of the
// routing tables and rows [grp * rows_per_wg, ...) of it; each row is dotted
// with the expert's pairs TC at a time. Activations: global planes of all
// input rows. Rows of one pass (PIPE) stay in registers for all the pairs,
// and the next row's blocks are loaded meanwhile; longer rows are streamed
// again per chunk of pairs (from cache).
template <int LPR, int NITC, int TC>
__device__ __forceinline__ void q80_group_pairs(const Q80Params& p, int poff, int c0, int cnt, int (&pr)[TC],
                                                int (&xr)[TC]) {
#pragma unroll
    for (int t = 0; t < TC; ++t) {
        pr[t] = p.route.pairs[poff + c0 + min(t, cnt - 1)];
        const int tok = pr[t] / p.n_used, s = pr[t] - tok * p.n_used;
        xr[t] = tok * p.ne11 + s % p.ne11;
    }
}

template <int LPR, int TC>
__device__ __forceinline__ void q80_group_store(const Q80Params& p, int g, bool live, int rr, int cnt,
                                                const int (&pr)[TC], float (&acc)[TC]) {
#pragma unroll
    for (int t = 0; t < TC; ++t) acc[t] = group_sum_last<LPR>(acc[t]);
    if (g == LPR - 1 && live) {
#pragma unroll
        for (int t = 0; t < TC; ++t)
            if (t < cnt) p.Y[(int64_t)pr[t] * p.M + rr] = acc[t];
    }
}

template <int LPR, int NITC, int TC, bool PIPE>
__global__ __launch_bounds__(Q80_WAVES * 64) void moe_q8_0_grouped_kernel(Q80Params p) {
    constexpr int RPW = 64 / LPR;
    const int a = blockIdx.x / p.groups;
    const int grp = blockIdx.x - a * p.groups;
    if (a >= *p.route.n_act) return;   // uniform over the workgroup
    const int e = p.route.act[a];
    const int poff = p.route.act_off[a];
    const int pcnt = p.route.act_cnt[a];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane & (LPR - 1);
    const int sub = lane / LPR;
    const int nb = p.nb;
    const size_t row_bytes = (size_t)nb * Q80_BYTES;
    const int begin = grp * p.rows_per_wg;
    const int end = min(p.M, begin + p.rows_per_wg);
    const uint8_t* base = p.bank + (size_t)e * p.expert_bytes;
    constexpr int S = Q80_WAVES * RPW;
    int r0 = begin + wave * RPW;
    auto rowp = [&](int rw) { return base + (size_t)min(rw + sub, end - 1) * row_bytes; };
    auto use = [&](const Q80W<NITC>& w, int rw) {
        for (int c0 = 0; c0 < pcnt; c0 += TC) {
            const int cnt = min(TC, pcnt - c0);
            int pr[TC], xr[TC];
            float acc[TC];
            q80_group_pairs<LPR, NITC, TC>(p, poff, c0, cnt, pr, xr);
#pragma unroll
            for (int t = 0; t < TC; ++t) acc[t] = 0.0f;
            q80_mac<LPR, NITC, TC>(w, nb, g, p.Aq, p.Ad, xr, cnt, acc);
            q80_group_store<LPR, TC>(p, g, rw + sub < end, min(rw + sub, end - 1), cnt, pr, acc);
        }
    };
    if (PIPE) {
        Q80W<NITC> wa, wb;
        if (r0 < end) q80_load<LPR, NITC>(wa, rowp(r0), nb, g);
        while (r0 < end) {
            if (r0 + S < end) q80_load<LPR, NITC>(wb, rowp(r0 + S), nb, g);
            use(wa, r0);
            r0 += S;
            if (r0 >= end) break;
            if (r0 + S < end) q80_load<LPR, NITC>(wa, rowp(r0 + S), nb, g);
            use(wb, r0);
            r0 += S;
        }
    } else {
        for (; r0 < end; r0 += S) {
            for (int c0 = 0; c0 < pcnt; c0 += TC) {
                const int cnt = min(TC, pcnt - c0);
                int pr[TC], xr[TC];
                float acc[TC];
                q80_group_pairs<LPR, NITC, TC>(p, poff, c0, cnt, pr, xr);
#pragma unroll
                for (int t = 0; t < TC; ++t) acc[t] = 0.0f;
                q80_dot<LPR, NITC, TC>(rowp(r0), nb, g, p.Aq, p.Ad, xr, cnt, acc);
                q80_group_store<LPR, TC>(p, g, r0 + sub < end, min(r0 + sub, end - 1), cnt, pr, acc);
            }
        }
    }
}

// ---------------------------------------------------------------------------
hipError_t launch_quantize_q8_0(const float* x, uint8_t* y, int64_t nblocks, bool ref_encoder, hipStream_t st) {
    if (nblocks <= 0) return hipSuccess;
    const int64_t grid = (nblocks * 8 + 255) / 256;
    if (ref_encoder)
        hipLaunchKernelGGL(quantize_q8_0_ref_kernel, dim3((unsigned)grid), dim3(256), 0, st, x, y, nblocks);
    else
        hipLaunchKernelGGL(quantize_q8_0_kernel, dim3((unsigned)grid), dim3(256), 0, st, x, y, nblocks);
    return hipGetLastError();
}

hipError_t launch_dequant_q8_0(const uint8_t* x, float* y, int64_t nblocks, hipStream_t st) {
    if (nblocks <= 0) return hipSuccess;
    const int64_t grid = (nblocks * 8 + 255) / 256;
    hipLaunchKernelGGL(dequant_q8_0_kernel, dim3((unsigned)grid), dim3(256), 0, st, x, y, nblocks);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_0_planes(const float* x, int64_t x_tstride, int rows, int nb, int8_t* q, float* d,
                                       hipStream_t st) {
    const int64_t items = (int64_t)rows * nb;
    if (items <= 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8_0_planes_kernel, dim3((unsigned)((items * 8 + 255) / 256)), dim3(256), 0, st, x,
                       x_tstride, rows, nb, q, d);
    return hipGetLastError();
}

hipError_t launch_block_sums_q8_0(const uint8_t* W, int M, int nb, const float* x, int32_t* S, hipStream_t st) {
    const int64_t items = (int64_t)M * nb;
    if (items <= 0) return hipSuccess;
    hipLaunchKernelGGL(block_sums_q8_0_kernel, dim3((unsigned)((items * 8 + 255) / 256)), dim3(256), 0, st, W, M,
                       nb, x, S);
    return hipGetLastError();
}

hipError_t launch_vec_dot_q8_0(const uint8_t* wx, const uint8_t* a, int nb, float* out, hipStream_t st) {
    hipLaunchKernelGGL(vec_dot_q8_0_kernel, dim3(1), dim3(64), 0, st, wx, a, nb, out);
    return hipGetLastError();
}

size_t q80_lds_bytes(int xrows, int nb) { return (size_t)xrows * nb * (QK80 + 4); }

// Lanes per row: 8 below 64 blocks, 16 below 128, 32 below 256, else 64,
// so that a lane holds four blocks or more (fewer only for short rows).
int q80_lanes_per_row(int nb) { return nb < 64 ? 8 : nb < 128 ? 16 : nb < 256 ? 32 : 64; }

int q80_rows_per_wg(int nb) { return Q80_WAVES * (64 / q80_lanes_per_row(nb)); }

// (LPR, NITC) of a row length, LPR as q80_lanes_per_row: NITC = 4 blocks a
// lane at a time when the row fits in one such pass, else 8
#define SPQ_Q80_SHAPES(X)                                          \
    if (nb < 64) { if (nb <= 32) { X(8, 4) } else { X(8, 8) } }    \
    else if (nb < 128) { if (nb <= 64) { X(16, 4) } else { X(16, 8) } } \
    else if (nb < 256) { if (nb <= 128) { X(32, 4) } else { X(32, 8) } } \
    else { if (nb <= 256) { X(64, 4) } else { X(64, 8) } }

static bool q80_pipe(int nb) { return nb <= 4 * q80_lanes_per_row(nb); }

template <int T, bool GX>
static hipError_t launch_gemv_q80_t(const Q80Params& p, int grid, hipStream_t st) {
    const int nb = p.nb;
    const size_t lds = GX ? 0 : q80_lds_bytes(p.n_xrows, nb);
    // rows of one pass are pipelined at T <= 2, where a row's integer work is short
    const bool pipe = T <= 2 && q80_pipe(nb);
#define SPQ_GO(L, N)                                                                                              \
    if (pipe && N == 4)                                                                                           \
        hipLaunchKernelGGL((gemv_q8_0_kernel<L, N, T, GX, (N == 4 && T <= 2)>), dim3(grid), dim3(Q80_WAVES * 64), \
                           lds, st, p);                                                                           \
    else                                                                                                          \
        hipLaunchKernelGGL((gemv_q8_0_kernel<L, N, T, GX, false>), dim3(grid), dim3(Q80_WAVES * 64), lds, st, p); \
    return hipGetLastError();
    SPQ_Q80_SHAPES(SPQ_GO)
#undef SPQ_GO
}

template <int T>
static hipError_t launch_q80_staged_t(const Q80Params& p, int grid, hipStream_t st) {
    const size_t lds = ((q80_lds_bytes(p.n_xrows, p.nb) + 1023) & ~(size_t)1023) + q80s_weight_lds();
    hipLaunchKernelGGL((gemv_q8_0_staged_kernel<T>), dim3(grid), dim3(Q80_WAVES * 64), lds, st, p);
    return hipGetLastError();
}

bool q80_staged_fits(int T, int nb) {
    return nb % 8 == 0 && nb >= Q80S_CB && T >= 1 && T <= 8 &&
           ((q80_lds_bytes(T, nb) + 1023) & ~(size_t)1023) + q80s_weight_lds() <= (size_t)Q80_LDS_MAX;
}

int q80_staged_grid(int64_t rows, int T, int nb, int num_cus, size_t lds_max) {
    const int64_t need = (rows + Q80_WAVES - 1) / Q80_WAVES;   // one row a wave at a time
    const size_t per = ((q80_lds_bytes(T, nb) + 1023) & ~(size_t)1023) + q80s_weight_lds();
    const int64_t fit = lds_max / per >= 2 ? 2 : 1;           // workgroups a CU can hold, up to two
    const int64_t cap = fit * num_cus;
    return (int)(need < cap ? need : cap);
}

size_t q80_staged_lds_bytes(int T, int nb) {
    return ((q80_lds_bytes(T, nb) + 1023) & ~(size_t)1023) + q80s_weight_lds();
}

hipError_t launch_gemv_q8_0_staged(const Q80Params& p, int T, int grid, hipStream_t st) {
    if (grid < 1 || p.n_xrows != T || !q80_staged_fits(T, p.nb)) return hipErrorInvalidValue;
    switch (T) {
        case 1: return launch_q80_staged_t<1>(p, grid, st);
        case 2: return launch_q80_staged_t<2>(p, grid, st);
        case 3: return launch_q80_staged_t<3>(p, grid, st);
        case 4: return launch_q80_staged_t<4>(p, grid, st);
        case 5: return launch_q80_staged_t<5>(p, grid, st);
        case 6: return launch_q80_staged_t<6>(p, grid, st);
        case 7: return launch_q80_staged_t<7>(p, grid, st);
        case 8: return launch_q80_staged_t<8>(p, grid, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_q8_0(const Q80Params& p, int T, bool global_acts, int grid, hipStream_t st) {
    if (p.nb < 1 || grid < 1 || p.n_xrows != T) return hipErrorInvalidValue;
    if (global_acts) {
        if (T != 1 || !p.Aq) return hipErrorInvalidValue;
        return launch_gemv_q80_t<1, true>(p, grid, st);
    }
    if (q80_lds_bytes(T, p.nb) > Q80_LDS_MAX) return hipErrorInvalidValue;
    switch (T) {
        case 1: return launch_gemv_q80_t<1, false>(p, grid, st);
        case 2: return launch_gemv_q80_t<2, false>(p, grid, st);
        case 3: return launch_gemv_q80_t<3, false>(p, grid, st);
        case 4: return launch_gemv_q80_t<4, false>(p, grid, st);
        case 5: return launch_gemv_q80_t<5, false>(p, grid, st);
        case 6: return launch_gemv_q80_t<6, false>(p, grid, st);
        case 7: return launch_gemv_q80_t<7, false>(p, grid, st);
        case 8: return launch_gemv_q80_t<8, false>(p, grid, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_q8_0_sweep(const Q80Params& p, int grid, hipStream_t st) {
    const int nb = p.nb;
    if (nb < 1 || grid < 1 || p.M < 1 || !p.ids) return hipErrorInvalidValue;
    const size_t lds = q80_lds_bytes(p.n_xrows, nb);
    if (lds > Q80_LDS_MAX) return hipErrorInvalidValue;
    const bool pipe = q80_pipe(nb);
#define SPQ_GO(L, N)                                                                                              \
    if (pipe && N == 4)                                                                                           \
        hipLaunchKernelGGL((moe_q8_0_sweep_kernel<L, N, (N == 4)>), dim3(grid), dim3(Q80_WAVES * 64), lds, st, p); \
    else                                                                                                          \
        hipLaunchKernelGGL((moe_q8_0_sweep_kernel<L, N, false>), dim3(grid), dim3(Q80_WAVES * 64), lds, st, p);   \
    return hipGetLastError();
    SPQ_Q80_SHAPES(SPQ_GO)
#undef SPQ_GO
}

template <int TC>
static hipError_t launch_moe_grouped_t(const Q80Params& p, int grid, hipStream_t st) {
    const int nb = p.nb;
    const bool pipe = q80_pipe(nb);
#define SPQ_GO(L, N)                                                                                              \
    if (pipe && N == 4)                                                                                           \
        hipLaunchKernelGGL((moe_q8_0_grouped_kernel<L, N, TC, (N == 4)>), dim3(grid), dim3(Q80_WAVES * 64), 0, st, \
                           p);                                                                                    \
    else                                                                                                          \
        hipLaunchKernelGGL((moe_q8_0_grouped_kernel<L, N, TC, false>), dim3(grid), dim3(Q80_WAVES * 64), 0, st, p); \
    return hipGetLastError();
    SPQ_Q80_SHAPES(SPQ_GO)
#undef SPQ_GO
}

hipError_t launch_moe_q8_0_grouped(const Q80Params& p, int tc, int grid, hipStream_t st) {
    if (p.nb < 1 || grid < 1 || p.M < 1 || !p.Aq || p.groups < 1 || p.rows_per_wg < 1) return hipErrorInvalidValue;
    switch (tc) {
        case 1: return launch_moe_grouped_t<1>(p, grid, st);
        case 2: return launch_moe_grouped_t<2>(p, grid, st);
        case 4: return launch_moe_grouped_t<4>(p, grid, st);
        case 8: return launch_moe_grouped_t<8>(p, grid, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace spq4k
