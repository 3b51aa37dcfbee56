// gemv_core.h — the Q4_K x Q8_K matvec building blocks shared by the dense,
// grouped and expert-gathered GEMV kernels.
//
// Lane mapping (wave64): lanes work in quads on a 144 B super-block. Lane
// l4 = lane & 3 of a quad reads the 16 B header (d, dmin, scales) and the 32
// contiguous bytes qs[32*l4 .. 32*l4+31]. Those bytes carry the whole of
// sub-blocks j0 = 2*l4 (low nibbles, elements 64*l4 + 0..31) and j1 = 2*l4 + 1
// (high nibbles, elements 64*l4 + 32..63), so each lane forms the two exact
// integer sub-block sums S_{b,j0}, S_{b,j1} with eight v_dot4_i32_i8 each,
// applies its two 6-bit scales and mins, and folds the block into an fp32
// accumulator:
//     acc += (fp16(d) * d8) * (sc0*S0 + sc1*S1) - (fp16(dmin) * d8) * (m0*bs01 + m1*bs23)
// This is the arithmetic of ggml_vec_dot_q4_K_q8_K
// (vendor/ggml/src/ggml-cpu/quants.c:645-718, arch/x86/quants.c:1919-1982)
// with the integer parts exact and only the fp32 summation order changed.
//
// Activations are Q8_K, staged in LDS as planes
//   q8[slot][256] int8 | bsum[slot][16] int16 | d8[slot] f32,  slot = t*CB + block
// either quantised on chip from fp32 (stage_q8_from_f32) or copied from a
// Q8_K plane buffer written by quantize_q8k_planes_kernel (stage_q8_from_planes).
#pragma once

#include "q4k_device.h"

namespace spq4k {

// Registers of one lane for one super-block of one row.
struct W4 {
    uint4 hdr;   // d | dmin << 16, scale bytes 0-3, 4-7, 8-11
    uint4 qa;    // qs[32*l4 + 0 .. 15]
    uint4 qb;    // qs[32*l4 + 16 .. 31]
};

__device__ __forceinline__ W4 load_w4(const uint8_t* __restrict__ blk, int l4) {
    W4 w;
    w.hdr = *reinterpret_cast<const uint4*>(blk);
    const uint4* q = reinterpret_cast<const uint4*>(blk + 16 + 32 * l4);
    w.qa = q[0];
    w.qb = q[1];
    return w;
}

// Per-lane, per-block constants derived from the header.
struct BlkC {
    float d, dmin;
    int sc0, sc1, m0, m1;
};

__device__ __forceinline__ BlkC block_consts(const uint4& h, int l4) {
    BlkC c;
    c.d = half_bits_to_float(h.x & 0xFFFFu);
    c.dmin = half_bits_to_float(h.x >> 16);
    const ScaleMin sm = unpack_scale_min(h.y, h.z, h.w);
    const bool hi = l4 >= 2;
    const uint32_t scw = hi ? sm.sc_hi : sm.sc_lo;
    const uint32_t mw = hi ? sm.m_hi : sm.m_lo;
    const int sh = 16 * (l4 & 1);
    c.sc0 = (int)((scw >> sh) & 0xFFu);
    c.sc1 = (int)((scw >> (sh + 8)) & 0xFFu);
    c.m0 = (int)((mw >> sh) & 0xFFu);
    c.m1 = (int)((mw >> (sh + 8)) & 0xFFu);
    return c;
}

// Nibble planes of the lane's 32 qs bytes: lo[i] holds elements 64*l4 + 4i..4i+3,
// hi[i] elements 64*l4 + 32 + 4i..4i+3, as unsigned bytes 0..15.
struct Nib {
    int lo[8], hi[8];
};

__device__ __forceinline__ Nib split_nibbles(const W4& w) {
    Nib n;
    const uint32_t q[8] = {w.qa.x, w.qa.y, w.qa.z, w.qa.w, w.qb.x, w.qb.y, w.qb.z, w.qb.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        n.lo[i] = (int)(q[i] & 0x0F0F0F0Fu);
        n.hi[i] = (int)((q[i] >> 4) & 0x0F0F0F0Fu);
    }
    return n;
}

// LDS view of the staged Q8_K activations for one chunk.
struct Q8Lds {
    int8_t* q8;     // [slots][256]
    int16_t* bs;    // [slots][16]
    float* d8;      // [slots]
};

__host__ __device__ constexpr int q8lds_bytes(int slots) { return slots * (256 + 32 + 4); }

__device__ __forceinline__ Q8Lds q8lds_carve(char* base, int slots) {
    Q8Lds v;
    v.q8 = reinterpret_cast<int8_t*>(base);
    v.bs = reinterpret_cast<int16_t*>(base + slots * 256);
    v.d8 = reinterpret_cast<float*>(base + slots * (256 + 32));
    return v;
}

// Q8_K activations as planes in global memory: T rows of nb blocks.
struct Q8Planes {
    const int8_t* qs;    // [T][nb][256], 16-byte aligned
    const int16_t* bs;   // [T][nb][16]
    const float* d;      // [T][nb]
    // [T][nb][48 bytes], 16-byte aligned: the min-term operand of the matrix-core
    // kernels, BS_j = bs[2j] + bs[2j+1] split as 32 hi_j + lo_j (lo_j in 0..31):
    // fp16 hi_0..hi_7, fp16 lo_0..lo_7, then d as fp32 at byte 32
    const uint8_t* mn;
};
constexpr int Q8MN_BYTES = 48;

// fp32 rows -> Q8_K planes (qs [T][nb][256], bs [T][nb][16], d [T][nb] and the
// min-term operand mn [T][nb][48 B]): the activation operand of the
// pre-quantised GEMV/MoE/GEMM paths. Items (t, block) 16 * blk .. +15, 16 lanes
// an item (256 threads). With `perm` each 64-value group g of qs is stored as
// the matrix-core ring kernels read it: bytes 64g + 16s .. +15 hold values
// 64g + 8s .. +7 then 64g + 32 + 8s .. +7 (s = 0..3).
__device__ __forceinline__ void quantize_planes_items(const float* __restrict__ x, int64_t x_tstride, int T, int nb,
                                                      int8_t* __restrict__ qs, int16_t* __restrict__ bs,
                                                      float* __restrict__ d, uint8_t* __restrict__ mn, int perm,
                                                      int64_t blk) {
    const int e = threadIdx.x & 15;
    const int64_t nitems = (int64_t)T * nb;
    const int64_t item0 = blk * 16 + (threadIdx.x >> 4);
    const bool valid = item0 < nitems;
    const int64_t item = valid ? item0 : nitems - 1;
    const int64_t t = item / nb;
    const int64_t b = item - t * nb;
    const float4* src = reinterpret_cast<const float4*>(x + t * x_tstride + b * QK + 16 * e);
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 a = src[i];
        v[4 * i] = a.x; v[4 * i + 1] = a.y; v[4 * i + 2] = a.z; v[4 * i + 3] = a.w;
    }
    const Q8Lane q = quantize_q8k_16(v, e);
    // sub-block j = e / 2 sums the bsums of lanes 2j and 2j + 1
    const int bsum_pair = q.bsum + __shfl_xor(q.bsum, 1, 16);
    if (!valid) return;
    if (perm) {
        // values 16e .. 16e+15 = 64g + 32h + 8s .. for g = e/4, h = (e/2)&1, s = 2(e&1), 2(e&1)+1
        int8_t* dst = qs + item * 256 + 64 * (e >> 2) + 32 * (e & 1) + 8 * ((e >> 1) & 1);
        *reinterpret_cast<uint2*>(dst) = make_uint2(q.q[0], q.q[1]);
        *reinterpret_cast<uint2*>(dst + 16) = make_uint2(q.q[2], q.q[3]);
    } else {
        *reinterpret_cast<uint4*>(qs + item * 256 + 16 * e) = make_uint4(q.q[0], q.q[1], q.q[2], q.q[3]);
    }
    bs[item * 16 + e] = (int16_t)q.bsum;
    if (e == 0) d[item] = q.d;
    _Float16* m = reinterpret_cast<_Float16*>(mn + item * Q8MN_BYTES);
    if ((e & 1) == 0) {
        m[e >> 1] = (_Float16)(bsum_pair >> 5);       // hi_j, floor division (|BS_j| <= 4064)
        m[8 + (e >> 1)] = (_Float16)(bsum_pair & 31);  // lo_j
    }
    if (e == 1) *reinterpret_cast<float*>(mn + item * Q8MN_BYTES + 32) = q.d;
}

// Two integer sub-block sums of one lane against one staged activation block.
__device__ __forceinline__ void subblock_pair(const Nib& n, const int8_t* q8blk, int l4, int& S0, int& S1) {
    const int4* p = reinterpret_cast<const int4*>(q8blk + 64 * l4);
    const int4 a0 = p[0], a1 = p[1], b0 = p[2], b1 = p[3];
    int s = 0;
    s = dot4(n.lo[0], a0.x, s); s = dot4(n.lo[1], a0.y, s);
    s = dot4(n.lo[2], a0.z, s); s = dot4(n.lo[3], a0.w, s);
    s = dot4(n.lo[4], a1.x, s); s = dot4(n.lo[5], a1.y, s);
    s = dot4(n.lo[6], a1.z, s); s = dot4(n.lo[7], a1.w, s);
    int u = 0;
    u = dot4(n.hi[0], b0.x, u); u = dot4(n.hi[1], b0.y, u);
    u = dot4(n.hi[2], b0.z, u); u = dot4(n.hi[3], b0.w, u);
    u = dot4(n.hi[4], b1.x, u); u = dot4(n.hi[5], b1.y, u);
    u = dot4(n.hi[6], b1.z, u); u = dot4(n.hi[7], b1.w, u);
    S0 = s;
    S1 = u;
}

// Min-term integer: m0 * (bsums[4 l4] + bsums[4 l4 + 1]) + m1 * (bsums[4 l4 + 2] + bsums[4 l4 + 3]).
__device__ __forceinline__ int min_term(const int16_t* bsblk, int l4, int m0, int m1) {
    const uint2 v = *reinterpret_cast<const uint2*>(bsblk + 4 * l4);
    const int b0 = (int)(int16_t)(v.x & 0xFFFFu), b1 = (int)(int16_t)(v.x >> 16);
    const int b2 = (int)(int16_t)(v.y & 0xFFFFu), b3 = (int)(int16_t)(v.y >> 16);
    return m0 * (b0 + b1) + m1 * (b2 + b3);
}

// One block of one row against T staged activation rows.
template <int T>
__device__ __forceinline__ void block_dot(const W4& w, int l4, const Q8Lds& L, int bb, int CB, bool live,
                                          float (&acc)[T]) {
    const BlkC k = block_consts(w.hdr, l4);
    const Nib n = split_nibbles(w);
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

// Streams one row's super-blocks (this lane's share: blocks bsub, bsub + BPR,
// ... of each LDS chunk) against the staged activations and accumulates.
// Staging of chunk [c0, c0 + nblk) is split in two so that its global loads
// are issued before the weight prefetch: `pre(c0, nblk)` issues this lane's
// first activation loads and returns them in registers, `fin(c0, nblk, r)`
// turns them into the LDS slots [t * CB + 0 .. nblk) (whole workgroup, between
// barriers). Loads return in issue order, so an activation load queued behind
// the weight prefetch would stall staging until every weight byte had landed.
// Weight loads are software-pipelined in two register sets of U blocks;
// addresses are clamped in bounds and out-of-range blocks contribute zero.
// Fmt is the weight format (FmtQ4K below, FmtQ6K in q6k_core.h): its block
// size, lane loads and the per-block dot against staged activations.
template <typename Fmt, int T, int BPR, int U, typename PreFn, typename FinFn>
__device__ __forceinline__ void stream_row(const uint8_t* __restrict__ wrow, bool row_ok, int l4, int bsub, int nb,
                                           int CB, const Q8Lds& L, float (&acc)[T], PreFn pre, FinFn fin) {
    using W = typename Fmt::W;
    for (int c0 = 0; c0 < nb; c0 += CB) {
        const int nblk = min(nb, c0 + CB) - c0;
        const int niter = (nblk + BPR - 1) / BPR;   // same for every lane
        const uint8_t* __restrict__ wc = wrow + (size_t)c0 * Fmt::BYTES;
        auto blk_of = [&](int it) { return min(bsub + BPR * it, nblk - 1); };

        auto xr = pre(c0, nblk);
        W A[U], B[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (u < niter) A[u] = Fmt::load(wc + (size_t)blk_of(u) * Fmt::BYTES, l4);

        __syncthreads();  // previous chunk's LDS reads are done
        fin(c0, nblk, xr);
        __syncthreads();

        for (int i = 0; i < niter; i += 2 * U) {
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (i + U + u < niter) B[u] = Fmt::load(wc + (size_t)blk_of(i + U + u) * Fmt::BYTES, l4);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int it = i + u;
                if (it < niter) {
                    const int raw = bsub + BPR * it;
                    Fmt::template dot<T>(A[u], l4, L, min(raw, nblk - 1), CB, row_ok && raw < nblk, acc);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (i + 2 * U + u < niter) A[u] = Fmt::load(wc + (size_t)blk_of(i + 2 * U + u) * Fmt::BYTES, l4);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int it = i + U + u;
                if (it < niter) {
                    const int raw = bsub + BPR * it;
                    Fmt::template dot<T>(B[u], l4, L, min(raw, nblk - 1), CB, row_ok && raw < nblk, acc);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Register-resident activations (decode kernels). A lane that works on quarter
// l4 of block b for many rows keeps the Q8_K data that quarter needs in VGPRs:
//   a[0..7]  = q8[64 l4 + 0 .. 31]   (the low-nibble sub-block 2 l4)
//   a[8..15] = q8[64 l4 + 32 .. 63]  (the high-nibble sub-block 2 l4 + 1)
//   bsA = bsums[4 l4] + bsums[4 l4 + 1], bsB = bsums[4 l4 + 2] + bsums[4 l4 + 3]
struct Q8Reg {
    int a[16];
    int bsA, bsB;
    float d8;
};

__device__ __forceinline__ void load_q8reg(const Q8Lds& L, int b, int l4, Q8Reg& q) {
    const int4* p = reinterpret_cast<const int4*>(L.q8 + b * 256 + 64 * l4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int4 v = p[i];
        q.a[4 * i] = v.x; q.a[4 * i + 1] = v.y; q.a[4 * i + 2] = v.z; q.a[4 * i + 3] = v.w;
    }
    const uint2 bs = *reinterpret_cast<const uint2*>(L.bs + b * 16 + 4 * l4);
    q.bsA = (int)(int16_t)(bs.x & 0xFFFFu) + (int)(int16_t)(bs.x >> 16);
    q.bsB = (int)(int16_t)(bs.y & 0xFFFFu) + (int)(int16_t)(bs.y >> 16);
    q.d8 = L.d8[b];
}

// The two exact integer sub-block sums of quarter l4 of a block:
// S0 over sub-block 2 l4 (low nibbles), S1 over sub-block 2 l4 + 1 (high).
__device__ __forceinline__ void subblock_sums_reg(const W4& w, const int (&a)[16], int& S0, int& S1) {
    const uint32_t qq[8] = {w.qa.x, w.qa.y, w.qa.z, w.qa.w, w.qb.x, w.qb.y, w.qb.z, w.qb.w};
    int s = 0, u = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        s = dot4((int)(qq[i] & 0x0F0F0F0Fu), a[i], s);
        u = dot4((int)((qq[i] >> 4) & 0x0F0F0F0Fu), a[8 + i], u);
    }
    S0 = s;
    S1 = u;
}

// Scales and mins of sub-blocks 2 l4 and 2 l4 + 1 (get_scale_min_k4,
// ggml-quants.c:818-825) from the header words h.y, h.z, h.w.
__device__ __forceinline__ void scales_of_quarter(const uint4& h, int l4, int& sc0, int& sc1, int& m0, int& m1) {
    const int sh = 16 * (l4 & 1);
    const uint32_t s0 = h.y >> sh, s1 = h.z >> sh, s2 = h.w >> sh;
    uint32_t scp, mp;
    if (l4 < 2) {
        scp = s0 & 0x3F3Fu;
        mp = s1 & 0x3F3Fu;
    } else {
        scp = (s2 & 0x0F0Fu) | ((s0 >> 2) & 0x3030u);
        mp = ((s2 >> 4) & 0x0F0Fu) | ((s1 >> 2) & 0x3030u);
    }
    sc0 = (int)(scp & 0xFFu);
    sc1 = (int)((scp >> 8) & 0xFFu);
    m0 = (int)(mp & 0xFFu);
    m1 = (int)((mp >> 8) & 0xFFu);
}

// acc + this lane's share of ggml_vec_dot_q4_K_q8_K for one block:
// (d d8) (sc0 S0 + sc1 S1) - (dmin d8) (m0 bsA + m1 bsB), integers exact.
__device__ __forceinline__ float block_dot_reg(const W4& w, int l4, const Q8Reg& q, float acc) {
    const float d = half_bits_to_float(w.hdr.x & 0xFFFFu);
    const float dmin = half_bits_to_float(w.hdr.x >> 16);
    int sc0, sc1, m0, m1, S0, S1;
    scales_of_quarter(w.hdr, l4, sc0, sc1, m0, m1);
    subblock_sums_reg(w, q.a, S0, S1);
    // |S| <= 32 * 15 * 127 and sc <= 63: exact in 24-bit multiplies (full rate)
    const int A = __mul24(sc0, S0) + __mul24(sc1, S1);
    const int B = m0 * q.bsA + m1 * q.bsB;
    acc = fmaf(d * q.d8, (float)A, acc);
    acc = fmaf(-(dmin * q.d8), (float)B, acc);
    return acc;
}

template <int N>
struct RegWords {
    uint32_t v[N];
};

// Marks every register of the row buffers b as needed here, so that the
// compiler waits for their loads at this point (loads complete in order: the
// wait covers those loads and the ones before them, not the later ones).
template <int NIT, typename W>
__device__ __forceinline__ void arrived(const W (&b)[NIT]) {
    static_assert(sizeof(W) % 4 == 0, "row buffers are whole registers");
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const auto w = __builtin_bit_cast(RegWords<sizeof(W) / 4>, b[it]);
#pragma unroll
        for (int k = 0; k < (int)(sizeof(W) / 4); ++k) asm volatile("" ::"v"(w.v[k]));
    }
}

// Quantise activation blocks into LDS. Work items are (t, block) pairs,
// item i -> t = i / nblk, block kb0 + i % nblk. Each 16-lane row of a wave
// quantises one item per pass. X rows are 16-byte aligned (checked on host).
// stage_f32_load issues this lane's loads for the first pass; stage_f32_fin
// quantises them and runs any further passes.
struct XRegs {
    float x[16];
};

template <int WAVES>
__device__ __forceinline__ void stage_f32_item(int pass_base, int nitems, int nblk, int& t, int& bb, bool& valid) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int item0 = pass_base + wave * 4 + (lane >> 4);
    valid = item0 < nitems;
    const int item = valid ? item0 : nitems - 1;   // clamp: in-bounds, result discarded
    t = item / nblk;
    bb = item - t * nblk;
}

__device__ __forceinline__ XRegs load_x16(const float* __restrict__ X, int64_t x_tstride, int t, int kb) {
    XRegs r;
    const int e = threadIdx.x & 15;
    const float4* src = reinterpret_cast<const float4*>(X + (int64_t)t * x_tstride + (int64_t)kb * QK + 16 * e);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 v = src[i];
        r.x[4 * i + 0] = v.x; r.x[4 * i + 1] = v.y; r.x[4 * i + 2] = v.z; r.x[4 * i + 3] = v.w;
    }
    return r;
}

__device__ __forceinline__ void store_q8_item(const XRegs& r, bool valid, int slot, const Q8Lds& L) {
    const int e = threadIdx.x & 15;
    const Q8Lane q = quantize_q8k_16(r.x, e);
    if (valid) {
        *reinterpret_cast<uint4*>(L.q8 + slot * 256 + 16 * e) = make_uint4(q.q[0], q.q[1], q.q[2], q.q[3]);
        L.bs[slot * 16 + e] = (int16_t)q.bsum;
        if (e == 0) L.d8[slot] = q.d;
    }
}

template <int WAVES>
__device__ __forceinline__ XRegs stage_f32_load(const float* __restrict__ X, int64_t x_tstride, int T, int kb0,
                                                int nblk) {
    int t, bb;
    bool valid;
    stage_f32_item<WAVES>(0, T * nblk, nblk, t, bb, valid);
    return load_x16(X, x_tstride, t, kb0 + bb);
}

template <int WAVES>
__device__ __forceinline__ void stage_f32_fin(const float* __restrict__ X, int64_t x_tstride, int T, int kb0,
                                              int nblk, const Q8Lds& L, int slot_stride, const XRegs& first) {
    const int nitems = T * nblk;
    int t, bb;
    bool valid;
    stage_f32_item<WAVES>(0, nitems, nblk, t, bb, valid);
    store_q8_item(first, valid, t * slot_stride + bb, L);
    for (int base = 4 * WAVES; base < nitems; base += 4 * WAVES) {
        stage_f32_item<WAVES>(base, nitems, nblk, t, bb, valid);
        const XRegs r = load_x16(X, x_tstride, t, kb0 + bb);
        store_q8_item(r, valid, t * slot_stride + bb, L);
    }
}

template <int WAVES>
__device__ __forceinline__ void stage_q8_from_f32(const float* __restrict__ X, int64_t x_tstride, int T, int kb0,
                                                  int nblk, const Q8Lds& L, int slot_stride) {
    stage_f32_fin<WAVES>(X, x_tstride, T, kb0, nblk, L, slot_stride, stage_f32_load<WAVES>(X, x_tstride, T, kb0, nblk));
}

// Copy Q8_K planes [t][kb0 .. kb0+nblk) into the LDS layout.
template <int NT>
__device__ __forceinline__ void stage_q8_from_planes(const Q8Planes& P, int nb, int T, int kb0, int nblk,
                                                     const Q8Lds& L, int slot_stride) {
    const int tid = threadIdx.x;
    for (int t = 0; t < T; ++t) {
        // qs: nblk*256 bytes, 16 B per thread per step
        const uint4* s = reinterpret_cast<const uint4*>(P.qs + ((int64_t)t * nb + kb0) * 256);
        uint4* d = reinterpret_cast<uint4*>(L.q8 + t * slot_stride * 256);
        for (int i = tid; i < nblk * 16; i += NT) d[i] = s[i];
        // bsums: nblk*32 bytes, 4 B per thread per step
        const uint32_t* sb = reinterpret_cast<const uint32_t*>(P.bs + ((int64_t)t * nb + kb0) * 16);
        uint32_t* db = reinterpret_cast<uint32_t*>(L.bs + t * slot_stride * 16);
        for (int i = tid; i < nblk * 8; i += NT) db[i] = sb[i];
        const float* sd = P.d + (int64_t)t * nb + kb0;
        for (int i = tid; i < nblk; i += NT) L.d8[t * slot_stride + i] = sd[i];
    }
}

// ---------------------------------------------------------------------------
// Weight-format policy of Q4_K for the kernels shared with other formats
// (stream_row, the decode kernels): block bytes, a lane's loads, the
// register-activation dot and the LDS-activation dot over T tokens.
struct FmtQ4K {
    static constexpr int BYTES = Q4K_BYTES;
    using W = W4;
    using R = Q8Reg;
    static __device__ __forceinline__ W load(const uint8_t* blk, int l4) { return load_w4(blk, l4); }
    static __device__ __forceinline__ void load_reg(const Q8Lds& L, int b, int l4, R& q) { load_q8reg(L, b, l4, q); }
    static __device__ __forceinline__ float dot_reg(const W& w, int l4, const R& q, float acc) {
        return block_dot_reg(w, l4, q, acc);
    }
    template <int T>
    static __device__ __forceinline__ void dot(const W& w, int l4, const Q8Lds& L, int bb, int CB, bool live,
                                               float (&acc)[T]) {
        block_dot<T>(w, l4, L, bb, CB, live, acc);
    }
};

}  // namespace spq4k
