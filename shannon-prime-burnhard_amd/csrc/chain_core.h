// chain_core.h — building blocks shared by the persistent decode-chain
// kernels (k_chain.hip, k_chain2.hip): agent-coherent scalar access, the
// window piece (one lane's share of a Q4_K block) and its dot product, and the
// lane-major Q8_K activation layout the compute waves read.
#pragma once

#include "gemv_core.h"
#include "launch.h"

namespace spq4k {
namespace {

constexpr int CH_MAXIT = CHAIN_MAX_NB / 16;    // block-quarters a lane per row
constexpr unsigned CH_SPIN = 1u << 20;         // polls before a wait gives up
static_assert(CH_MAXIT == 3, "the consume step selects among three activation register sets");


__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) float gfloat;

// agent-coherent store (global_store sc1) through a global-address-space
// pointer (a generic pointer would make it a flat store)
__device__ __forceinline__ void st_agent(float* p, float v) {
    __hip_atomic_store((gfloat*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// n floats (n a multiple of 256) from global memory into LDS, agent-coherent,
// 1 KB an instruction; the caller waits (vmcnt) before the data is read
__device__ __forceinline__ void stage_vec_lds(const float* __restrict__ src, float* dst, int n) {
    const int lane = threadIdx.x & 63;
    for (int j = 0; j < n; j += 256)
        __builtin_amdgcn_global_load_lds((const void*)(src + j + 4 * lane), (lds_void*)(dst + j), 16, 0,
                                         /*sc1*/ 16);
}

__device__ __forceinline__ void barrier_lds() {
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's LDS writes done
    __builtin_amdgcn_s_barrier();
}

// silu(x) = x / (1 + e^-x) (ggml_silu_f32, ggml-cpu/vec.h:1064-1066)
__device__ __forceinline__ float chain_silu(float x) { return x / (1.0f + expf(-x)); }

// rows of a stage of `rows` rows that compute wave g (of G) owns: g, g + G, ...
__device__ __forceinline__ int rows_of(int rows, int g, int G) { return g < rows ? (rows - 1 - g) / G + 1 : 0; }

// ---------------------------------------------------------------------------
// compute-wave helpers
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// One lane's share of a block for the window: the quad of lanes with the
// same bsub reads the block's 144 bytes exactly once -- lane l4 the header
// dword l4 (d | dmin, then the three scale words) and the 32 qs bytes of
// quarter l4. The header is shared across the quad by DPP when the piece is
// consumed (doing it at load time would wait for the load).
struct Piece {
    uint32_t h;
    u32x4 qa, qb;
};

__device__ __forceinline__ Piece load_piece(const uint8_t* blk, int l4) {
    // global-address-space loads of plain vector types: a generic pointer
    // (or a class type's copy through a generic reference) gives flat
    // loads, which also count against lgkmcnt
    typedef __attribute__((address_space(1))) const uint32_t gu32;
    typedef __attribute__((address_space(1))) const u32x4 gu32x4;
    Piece w;
    w.h = *(gu32*)(blk + 4 * l4);
    const gu32x4* q = (gu32x4*)(blk + 16 + 32 * l4);
    w.qa = q[0];
    w.qb = q[1];
    return w;
}

template <int CTRL>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}

// acc + this lane's share of ggml_vec_dot_q4_K_q8_K for the piece's block
// (block_dot_reg on the reassembled W4)
__device__ __forceinline__ float piece_dot(const Piece& p, int l4, const Q8Reg& q, float acc) {
    W4 w;
    w.hdr.x = quad_bcast<0x00>(p.h);   // quad_perm [0,0,0,0]
    w.hdr.y = quad_bcast<0x55>(p.h);   // [1,1,1,1]
    w.hdr.z = quad_bcast<0xAA>(p.h);   // [2,2,2,2]
    w.hdr.w = quad_bcast<0xFF>(p.h);   // [3,3,3,3]
    w.qa = make_uint4(p.qa.x, p.qa.y, p.qa.z, p.qa.w);
    w.qb = make_uint4(p.qb.x, p.qb.y, p.qb.z, p.qb.w);
    return block_dot_reg(w, l4, q, acc);
}

// Q8_K activations in LDS, lane-major: for pass it (blocks 16 it .. 16 it + 15)
// a region of CH_Q8L_PASS bytes holding, for lane L = 4 bsub + l4, the 64
// bytes q8[64 l4 .. 64 l4 + 63] of block 16 it + bsub as four 1 KB planes
// (plane k at k * 1024 + 16 L) and then {bsA, bsB, d8, 0} at 4096 + 16 L,
// bsA = bsums[4 l4] + bsums[4 l4 + 1], bsB = bsums[4 l4 + 2] + bsums[4 l4 + 3].
// A wave reads a piece's activations as five conflict-free 16-byte reads a
// lane at a uniform offset, so the pass of a piece is an address, not a
// choice among register sets.
constexpr int CH_Q8L_PASS = 5 * 1024;
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i32x4 lint4;

__device__ __forceinline__ void q8l_read(const char* q8l_gen, int it, int lane, Q8Reg& q) {
    const __attribute__((address_space(3))) char* base =
        (const __attribute__((address_space(3))) char*)q8l_gen + it * CH_Q8L_PASS + 16 * lane;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const i32x4 v = *(const lint4*)(base + 1024 * k);
        q.a[4 * k] = v.x; q.a[4 * k + 1] = v.y; q.a[4 * k + 2] = v.z; q.a[4 * k + 3] = v.w;
    }
    const i32x4 m = *(const lint4*)(base + 4096);
    q.bsA = m.x;
    q.bsB = m.y;
    q.d8 = __int_as_float(m.z);
}

// Quantise block b of x (this 16-lane row holds values 16 e .. 16 e + 15,
// e = lane & 15) to Q8_K (quantize_q8k_16: quantize_row_q8_K_ref bit for
// bit) and store it in the lane-major layout.
__device__ __forceinline__ void q8l_store_block(const XRegs& r, bool valid, int b, char* q8l_gen) {
    const int e = threadIdx.x & 15;
    const Q8Lane q = quantize_q8k_16(r.x, e);
    // bsums of the sub-block pairs: lanes e = 4 l4 hold bsA, fetch bsB from e + 2
    const int pair = q.bsum + __shfl_xor(q.bsum, 1, 16);
    const int pair2 = __shfl_xor(pair, 2, 16);
    if (!valid) return;
    __attribute__((address_space(3))) char* base = (__attribute__((address_space(3))) char*)q8l_gen +
                                                   (b >> 4) * CH_Q8L_PASS + 16 * (4 * (b & 15) + (e >> 2));
    *(lint4*)(base + 1024 * (e & 3)) = i32x4{(int)q.q[0], (int)q.q[1], (int)q.q[2], (int)q.q[3]};
    if ((e & 3) == 0) *(lint4*)(base + 4096) = i32x4{pair, pair2, __float_as_int(q.d), 0};
}

__device__ __forceinline__ int ufl(int v) { return __builtin_amdgcn_readfirstlane(v); }

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) const f32x4 lfloat4;

}  // namespace
}  // namespace spq4k
