// k_moe.hip — expert-gathered Q4_K matvec (GGML_OP_MUL_MAT_ID) on gfx950.
//
// Semantics of ggml_compute_forward_mul_mat_id
// (vendor/ggml/src/ggml-cpu/ggml-cpu.c:1441-1511, 1521-1690): for token t and
// slot s the expert is ids[t][s], its input row is X[t][s % ne11] quantised to
// Q8_K, and Y[t][s][r] = row r of that expert . Q8_K(input). Like the CPU
// driver (ggml-cpu.c:1609-1626), (token, slot) pairs are grouped by expert so
// that each selected expert's weights are streamed once per call, whatever
// the number of tokens routed to it.
//
//   1. moe_route_kernel (one workgroup): per-expert counts, an exclusive scan,
//      the compacted list of active experts and, per expert, its pairs in
//      (token, slot) order. Out-of-range ids are not routed (their outputs are
//      left untouched; the host entry points reject them).
//   2. quantize_q8k_planes_kernel: the T*ne11 input rows to Q8_K planes.
//   3. moe_gemv_kernel: workgroup (a, tile) takes active expert a and a tile
//      of its rows; its pairs are processed TC at a time, each chunk staged
//      from the Q8_K planes into LDS and streamed with the dense GEMV's code.
#include "gemv_core.h"
#include "launch.h"

namespace spq4k {

__global__ __launch_bounds__(256) void moe_route_kernel(const int32_t* __restrict__ ids, int n_pairs, int E,
                                                        MoeRoute r) {
    extern __shared__ int sh[];   // cnt[E], off[E]
    int* cnt = sh;
    int* off = sh + E;
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        int c = 0;
        for (int i = 0; i < n_pairs; ++i) c += (ids[i] == e);
        cnt[e] = c;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0, act = 0;
        for (int e = 0; e < E; ++e) {
            off[e] = run;
            run += cnt[e];
            if (cnt[e] > 0) {
                r.act[act] = e;
                r.act_off[act] = off[e];
                r.act_cnt[act] = cnt[e];
                ++act;
            }
        }
        *r.n_act = act;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        if (cnt[e] == 0) continue;
        int p = off[e];
        for (int i = 0; i < n_pairs; ++i)
            if (ids[i] == e) r.pairs[p++] = i;
    }
}

template <int TC, int BPR, int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void moe_gemv_kernel(MoeParams p) {
    extern __shared__ __align__(16) char smem[];
    constexpr int LPR = 4 * BPR;
    constexpr int RPW = 64 / LPR;
    constexpr int ROWS = WAVES * RPW;

    const int a = blockIdx.x / p.tiles_per_expert;
    const int tile = blockIdx.x - a * p.tiles_per_expert;
    if (a >= *p.route.n_act) return;           // uniform over the workgroup
    const int e = p.route.act[a];
    const int poff = p.route.act_off[a];
    const int pcnt = p.route.act_cnt[a];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int l4 = lane & 3;
    const int bsub = (lane >> 2) & (BPR - 1);
    const int M = p.M;
    const int row = tile * ROWS + wave * RPW + lane / LPR;
    const bool row_ok = row < M;
    const int nb = p.nb;
    const size_t row_bytes = (size_t)nb * Q4K_BYTES;
    const uint8_t* __restrict__ wrow =
        p.bank + (size_t)e * p.expert_bytes + (size_t)(row_ok ? row : M - 1) * row_bytes;

    const int CB = p.chunk_blocks;
    const Q8Lds L = q8lds_carve(smem, TC * CB);
    __shared__ int s_q8row[TC];
    __shared__ int s_pair[TC];

    for (int c = 0; c < pcnt; c += TC) {
        const int nt = min(TC, pcnt - c);
        __syncthreads();   // the previous chunk's readers of s_pair are done
        if (threadIdx.x < TC) {
            const int i = min((int)threadIdx.x, nt - 1);   // clamp: duplicate slots are computed, not stored
            const int pair = p.route.pairs[poff + c + i];
            const int t = pair / p.n_used;
            const int s = pair - t * p.n_used;
            s_pair[threadIdx.x] = pair;
            s_q8row[threadIdx.x] = t * p.ne11 + (s % p.ne11);
        }
        __syncthreads();
        float acc[TC];
#pragma unroll
        for (int t = 0; t < TC; ++t) acc[t] = 0.0f;
        stream_row<TC, BPR, U>(wrow, row_ok, l4, bsub, nb, CB, L, acc, [&](int, int) { return 0; },
                               [&](int c0, int nblk, int) {
            // copy the chunk's Q8_K rows (planes) into LDS slots t * CB + b
            for (int t = 0; t < TC; ++t) {
                const int q8r = s_q8row[t];
                const uint4* s = reinterpret_cast<const uint4*>(p.Q.qs + ((int64_t)q8r * nb + c0) * 256);
                uint4* d = reinterpret_cast<uint4*>(L.q8 + t * CB * 256);
                for (int i = threadIdx.x; i < nblk * 16; i += WAVES * 64) d[i] = s[i];
                const uint32_t* sb = reinterpret_cast<const uint32_t*>(p.Q.bs + ((int64_t)q8r * nb + c0) * 16);
                uint32_t* db = reinterpret_cast<uint32_t*>(L.bs + t * CB * 16);
                for (int i = threadIdx.x; i < nblk * 8; i += WAVES * 64) db[i] = sb[i];
                const float* sd = p.Q.d + (int64_t)q8r * nb + c0;
                for (int i = threadIdx.x; i < nblk; i += WAVES * 64) L.d8[t * CB + i] = sd[i];
            }
        });
#pragma unroll
        for (int t = 0; t < TC; ++t) acc[t] = group_sum_last<LPR>(acc[t]);
        if (row_ok && (lane & (LPR - 1)) == LPR - 1) {
#pragma unroll
            for (int t = 0; t < TC; ++t)
                if (t < nt) p.Y[(int64_t)s_pair[t] * M + row] = acc[t];
        }
    }
}

// ---------------------------------------------------------------------------
hipError_t launch_moe_route(const int32_t* ids, int n_pairs, int E, const MoeRoute& r, hipStream_t st) {
    hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(256), (size_t)2 * E * sizeof(int), st, ids, n_pairs, E, r);
    return hipGetLastError();
}

template <int TC, int BPR>
static hipError_t launch_moe_tb(const MoeParams& p, int grid, hipStream_t st) {
    constexpr int WAVES = 4, U = 2;
    const size_t lds = (size_t)q8lds_bytes(TC * p.chunk_blocks);
    hipLaunchKernelGGL((moe_gemv_kernel<TC, BPR, WAVES, U>), dim3(grid), dim3(WAVES * 64), lds, st, p);
    return hipGetLastError();
}

template <int TC>
static hipError_t launch_moe_t(const MoeParams& p, int bpr, int grid, hipStream_t st) {
    switch (bpr) {
        case 1: return launch_moe_tb<TC, 1>(p, grid, st);
        case 2: return launch_moe_tb<TC, 2>(p, grid, st);
        case 4: return launch_moe_tb<TC, 4>(p, grid, st);
        case 8: return launch_moe_tb<TC, 8>(p, grid, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_gemv(const MoeParams& p, int tc, int bpr, int grid, hipStream_t st) {
    switch (tc) {
        case 1: return launch_moe_t<1>(p, bpr, grid, st);
        case 2: return launch_moe_t<2>(p, bpr, grid, st);
        case 4: return launch_moe_t<4>(p, bpr, grid, st);
        case 8: return launch_moe_t<8>(p, bpr, grid, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace spq4k
