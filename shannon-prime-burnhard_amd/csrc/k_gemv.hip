// k_gemv.hip — fused Q4_K GEMV for decode (T <= 8 tokens) on gfx950.
//
// Replaces, for GGML_TYPE_Q4_K, the work of ggml_compute_forward_mul_mat
// (vendor/ggml/src/ggml-cpu/ggml-cpu.c:1241-1439: Q8_K conversion of src1, then
// ggml_vec_dot_q4_K_q8_K per output) and of the CUDA backend's
// quantize_q8_1 + mul_mat_vec_q<Q4_K> (ggml-cuda/mmvq.cu:393, quantize.cu:4),
// with the CPU path's Q8_K numerics.
//
// One launch covers up to four weight matrices that share the same input
// (e.g. q/k/v or gate/up). Work unit = (row tile of 16*WAVES rows, K split):
//   1. the workgroup issues the weight loads of its first blocks,
//   2. quantises its K range of the T input rows to Q8_K into LDS,
//   3. streams its rows' 144 B blocks and accumulates per lane in fp32,
//   4. reduces the four lanes of each row; with one K split it stores y,
//      otherwise it stores a partial and the last workgroup of the tile
//      (atomic arrival counter) sums the partials in split order and stores y.
// The arrival counter is reset by that last workgroup, so no per-launch clear
// is needed and the result does not depend on workgroup timing.
#include "gemv_core.h"
#include "launch.h"

namespace spq4k {

template <int T, int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void gemv_q4k_kernel(GemvParams p) {
    extern __shared__ __align__(16) char smem[];
    constexpr int ROWS = WAVES * 16;

    const int wg = blockIdx.x;
    const int tile = wg / p.ksplit;
    const int split = wg - tile * p.ksplit;

    // segment of this tile
    int sidx = 0;
#pragma unroll
    for (int s = 1; s < GEMV_MAX_SEG; ++s)
        if (s < p.nseg && tile >= p.seg[s].tile_begin) sidx = s;
    const uint8_t* __restrict__ W = p.seg[sidx].W;
    float* __restrict__ Y = p.seg[sidx].Y;
    const int M = p.seg[sidx].M;
    const int64_t y_tstride = p.seg[sidx].y_tstride;
    const int row0 = (tile - p.seg[sidx].tile_begin) * ROWS;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int l4 = lane & 3;
    const int grp = lane >> 2;
    const int row = row0 + wave * 16 + grp;
    const bool row_ok = row < M;

    const int nb = p.nb;
    const int kb0 = split * p.kb_per_split;
    const int kb1 = min(nb, kb0 + p.kb_per_split);
    const size_t row_bytes = (size_t)nb * Q4K_BYTES;
    const uint8_t* __restrict__ wrow = W + (size_t)(row_ok ? row : 0) * row_bytes;

    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.0f;

    const int CB = p.chunk_blocks;
    const Q8Lds L = q8lds_carve(smem, T * CB);

    for (int c0 = kb0; c0 < kb1; c0 += CB) {
        const int c1 = min(kb1, c0 + CB);
        const int nblk = c1 - c0;

        // prefetch the first U blocks of the chunk, then stage activations
        W4 wr[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            wr[u] = (row_ok && u < nblk) ? load_w4(wrow + (size_t)(c0 + u) * Q4K_BYTES, l4) : zero_w4();

        __syncthreads();  // previous chunk's LDS reads are done
        stage_q8<WAVES>(p.X, p.x_tstride, T, c0, nblk, L, CB);
        __syncthreads();

        for (int b = 0; b < nblk; b += U) {
            W4 cur[U];
#pragma unroll
            for (int u = 0; u < U; ++u) cur[u] = wr[u];
            // issue the next group's loads before using this one
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int nbk = b + U + u;
                wr[u] = (row_ok && nbk < nblk) ? load_w4(wrow + (size_t)(c0 + nbk) * Q4K_BYTES, l4) : zero_w4();
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int bb = b + u;
                if (bb < nblk) {
                    const BlkC k = block_consts(cur[u].hdr, l4);
                    const Nib n = split_nibbles(cur[u]);
#pragma unroll
                    for (int t = 0; t < T; ++t) {
                        const int slot = t * CB + bb;
                        int S0, S1;
                        subblock_pair(n, L.q8 + slot * 256, l4, S0, S1);
                        const int A = k.sc0 * S0 + k.sc1 * S1;
                        const int B = min_term(L.bs + slot * 16, l4, k.m0, k.m1);
                        const float d8 = L.d8[slot];
                        acc[t] = fmaf(k.d * d8, (float)A, acc[t]);
                        acc[t] = fmaf(-(k.dmin * d8), (float)B, acc[t]);
                    }
                }
            }
        }
    }

    // reduce the four lanes of each row
#pragma unroll
    for (int t = 0; t < T; ++t) {
        acc[t] += __shfl_xor(acc[t], 1, 64);
        acc[t] += __shfl_xor(acc[t], 2, 64);
    }

    if (p.ksplit == 1) {
        if (row_ok && l4 == 0) {
#pragma unroll
            for (int t = 0; t < T; ++t) Y[(int64_t)t * y_tstride + row] = acc[t];
        }
        return;
    }

    // split-K: partial[tile][split][t][ROWS]
    float* part = p.partial + ((size_t)tile * p.ksplit + split) * (size_t)(T * ROWS);
    const int rit = wave * 16 + grp;
    if (l4 == 0) {
#pragma unroll
        for (int t = 0; t < T; ++t) part[t * ROWS + rit] = acc[t];
    }
    __threadfence();
    __syncthreads();
    __shared__ int s_last;
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(p.counters + tile, 1u, __ATOMIC_ACQ_REL,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == (unsigned)(p.ksplit - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const float* tbase = p.partial + (size_t)tile * p.ksplit * (size_t)(T * ROWS);
    for (int i = threadIdx.x; i < T * ROWS; i += WAVES * 64) {
        const int t = i / ROWS;
        const int r = row0 + (i - t * ROWS);
        float s = 0.0f;
        for (int sp = 0; sp < p.ksplit; ++sp)
            s += __builtin_nontemporal_load(tbase + (size_t)sp * (T * ROWS) + i);
        if (r < M) Y[(int64_t)t * y_tstride + r] = s;
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(p.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Diagnostic: the exact integer sub-block sums S[row][b][j] exactly as the GEMV
// lanes form them (same loads, unpacking and dot products), for one Q8_K row.
template <int WAVES>
__global__ __launch_bounds__(WAVES * 64) void subblock_sums_kernel(const uint8_t* __restrict__ W, int M,
                                                                   int nb, const float* __restrict__ X,
                                                                   int32_t* __restrict__ S, int CB) {
    extern __shared__ __align__(16) char smem[];
    constexpr int ROWS = WAVES * 16;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int l4 = lane & 3;
    const int row = blockIdx.x * ROWS + wave * 16 + (lane >> 2);
    const bool row_ok = row < M;
    const Q8Lds L = q8lds_carve(smem, CB);
    for (int c0 = 0; c0 < nb; c0 += CB) {
        const int nblk = min(nb, c0 + CB) - c0;
        __syncthreads();
        stage_q8<WAVES>(X, 0, 1, c0, nblk, L, CB);
        __syncthreads();
        if (!row_ok) continue;
        for (int bb = 0; bb < nblk; ++bb) {
            const W4 w = load_w4(W + ((size_t)row * nb + c0 + bb) * Q4K_BYTES, l4);
            const Nib n = split_nibbles(w);
            int S0, S1;
            subblock_pair(n, L.q8 + bb * 256, l4, S0, S1);
            int32_t* o = S + ((size_t)row * nb + c0 + bb) * 8 + 2 * l4;
            o[0] = S0;
            o[1] = S1;
        }
    }
}

// ---------------------------------------------------------------------------
template <int T, int WAVES>
static hipError_t launch_t(const GemvParams& p, int ntiles, hipStream_t st) {
    const size_t lds = (size_t)q8lds_bytes(T * p.chunk_blocks);
    hipLaunchKernelGGL((gemv_q4k_kernel<T, WAVES, 2>), dim3(ntiles * p.ksplit), dim3(WAVES * 64), lds, st, p);
    return hipGetLastError();
}

hipError_t launch_gemv(const GemvParams& p, int T, int waves, int ntiles, hipStream_t st) {
#define SPQ_CASE(TT)                                                   \
    case TT:                                                           \
        return waves == 2 ? launch_t<TT, 2>(p, ntiles, st) : launch_t<TT, 4>(p, ntiles, st);
    switch (T) {
        SPQ_CASE(1) SPQ_CASE(2) SPQ_CASE(3) SPQ_CASE(4)
        SPQ_CASE(5) SPQ_CASE(6) SPQ_CASE(7) SPQ_CASE(8)
        default: return hipErrorInvalidValue;
    }
#undef SPQ_CASE
}

hipError_t launch_subblock_sums(const uint8_t* W, int M, int nb, const float* X, int32_t* S, hipStream_t st) {
    constexpr int WAVES = 4;
    const int CB = nb < 64 ? nb : 64;
    const size_t lds = (size_t)q8lds_bytes(CB);
    const int grid = (M + WAVES * 16 - 1) / (WAVES * 16);
    hipLaunchKernelGGL((subblock_sums_kernel<WAVES>), dim3(grid), dim3(WAVES * 64), lds, st, W, M, nb, X, S, CB);
    return hipGetLastError();
}

}  // namespace spq4k
