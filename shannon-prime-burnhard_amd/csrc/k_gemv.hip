// k_gemv.hip — fused Q4_K GEMV for decode (T <= 8 tokens) on gfx950.
//
// Replaces, for GGML_TYPE_Q4_K, the work of ggml_compute_forward_mul_mat
// (vendor/ggml/src/ggml-cpu/ggml-cpu.c:1241-1439: Q8_K conversion of src1, then
// ggml_vec_dot_q4_K_q8_K per output) and of the CUDA backend's
// quantize_q8_1 + mul_mat_vec_q<Q4_K> (ggml-cuda/mmvq.cu:393, quantize.cu:4),
// with the CPU path's Q8_K numerics.
//
// One launch covers up to four weight matrices that share the same input
// (q/k/v or gate/up). A workgroup of WAVES waves owns WAVES * 16/BPR rows and
// the whole K range:
//   - 4*BPR lanes work on one row; lane (bsub, l4) takes blocks
//     b = bsub, bsub + BPR, ... and within each block the 32 qs bytes of
//     quarter l4 (two whole sub-blocks; see gemv_core.h);
//   - the workgroup first issues the loads of its first U blocks per lane,
//     then quantises the T input rows to Q8_K into LDS while they are in
//     flight, then streams the rest of its rows with U blocks of loads in
//     flight per lane;
//   - the 4*BPR lane partials of a row are combined by a butterfly and
//     stored. No cross-workgroup traffic, no atomics: the result depends
//     only on the inputs.
// BPR trades rows per workgroup against redundant activation quantisation:
// the host picks it so that small matrices still launch >= 2 workgroups
// per CU and large ones quantise x as few times as possible.
#include "gemv_core.h"
#include "launch.h"

namespace spq4k {

template <int T, int BPR, int WAVES, int U, bool PREQ>
__global__ __launch_bounds__(WAVES * 64) void gemv_q4k_kernel(GemvParams p) {
    extern __shared__ __align__(16) char smem[];
    constexpr int LPR = 4 * BPR;         // lanes per row
    constexpr int RPW = 64 / LPR;        // rows per wave
    constexpr int ROWS = WAVES * RPW;    // rows per workgroup

    const int tile = blockIdx.x;
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
    const int bsub = (lane >> 2) & (BPR - 1);
    const int row = row0 + wave * RPW + lane / LPR;
    const bool row_ok = row < M;

    const int nb = p.nb;
    const size_t row_bytes = (size_t)nb * Q4K_BYTES;
    // rows past M re-read row M-1 (in bounds) and contribute nothing
    const uint8_t* __restrict__ wrow = W + (size_t)(row_ok ? row : M - 1) * row_bytes;

    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.0f;

    const int CB = p.chunk_blocks;
    const Q8Lds L = q8lds_carve(smem, T * CB);
    if (PREQ) {
        stream_row<T, BPR, U>(
            wrow, row_ok, l4, bsub, nb, CB, L, acc, [&](int, int) { return 0; },
            [&](int c0, int nblk, int) { stage_q8_from_planes<WAVES * 64>(p.Q, nb, T, c0, nblk, L, CB); });
    } else {
        stream_row<T, BPR, U>(
            wrow, row_ok, l4, bsub, nb, CB, L, acc,
            [&](int c0, int nblk) { return stage_f32_load<WAVES>(p.X, p.x_tstride, T, c0, nblk); },
            [&](int c0, int nblk, const XRegs& xr) {
                stage_f32_fin<WAVES>(p.X, p.x_tstride, T, c0, nblk, L, CB, xr);
            });
    }

    // reduce the LPR lanes of each row (DPP, fixed order: deterministic)
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = group_sum_last<LPR>(acc[t]);
    if (row_ok && (lane & (LPR - 1)) == LPR - 1) {
#pragma unroll
        for (int t = 0; t < T; ++t) Y[(int64_t)t * y_tstride + row] = acc[t];
    }
}

// T = 1 decode kernel specialised on the number of blocks per row (see
// stream_row_fixed); same tiling, lane mapping and arithmetic as above.
template <int NB, int BPR, int WAVES, int D>
__global__ __launch_bounds__(WAVES * 64) void gemv_q4k_fixed_kernel(GemvParams p) {
    __shared__ __align__(16) char smem[q8lds_bytes(NB)];
    constexpr int LPR = 4 * BPR;
    constexpr int RPW = 64 / LPR;
    constexpr int ROWS = WAVES * RPW;
    const int tile = blockIdx.x;
    int sidx = 0;
#pragma unroll
    for (int s = 1; s < GEMV_MAX_SEG; ++s)
        if (s < p.nseg && tile >= p.seg[s].tile_begin) sidx = s;
    const uint8_t* __restrict__ W = p.seg[sidx].W;
    float* __restrict__ Y = p.seg[sidx].Y;
    const int M = p.seg[sidx].M;
    const int row0 = (tile - p.seg[sidx].tile_begin) * ROWS;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int l4 = lane & 3;
    const int bsub = (lane >> 2) & (BPR - 1);
    const int row = row0 + wave * RPW + lane / LPR;
    const bool row_ok = row < M;
    const uint8_t* __restrict__ wrow = W + (size_t)(row_ok ? row : M - 1) * (NB * Q4K_BYTES);
    const Q8Lds L = q8lds_carve(smem, NB);
    float acc = stream_row_fixed<NB, BPR, D, WAVES>(wrow, row_ok, l4, bsub, p.X, L);
    acc = group_sum_last<LPR>(acc);
    if (row_ok && (lane & (LPR - 1)) == LPR - 1) Y[row] = acc;
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
        stage_q8_from_f32<WAVES>(X, 0, 1, c0, nblk, L, CB);
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
template <int T, int BPR, bool PREQ>
static hipError_t launch_tb(const GemvParams& p, int ntiles, hipStream_t st) {
    constexpr int WAVES = 4;
    constexpr int U = 2;
    const size_t lds = (size_t)q8lds_bytes(T * p.chunk_blocks);
    hipLaunchKernelGGL((gemv_q4k_kernel<T, BPR, WAVES, U, PREQ>), dim3(ntiles), dim3(WAVES * 64), lds, st, p);
    return hipGetLastError();
}

template <int T, bool PREQ>
static hipError_t launch_t(const GemvParams& p, int bpr, int ntiles, hipStream_t st) {
    switch (bpr) {
        case 1: return launch_tb<T, 1, PREQ>(p, ntiles, st);
        case 2: return launch_tb<T, 2, PREQ>(p, ntiles, st);
        case 4: return launch_tb<T, 4, PREQ>(p, ntiles, st);
        case 8: return launch_tb<T, 8, PREQ>(p, ntiles, st);
        default: return hipErrorInvalidValue;
    }
}

int gemv_rows_per_tile(int bpr) { return 4 * (64 / (4 * bpr)); }

template <int NB>
static hipError_t launch_fixed(const GemvParams& p, int bpr, int ntiles, hipStream_t st) {
    constexpr int WAVES = 4, D = 4;
    switch (bpr) {
        case 1: hipLaunchKernelGGL((gemv_q4k_fixed_kernel<NB, 1, WAVES, D>), dim3(ntiles), dim3(256), 0, st, p); break;
        case 2: hipLaunchKernelGGL((gemv_q4k_fixed_kernel<NB, 2, WAVES, D>), dim3(ntiles), dim3(256), 0, st, p); break;
        case 4: hipLaunchKernelGGL((gemv_q4k_fixed_kernel<NB, 4, WAVES, D>), dim3(ntiles), dim3(256), 0, st, p); break;
        case 8: hipLaunchKernelGGL((gemv_q4k_fixed_kernel<NB, 8, WAVES, D>), dim3(ntiles), dim3(256), 0, st, p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv(const GemvParams& p, int T, int bpr, int ntiles, hipStream_t st) {
    const bool pq = p.Q.qs != nullptr;
    // decode fast path: one token, activations quantised on chip, the K of
    // the 8B-class shapes (4096 and 12288) known at compile time
    // (the fully unrolled variants with few lanes per row need too many
    // registers; those shapes have enough rows for the generic kernel)
    if (T == 1 && !pq && p.fixed_ok) {
        if (p.nb == 16 && bpr >= 2) return launch_fixed<16>(p, bpr, ntiles, st);
        if (p.nb == 48 && bpr >= 4) return launch_fixed<48>(p, bpr, ntiles, st);
    }
#define SPQ_T(TT) \
    case TT: return pq ? launch_t<TT, true>(p, bpr, ntiles, st) : launch_t<TT, false>(p, bpr, ntiles, st);
    switch (T) {
        SPQ_T(1) SPQ_T(2) SPQ_T(3) SPQ_T(4) SPQ_T(5) SPQ_T(6) SPQ_T(7) SPQ_T(8)
        default: return hipErrorInvalidValue;
    }
#undef SPQ_T
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
