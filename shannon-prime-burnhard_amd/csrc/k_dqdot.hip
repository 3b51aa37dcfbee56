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

// acc[t] += this lane's 64 products of block (bsub + 16 it) for each token
template <int T>
__device__ __forceinline__ void dq_block(const DqRow& w, int l4, const lf32x4* xl, int npass, int it, int lane,
                                         float (&acc)[T]) {
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
            const uint32_t qw = q[i4];
            float wv[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t byte = (qw >> (8 * k)) & 0xFFu;
                wv[k] = dd * (float)(half ? byte >> 4 : byte & 0x0Fu) - mm;
            }
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const f32x4 x = xl[(((size_t)t * npass + it) * 16 + 8 * half + i4) * 64 + lane];
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

// x (one row of nb blocks) into the lane-major staging of dequant_matvec_kernel
__device__ __forceinline__ void dq_stage_row(const float* __restrict__ x, int nb, f32x4* dq_x) {
    const f32x4* xr = reinterpret_cast<const f32x4*>(x);
    for (int e4 = threadIdx.x; e4 < nb * 64; e4 += blockDim.x) {
        const int b = e4 >> 6, g = (e4 >> 4) & 3, i4 = e4 & 15;
        dq_x[((size_t)(b >> 4) * 16 + i4) * 64 + 4 * (b & 15) + g] = xr[e4];
    }
}

// one row's dequant-then-dot against the staged x, summed over the wave
// (every lane gets the sum)
__device__ __forceinline__ float dq_row_dot(const uint8_t* __restrict__ row, int nb, const lf32x4* xl, int lane) {
    const int l4 = lane & 3, bsub = lane >> 2;
    const int npass = (nb + 15) >> 4;
    float acc[1] = {0.0f};
    for (int it = 0; it < npass; ++it) {
        const DqRow w = dq_load(row, nb, bsub, l4, it);
        if (bsub + 16 * it < nb) dq_block<1>(w, l4, xl, npass, it, lane, acc);
    }
    const float s = group_sum_last<64>(acc[0]);
    return __shfl(s, 63, 64);
}

// sp_beast_route_experts (:385-443) in one wave: the largest logit (NaNs
// skipped, -1e30 when none), exp_i = expf(l_i - max), their fp32 sum in index
// order, score_i = exp_i / sum; top_k rounds, each taking the unselected
// expert of the largest score (the lowest index among equal ones, as the
// reference's strictly-greater scan); the chosen scores renormalised by
// 1 / (their fp32 sum in rank order) when that sum is positive.
__global__ __launch_bounds__(64) void beast_route_kernel(const float* __restrict__ logits, int E, int top_k,
                                                         int32_t* __restrict__ ids, float* __restrict__ scores) {
    extern __shared__ float rt_score[];            // E scores, then E selection flags
    int* const sel = reinterpret_cast<int*>(rt_score + E);
    __shared__ float s_sum;
    const int lane = threadIdx.x;
    float m = -1e30f;
    for (int i = lane; i < E; i += 64)
        if (logits[i] > m) m = logits[i];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        if (o > m) m = o;
    }
    for (int i = lane; i < E; i += 64) {
        rt_score[i] = expf(logits[i] - m);
        sel[i] = 0;
    }
    __syncthreads();
    if (lane == 0) {
        float sum = 0.0f;
        for (int i = 0; i < E; ++i) sum += rt_score[i];
        s_sum = sum;
    }
    __syncthreads();
    const float sum = s_sum;
    for (int i = lane; i < E; i += 64) rt_score[i] = rt_score[i] / sum;
    __syncthreads();
    __shared__ float chosen[BEAST_MAX_TOPK];
    for (int k = 0; k < top_k; ++k) {
        float bv = -1e30f;
        int bi = -1;
        for (int i = lane; i < E; i += 64)
            if (!sel[i] && rt_score[i] > bv) {
                bv = rt_score[i];
                bi = i;
            }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            if (oi >= 0 && (ov > bv || (ov == bv && (bi < 0 || oi < bi)))) {
                bv = ov;
                bi = oi;
            }
        }
        if (lane == 0) {
            chosen[k] = bv;
            ids[k] = bi;
            if (bi >= 0) sel[bi] = 1;
        }
        __syncthreads();
    }
    if (lane == 0) {
        float ssum = 0.0f;
        for (int k = 0; k < top_k; ++k) ssum += chosen[k];
        const float inv = ssum > 0.0f ? 1.0f / ssum : 1.0f;
        for (int k = 0; k < top_k; ++k) scores[k] = ssum > 0.0f ? chosen[k] * inv : chosen[k];
    }
}

// gate and up rows of every selected expert against the hidden state, and
// silu(gate) * up (beast_silu_mul, :1168-1173): H[s][r], s < top_k, r < n_ff;
// a wave per sweep row (s, r) at a time, rows_per_wg consecutive sweep rows a
// workgroup of 4 waves.
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
    const int total = top_k * n_ff;
    const int q0 = blockIdx.x * rows_per_wg;
    const int q1 = q0 + rows_per_wg < total ? q0 + rows_per_wg : total;
    const size_t row_bytes = (size_t)nb * Q4K_BYTES;
    for (int q = q0 + wave; q < q1; q += 4) {
        const int s = q / n_ff, r = q - s * n_ff;
        const int e = ids[s];
        float h = 0.0f;                        // no expert (a routing with no candidate): nothing
        if (e >= 0 && e < E) {
            const size_t off = (size_t)e * expert_bytes + (size_t)r * row_bytes;
            const float g = dq_row_dot(gate + off, nb, xl, lane);
            const float u = dq_row_dot(up + off, nb, xl, lane);
            h = (g / (1.0f + expf(-g))) * u;
        }
        if (lane == 0) H[q] = h;
    }
}

// down rows of every selected expert against that expert's H row, summed in
// rank order as output += score * down (:541-543, fused multiply-add as the
// reference's GCC build contracts it): out[i], rows_per_wg consecutive rows
// a workgroup of 4 waves, at most BEAST_DOWN_RPW a wave; the H rows are
// staged one expert at a time.
__global__ __launch_bounds__(256) void beast_down_sum_kernel(const uint8_t* __restrict__ down, size_t expert_bytes,
                                                             int n_embd, int nb, const int32_t* __restrict__ ids,
                                                             int E, const float* __restrict__ scores, int top_k,
                                                             const float* __restrict__ H, int n_ff,
                                                             float* __restrict__ out, int rows_per_wg) {
    extern __shared__ __align__(16) f32x4 dq_x[];
    const lf32x4* xl = (const lf32x4*)dq_x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = blockIdx.x * rows_per_wg;
    const int r1 = r0 + rows_per_wg < n_embd ? r0 + rows_per_wg : n_embd;
    const size_t row_bytes = (size_t)nb * Q4K_BYTES;
    float acc[BEAST_DOWN_RPW];
#pragma unroll
    for (int j = 0; j < BEAST_DOWN_RPW; ++j) acc[j] = 0.0f;
    for (int s = 0; s < top_k; ++s) {
        const int e = ids[s];
        if (e < 0 || e >= E) continue;         // uniform over the workgroup
        __syncthreads();                       // the previous expert's readers are done
        dq_stage_row(H + (size_t)s * n_ff, nb, dq_x);
        __syncthreads();
        const uint8_t* base = down + (size_t)e * expert_bytes;
        const float sc = scores[s];
#pragma unroll
        for (int j = 0; j < BEAST_DOWN_RPW; ++j) {
            const int i = r0 + wave + 4 * j;
            if (i < r1) {
                const float d = dq_row_dot(base + (size_t)i * row_bytes, nb, xl, lane);
                acc[j] = fmaf(sc, d, acc[j]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < BEAST_DOWN_RPW; ++j) {
        const int i = r0 + wave + 4 * j;
        if (i < r1 && lane == 0) out[i] = acc[j];
    }
}

}  // namespace

size_t dequant_matvec_lds_bytes(int T, int nb) { return (size_t)T * ((nb + 15) / 16) * 16 * 64 * 16; }

hipError_t launch_beast_moe(const uint8_t* gate, const uint8_t* up, const uint8_t* down, int E, int n_embd, int n_ff,
                            const float* logits, int top_k, const float* hidden, float* out, int32_t* ids,
                            float* scores, float* H, int num_cus, hipStream_t st) {
    if (E < 1 || E > BEAST_MAX_EXPERTS || top_k < 1 || top_k > BEAST_MAX_TOPK || n_embd % 256 || n_ff % 256)
        return hipErrorInvalidValue;
    const int nb_e = n_embd / 256, nb_f = n_ff / 256;
    const size_t lds_e = dequant_matvec_lds_bytes(1, nb_e), lds_f = dequant_matvec_lds_bytes(1, nb_f);
    if (lds_e > DQ_MATVEC_LDS_MAX || lds_f > DQ_MATVEC_LDS_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(beast_route_kernel, dim3(1), dim3(64), (size_t)E * 2 * sizeof(float), st, logits, E, top_k,
                       ids, scores);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // gate / up: about four workgroups a CU over top_k * n_ff sweep rows
    const size_t gu_bytes = (size_t)n_ff * nb_e * Q4K_BYTES;
    const int64_t total = (int64_t)top_k * n_ff;
    int64_t want = (int64_t)num_cus * 4;
    int64_t rpw = (total + want - 1) / want;
    rpw = (rpw + 3) & ~(int64_t)3;
    if (lds_e > 64 * 1024) {
        e = hipFuncSetAttribute((const void*)beast_gate_up_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds_e);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(beast_gate_up_kernel, dim3((unsigned)((total + rpw - 1) / rpw)), dim3(256), lds_e, st, gate,
                       up, gu_bytes, n_ff, nb_e, ids, E, top_k, hidden, H, (int)rpw);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    // down and the weighted sum: rows in runs of a multiple of 4, at most
    // BEAST_DOWN_RPW a wave
    const size_t dn_bytes = (size_t)n_embd * nb_f * Q4K_BYTES;
    int64_t drw = ((int64_t)n_embd + want - 1) / want;
    drw = (drw + 3) & ~(int64_t)3;
    if (drw > 4 * BEAST_DOWN_RPW) drw = 4 * BEAST_DOWN_RPW;
    if (lds_f > 64 * 1024) {
        e = hipFuncSetAttribute((const void*)beast_down_sum_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds_f);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(beast_down_sum_kernel, dim3((unsigned)((n_embd + drw - 1) / drw)), dim3(256), lds_f, st, down,
                       dn_bytes, n_embd, nb_f, ids, E, scores, top_k, H, n_ff, out, (int)drw);
    return hipGetLastError();
}

hipError_t launch_dequant_matvec(const uint8_t* W, int M, int nb, const float* X, int64_t x_tstride, float* Y,
                                 int64_t y_tstride, int T, int num_cus, hipStream_t st) {
    if (M <= 0 || nb <= 0 || T < 1 || T > DQ_MATVEC_MAX_T) return hipErrorInvalidValue;
    const size_t lds = dequant_matvec_lds_bytes(T, nb);
    if (lds > DQ_MATVEC_LDS_MAX) return hipErrorInvalidValue;
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
