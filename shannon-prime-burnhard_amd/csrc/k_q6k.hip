// k_q6k.hip — Q6_K format conversions on gfx950:
//   Q6_K -> fp32   (dequantize_row_q6_K, ggml-quants.c:1877-1906)
//   fp32 -> Q6_K   (quantize_row_q6_K_ref + make_qx_quants,
//                   ggml-quants.c:1807-1875, :566-635)
//   Q6_K . Q8_K    (ggml_vec_dot_q6_K_q8_K shape, one row)
//   exact integer sub-block sums (diagnostic)
// Compiled with -ffp-contract=off and IEEE division: the conversions are
// bit-identical to the CPU path. The matvec kernels are the format templates
// of k_gemv.hip and k_moe.hip instantiated with FmtQ6K (q6k_core.h).
#include "launch.h"
#include "q6k_core.h"

namespace spq4k {

// ---------------------------------------------------------------------------
// Q6_K -> fp32. Thread i of a block's 64 writes elements 4i .. 4i+3, which
// share the half n, quarter h and sub-block: y = (d * scale) * (q - 32), each
// product rounded once as in the reference.
__global__ __launch_bounds__(256) void dequant_q6k_kernel(const uint8_t* __restrict__ x, float* __restrict__ y,
                                                          int64_t nblocks) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t blk = gid >> 6;
    if (blk >= nblocks) return;
    const int e0 = 4 * (int)(gid & 63);
    const int n = e0 >> 7, h = (e0 >> 5) & 3, l = e0 & 31;
    const uint8_t* b = x + blk * Q6K_BYTES;
    typedef uint32_t u32_a2 __attribute__((aligned(2)));
    const uint32_t lo = *reinterpret_cast<const u32_a2*>(b + 64 * n + 32 * (h & 1) + l);
    const uint32_t hi = *reinterpret_cast<const u32_a2*>(b + 128 + 32 * n + l);
    const int sc = (int)(int8_t)b[192 + 8 * n + 2 * h + (l >> 4)];
    const float ds = half_bits_to_float(*reinterpret_cast<const u16_a2*>(b + 208)) * (float)sc;
    const uint32_t nib = (h >> 1) ? (lo >> 4) & 0x0F0F0F0Fu : lo & 0x0F0F0F0Fu;
    const uint32_t q = nib | (((hi >> (2 * h)) & 0x03030303u) << 4);
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = ds * (float)((int)((q >> (8 * k)) & 0xFFu) - 32);
    *reinterpret_cast<float4*>(y + blk * QK + e0) = make_float4(v[0], v[1], v[2], v[3]);
}

// ---------------------------------------------------------------------------
// fp32 -> Q6_K. Sixteen lanes per block: lane j fits sub-block j
// (make_qx_quants(16, 32, x, L, 1, NULL), same operation order), the sixteen
// lanes agree on the fit scale of largest magnitude, then each lane requantises
// its values against the stored d * scale_j; the block is packed through LDS.
__device__ __forceinline__ int clamp_i(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

__device__ float qx_fit16(const float (&x)[16], int (&L)[16]) {
    constexpr int n = 16, nmax = 32;
    float max = 0, amax = 0;
#pragma unroll
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax < 1e-15f) {
#pragma unroll
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = (float)(-nmax) / max;
    float sumlx = 0, suml2 = 0;
#pragma unroll
    for (int i = 0; i < n; ++i) {
        const int l = clamp_i(nearest_int_ref(iscale * x[i]), -nmax, nmax - 1);
        L[i] = l + nmax;
        const float w = x[i] * x[i];
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    float scale = suml2 != 0.f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -((float)nmax + 0.1f * (float)is) / max;
        sumlx = suml2 = 0;
        int La[16];
#pragma unroll
        for (int i = 0; i < n; ++i) {
            const int l = clamp_i(nearest_int_ref(iscale * x[i]), -nmax, nmax - 1);
            La[i] = l + nmax;
            const float w = x[i] * x[i];
            sumlx += w * x[i] * (float)l;
            suml2 += w * (float)l * (float)l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
#pragma unroll
            for (int i = 0; i < n; ++i) L[i] = La[i];
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

__global__ __launch_bounds__(256) void quantize_q6k_kernel(const float* __restrict__ xin, uint8_t* __restrict__ y,
                                                           int64_t nblocks) {
    __shared__ uint8_t Ls[16][256];
    __shared__ __align__(4) uint8_t ob[16][212];
    const int j = threadIdx.x & 15;
    const int lb = threadIdx.x >> 4;
    const int64_t blk0 = (int64_t)blockIdx.x * 16 + lb;
    const bool valid = blk0 < nblocks;
    const int64_t blk = valid ? blk0 : nblocks - 1;   // in bounds; never stored

    float x[16];
    const float4* src = reinterpret_cast<const float4*>(xin + blk * QK + 16 * j);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 a = src[i];
        x[4 * i] = a.x; x[4 * i + 1] = a.y; x[4 * i + 2] = a.z; x[4 * i + 3] = a.w;
    }
    int L[16];
    const float scale = qx_fit16(x, L);

    // the first sub-block of largest |scale| (the reference's `abs > max_abs`
    // scan from 0; NaN never wins): key = |scale| bits : (15 - j)
    uint32_t ab = __float_as_uint(scale) & 0x7FFFFFFFu;
    uint32_t key_hi = ab > 0x7F800000u ? 0u : ab, key_lo = 15u - (uint32_t)j;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
        const uint32_t oh = (uint32_t)__shfl_xor((int)key_hi, off, 16);
        const uint32_t ol = (uint32_t)__shfl_xor((int)key_lo, off, 16);
        const bool t = oh > key_hi || (oh == key_hi && ol > key_lo);
        key_hi = t ? oh : key_hi;
        key_lo = t ? ol : key_lo;
    }
    const float max_scale = __shfl(scale, 15 - (int)key_lo, 16);
    const float max_abs_scale = __uint_as_float(key_hi);
    const bool zero = !(max_abs_scale >= 1e-15f);

    int sc = 0;
    uint16_t d16 = 0;
    if (!zero) {
        const float iscale = -128.f / max_scale;
        const _Float16 dh = (_Float16)(1 / iscale);
        __builtin_memcpy(&d16, &dh, 2);
        const int v = nearest_int_ref(iscale * scale);
        sc = (int)(int8_t)(v < 127 ? v : 127);
        const float d = half_bits_to_float(d16) * (float)sc;
        if (d != 0.0f) {
#pragma unroll
            for (int i = 0; i < 16; ++i) L[i] = clamp_i(nearest_int_ref(x[i] / d), -32, 31) + 32;
        }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) Ls[lb][16 * j + i] = zero ? 0 : (uint8_t)L[i];
    __syncthreads();

    // lane j packs ql bytes 8j .. 8j+7 and qh bytes 4j .. 4j+3
    const uint8_t* Lb = Ls[lb];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int p = 8 * j + k;
        const int n = p >> 6, r = p & 63;
        const int e = 128 * n + 32 * (r >> 5) + (r & 31);
        ob[lb][p] = (uint8_t)((Lb[e] & 0x0F) | ((Lb[e + 64] & 0x0F) << 4));
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int p = 4 * j + k;
        const int e = 128 * (p >> 5) + (p & 31);
        ob[lb][128 + p] =
            (uint8_t)((Lb[e] >> 4) | ((Lb[e + 32] >> 4) << 2) | ((Lb[e + 64] >> 4) << 4) | ((Lb[e + 96] >> 4) << 6));
    }
    ob[lb][192 + j] = (uint8_t)sc;
    if (j == 0) {
        ob[lb][208] = (uint8_t)(d16 & 0xFF);
        ob[lb][209] = (uint8_t)(d16 >> 8);
    }
    __syncthreads();
    if (!valid) return;
    // 105 two-byte words a block (block starts are 2-byte aligned)
    uint16_t* o = reinterpret_cast<uint16_t*>(y + blk * Q6K_BYTES);
    const uint16_t* s16 = reinterpret_cast<const uint16_t*>(ob[lb]);
    for (int k = j; k < Q6K_BYTES / 2; k += 16) o[k] = s16[k];
}

// ---------------------------------------------------------------------------
// One Q6_K row . one Q8_K row (global 292 B blocks). One wave, four lanes per
// block as in the GEMV; wave-wide fp32 reduction in a fixed order.
__global__ __launch_bounds__(64) void vec_dot_q6k_kernel(const uint8_t* __restrict__ wx,
                                                         const uint8_t* __restrict__ q8, int nb,
                                                         float* __restrict__ out) {
    const int lane = threadIdx.x;
    const int l4 = lane & 3, n = l4 >> 1, s = l4 & 1;
    float acc = 0.0f;
    for (int b = lane >> 2; b < nb; b += 16) {
        const W6 w = load_w6(wx + (size_t)b * Q6K_BYTES, l4);
        const uint8_t* yb = q8 + (size_t)b * Q8K_BYTES;
        const int* qs = reinterpret_cast<const int*>(yb + 4 + 128 * n + 16 * s);   // 4-byte aligned
        const int16_t* bs = reinterpret_cast<const int16_t*>(yb + 260);
        Q8Reg6 r;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
#pragma unroll
            for (int i = 0; i < 4; ++i) r.a[4 * h + i] = qs[8 * h + i];
            r.o[h] = -32 * (int)bs[8 * n + 2 * h + s];
        }
        r.d8 = *reinterpret_cast<const float*>(yb);
        acc = block_dot6_reg(w, l4, r, acc);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) *out = acc;
}

// ---------------------------------------------------------------------------
// Diagnostic: the exact integer sub-block sums S[row][b][j] = sum over the 16
// weights of sub-block j of (q - 32) * q8, formed by the GEMV's lane code
// (q6_extract, the offset-initialised dot4 chains) against Q8_K(x), one row.
template <int WAVES>
__global__ __launch_bounds__(WAVES * 64) void subblock_sums_q6k_kernel(const uint8_t* __restrict__ W, int M, int nb,
                                                                       const float* __restrict__ X,
                                                                       int32_t* __restrict__ S, int CB) {
    extern __shared__ __align__(16) char smem[];
    constexpr int ROWS = WAVES * 16;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int l4 = lane & 3, n = l4 >> 1, s = l4 & 1;
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
            const W6 w = load_w6(W + ((size_t)row * nb + c0 + bb) * Q6K_BYTES, l4);
            Q8Reg6 r;
            load_q8reg6(L, bb, l4, r);
            uint32_t q[16];
            q6_extract(w, q);
            int32_t* o = S + ((size_t)row * nb + c0 + bb) * 16 + 8 * n + s;
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                int acc = r.o[h];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc = dot4((int)q[4 * h + i], r.a[4 * h + i], acc);
                o[2 * h] = acc;
            }
        }
    }
}

// ---------------------------------------------------------------------------
hipError_t launch_dequant_q6k(const uint8_t* x, float* y, int64_t nblocks, hipStream_t st) {
    if (nblocks <= 0) return hipSuccess;
    const int64_t grid = (nblocks * 64 + 255) / 256;
    hipLaunchKernelGGL(dequant_q6k_kernel, dim3((unsigned)grid), dim3(256), 0, st, x, y, nblocks);
    return hipGetLastError();
}

hipError_t launch_quantize_q6k(const float* x, uint8_t* y, int64_t nblocks, hipStream_t st) {
    if (nblocks <= 0) return hipSuccess;
    const int64_t grid = (nblocks + 15) / 16;
    hipLaunchKernelGGL(quantize_q6k_kernel, dim3((unsigned)grid), dim3(256), 0, st, x, y, nblocks);
    return hipGetLastError();
}

hipError_t launch_vec_dot_q6k(const uint8_t* wx, const uint8_t* q8, int nb, float* out, hipStream_t st) {
    hipLaunchKernelGGL(vec_dot_q6k_kernel, dim3(1), dim3(64), 0, st, wx, q8, nb, out);
    return hipGetLastError();
}

hipError_t launch_subblock_sums_q6k(const uint8_t* W, int M, int nb, const float* X, int32_t* S, hipStream_t st) {
    constexpr int WAVES = 4;
    const int CB = nb < 64 ? nb : 64;
    const size_t lds = (size_t)q8lds_bytes(CB);
    const int grid = (M + WAVES * 16 - 1) / (WAVES * 16);
    hipLaunchKernelGGL((subblock_sums_q6k_kernel<WAVES>), dim3(grid), dim3(WAVES * 64), lds, st, W, M, nb, X, S, CB);
    return hipGetLastError();
}

}  // namespace spq4k
