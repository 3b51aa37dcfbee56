// k_gemm.hip — Q4_K x Q8_K matmul for prefill on gfx950 matrix cores.
//
// Computes GGML_OP_MUL_MAT for a T-token batch with the numerics of the
// reference CPU path (ggml_compute_forward_mul_mat, ggml-cpu.c:1241-1439:
// Q8_K activations, integer sub-block sums exact, fp32 combine):
//   Y[t][r] = sum_b  d_rb d8_tb I_rbt  -  sum_b sum_j (dmin_rb m_rbj)(d8_tb BS_tbj)
//   I_rbt   = sum_j sc_rbj S_rbtj,    S_rbtj = sum_{k in sub-block j} q4_rk q8_tk
//   BS_tbj  = bsums_tb[2j] + bsums_tb[2j+1]
// The CUDA backend's equivalent is mul_mat_q<Q4_K> (ggml-cuda/mmq.cuh:3478),
// which uses Q8_1 activations; this kernel keeps Q8_K.
//
// Matrix-core mapping (wave64, v_mfma_i32_16x16x64_i8, lane l: row/col l%16,
// k-quarter q = l/16 holding 16 consecutive k):
//   - a 6-bit scale sc = 8*sh + sl (sh, sl in 0..7) is folded into two int8
//     A operands A_hi = sh*q4 and A_lo = sl*q4 (both <= 105), so the matrix
//     cores accumulate H = sum A_hi q8 and L = sum A_lo q8 over a whole
//     256-value super-block with no per-sub-block VALU work, and I = 8H + L
//     exactly;
//   - the min-term integer M = sum_j m_j BS_j of each super-block comes from
//     v_mfma_f32_16x16x4f32 fed with the integers m_j (<= 63) and BS_j
//     (|BS| <= 4064): every product and partial sum stays below 2^24, so M is
//     exact;
//   - per super-block acc += (d*d8) I - (dmin*d8) M in fp32, the reference's
//     per-block combine.
// Workgroup tile: 4 waves x 16 rows, NCT x 16 tokens; activations (Q8_K
// planes written by quantize_q8k_planes_kernel) staged per super-block in LDS
// (double-buffered: the next block's loads are issued before this block's
// MFMAs and stored after them), weights streamed from HBM into registers one
// super-block ahead.
#include "gemv_core.h"
#include "launch.h"

namespace spq4k {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// per-lane weight registers for one super-block: header + 64 B of qs
struct WG4 {
    uint4 hdr;
    uint4 q[4];   // step s: qs[32 s + 16 (q & 1) .. + 16]
};

template <int NCT>
__global__ __launch_bounds__(256) void gemm_q4k_kernel(GemmParams p) {
    constexpr int TOK = NCT * 16;          // tokens per workgroup
    __shared__ __align__(16) int8_t s_q8[2][TOK * 256];
    __shared__ float s_d8[2][TOK];
    __shared__ float s_bm[2][TOK * 8];    // BS_j as exact floats
    __shared__ float s_dr[2][64];         // d of the workgroup's rows
    __shared__ float s_dmr[2][64];        // dmin of the workgroup's rows

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c16 = lane & 15;             // A row / B column within a 16-tile
    const int q = lane >> 4;               // k-quarter of a 64-k step; output row group
    const int M = p.M, T = p.T, nb = p.nb;

    // token tile fastest: the workgroups sharing a weight tile run together
    const int ttiles = (T + TOK - 1) / TOK;
    const int tt = blockIdx.x % ttiles;
    const int rt = blockIdx.x / ttiles;
    const int row_a = rt * 64 + wave * 16 + c16;            // this lane's A row
    const int row_a_c = min(row_a, M - 1);
    const int tok0 = tt * TOK;

    const uint8_t* __restrict__ wrow = p.W + (size_t)row_a_c * nb * Q4K_BYTES;

    auto load_wblock = [&](int b) {
        WG4 w;
        const uint8_t* blk = wrow + (size_t)b * Q4K_BYTES;
        w.hdr = *reinterpret_cast<const uint4*>(blk);
#pragma unroll
        for (int s = 0; s < 4; ++s) w.q[s] = *reinterpret_cast<const uint4*>(blk + 16 + 32 * s + 16 * (q & 1));
        return w;
    };

    // staging of super-block b's activations into LDS buffer `buf`, split in
    // a load half (into registers) and a store half, so that the next
    // block's loads are in flight during the current block's MFMAs
    constexpr int QV = (TOK * 16 + 255) / 256;   // uint4 per thread
    constexpr int BV = (TOK * 8 + 255) / 256;    // bsum pairs per thread
    struct StageRegs {
        v4i q[QV];   // native vectors: HIP's uint4 copies go through a stack slot
        float bm[BV];
        float d8[BV];
    };
    auto stage_load = [&](int b, StageRegs& r) {
#pragma unroll
        for (int k = 0; k < QV; ++k) {
            const int i = threadIdx.x + 256 * k;
            const int t = min(i >> 4, TOK - 1), c = i & 15;
            const int tg = min(tok0 + t, T - 1);
            r.q[k] = reinterpret_cast<const v4i*>(p.Q.qs + ((int64_t)tg * nb + b) * 256)[c];
        }
#pragma unroll
        for (int k = 0; k < BV; ++k) {
            const int i = threadIdx.x + 256 * k;
            const int t = min(i >> 3, TOK - 1), j = i & 7;
            const int tg = min(tok0 + t, T - 1);
            const int16_t* bs = p.Q.bs + ((int64_t)tg * nb + b) * 16;
            r.bm[k] = (float)((int)bs[2 * j] + (int)bs[2 * j + 1]);
            r.d8[k] = p.Q.d[(int64_t)tg * nb + b];
        }
    };
    auto stage_store = [&](const StageRegs& r, int buf) {
#pragma unroll
        for (int k = 0; k < QV; ++k) {
            const int i = threadIdx.x + 256 * k;
            if (i < TOK * 16) reinterpret_cast<v4i*>(s_q8[buf])[i] = r.q[k];
        }
#pragma unroll
        for (int k = 0; k < BV; ++k) {
            const int i = threadIdx.x + 256 * k;
            if (i < TOK * 8) {
                s_bm[buf][i] = r.bm[k];
                if ((i & 7) == 0) s_d8[buf][i >> 3] = r.d8[k];
            }
        }
    };
    auto stage = [&](int b, int buf) {
        StageRegs r;
        stage_load(b, r);
        stage_store(r, buf);
    };

    v4f acc[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) acc[ct] = v4f{0, 0, 0, 0};

    WG4 wcur = load_wblock(0);
    stage(0, 0);
    for (int b = 0; b < nb; ++b) {
        const int buf = b & 1;
        // row constants of this super-block (A-lane row)
        const float d = half_bits_to_float(wcur.hdr.x & 0xFFFFu);
        const float dmin = half_bits_to_float(wcur.hdr.x >> 16);
        const ScaleMin sm = unpack_scale_min(wcur.hdr.y, wcur.hdr.z, wcur.hdr.w);
        if (q == 0) {
            s_dr[buf][wave * 16 + c16] = d;
            s_dmr[buf][wave * 16 + c16] = dmin;
        }
        __syncthreads();   // stage(b) and s_dr visible; previous block's readers done
        WG4 wnext;
        StageRegs snext;
        if (b + 1 < nb) {
            wnext = load_wblock(b + 1);
            stage_load(b + 1, snext);
        }

        v4i ch[NCT], cl[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            ch[ct] = v4i{0, 0, 0, 0};
            cl[ct] = v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            // sub-block of this lane's 16 k: j = 2s + (q >= 2)
            const int j = 2 * s + (q >> 1);
            const uint32_t scw = j < 4 ? sm.sc_lo : sm.sc_hi;
            const uint32_t sc = (scw >> (8 * (j & 3))) & 0xFFu;
            const u16x2 sh = {(uint16_t)(sc >> 3), (uint16_t)(sc >> 3)};
            const u16x2 sl = {(uint16_t)(sc & 7u), (uint16_t)(sc & 7u)};
            const uint32_t w4[4] = {wcur.q[s].x, wcur.q[s].y, wcur.q[s].z, wcur.q[s].w};
            int ahs[4], als[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t nib = (q >= 2) ? ((w4[i] >> 4) & 0x0F0F0F0Fu) : (w4[i] & 0x0F0F0F0Fu);
                // packed 16-bit multiply (v_pk_mul_lo_u16): each byte < 16 times
                // a factor < 8 stays below 128, so no carry crosses a byte
                u16x2 n2;
                __builtin_memcpy(&n2, &nib, 4);
                const u16x2 h2 = n2 * sh, l2 = n2 * sl;
                __builtin_memcpy(&ahs[i], &h2, 4);
                __builtin_memcpy(&als[i], &l2, 4);
            }
            const v4i ahi = {ahs[0], ahs[1], ahs[2], ahs[3]};
            const v4i alo = {als[0], als[1], als[2], als[3]};
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                const v4i bv = *reinterpret_cast<const v4i*>(s_q8[buf] + (ct * 16 + c16) * 256 + 64 * s + 16 * q);
                ch[ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi, bv, ch[ct], 0, 0, 0);
                cl[ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo, bv, cl[ct], 0, 0, 0);
            }
        }
        // min-term integers: A_m[r][j] = m_j (k-quarter q holds j = q and j = 4 + q)
        const float am0 = (float)((sm.m_lo >> (8 * q)) & 0xFFu);
        const float am1 = (float)((sm.m_hi >> (8 * q)) & 0xFFu);
        const float4 drow = *reinterpret_cast<const float4*>(&s_dr[buf][wave * 16 + 4 * q]);
        const float4 dmrow = *reinterpret_cast<const float4*>(&s_dmr[buf][wave * 16 + 4 * q]);
        const float dd[4] = {drow.x, drow.y, drow.z, drow.w};
        const float dm[4] = {dmrow.x, dmrow.y, dmrow.z, dmrow.w};
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            const int tl = ct * 16 + c16;
            v4f cm = {0, 0, 0, 0};
            cm = __builtin_amdgcn_mfma_f32_16x16x4f32(am0, s_bm[buf][tl * 8 + q], cm, 0, 0, 0);
            cm = __builtin_amdgcn_mfma_f32_16x16x4f32(am1, s_bm[buf][tl * 8 + 4 + q], cm, 0, 0, 0);
            const float d8 = s_d8[buf][tl];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int I = (ch[ct][i] << 3) + cl[ct][i];
                acc[ct][i] = fmaf(dd[i] * d8, (float)I, acc[ct][i]);
                acc[ct][i] = fmaf(-(dm[i] * d8), cm[i], acc[ct][i]);
            }
        }
        if (b + 1 < nb) {
            // buffer buf ^ 1 was last read in block b - 1, before this block's barrier
            stage_store(snext, buf ^ 1);
            wcur = wnext;
        }
    }

    // output: lane holds rows 4q..4q+3 of its wave tile for token c16 of each column tile
    const int row_o = rt * 64 + wave * 16 + 4 * q;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
        const int t = tok0 + ct * 16 + c16;
        if (t >= T) continue;
        float* y = p.Y + (int64_t)t * M;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (row_o + i < M) y[row_o + i] = acc[ct][i];
    }
}

// ---------------------------------------------------------------------------
// Skinny form for T <= 64 (prefill of short prompts): the weights stream is the
// cost, so the grid needs many waves. A workgroup owns 16 rows x 16*NCT tokens
// of one of up to four matrices sharing the input (row tiles of the segments
// are numbered one after the other) and its KW waves split K: wave w takes
// super-blocks w, w + KW, ..., CH of them at a time with every load of the
// chunk (weights and the activation fragments, read straight from the L2
// resident Q8_K planes) issued before any is used. The exact scale folding and
// min-term MFMA are the tiled kernel's. The KW partial tiles are summed
// through LDS in wave order (deterministic) and stored.
struct SkinnyFrag {
    v4i bq[4];
    float bs0, bs1, d8;
};

template <int NCT, int KW, int CH>
__global__ __launch_bounds__(KW * 64) void gemm_skinny_kernel(GemmParams p) {
    constexpr int TOK = NCT * 16;
    __shared__ v4f red[KW][NCT][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c16 = lane & 15;
    const int q = lane >> 4;
    const int T = p.T, nb = p.nb;
    const int ttiles = (T + TOK - 1) / TOK;
    const int tt = blockIdx.x % ttiles;
    const int gt = blockIdx.x / ttiles;            // row tile over all segments
    int sidx = 0;
#pragma unroll
    for (int k = 1; k < GEMM_MAX_SEG; ++k)
        if (k < p.nseg && gt >= p.seg[k].tile_begin) sidx = k;
    const uint8_t* __restrict__ W = p.seg[sidx].W;
    float* __restrict__ Y = p.seg[sidx].Y;
    const int M = p.seg[sidx].M;
    const int rt = gt - p.seg[sidx].tile_begin;
    const int row_a = min(rt * 16 + c16, M - 1);
    const int tok0 = tt * TOK;
    const uint8_t* __restrict__ wrow = W + (size_t)row_a * nb * Q4K_BYTES;

    int tg[NCT];   // this lane's B column (token) in each 16-token tile, clamped
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) tg[ct] = min(tok0 + ct * 16 + c16, T - 1);

    auto load_w = [&](int b) {
        WG4 w;
        const uint8_t* blk = wrow + (size_t)b * Q4K_BYTES;
        w.hdr = *reinterpret_cast<const uint4*>(blk);
#pragma unroll
        for (int s = 0; s < 4; ++s) w.q[s] = *reinterpret_cast<const uint4*>(blk + 16 + 32 * s + 16 * (q & 1));
        return w;
    };
    auto load_b = [&](int b, int ct) {
        SkinnyFrag f;
        const int64_t it = (int64_t)tg[ct] * nb + b;
        const int8_t* q8 = p.Q.qs + it * 256 + 16 * q;
#pragma unroll
        for (int s = 0; s < 4; ++s) f.bq[s] = *reinterpret_cast<const v4i*>(q8 + 64 * s);
        const uint32_t* bs = reinterpret_cast<const uint32_t*>(p.Q.bs + it * 16);
        const uint32_t u0 = bs[q], u1 = bs[4 + q];   // bsums[2j], [2j+1] for j = q and j = 4 + q
        f.bs0 = (float)((int)(int16_t)(u0 & 0xFFFFu) + (int)(int16_t)(u0 >> 16));
        f.bs1 = (float)((int)(int16_t)(u1 & 0xFFFFu) + (int)(int16_t)(u1 >> 16));
        f.d8 = p.Q.d[it];
        return f;
    };

    v4f acc[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) acc[ct] = v4f{0, 0, 0, 0};

    for (int b0 = wave; b0 < nb; b0 += KW * CH) {
        // every load of the chunk first (blocks past the end re-read the last
        // block of the wave's slice and are not accumulated)
        WG4 wv[CH];
        SkinnyFrag fr[CH][NCT];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int braw = b0 + c * KW;
            const int b = braw < nb ? braw : b0;
            wv[c] = load_w(b);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) fr[c][ct] = load_b(b, ct);
        }
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            if (b0 + c * KW >= nb) break;
            const WG4& wcur = wv[c];
            const float d = half_bits_to_float(wcur.hdr.x & 0xFFFFu);
            const float dmin = half_bits_to_float(wcur.hdr.x >> 16);
            const ScaleMin sm = unpack_scale_min(wcur.hdr.y, wcur.hdr.z, wcur.hdr.w);
            v4i ch[NCT], cl[NCT];
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                ch[ct] = v4i{0, 0, 0, 0};
                cl[ct] = v4i{0, 0, 0, 0};
            }
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int j = 2 * s + (q >> 1);
                const uint32_t scw = j < 4 ? sm.sc_lo : sm.sc_hi;
                const uint32_t sc = (scw >> (8 * (j & 3))) & 0xFFu;
                const u16x2 sh = {(uint16_t)(sc >> 3), (uint16_t)(sc >> 3)};
                const u16x2 sl = {(uint16_t)(sc & 7u), (uint16_t)(sc & 7u)};
                const uint32_t w4[4] = {wcur.q[s].x, wcur.q[s].y, wcur.q[s].z, wcur.q[s].w};
                int ahs[4], als[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t nib = (q >= 2) ? ((w4[i] >> 4) & 0x0F0F0F0Fu) : (w4[i] & 0x0F0F0F0Fu);
                    u16x2 n2;
                    __builtin_memcpy(&n2, &nib, 4);
                    const u16x2 h2 = n2 * sh, l2 = n2 * sl;
                    __builtin_memcpy(&ahs[i], &h2, 4);
                    __builtin_memcpy(&als[i], &l2, 4);
                }
                const v4i ahi = {ahs[0], ahs[1], ahs[2], ahs[3]};
                const v4i alo = {als[0], als[1], als[2], als[3]};
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) {
                    ch[ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi, fr[c][ct].bq[s], ch[ct], 0, 0, 0);
                    cl[ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo, fr[c][ct].bq[s], cl[ct], 0, 0, 0);
                }
            }
            // d, dmin of output rows 4q .. 4q+3 (held by lanes 4q+i, whose c16 is that row)
            float dd[4], dm[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                dd[i] = __shfl(d, 4 * q + i);
                dm[i] = __shfl(dmin, 4 * q + i);
            }
            const float am0 = (float)((sm.m_lo >> (8 * q)) & 0xFFu);
            const float am1 = (float)((sm.m_hi >> (8 * q)) & 0xFFu);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                v4f cm = {0, 0, 0, 0};
                cm = __builtin_amdgcn_mfma_f32_16x16x4f32(am0, fr[c][ct].bs0, cm, 0, 0, 0);
                cm = __builtin_amdgcn_mfma_f32_16x16x4f32(am1, fr[c][ct].bs1, cm, 0, 0, 0);
                // C lane layout: rows 4q + i, column (token) c16: this lane's own d8
                const float d8c = fr[c][ct].d8;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int I = (ch[ct][i] << 3) + cl[ct][i];
                    acc[ct][i] = fmaf(dd[i] * d8c, (float)I, acc[ct][i]);
                    acc[ct][i] = fmaf(-(dm[i] * d8c), cm[i], acc[ct][i]);
                }
            }
        }
    }
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) red[wave][ct][lane] = acc[ct];
    __syncthreads();
    // wave w reduces tile ct = w (if any) over the KW partials in wave order
    for (int ct = wave; ct < NCT; ct += KW) {
        v4f s = red[0][ct][lane];
#pragma unroll
        for (int w = 1; w < KW; ++w) s += red[w][ct][lane];
        const int t = tok0 + ct * 16 + c16;
        if (t < T) {
            float* y = Y + (int64_t)t * M;
            const int row_o = rt * 16 + 4 * q;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (row_o + i < M) y[row_o + i] = s[i];
        }
    }
}

template <int NCT, int KW, int CH>
static hipError_t launch_skinny(const GemmParams& p, hipStream_t st) {
    constexpr int TOK = NCT * 16;
    const int64_t grid = (int64_t)p.total_tiles * ((p.T + TOK - 1) / TOK);
    hipLaunchKernelGGL((gemm_skinny_kernel<NCT, KW, CH>), dim3((unsigned)grid), dim3(KW * 64), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_gemm_skinny(const GemmParams& p, hipStream_t st) {
    // KW waves split K so that a wave has at most CH blocks per chunk
    const bool longk = p.nb > 16;
    if (p.T <= 16) return longk ? launch_skinny<1, 16, 3>(p, st) : launch_skinny<1, 8, 2>(p, st);
    if (p.T <= 32) return longk ? launch_skinny<2, 16, 2>(p, st) : launch_skinny<2, 8, 2>(p, st);
    return longk ? launch_skinny<4, 16, 1>(p, st) : launch_skinny<4, 8, 1>(p, st);
}

template <int NCT>
static hipError_t launch_gemm_n(const GemmParams& p, hipStream_t st) {
    constexpr int TOK = NCT * 16;
    const int64_t grid = (int64_t)((p.M + 63) / 64) * ((p.T + TOK - 1) / TOK);
    hipLaunchKernelGGL((gemm_q4k_kernel<NCT>), dim3((unsigned)grid), dim3(256), 0, st, p);
    return hipGetLastError();
}

bool gemm_use_skinny(int T, int mode) { return mode == 1 || (mode != 2 && T <= 64); }

hipError_t launch_gemm(const GemmParams& p, hipStream_t st) {
    if (p.T <= 16) return launch_gemm_n<1>(p, st);
    if (p.T <= 32) return launch_gemm_n<2>(p, st);
    return launch_gemm_n<4>(p, st);
}

}  // namespace spq4k
