// k_gemm.hip — Q4_K x Q8_K matmul for prefill on gfx950 matrix cores.
//
// Computes GGML_OP_MUL_MAT for a T-token batch with the numerics of the
// reference CPU path (ggml_compute_forward_mul_mat, ggml-cpu.c:1241-1439:
// Q8_K activations, integer sub-block sums exact, fp32 combine):
//   Y[t][r] = sum_b  d8_tb (d_rb I_rbt  -  dmin_rb M_rbt)
//   I_rbt   = sum_j sc_rbj S_rbtj,    S_rbtj = sum_{k in sub-block j} q4_rk q8_tk
//   M_rbt   = sum_j m_rbj BS_tbj,     BS_tbj = bsums_tb[2j] + bsums_tb[2j+1]
// The CUDA backend's equivalent is mul_mat_q<Q4_K> (ggml-cuda/mmq.cuh:3478),
// which uses Q8_1 activations; these kernels keep Q8_K.
//
// Matrix-core mapping (wave64, 16x16 output tiles; lane l has column l % 16
// and k-slot group q = l / 16; the output lane holds rows 4q .. 4q+3):
//   - a 6-bit scale sc = 8*sh + sl (sh, sl in 0..7) is folded into two int8
//     operands sh*q4 and sl*q4 (both <= 105), so v_mfma_i32_16x16x64_i8
//     accumulates H = sum sh q4 q8 and L = sum sl q4 q8 over a whole 256-value
//     super-block with no per-sub-block work, and I = 8H + L exactly;
//   - the min-term integer M comes from one v_mfma_f32_16x16x16_f16 per tile:
//     BS_j = 32 hi_j + lo_j (hi_j in -127..127, lo_j in 0..31) and the k slots
//     hold (32 m_j, hi_j) for j = 0..7 and (m_j, lo_j) for j = 0..7; every
//     operand, product (<= 2016 * 127) and partial sum (< 2^22) is an integer
//     that fp16 / fp32 represent exactly, so M is exact;
//   - per super-block acc += d8 (d I - dmin M) in fp32.
#include "gemv_core.h"
#include "launch.h"
#include "q6k_core.h"
#include "ring_core.h"

#include <type_traits>

namespace spq4k {

// per-lane weight registers for one super-block: header + 64 B of qs (skinny kernel)
struct WG4 {
    uint4 hdr;
    uint4 q[4];   // step s: qs[32 s + 16 (q & 1) .. + 16]
};

// Workgroup i runs on XCD i % 8. Logical tile L numbers the workgroups of one
// XCD consecutively, so neighbouring tiles (the token tiles of one row tile,
// which read the same weights) share that XCD's L2.
__device__ __forceinline__ int xcd_tile(int bid, int G) {
    const int x = bid & 7;
    return x * (G >> 3) + min(x, G & 7) + (bid >> 3);
}


// ---------------------------------------------------------------------------
// Tiled form. A workgroup of four waves owns ROWS = WR*RT*16 rows of one of up
// to four matrices sharing the input (row tiles of the segments are numbered
// one after the other) and TOK = CT*16 tokens; wave (wr, wk) computes RT x CT
// output tiles of 16x16 over super-blocks wk, wk + WK, ... and the WK partial
// tiles are summed through LDS in wave order (deterministic).
//
// k order inside a super-block: k-slot group q of step s (s = 0..3) holds the
// low and the high nibbles of bytes 8s .. 8s+7 of the 32-byte nibble group q,
// i.e. k = 64q + 8s + e and 64q + 32 + 8s + e (e = 0..7): a lane loads its own
// 32 bytes of qs once per super-block and its two sub-blocks (2q, 2q+1) keep
// one scale pair for all four steps. The activations are staged in LDS in the
// same order (a 16-byte read per fragment, rows padded to 272 bytes so that
// the 16 tokens of a fragment read hit distinct banks), double-buffered: the
// next iteration's loads are issued before this one's MFMAs and stored after.
template <int RT, int CT, int WR, int WK>
__global__ __launch_bounds__(256) void gemm_tiled_kernel(GemmParams p) {
    static_assert(WR * WK == 4, "four waves per workgroup");
    constexpr int TOK = CT * 16;
    constexpr int ROWS = WR * RT * 16;
    constexpr int QS = 272;     // LDS bytes per token row of q8
    constexpr int MS = 20;      // LDS halves per token of the min operand (16 used)
    __shared__ __align__(16) int8_t s_q8[2][WK][TOK * QS];
    __shared__ __align__(16) _Float16 s_mn[2][WK][TOK * MS];
    __shared__ __align__(16) float s_d8[2][WK][TOK];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wr = wave % WR, wk = wave / WR;
    const int c16 = lane & 15;
    const int q = lane >> 4;
    const int T = p.T, nb = p.nb;
    const int ttiles = (T + TOK - 1) / TOK;
    const int L = xcd_tile(blockIdx.x, gridDim.x);
    const int tt = L % ttiles;
    const int gt = L / ttiles;                      // row tile over all segments
    int sidx = 0;
#pragma unroll
    for (int k = 1; k < GEMM_MAX_SEG; ++k)
        if (k < p.nseg && gt >= p.seg[k].tile_begin) sidx = k;
    const uint8_t* __restrict__ W = p.seg[sidx].W;
    float* __restrict__ Y = p.seg[sidx].Y;
    const int M = p.seg[sidx].M;
    const int row0 = (gt - p.seg[sidx].tile_begin) * ROWS + wr * RT * 16;
    const int tok0 = tt * TOK;

    const uint8_t* wrow[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) wrow[r] = W + (size_t)min(row0 + r * 16 + c16, M - 1) * nb * Q4K_BYTES;

    struct WQ {
        v4i hdr, lo, hi;   // header; bytes 0..15 and 16..31 of the lane's 32-byte nibble group
    };
    auto load_w = [&](int b, WQ* w) {
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const uint8_t* blk = wrow[r] + (size_t)b * Q4K_BYTES;
            w[r].hdr = *reinterpret_cast<const v4i*>(blk);
            w[r].lo = *reinterpret_cast<const v4i*>(blk + 16 + 32 * q);
            w[r].hi = *reinterpret_cast<const v4i*>(blk + 32 + 32 * q);
        }
    };

    // staging of iteration `it` (super-blocks it*WK .. it*WK + WK-1)
    constexpr int NQ = WK * TOK * 16;   // 16-byte chunks of q8
    constexpr int NM = WK * TOK * 8;    // (token, sub-block) items of the min operand
    constexpr int QV = (NQ + 255) / 256;
    constexpr int MV = (NM + 255) / 256;
    struct Stage {
        v4i q[QV];
        uint32_t bs[MV];
        float d8[MV];
    };
    auto stage_load = [&](int it, Stage& s) {
#pragma unroll
        for (int k = 0; k < QV; ++k) {
            const int i = min((int)threadIdx.x + 256 * k, NQ - 1);
            const int kb = i / (TOK * 16), t = (i >> 4) % TOK, c = i & 15;
            const int b = min(it * WK + kb, nb - 1), tg = min(tok0 + t, T - 1);
            s.q[k] = reinterpret_cast<const v4i*>(p.Q.qs + ((int64_t)tg * nb + b) * 256)[c];
        }
#pragma unroll
        for (int k = 0; k < MV; ++k) {
            const int i = min((int)threadIdx.x + 256 * k, NM - 1);
            const int kb = i / (TOK * 8), t = (i >> 3) % TOK, j = i & 7;
            const int b = min(it * WK + kb, nb - 1), tg = min(tok0 + t, T - 1);
            const int64_t ib = (int64_t)tg * nb + b;
            s.bs[k] = reinterpret_cast<const uint32_t*>(p.Q.bs + ib * 16)[j];
            s.d8[k] = p.Q.d[ib];
        }
    };
    auto stage_store = [&](const Stage& s, int buf) {
#pragma unroll
        for (int k = 0; k < QV; ++k) {
            const int i = (int)threadIdx.x + 256 * k;
            if (NQ % 256 == 0 || i < NQ) {
                const int kb = i / (TOK * 16), t = (i >> 4) % TOK, c = i & 15;
                // chunk c = k 16c .. 16c+15: group c/4, nibble half (c/2)&1, steps 2(c&1), 2(c&1)+1
                int8_t* dst = s_q8[buf][kb] + t * QS + 64 * (c >> 2) + 32 * (c & 1) + 8 * ((c >> 1) & 1);
                *reinterpret_cast<uint64_t*>(dst) = (uint64_t)(uint32_t)s.q[k].x | ((uint64_t)(uint32_t)s.q[k].y << 32);
                *reinterpret_cast<uint64_t*>(dst + 16) =
                    (uint64_t)(uint32_t)s.q[k].z | ((uint64_t)(uint32_t)s.q[k].w << 32);
            }
        }
#pragma unroll
        for (int k = 0; k < MV; ++k) {
            const int i = (int)threadIdx.x + 256 * k;
            if (NM % 256 == 0 || i < NM) {
                const int kb = i / (TOK * 8), t = (i >> 3) % TOK, j = i & 7;
                const int bsum = (int)(int16_t)(s.bs[k] & 0xFFFFu) + (int)(int16_t)(s.bs[k] >> 16);
                _Float16* m = s_mn[buf][kb] + t * MS;
                m[j] = (_Float16)(bsum >> 5);          // hi_j (floor division)
                m[8 + j] = (_Float16)(bsum & 31);      // lo_j
                if (j == 0) s_d8[buf][kb][t] = s.d8[k];
            }
        }
    };

    v4f acc[RT][CT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[r][ct] = v4f{0, 0, 0, 0};

    const int n_it = (nb + WK - 1) / WK;
    WQ wcur[RT];
    load_w(min(wk, nb - 1), wcur);
    {
        Stage s0;
        stage_load(0, s0);
        stage_store(s0, 0);
    }
    for (int it = 0; it < n_it; ++it) {
        const int buf = it & 1;
        __syncthreads();   // staging of `it` visible; readers of buf ^ 1 (iteration it - 1) done
        // next iteration's loads (clamped at the end: unconditional, so no wait
        // is forced at a branch join)
        WQ wnext[RT];
        Stage snext;
        const int itn = min(it + 1, n_it - 1);
        load_w(min(itn * WK + wk, nb - 1), wnext);
        stage_load(itn, snext);

        if (it * WK + wk < nb) {   // wave-uniform
            float d[RT], dmin[RT];
            uint32_t SH0[RT], SL0[RT], SH1[RT], SL1[RT];
            h4 bm[RT];
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const uint32_t h0 = (uint32_t)wcur[r].hdr.x;
                d[r] = half_bits_to_float(h0 & 0xFFFFu);
                dmin[r] = half_bits_to_float(h0 >> 16);
                const ScaleMin sm = unpack_scale_min((uint32_t)wcur[r].hdr.y, (uint32_t)wcur[r].hdr.z,
                                                     (uint32_t)wcur[r].hdr.w);
                // sub-blocks 2q (low nibbles) and 2q + 1 (high nibbles)
                const uint32_t sc01 = (q < 2 ? sm.sc_lo : sm.sc_hi) >> (16 * (q & 1));
                SH0[r] = ((sc01 >> 3) & 7u) * 0x10001u;
                SL0[r] = (sc01 & 7u) * 0x10001u;
                SH1[r] = ((sc01 >> 11) & 7u) * 0x10001u;
                SL1[r] = ((sc01 >> 8) & 7u) * 0x10001u;
                // min operand: (32 m_j) for slots 0..7, (m_j) for slots 8..15;
                // 0x6400 | m is the fp16 1024 + m, rescaled exactly
                const uint32_t mw = (q & 1) ? sm.m_hi : sm.m_lo;
                const uint32_t x01 = __builtin_amdgcn_perm(0x64646464u, mw, 0x04010400u);
                const uint32_t x23 = __builtin_amdgcn_perm(0x64646464u, mw, 0x04030402u);
                h2 a01, a23;
                __builtin_memcpy(&a01, &x01, 4);
                __builtin_memcpy(&a23, &x23, 4);
                const _Float16 f = q < 2 ? (_Float16)32.0f : (_Float16)1.0f;
                const _Float16 o = q < 2 ? (_Float16)-32768.0f : (_Float16)-1024.0f;
                const h2 fv = {f, f}, ov = {o, o};
                const h2 b01 = a01 * fv + ov, b23 = a23 * fv + ov;
                bm[r] = h4{b01.x, b01.y, b23.x, b23.y};
            }

            v4i ch[RT][CT], cl[RT][CT];
#pragma unroll
            for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    ch[r][ct] = v4i{0, 0, 0, 0};
                    cl[r][ct] = v4i{0, 0, 0, 0};
                }
            const int8_t* qb = s_q8[buf][wk] + c16 * QS + 64 * q;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                v4i a[CT];
#pragma unroll
                for (int ct = 0; ct < CT; ++ct)
                    a[ct] = *reinterpret_cast<const v4i*>(qb + ct * 16 * QS + 16 * s);
#pragma unroll
                for (int r = 0; r < RT; ++r) {
                    const uint32_t w0 = (uint32_t)(s < 2 ? wcur[r].lo[2 * s] : wcur[r].hi[2 * s - 4]);
                    const uint32_t w1 = (uint32_t)(s < 2 ? wcur[r].lo[2 * s + 1] : wcur[r].hi[2 * s - 3]);
                    const uint32_t l0 = w0 & 0x0F0F0F0Fu, l1 = w1 & 0x0F0F0F0Fu;
                    const uint32_t u0 = (w0 >> 4) & 0x0F0F0F0Fu, u1 = (w1 >> 4) & 0x0F0F0F0Fu;
                    const v4i bh = {(int)pk_mul_u16(l0, SH0[r]), (int)pk_mul_u16(l1, SH0[r]),
                                    (int)pk_mul_u16(u0, SH1[r]), (int)pk_mul_u16(u1, SH1[r])};
                    const v4i bl = {(int)pk_mul_u16(l0, SL0[r]), (int)pk_mul_u16(l1, SL0[r]),
                                    (int)pk_mul_u16(u0, SL1[r]), (int)pk_mul_u16(u1, SL1[r])};
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct) {
                        ch[r][ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[ct], bh, ch[r][ct], 0, 0, 0);
                        cl[r][ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[ct], bl, cl[r][ct], 0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const h4 am = *reinterpret_cast<const h4*>(s_mn[buf][wk] + (ct * 16 + c16) * MS + 4 * q);
                const v4f d8 = *reinterpret_cast<const v4f*>(&s_d8[buf][wk][ct * 16 + 4 * q]);
#pragma unroll
                for (int r = 0; r < RT; ++r) {
                    const v4f cm = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm[r], v4f{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int I = (ch[r][ct][i] << 3) + cl[r][ct][i];
                        acc[r][ct][i] = fmaf(d8[i], fmaf(-dmin[r], cm[i], d[r] * (float)I), acc[r][ct][i]);
                    }
                }
            }
        }
        // buffer buf ^ 1 was last read in iteration it - 1, before this iteration's barrier
        stage_store(snext, buf ^ 1);
#pragma unroll
        for (int r = 0; r < RT; ++r) wcur[r] = wnext[r];
    }

    // output: lane holds tokens 4q .. 4q+3 of each token tile, row c16 of each row tile
    if constexpr (WK > 1) {
        __syncthreads();   // every wave is done with the staging buffers
        v4f* red = reinterpret_cast<v4f*>(&s_q8[0][0][0]);   // [WK-1][WR][RT*CT][64]
        static_assert((WK - 1) * WR * RT * CT * 64 * 16 <= (int)sizeof(s_q8), "reduction fits the staging LDS");
        if (wk > 0) {
#pragma unroll
            for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int ct = 0; ct < CT; ++ct)
                    red[(((wk - 1) * WR + wr) * RT * CT + r * CT + ct) * 64 + lane] = acc[r][ct];
        }
        __syncthreads();
        if (wk > 0) return;
#pragma unroll
        for (int w = 1; w < WK; ++w)
#pragma unroll
            for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) acc[r][ct] += red[(((w - 1) * WR + wr) * RT * CT + r * CT + ct) * 64 + lane];
    }
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int row = row0 + r * 16 + c16;
        if (row >= M) continue;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = tok0 + ct * 16 + 4 * q + i;
                if (t < T) Y[(int64_t)t * M + row] = acc[r][ct][i];
            }
    }
}

// ---------------------------------------------------------------------------
// Ring form. Every operand of a super-block reaches LDS through direct global
// -> LDS loads (global_load_lds_dwordx4), S - 1 super-blocks ahead, so a
// wave's registers hold only accumulators and the operands of one step.
// A workgroup of NW waves owns ROWS = 16*RT*NW rows of one of up to four
// matrices sharing the input, TOK = 16*CT tokens and one of p.ksplit ranges of
// p.kchunk super-blocks; wave w computes rows 16*RT*w .. +16*RT of the tile
// against all TOK tokens (C = weights x activations: output lane rows
// 4q .. 4q+3, token c16). With one K range the tile is stored to Y; with
// several, to the partial plane p.P, which gemm_reduce_kernel sums in range
// order (deterministic).
//
// A stage holds, as 16-byte slots (64 slots = one wave-wide load), each
// region rounded up to whole loads:
//   ROWS x 9 slots   the super-block of each row (144 bytes, row-major);
//   TOK x 17 slots   the Q8_K values of each token (the permuted order of
//                    quantize_q8k_planes: one 16-byte read per fragment), one
//                    spare slot a row so that the 16 tokens of a fragment read
//                    hit distinct banks;
//   TOK x 3 slots    the min-term operand and d of each token (Q8Planes::mn);
// the NPW loads a wave issues per stage cover them (the surplus and padding
// slots re-read a valid address). A wave waits for its own loads of a stage
// with s_waitcnt vmcnt (loads complete in order) before the barrier that
// publishes the stage to the other waves.
//
// F selects the weight format: 0 = Q4_K (9 slots a row, ring_block /
// ring_block32), 1 = Q6_K (14 slots a row of Q6K_LDS = 224 bytes: slots 0..12
// are block bytes 0..207 and slot 13 re-reads bytes 194..209, so no load
// leaves its 210-byte block; ring_block_q6, 16x16 tiles). Q6_K block starts
// are 2-byte aligned; global loads on gfx950 take unaligned addresses.
// 2 = Q5_K (11 slots of its 176-byte block; ring_block_q5, 16x16 tiles).
// 3 = Q8_0 with K a multiple of 256: a super-block is eight 34-byte blocks,
// 272 bytes = 17 slots a row; the activations are Q8_0 planes (p.Q.qs int8
// [T][K], p.Q.d fp32 [T][K/32]): the token's values as for Q8_K, its eight
// scales in the first two of its three min-term slots (ring_block_q80).
template <int RT, int CT, int NW, int S, int TW = 16, int F = 0>
__global__ __launch_bounds__(NW * 64) void gemm_ring_kernel(GemmParams p) {
    static_assert(TW == 16 || TW == 32, "16x16 or 32x32 output tiles");
    static_assert(F == 0 || TW == 16, "Q6_K, Q5_K and Q8_0 run on 16x16 tiles");
    constexpr int WSL = F == 1 ? 14 : F == 2 ? 11 : F == 3 ? 17 : 9;                 // 16-byte slots of a row's block
    constexpr int BB = F == 1 ? Q6K_BYTES : F == 2 ? Q5K_BYTES : F == 3 ? Q80_RING_ROW : Q4K_BYTES;   // bytes in memory
    constexpr int ROWB = 16 * WSL;                   // bytes of a row in the stage
    constexpr int TOK = CT * TW;
    constexpr int ROWS = RT * TW * NW;
    constexpr int W_SLOTS = ROWS * WSL, Q_SLOTS = TOK * 17, M_SLOTS = TOK * 3;
    constexpr int W_LOADS = (W_SLOTS + 63) / 64, Q_LOADS = (Q_SLOTS + 63) / 64, M_LOADS = (M_SLOTS + 63) / 64;
    constexpr int NLOAD = W_LOADS + Q_LOADS + M_LOADS;
    constexpr int NPW = (NLOAD + NW - 1) / NW;    // loads per wave per stage
    constexpr int STAGE = NPW * NW * 1024;
    constexpr int Q_OFF = W_LOADS * 1024, M_OFF = Q_OFF + Q_LOADS * 1024;
    __shared__ __align__(1024) uint8_t lds[S][STAGE];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c16 = lane & 15;
    const int q = lane >> 4;
    const int T = p.T, nb = p.nb;
    const int ttiles = (T + TOK - 1) / TOK;
    const int L = xcd_tile(blockIdx.x, gridDim.x);
    const int tt = L % ttiles;
    const int gt = (L / ttiles) % p.total_tiles;
    const int ks = L / (ttiles * p.total_tiles);
    int sidx = 0;
#pragma unroll
    for (int k = 1; k < GEMM_MAX_SEG; ++k)
        if (k < p.nseg && gt >= p.seg[k].tile_begin) sidx = k;
    const uint8_t* __restrict__ W = p.seg[sidx].W;
    const int M = p.seg[sidx].M;
    const int row0 = (gt - p.seg[sidx].tile_begin) * ROWS;
    const int tok0 = tt * TOK;
    const int kb0 = ks * p.kchunk;
    const int nbl = min(nb - kb0, p.kchunk);       // super-blocks of this range (>= 1)

    // per load: source of the range's first super-block, byte stride between super-blocks
    const uint8_t* src[NPW];
    uint32_t stride[NPW];
#pragma unroll
    for (int i = 0; i < NPW; ++i) {
        const int J = NW * i + wave;              // load index within the stage
        const int slot = J * 64 + lane;
        // surplus and padding: any valid address (Q8_0 planes have no min-term plane)
        src[i] = F == 3 ? reinterpret_cast<const uint8_t*>(p.Q.qs) : p.Q.mn;
        stride[i] = 0;
        if (J < W_LOADS) {
            const int r = min(row0 + slot / WSL, M - 1);
            const int sub = slot % WSL;
            src[i] = W + ((size_t)r * nb + kb0) * BB + (F == 1 && sub == 13 ? 194 : 16 * sub);
            stride[i] = BB;
        } else if (J < W_LOADS + Q_LOADS) {
            const int sl = slot - W_LOADS * 64;
            if (sl < Q_SLOTS) {
                const int tg = min(tok0 + sl / 17, T - 1);
                src[i] = reinterpret_cast<const uint8_t*>(p.Q.qs) + ((size_t)tg * nb + kb0) * 256 +
                         16 * min(sl % 17, 15);
                stride[i] = 256;
            }
        } else if (J < NLOAD) {
            const int sl = slot - (W_LOADS + Q_LOADS) * 64;
            if (sl < M_SLOTS) {
                const int tg = min(tok0 + sl / 3, T - 1);
                if constexpr (F == 3) {
                    src[i] = reinterpret_cast<const uint8_t*>(p.Q.d) + ((size_t)tg * nb + kb0) * 32 + 16 * min(sl % 3, 1);
                    stride[i] = 32;
                } else {
                    src[i] = p.Q.mn + ((size_t)tg * nb + kb0) * Q8MN_BYTES + 16 * (sl % 3);
                    stride[i] = Q8MN_BYTES;
                }
            }
        }
    }
    auto issue = [&](int b, int buf) {
#pragma unroll
        for (int i = 0; i < NPW; ++i)
            __builtin_amdgcn_global_load_lds(
                (const void*)(src[i] + (size_t)b * stride[i]),
                (__attribute__((address_space(3))) void*)(lds[buf] + (NW * i + wave) * 1024), 16, 0, 0);
    };

    typedef typename std::conditional<TW == 16, v4f, v16f>::type acc_t;
    acc_t acc[RT][CT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[r][ct] = acc_t{};

#pragma unroll
    for (int k = 0; k < S - 1; ++k) issue(min(k, nbl - 1), k);
    for (int b = 0; b < nbl; ++b) {
        const int buf = b % S;
        // this wave's loads of stage b are done (the S - 2 later stages may
        // still be in flight); the barrier publishes everyone's and retires
        // the readers of the buffer refilled next
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((S - 2) * NPW) : "memory");
        issue(min(b + S - 1, nbl - 1), (b + S - 1) % S);

        if constexpr (F == 1)
            ring_block_q6<RT, CT>(lds[buf] + (wave * RT * 16) * ROWB, lds[buf] + Q_OFF, lds[buf] + M_OFF, c16, q, acc);
        else if constexpr (F == 2)
            ring_block_q5<RT, CT>(lds[buf] + (wave * RT * 16) * ROWB, lds[buf] + Q_OFF, lds[buf] + M_OFF, c16, q, acc);
        else if constexpr (F == 3)
            ring_block_q80<RT, CT>(lds[buf] + (wave * RT * 16) * ROWB, lds[buf] + Q_OFF, lds[buf] + M_OFF, c16, q, acc);
        else if constexpr (TW == 16)
            ring_block<RT, CT>(lds[buf] + (wave * RT * 16) * Q4K_BYTES, lds[buf] + Q_OFF, lds[buf] + M_OFF, c16, q, acc);
        else
            ring_block32<RT, CT>(lds[buf] + (wave * RT * 32) * Q4K_BYTES, lds[buf] + Q_OFF, lds[buf] + M_OFF, lane, acc);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the clamped loads past the last stage

    // destination: Y of the segment, or this range's slice of the partial plane
    // (rows of all segments one after the other, p.rows in all)
    float* __restrict__ out;
    int64_t ld;
    int rbase;
    if (p.ksplit > 1) {
        out = p.P + (int64_t)ks * T * p.rows;
        ld = p.rows;
        rbase = p.seg[sidx].row_begin;
    } else {
        out = p.seg[sidx].Y;
        ld = M;
        rbase = 0;
    }
    const bool vec = ((ld | rbase) & 3) == 0;
    // a lane holds runs of 4 consecutive rows of one token: TW = 16, rows
    // 4q .. 4q+3 of each tile; TW = 32, rows 8j + 4h .. +3 for j = 0..3
    constexpr int RUNS = TW == 16 ? 1 : 4;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const int t = tok0 + ct * TW + (TW == 16 ? c16 : (lane & 31));
            if (t >= T) continue;
#pragma unroll
            for (int j = 0; j < RUNS; ++j) {
                const int rq = TW == 16 ? row0 + wave * RT * 16 + r * 16 + 4 * q
                                        : row0 + wave * RT * 32 + r * 32 + 8 * j + 4 * (lane >> 5);
                float* y = out + (int64_t)t * ld + rbase + rq;
                const v4f v = {acc[r][ct][4 * j], acc[r][ct][4 * j + 1], acc[r][ct][4 * j + 2], acc[r][ct][4 * j + 3]};
                if (vec && rq + 3 < M) {
                    *reinterpret_cast<v4f*>(y) = v;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (rq + i < M) y[i] = v[i];
                }
            }
        }
    }
}

// Y[t][r] of each segment = sum over the K ranges, in range order, of the
// partial plane P[range][t][row_begin + r]: one element a thread, every
// range's load issued before the sums.
constexpr int REDUCE_MAX_SPLIT = 32;
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmParams p) {
    const int64_t n = (int64_t)p.T * p.rows;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const int ks = p.ksplit;
    float part[REDUCE_MAX_SPLIT];
#pragma unroll
    for (int k = 0; k < REDUCE_MAX_SPLIT; ++k)
        if (k < ks) part[k] = p.P[(int64_t)k * n + i];
    float sum = part[0];
#pragma unroll
    for (int k = 1; k < REDUCE_MAX_SPLIT; ++k)
        if (k < ks) sum += part[k];
    const int t = (int)(i / p.rows);
    const int rg = (int)(i - (int64_t)t * p.rows);
    int sidx = 0;
#pragma unroll
    for (int k = 1; k < GEMM_MAX_SEG; ++k)
        if (k < p.nseg && rg >= p.seg[k].row_begin) sidx = k;
    p.seg[sidx].Y[(int64_t)t * p.seg[sidx].M + (rg - p.seg[sidx].row_begin)] = sum;
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

bool gemm_use_skinny(int T, int mode) { return mode == 1; }

// Tiled-kernel launch shapes, indexed by GemmParams::cfg (-1: chosen here).
struct TiledShape {
    int rows, tok;   // workgroup tile
    bool ring;       // ring kernel: permuted Q8_K values, K ranges
    hipError_t (*launch)(const GemmParams&, int grid, hipStream_t);
    int fmt = WF_Q4K;   // weight format the shape runs
};
template <int RT, int CT, int WR, int WK>
static hipError_t launch_tiled_(const GemmParams& p, int grid, hipStream_t st) {
    hipLaunchKernelGGL((gemm_tiled_kernel<RT, CT, WR, WK>), dim3((unsigned)grid), dim3(256), 0, st, p);
    return hipGetLastError();
}
template <int RT, int CT, int NW, int S, int TW = 16, int F = 0>
static hipError_t launch_ring_(const GemmParams& p, int grid, hipStream_t st) {
    hipLaunchKernelGGL((gemm_ring_kernel<RT, CT, NW, S, TW, F>), dim3((unsigned)grid), dim3(NW * 64), 0, st, p);
    return hipGetLastError();
}
static const TiledShape kTiled[] = {
    {256, 64, true, launch_ring_<2, 4, 8, 2>},      // 0: ring 16x16, 8 waves, 2 stages
    {128, 64, true, launch_ring_<1, 4, 8, 3>},      // 1: ring, 8 waves, 3 stages
    {128, 64, true, launch_ring_<2, 4, 4, 3>},      // 2: ring, 4 waves, 3 stages
    {64, 32, false, launch_tiled_<2, 2, 2, 2>},     // 3: register-staged, K split in two
    {32, 16, false, launch_tiled_<2, 1, 1, 4>},     // 4: register-staged, K split in four
    {128, 64, false, launch_tiled_<2, 4, 4, 1>},    // 5: register-staged
    {128, 16, true, launch_ring_<1, 1, 8, 3>},      // 6: ring, T <= 16
    {128, 32, true, launch_ring_<1, 2, 8, 3>},      // 7: ring, T <= 32
    {64, 16, true, launch_ring_<1, 1, 4, 3>},       // 8: ring, T <= 16, 4 waves
    {256, 128, true, launch_ring_<2, 8, 8, 2>},     // 9: ring, 8 waves, 2 stages of 80 KB
    {128, 128, true, launch_ring_<1, 8, 8, 2>},     // 10: ring, 8 waves, 2 stages
    {256, 64, true, launch_ring_<1, 2, 8, 2, 32>},  // 11: ring 32x32, 8 waves, 2 stages
    {128, 64, true, launch_ring_<1, 2, 4, 3, 32>},  // 12: ring 32x32, 4 waves, 3 stages
    {128, 32, true, launch_ring_<1, 1, 4, 3, 32>},  // 13: ring 32x32, T <= 32
    // Q6_K (ring_block_q6)
    {128, 64, true, launch_ring_<1, 4, 8, 3, 16, 1>, WF_Q6K},   // 14: 8 waves, 3 stages of 48 KB
    {128, 16, true, launch_ring_<1, 1, 8, 3, 16, 1>, WF_Q6K},   // 15: T <= 16
    {128, 32, true, launch_ring_<1, 2, 8, 3, 16, 1>, WF_Q6K},   // 16: T <= 32
    {256, 64, true, launch_ring_<2, 4, 8, 2, 16, 1>, WF_Q6K},   // 17: 8 waves, 2 stages of 80 KB
    {64, 64, true, launch_ring_<1, 4, 4, 3, 16, 1>, WF_Q6K},    // 18: 4 waves
    // Q5_K (ring_block_q5)
    {128, 64, true, launch_ring_<1, 4, 8, 3, 16, 2>, WF_Q5K},   // 19: 8 waves, 3 stages
    {128, 16, true, launch_ring_<1, 1, 8, 3, 16, 2>, WF_Q5K},   // 20: T <= 16
    {128, 32, true, launch_ring_<1, 2, 8, 3, 16, 2>, WF_Q5K},   // 21: T <= 32
    {128, 64, true, launch_ring_<1, 4, 8, 2, 16, 2>, WF_Q5K},   // 22: 8 waves, 2 stages
    {64, 64, true, launch_ring_<1, 4, 4, 3, 16, 2>, WF_Q5K},    // 23: 4 waves
    // Q8_0, K a multiple of 256 (F = 3)
    {128, 16, true, launch_ring_<1, 1, 8, 3, 16, 3>, WF_Q80},   // 24: T <= 16
    {128, 32, true, launch_ring_<1, 2, 8, 3, 16, 3>, WF_Q80},   // 25: T <= 32
    {128, 64, true, launch_ring_<1, 4, 8, 2, 16, 3>, WF_Q80},   // 26: 8 waves, 2 stages of 56 KB
    {64, 64, true, launch_ring_<1, 4, 4, 3, 16, 3>, WF_Q80},    // 27: 4 waves, 3 stages
    {128, 16, true, launch_ring_<1, 1, 8, 2, 16, 3>, WF_Q80},   // 28: T <= 16, 2 stages (two workgroups a CU)
    // 64 x 16 tiles, 4 waves, 3 stages (the Q4_K shape 8 of each format)
    {64, 16, true, launch_ring_<1, 1, 4, 3, 16, 1>, WF_Q6K},    // 29
    {64, 16, true, launch_ring_<1, 1, 4, 3, 16, 2>, WF_Q5K},    // 30
    {64, 16, true, launch_ring_<1, 1, 4, 3, 16, 3>, WF_Q80},    // 31
    {128, 64, true, launch_ring_<1, 2, 4, 2, 32>},   // 32: ring 32x32, 4 waves, 2 stages (two workgroups a CU)
};
constexpr int N_TILED = (int)(sizeof(kTiled) / sizeof(kTiled[0]));

int gemm_tiled_shapes() { return N_TILED; }

static int64_t row_tiles(const GemmParams& p, int rows) {
    int64_t tiles = 0;
    for (int i = 0; i < p.nseg; ++i) tiles += (p.seg[i].M + rows - 1) / rows;
    return tiles;
}

GemmPlan gemm_plan(const GemmParams& p, int num_cus, size_t max_partial_bytes) {
    GemmPlan g;
    int cfg = p.cfg;
    if (cfg >= 0 && cfg < N_TILED && kTiled[cfg].fmt != p.fmt) cfg = -1;   // a shape of the other format
    // T <= 32 (Q8_0: T <= 16, or <= 32 on 4096 rows or fewer): 64 x 16 tiles
    // of 4 waves, measured (us, against the 128-row shapes) at T = 16 on
    // 24576 x 4096 / 4096 x 12288 / 1024 x 4096: Q6_K 34.1 / 22.3 / 13.1
    // against 47.9 / 28.4 / 16.5, Q5_K 29.7 / 20.3 / 12.2 against
    // 36.6 / 23.0 / 14.0, Q8_0 44.8 / 26.5 / 15.5 against 49.9 / 28.7 / 19.5;
    // at T = 32 Q6_K 47.4 against 52.5 and Q5_K 37.9 against 46.2 on 24576
    // rows, Q8_0 66.7 against 62.3 there
    if ((cfg < 0 || cfg >= N_TILED) && p.fmt == WF_Q6K) {
        cfg = p.T <= 32 ? 29 : 14;
    } else if ((cfg < 0 || cfg >= N_TILED) && p.fmt == WF_Q5K) {
        cfg = p.T <= 32 ? 30 : 19;
    } else if ((cfg < 0 || cfg >= N_TILED) && p.fmt == WF_Q80) {
        // above 32 tokens: 128 x 64 tiles, 2 stages (4096 x 12288 at T = 512:
        // 227 us); 17..32 tokens on more than 4096 rows: 128 x 16, 2 stages
        cfg = (p.T <= 16 || (p.T <= 32 && p.rows <= 4096)) ? 31 : (p.T <= 32 ? 28 : 26);
    } else if (cfg < 0 || cfg >= N_TILED) {
        // tall (12288 rows or more) or long-K (48 super-blocks or more)
        const bool big = p.rows >= 12288 || p.nb >= 48;
        // measured on the 8B shapes (us, the choice against the next best):
        //   T = 16: 64 x 16 tiles, 4 waves: 24576 x 4096 24.5 / 28.3,
        //           4096 x 12288 17.4 / 18.7, 4096 x 4096 12.5 / 13.4
        //           (6144 x 4096 14.7 / 14.3);
        //   T = 32: the same on big matrices (24576 rows 29.2 / 38.8,
        //           4096 x 12288 21.4 / 23.6), 128 x 32 otherwise;
        //   32 < T < 128: 32x32 tiles on big matrices (24576 rows at T = 64
        //           41.4 / 48.2, 4096 x 12288 26.2 / 30.8), 128 x 32 on 4096
        //           rows (16.8 / 19.2), else 128 x 64
        if (p.T <= 16) {
            cfg = 8;
        } else if (p.T <= 32) {
            cfg = big ? 8 : 7;
        } else if (p.T < 128 && big) {
            cfg = 11;
        } else if (p.T < 128 && p.rows <= 4096) {
            cfg = 7;
        } else {
            // the largest tile that gives every CU a workgroup without a K
            // split, else 128 x 64 with one. Measured on MI355X at T = 512:
            // 256 x 64 on 32x32 MFMA tiles for 24576 rows (140 us against 155
            // on 16x16 tiles), 128 x 64 on 16x16 tiles for 4096 rows.
            // From T = 128 the 32x32 tiles also win on matrices of 6144 rows
            // or more (24 tiles of 256), measured at T = 128 / 512:
            //   6144 x 4096: 29.1 / 52.1 us against 32.1 / 64.0;
            //   24576 x 4096 at T = 128: 54.0 against 62.8.
            // They lose at 4096 rows: 4096 x 4096 at T = 512 is 50.0 against
            // 37.1, and 4096 x 12288 is 129 against 91.
            cfg = 1;
            const int64_t rt = row_tiles(p, 256);
            const int64_t g0 = rt * ((p.T + 63) / 64);
            if (g0 >= num_cus || (p.T >= 128 && rt >= 24)) cfg = 11;
            // From T = 256 on 12288 rows or more: the same 32x32 tiles in
            // 4-wave workgroups of 128 rows, two a CU, whose barriers do not
            // hold all eight waves of a CU in step (24576 x 4096 at T = 512,
            // cold weights: 164-165 against 169 us, in one run of both; 6144
            // rows: 54.3 against 52.2; T = 128 on 24576 rows: 55.0 against
            // 53.9)
            if (cfg == 11 && p.T >= 256 && p.rows >= 12288) cfg = 32;
        }
    }
    const TiledShape& s = kTiled[cfg];
    g.cfg = cfg;
    g.perm = s.ring;
    g.ksplit = 1;
    g.kchunk = p.nb;
    g.partial_bytes = 0;
    if (s.ring) {
        // split K until two workgroups per CU, keeping >= 4 super-blocks a range
        const int64_t grid0 = row_tiles(p, s.rows) * ((p.T + s.tok - 1) / s.tok);
        int64_t want = (2 * (int64_t)num_cus + grid0 - 1) / grid0;
        int64_t most = p.nb / 4 > 1 ? p.nb / 4 : 1;
        if (most > REDUCE_MAX_SPLIT) most = REDUCE_MAX_SPLIT;
        if (want > most) want = most;
        const size_t per_split = (size_t)p.T * p.rows * sizeof(float);
        while (want > 1 && (size_t)want * per_split > max_partial_bytes) --want;
        if (want > 1) {
            g.kchunk = (int)((p.nb + want - 1) / want);
            g.ksplit = (p.nb + g.kchunk - 1) / g.kchunk;
            g.partial_bytes = g.ksplit > 1 ? (size_t)g.ksplit * per_split : 0;
            if (g.ksplit == 1) g.kchunk = p.nb;
        }
    }
    return g;
}

hipError_t launch_gemm(const GemmParams& p0, hipStream_t st) {
    if (p0.cfg < 0 || p0.cfg >= N_TILED) return hipErrorInvalidValue;
    const TiledShape& s = kTiled[p0.cfg];
    if (s.fmt != p0.fmt) return hipErrorInvalidValue;
    if (!s.ring && p0.ksplit != 1) return hipErrorInvalidValue;
    GemmParams p = p0;
    int64_t tiles = 0;
    for (int i = 0; i < p.nseg; ++i) {
        p.seg[i].tile_begin = (int32_t)tiles;
        tiles += (p.seg[i].M + s.rows - 1) / s.rows;
    }
    for (int i = p.nseg; i < GEMM_MAX_SEG; ++i) p.seg[i].tile_begin = INT32_MAX;
    p.total_tiles = (int32_t)tiles;
    const int64_t grid = tiles * ((p.T + s.tok - 1) / s.tok) * p.ksplit;
    if (grid > INT32_MAX) return hipErrorInvalidValue;
    hipError_t e = s.launch(p, (int)grid, st);
    if (e != hipSuccess || p.ksplit == 1) return e;
    const int64_t n = (int64_t)p.T * p.rows;
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace spq4k
