// k_gemv.hip — fused Q4_K / Q6_K GEMV for decode (T <= 8 tokens) on gfx950.
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
// The kernels are templates over the weight format (FmtQ4K, FmtQ5K, FmtQ6K):
// the same lane mapping serves Q5_K and Q6_K blocks (q5k_core.h, q6k_core.h),
// whose CPU counterparts are ggml_vec_dot_q5_K_q8_K and _q6_K_q8_K
// (ggml-cpu/arch/x86/quants.c:2078, :2288).
#include "gemv_core.h"
#include "launch.h"
#include "q5k_core.h"
#include "q6k_core.h"

namespace spq4k {

template <typename Fmt, int T, int BPR, int WAVES, int U, bool PREQ>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(GemvParams p) {
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
    const size_t row_bytes = (size_t)nb * Fmt::BYTES;
    // rows past M re-read row M-1 (in bounds) and contribute nothing
    const uint8_t* __restrict__ wrow = W + (size_t)(row_ok ? row : M - 1) * row_bytes;

    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.0f;

    const int CB = p.chunk_blocks;
    const Q8Lds L = q8lds_carve(smem, T * CB);
    if (PREQ) {
        stream_row<Fmt, T, BPR, U>(
            wrow, row_ok, l4, bsub, nb, CB, L, acc, [&](int, int) { return 0; },
            [&](int c0, int nblk, int) { stage_q8_from_planes<WAVES * 64>(p.Q, nb, T, c0, nblk, L, CB); });
    } else {
        stream_row<Fmt, T, BPR, U>(
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

// Sum of squares of the lane's 16 x values in double (ggml_float), as the
// CPU's rms_norm accumulates them (ops.cpp:3757-3761: each square rounded to
// fp32, then added in double).
__device__ __forceinline__ double sumsq16(const XRegs& r) {
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < 16; ++j) s += (double)(r.x[j] * r.x[j]);
    return s;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// silu(x) = x / (1 + e^-x) (ggml_silu_f32, ggml-cpu/vec.h:1064-1066)
__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }

// T = 1 decode kernel. One wave per output row: lane (bsub, l4) = (lane >> 2,
// lane & 3) takes quarter l4 of blocks bsub, bsub + 16, ... of the row, so the
// Q8_K data those quarters need is loaded into registers once and reused for
// every row the wave processes. A workgroup of WAVES waves is one CU's share:
// x is quantised once per workgroup (by the first ceil(NB/4) waves, four
// blocks each) into LDS, and wave g = blockIdx * WAVES + w processes the rows
// g, g + G, g + 2G, ... of the concatenated segments (G = waves in the grid),
// with D rows of loads in flight. With XFW the quantising waves fetch and
// quantise x before issuing their own weight loads, so that x is not queued
// behind the weight requests of the whole CU. The row loop takes one of four
// forms: OP (every wave at most D rows: no loop), EI (one row in flight, the
// next row's loads issued on the current row's arrival, results stored once
// a wave), DYN2 (two rows at a time, the later rows claimed within the
// workgroup), or the static loop (the rest: fused forms, one row a wave).
// NORM: x is RMS-normalised and multiplied by p.norm_w before quantisation
// (ggml_rms_norm + ggml_mul, ggml-cpu/ops.cpp:3724-3784): the quantising
// waves reduce the sum of squares in double across the workgroup (one more
// barrier), then scale their values as (x * s) * w.
// GLU (D = 2): segments 0 and 1 are the gate and up matrices of equal M; wave
// g takes rows g, g + G, ... of both (the two rows in flight are gate r and
// up r) and stores silu(gate r . x) * (up r . x) to segment 0's output
// (ggml_silu + ggml_mul, forward.cpp:1703-1706).
// RT: the row length is p.nb, any value up to NB (NB a multiple of 16, the
// registers and LDS sized for NB); otherwise exactly NB blocks, known at
// compile time.
template <typename Fmt, int NB, int WAVES, int D, bool XFW, bool NORM, bool GLU, bool RT, bool STAMP = false,
          bool OP = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_decode_kernel(GemvParams p) {
    static_assert(!GLU || D == 2, "the fused gate/up pair is the two rows in flight");
    static_assert(!STAMP || !GLU, "timestamps cover the unfused form");
    static_assert(!OP || (D > 1 && !GLU), "one pass of D rows a wave (OP) is an unfused form with D > 1");
    // EI: one row in flight, the next row's loads issued early, results
    // stored once a wave (K <= 4096; at K = 12288 the two-row forms are faster)
    constexpr int NIT_ = (NB + 15) / 16;
    constexpr bool EI = D == 1 && !GLU && !OP && NIT_ == 1;
    // DYN2: two rows in flight, rows claimed from the workgroup's counter
    constexpr bool DYN2 = D == 2 && !GLU && !OP;
    // STAMP: the wave's start, its quantisation barrier, its first row done
    // and its last row's store issued (s_memrealtime, 100 MHz), written by lane 0 at
    // the end, after the last load (a store earlier would enter the vmcnt
    // accounting of the loads in flight)
    uint64_t st0 = 0, st1 = 0, st2 = 0;
    if constexpr (STAMP) st0 = __builtin_amdgcn_s_memrealtime();
    static_assert(!RT || NB % 16 == 0, "a runtime row length is bounded by whole 16-block passes");
    using W = typename Fmt::W;
    constexpr int NIT = (NB + 15) / 16;           // blocks per lane per row
    constexpr int QWMAX = (NB + 3) / 4;           // quantising waves at most
    constexpr int PASSES = (QWMAX + WAVES - 1) / WAVES;
    const int nb = RT ? p.nb : NB;                // blocks per row
    const int QW = (nb + 3) / 4;                  // quantising waves
    const size_t ROWB = (size_t)nb * Fmt::BYTES;
    __shared__ __align__(16) char q8s[q8lds_bytes(NB)];
    __shared__ int next_slot;                    // DYN2: the workgroup's next row slot
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l4 = lane & 3;
    const int bsub = lane >> 2;
    const int Mtot = GLU ? p.seg[0].M : p.total_rows;   // logical rows
    const int G = gridDim.x * WAVES;
    const int g = blockIdx.x * WAVES + wave;
    const int nrows = g < Mtot ? (Mtot - 1 - g) / G + 1 : 0;

    // segment table read once at kernel start into named scalars (an array
    // indexed by the segment would be placed in scratch); unused segments
    // have row_begin = INT32_MAX and are never selected
    const uint8_t* const W0 = p.seg[0].W;
    const uint8_t* const W1 = p.seg[1].W;
    const uint8_t* const W2 = p.seg[2].W;
    const uint8_t* const W3 = p.seg[3].W;
    float* const Y0 = p.seg[0].Y;
    float* const Y1 = p.seg[1].Y;
    float* const Y2 = p.seg[2].Y;
    float* const Y3 = p.seg[3].Y;
    const int R1 = p.seg[1].row_begin, R2 = p.seg[2].row_begin, R3 = p.seg[3].row_begin;
    struct Loc {
        const uint8_t* w;
        float* y;
        int row;
    };
    auto locate = [&](int r) {
        Loc l;
        if (r >= R3) { l.w = W3; l.y = Y3; l.row = r - R3; }
        else if (r >= R2) { l.w = W2; l.y = Y2; l.row = r - R2; }
        else if (r >= R1) { l.w = W1; l.y = Y1; l.row = r - R1; }
        else { l.w = W0; l.y = Y0; l.row = r; }
        return l;
    };
    W buf[EI ? 2 : D][NIT];
    // rows past the end re-read the last row (in bounds; never stored): the
    // first D loads are unconditional so that the compiler's wait counts for
    // x stay exact (a load under a branch makes it wait for every load)
    auto load_row = [&](int i, W (&b)[NIT]) {
        const int r0 = g + i * G;
        const int r = r0 < Mtot ? r0 : Mtot - 1;
        const Loc l = locate(r);
        const uint8_t* wr = l.w + (size_t)l.row * ROWB;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int bb = bsub + 16 * it;
            b[it] = Fmt::load(wr + (size_t)(bb < nb ? bb : nb - 1) * Fmt::BYTES, l4);
        }
    };
    // row r (< Mtot) of the concatenated segments
    auto load_at = [&](int r, W (&b)[NIT]) {
        const Loc l = locate(r);
        const uint8_t* wr = l.w + (size_t)l.row * ROWB;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int bb = bsub + 16 * it;
            b[it] = Fmt::load(wr + (size_t)(bb < nb ? bb : nb - 1) * Fmt::BYTES, l4);
        }
    };
    // GLU: row r of gate (which = 0) or up (which = 1)
    auto load_glu = [&](int i, int which, W (&b)[NIT]) {
        const int r0 = g + i * G;
        const int r = r0 < Mtot ? r0 : Mtot - 1;
        const uint8_t* wr = (which ? W1 : W0) + (size_t)r * ROWB;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int bb = bsub + 16 * it;
            b[it] = Fmt::load(wr + (size_t)(bb < nb ? bb : nb - 1) * Fmt::BYTES, l4);
        }
    };

    // activations: quantising waves load x first
    XRegs xr[PASSES];
    XRegs nw[NORM ? PASSES : 1];
    int xb[PASSES];
    bool xv[PASSES];
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
        const int qw = ps * WAVES + wave;
        const int item = qw * 4 + (lane >> 4);
        xv[ps] = qw < QW && item < nb;
        xb[ps] = item < nb ? item : nb - 1;
        if (qw < QW) xr[ps] = load_x16(p.X, 0, 0, xb[ps]);
        if (NORM && qw < QW) nw[NORM ? ps : 0] = load_x16(p.norm_w, 0, 0, xb[ps]);
    }
    const Q8Lds L = q8lds_carve(q8s, NB);
    if (NORM) {
        // sum of squares of x over the workgroup, in double; every wave adds
        // the WAVES partials in the same order, so all get the same scale
        __shared__ double ssq[WAVES];
        double s = 0.0;
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps)
            if (ps * WAVES + wave < QW && xv[ps]) s += sumsq16(xr[ps]);
        s = wave_sum_f64(s);
        if (lane == 0) ssq[wave] = s;
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        double S = 0.0;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) S += ssq[w];
        const float mean = (float)(S / (double)(nb * QK));
        const float scale = 1.0f / sqrtf(mean + p.eps);
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps)
#pragma unroll
            for (int j = 0; j < 16; ++j) xr[ps].x[j] = xr[ps].x[j] * scale * nw[NORM ? ps : 0].x[j];
    }
    auto quantise = [&]() {
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps) {
            if (ps * WAVES + wave < QW) store_q8_item(xr[ps], xv[ps], xb[ps], L);
        }
    };
    if (XFW) {
        quantise();
        __builtin_amdgcn_sched_barrier(0);
    }
    // LATE (two rows in flight, weights first): only the first row's loads go
    // out with x's; the second row's follow the quantisation barrier, before
    // the first row is consumed, so x does not queue behind both rows
    constexpr bool LATE = D == 2 && !XFW && !GLU;
    if (GLU) {
        load_glu(0, 0, buf[0]);
        load_glu(0, 1, buf[D - 1]);
    } else {
#pragma unroll
        for (int u = 0; u < D; ++u)
            if (!LATE || u == 0) load_row(u, buf[u]);
    }
    if (!XFW) quantise();
    if (DYN2 && threadIdx.x == 0) next_slot = 0;
    // all quantised blocks visible (LDS writes only: weight loads stay in flight)
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    if constexpr (STAMP) st1 = __builtin_amdgcn_s_memrealtime();
    if (LATE) load_row(1, buf[1]);

    typename Fmt::R qr[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int bb = bsub + 16 * it;
        Fmt::load_reg(L, bb < nb ? bb : nb - 1, l4, qr[it]);
    }
    if (GLU) {
        for (int i = 0; i < nrows; ++i) {
            float a2[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                float acc = 0.0f;
#pragma unroll
                for (int it = 0; it < NIT; ++it) {
                    const float a = Fmt::dot_reg(buf[u * (D - 1)][it], l4, qr[it], acc);
                    acc = (bsub + 16 * it < nb) ? a : acc;
                }
                a2[u] = group_sum_last<64>(acc);
            }
            if (lane == 63) Y0[g + i * G] = silu_f32(a2[0]) * a2[1];
            if (i + 1 < nrows) {
                load_glu(i + 1, 0, buf[0]);
                load_glu(i + 1, 1, buf[D - 1]);
            }
        }
        return;
    }
    // the dot product of the row in buffer b with x, in lane 63
    auto dot_row = [&](const W (&b)[NIT]) -> float {
        float acc = 0.0f;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const float a = Fmt::dot_reg(b[it], l4, qr[it], acc);
            acc = (bsub + 16 * it < nb) ? a : acc;
        }
        return group_sum_last<64>(acc);
    };
    // row r of the concatenated segments from the buffer b; first: the wave's first row
    auto consume_row = [&](int r, bool first, const W (&b)[NIT]) {
        const float acc = dot_row(b);
        if (lane == 63) {
            const Loc l = locate(r);
            l.y[l.row] = acc;
        }
        if constexpr (STAMP)
            if (first) st2 = __builtin_amdgcn_s_memrealtime();
    };
    auto consume = [&](int i, const W (&b)[NIT]) { consume_row(g + i * G, i == 0, b); };
    auto finish = [&]() {
        if constexpr (STAMP) {
            const uint64_t st3 = __builtin_amdgcn_s_memrealtime();
            if (lane == 0) {
                uint64_t* s = p.stamps + ((size_t)blockIdx.x * WAVES + wave) * 4;
                s[0] = st0;
                s[1] = st1;
                s[2] = st2;
                s[3] = st3;
            }
        }
    };
    if constexpr (OP) {
        // Every wave has at most D rows (the down projection's two): the
        // pass written out, with no loop. At a loop header (the tail loop
        // below), paths with different buffers loaded last meet and the
        // compiler waits there for every load in flight, so the first row
        // would wait for the second's loads too (issued late, after the
        // quantisation barrier) and both rows would be consumed only after
        // the second arrived.
#pragma unroll
        for (int u = 0; u < D; ++u)
            if (u < nrows) consume(u, buf[u]);
        finish();
        return;
    }
    if (EI && Mtot > G) {
        // One row in flight, the next row's loads issued as soon as the
        // current row has arrived, before its dot product: the wave's
        // compute no longer sits between one row's arrival and the next
        // row's request. (Issuing them earlier, two rows in flight, is slower
        // at these sizes; so is claiming rows from a workgroup counter.)
        // Taken when waves have two rows or more; a wave of one row runs the
        // loop below. Two buffers alternate. The results are collected in a
        // register, lane k holding the wave's row k, and stored together at
        // the end (every 64 rows): with no store in the loop, the wait for
        // each row is for that row's loads alone (a store in flight would be
        // waited for too, and a load into a register that a store in flight
        // reads waits for everything before it). A load past the wave's last
        // row re-reads that row (cached), so that the loop is entered and
        // re-entered with the same loads in flight.
        if (nrows > 0) {
            auto row_of = [&](int i) { return g + (i < nrows ? i : nrows - 1) * G; };
            float res = 0.0f;
            auto flush = [&](int i0, int n) {
                const int r = g + (i0 + lane) * G;
                if (lane < n) {
                    float* y = r >= R3 ? Y3 + (r - R3) : r >= R2 ? Y2 + (r - R2) : r >= R1 ? Y1 + (r - R1) : Y0 + r;
                    *y = res;
                }
            };
            auto put = [&](int i, float acc) {
                const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 63));
                res = lane == (i & 63) ? v : res;
                if ((i & 63) == 63) flush(i - 63, 64);
            };
            arrived<NIT>(buf[0]);
            load_at(row_of(1), buf[EI]);
            put(0, dot_row(buf[0]));
            if constexpr (STAMP) st2 = __builtin_amdgcn_s_memrealtime();
            int i = 1;
            for (; i + 1 < nrows; i += 2) {
                arrived<NIT>(buf[EI]);
                load_at(row_of(i + 1), buf[0]);
                put(i, dot_row(buf[EI]));
                arrived<NIT>(buf[0]);
                load_at(row_of(i + 2), buf[EI]);
                put(i + 1, dot_row(buf[0]));
            }
            if (i < nrows) put(i, dot_row(buf[EI]));
            if (nrows & 63) flush(nrows & ~63, nrows & 63);
        }
        finish();
        return;
    }
    if (DYN2 && Mtot > 2 * G) {
        // Two rows requested at a time, the rows after each wave's first two
        // (slots wave and wave + WAVES, rows g and g + G) claimed from the
        // workgroup's LDS counter: slot j of workgroup b is row
        // b * WAVES + j % WAVES + (j / WAVES) * G, so a wave whose rows arrive
        // early takes more of them and the waves of a CU end closer together
        // (lm_head's ended up to 7.5 us apart in the static order). Every
        // pass consumes each buffer and reloads it with a claimed row; the
        // first claim past the rows ends the loop and the other buffer's row
        // is consumed after it. The compiler waits for both buffers at the
        // loop header (the stores in the loop), so a wave consumes its two
        // rows after both have arrived, then requests two more; that measured
        // faster for lm_head than the static loop, which keeps two rows in
        // flight throughout. A wave with fewer than two rows has no claims to
        // make (every slot after its first two lies past the rows). Every row
        // is computed with the same arithmetic by whichever wave takes it.
        if (nrows >= 2) {
            int r0 = g, r1 = g + G;
            bool first = true;
            for (;;) {
                int slot = 0;
                if (lane == 0) slot = __hip_atomic_fetch_add(&next_slot, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                consume_row(r0, first, buf[0]);
                first = false;
                slot = __builtin_amdgcn_readfirstlane(slot) + 2 * WAVES;
                int next = blockIdx.x * WAVES + slot % WAVES + (slot / WAVES) * G;
                if (next >= Mtot) {
                    consume_row(r1, false, buf[1]);
                    break;
                }
                r0 = next;
                load_at(r0, buf[0]);
                slot = 0;
                if (lane == 0) slot = __hip_atomic_fetch_add(&next_slot, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                consume_row(r1, false, buf[1]);
                slot = __builtin_amdgcn_readfirstlane(slot) + 2 * WAVES;
                next = blockIdx.x * WAVES + slot % WAVES + (slot / WAVES) * G;
                if (next >= Mtot) {
                    consume_row(r0, false, buf[0]);
                    break;
                }
                r1 = next;
                load_at(r1, buf[1]);
            }
        } else if (nrows == 1) {
            consume_row(g, true, buf[0]);
        }
        finish();
        return;
    }
    int i0 = 0;
    if (D > 1) {
        // Whole passes whose reloads are all real rows: every pass reloads
        // every buffer, so at the loop header the oldest loads are always
        // buf[0]'s and the compiler waits for them alone. (A reload under a
        // condition inside the loop gives the header a path on which buf[0]
        // was loaded last, and the wait there becomes vmcnt(0): the rows in
        // flight would drain at every pass.)
        for (; i0 + 2 * D <= nrows; i0 += D) {
#pragma unroll
            for (int u = 0; u < D; ++u) {
                consume(i0 + u, buf[u]);
                load_row(i0 + u + D, buf[u]);
            }
        }
    }
    for (; i0 < nrows; i0 += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            const int i = i0 + u;
            if (i < nrows) {
                consume(i, buf[u]);
                if (i + D < nrows) load_row(i + D, buf[u]);
            }
        }
    }
    finish();
}

// RMS norm of T rows (one workgroup of 256 threads a row): the squares
// (fp32) summed in double by a fixed tree, mean = (float)(sum / K),
// s = 1 / sqrtf(mean + eps), y = (x * s) * w (ggml-cpu/ops.cpp:3757-3779).
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x, int64_t x_tstride, int K,
                                                       const float* __restrict__ w, float eps,
                                                       float* __restrict__ y) {
    __shared__ double part[4];
    const int t = blockIdx.x;
    const float* xr = x + (int64_t)t * x_tstride;
    double s = 0.0;
    for (int k = threadIdx.x; k < K; k += 256) s += (double)(xr[k] * xr[k]);
    s = wave_sum_f64(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    const double S = ((part[0] + part[1]) + part[2]) + part[3];
    const float mean = (float)(S / (double)K);
    const float scale = 1.0f / sqrtf(mean + eps);
    float* yr = y + (int64_t)t * K;
    for (int k = threadIdx.x; k < K; k += 256) yr[k] = xr[k] * scale * w[k];
}

__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                     float* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = silu_f32(g[i]) * u[i];
}

hipError_t launch_rms_norm(const float* x, int64_t x_tstride, int T, int K, const float* w, float eps, float* y,
                           hipStream_t st) {
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(T), dim3(256), 0, st, x, x_tstride, K, w, eps, y);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float* g, const float* u, float* y, int64_t n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, y, n);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Diagnostic: the exact integer sub-block sums S[row][b][j] exactly as the
// decode kernel's lanes form them (same loads, register layout and dot
// products: subblock_sums_reg), for one Q8_K row.
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
            Q8Reg q;
            load_q8reg(L, bb, l4, q);
            int S0, S1;
            subblock_sums_reg(w, q.a, S0, S1);
            int32_t* o = S + ((size_t)row * nb + c0 + bb) * 8 + 2 * l4;
            o[0] = S0;
            o[1] = S1;
        }
    }
}

// ---------------------------------------------------------------------------
template <typename Fmt, int T, int BPR, bool PREQ>
static hipError_t launch_tb(const GemvParams& p, int ntiles, hipStream_t st) {
    constexpr int WAVES = 4;
    constexpr int U = 2;
    const size_t lds = (size_t)q8lds_bytes(T * p.chunk_blocks);
    hipLaunchKernelGGL((gemv_kernel<Fmt, T, BPR, WAVES, U, PREQ>), dim3(ntiles), dim3(WAVES * 64), lds, st, p);
    return hipGetLastError();
}

template <typename Fmt, int T, bool PREQ>
static hipError_t launch_t(const GemvParams& p, int bpr, int ntiles, hipStream_t st) {
    switch (bpr) {
        case 1: return launch_tb<Fmt, T, 1, PREQ>(p, ntiles, st);
        case 2: return launch_tb<Fmt, T, 2, PREQ>(p, ntiles, st);
        case 4: return launch_tb<Fmt, T, 4, PREQ>(p, ntiles, st);
        case 8: return launch_tb<Fmt, T, 8, PREQ>(p, ntiles, st);
        default: return hipErrorInvalidValue;
    }
}

int gemv_rows_per_tile(int bpr) { return 4 * (64 / (4 * bpr)); }

template <typename Fmt, int NB, bool RT, int WAVES, int D, bool XFW, bool NORM = false, bool GLU = false,
          bool STAMP = false, bool OP = false>
static hipError_t launch_dec(const GemvParams& p, int grid, hipStream_t st) {
    hipLaunchKernelGGL((gemv_decode_kernel<Fmt, NB, WAVES, D, XFW, NORM, GLU, RT, STAMP, OP>), dim3(grid),
                       dim3(WAVES * 64), 0, st, p);
    return hipGetLastError();
}

// whether every wave of the launch has at most D rows (the one-pass form)
static bool one_pass(const GemvParams& p, const DecodeCfg& c) {
    return (int64_t)p.total_rows <= (int64_t)c.grid * c.waves * c.depth;
}

// the timestamped instances: the unfused Q4_K shapes the planner picks for
// rows of 4096 (o, q/k/v, gate/up, lm_head) and 12288 (down, one or two rows
// in flight)
#define SPQ_DEC_STAMPED(X) \
    X(16, 16, 1, false) X(16, 16, 1, true) X(16, 8, 2, true) X(48, 8, 2, false) X(48, 8, 1, false)

bool decode_stamps_supported(int fmt, int nb, const DecodeCfg& c) {
    if (fmt != WF_Q4K || c.norm || c.glu) return false;
#define SPQ_STOK(N, W, DD, XF) \
    if (nb == N && c.waves == W && c.depth == DD && c.xfirst == XF) return true;
    SPQ_DEC_STAMPED(SPQ_STOK)
#undef SPQ_STOK
    return false;
}

static hipError_t launch_dec_stamped(const GemvParams& p, const DecodeCfg& c, hipStream_t st) {
    if (!decode_stamps_supported(p.fmt, p.nb, c)) return hipErrorInvalidValue;
#define SPQ_STL(N, W, DD, XF)                                                                      \
    if (p.nb == N && c.waves == W && c.depth == DD && c.xfirst == XF) {                            \
        if constexpr (DD == 2 && !XF)                                                               \
            if (one_pass(p, c)) return launch_dec<FmtQ4K, N, false, W, DD, XF, false, false, true, true>(p, c.grid, st); \
        return launch_dec<FmtQ4K, N, false, W, DD, XF, false, false, true>(p, c.grid, st);         \
    }
    SPQ_DEC_STAMPED(SPQ_STL)
#undef SPQ_STL
    return hipErrorInvalidValue;
}

// launch shapes that fit the register file: K = 12288 with two rows in flight
// needs more than a 16-wave workgroup's 128 VGPRs; K = 27648 keeps 7 blocks of
// Q8_K per lane (133 VGPRs) and fits 8-wave workgroups with one row in flight
constexpr bool dec_shape_ok(int nb, int waves, int depth) {
    return !(nb >= 48 && waves == 16 && depth == 2) && !(nb > 48 && (waves > 8 || depth > 1));
}
// Q6_K holds 15 + 21 registers a block, Q5_K 20 + 19 (Q4_K 12 + 19): at
// K = 12288 a 16-wave workgroup (128 registers) or two rows in flight at 12
// waves would spill, and at K = 8192 two rows in flight at 16 waves
template <typename Fmt>
constexpr bool dec_shape_ok_fmt(int nb, int waves, int depth) {
    if (Fmt::BYTES != Q4K_BYTES && nb >= 48 && (waves == 16 || (waves == 12 && depth == 2))) return false;
    // and from 32 blocks a 16-wave workgroup holds one row in flight
    if (Fmt::BYTES != Q4K_BYTES && nb >= 32 && waves == 16 && depth == 2) return false;
    return dec_shape_ok(nb, waves, depth);
}

template <typename Fmt, int NB, bool RT = false>
static hipError_t launch_dec_nb(const GemvParams& p, const DecodeCfg& c, hipStream_t st) {
    if (c.glu || c.norm) {
        // the fused forms run x first; the gate/up pair is the two rows in flight
        if (!c.xfirst || (c.glu && c.depth != 2)) return hipErrorInvalidValue;
#define SPQ_DECF(W, DD)                                                                             \
        if constexpr (dec_shape_ok_fmt<Fmt>(NB, W, DD))                                             \
            if (c.waves == W && c.depth == DD) {                                                     \
                if (c.glu && c.norm) return launch_dec<Fmt, NB, RT, W, DD, true, true, DD == 2>(p, c.grid, st); \
                if (c.glu) return launch_dec<Fmt, NB, RT, W, DD, true, false, DD == 2>(p, c.grid, st);  \
                return launch_dec<Fmt, NB, RT, W, DD, true, true, false>(p, c.grid, st);                \
            }
        SPQ_DECF(16, 1) SPQ_DECF(16, 2) SPQ_DECF(12, 1) SPQ_DECF(12, 2) SPQ_DECF(8, 1) SPQ_DECF(8, 2)
#undef SPQ_DECF
        return hipErrorInvalidValue;
    }
#define SPQ_DEC(W, DD, X)                                                                  \
    if constexpr (dec_shape_ok_fmt<Fmt>(NB, W, DD))                                        \
        if (c.waves == W && c.depth == DD && c.xfirst == X) {                              \
            if constexpr (DD == 2 && !X)                                                   \
                if (one_pass(p, c)) return launch_dec<Fmt, NB, RT, W, DD, X, false, false, false, true>(p, c.grid, st); \
            return launch_dec<Fmt, NB, RT, W, DD, X>(p, c.grid, st);                      \
        }
    SPQ_DEC(16, 1, false) SPQ_DEC(16, 1, true) SPQ_DEC(16, 2, false) SPQ_DEC(16, 2, true)
    SPQ_DEC(12, 1, false) SPQ_DEC(12, 1, true) SPQ_DEC(12, 2, false) SPQ_DEC(12, 2, true)
    SPQ_DEC(8, 1, false) SPQ_DEC(8, 1, true) SPQ_DEC(8, 2, false) SPQ_DEC(8, 2, true)
#undef SPQ_DEC
    return hipErrorInvalidValue;
}

template <typename Fmt>
static bool dec_fused_ok(int nb, const DecodeCfg& c) {
    if (!c.xfirst || (c.glu && c.depth != 2)) return false;
    auto ok = [&](int n) {
        for (int w : {16, 12, 8})
            for (int d : {1, 2})
                if (c.waves == w && c.depth == d) return dec_shape_ok_fmt<Fmt>(n, w, d);
        return false;
    };
    return ok(nb);
}

bool decode_fused_supported(int fmt, int nb, const DecodeCfg& c) {
    if (!decode_supported(fmt, nb)) return false;
    const int nbk = decode_bucket(fmt, nb);
    if (fmt == WF_Q6K) return dec_fused_ok<FmtQ6K>(nbk, c);
    if (fmt == WF_Q5K) return dec_fused_ok<FmtQ5K>(nbk, c);
    if (fmt == WF_Q4K) return dec_fused_ok<FmtQ4K>(nbk, c);
    return false;
}

// Q4_K: K = 4096, 5120, 12288 and 27648 (the dense shapes of the 8B model and
// of the large-K configuration) compiled for their exact length; any other
// K up to 28672 runs the instance of the next multiple of 16 blocks with the
// length read at run time (decode_bucket). Q6_K / Q5_K (15 + 21 and 20 + 19
// registers a block a lane): K = 4096 and 12288 exactly, and K up to 8192 in
// the runtime-length instances of 16 and 32 blocks; longer rows would not
// fit the register file, and the generic kernel runs.
static bool decode_exact(int fmt, int nb) {
    if (fmt == WF_Q6K || fmt == WF_Q5K) return nb == 16 || nb == 48;
    return nb == 16 || nb == 20 || nb == 48 || nb == 108;
}

int decode_bucket(int fmt, int nb) {
    if (nb <= 0 || decode_exact(fmt, nb)) return nb;
    const int b = (nb + 15) / 16 * 16;
    if (fmt == WF_Q6K || fmt == WF_Q5K) return b <= 32 ? b : 0;
    return b <= DEC_MAX_NB ? b : 0;
}

bool decode_supported(int fmt, int nb) {
    if (fmt != WF_Q4K && fmt != WF_Q6K && fmt != WF_Q5K) return false;
    return decode_bucket(fmt, nb) > 0;
}

template <typename Fmt, int FMT>
static hipError_t launch_dec_bucket(const GemvParams& p, const DecodeCfg& c, hipStream_t st) {
    switch (decode_bucket(FMT, p.nb)) {
        case 16: return launch_dec_nb<Fmt, 16, true>(p, c, st);
        case 32: return launch_dec_nb<Fmt, 32, true>(p, c, st);
        default: break;
    }
    if constexpr (FMT == WF_Q4K) {
        switch (decode_bucket(WF_Q4K, p.nb)) {
            case 48: return launch_dec_nb<Fmt, 48, true>(p, c, st);
            case 64: return launch_dec_nb<Fmt, 64, true>(p, c, st);
            case 80: return launch_dec_nb<Fmt, 80, true>(p, c, st);
            case 96: return launch_dec_nb<Fmt, 96, true>(p, c, st);
            case 112: return launch_dec_nb<Fmt, 112, true>(p, c, st);
            default: break;
        }
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemv_decode(const GemvParams& p, const DecodeCfg& c, hipStream_t st) {
    if (p.stamps) return launch_dec_stamped(p, c, st);
    if (p.fmt == WF_Q6K) {
        if (p.nb == 16) return launch_dec_nb<FmtQ6K, 16>(p, c, st);
        if (p.nb == 48) return launch_dec_nb<FmtQ6K, 48>(p, c, st);
        return launch_dec_bucket<FmtQ6K, WF_Q6K>(p, c, st);
    }
    if (p.fmt == WF_Q5K) {
        if (p.nb == 16) return launch_dec_nb<FmtQ5K, 16>(p, c, st);
        if (p.nb == 48) return launch_dec_nb<FmtQ5K, 48>(p, c, st);
        return launch_dec_bucket<FmtQ5K, WF_Q5K>(p, c, st);
    }
    if (p.nb == 16) return launch_dec_nb<FmtQ4K, 16>(p, c, st);
    if (p.nb == 20) return launch_dec_nb<FmtQ4K, 20>(p, c, st);
    if (p.nb == 48) return launch_dec_nb<FmtQ4K, 48>(p, c, st);
    if (p.nb == 108) return launch_dec_nb<FmtQ4K, 108>(p, c, st);
    return launch_dec_bucket<FmtQ4K, WF_Q4K>(p, c, st);
}

template <typename Fmt>
static hipError_t launch_gemv_fmt(const GemvParams& p, int T, int bpr, int ntiles, hipStream_t st) {
    const bool pq = p.Q.qs != nullptr;
#define SPQ_T(TT) \
    case TT: return pq ? launch_t<Fmt, TT, true>(p, bpr, ntiles, st) : launch_t<Fmt, TT, false>(p, bpr, ntiles, st);
    switch (T) {
        SPQ_T(1) SPQ_T(2) SPQ_T(3) SPQ_T(4) SPQ_T(5) SPQ_T(6) SPQ_T(7) SPQ_T(8)
        default: return hipErrorInvalidValue;
    }
#undef SPQ_T
}

hipError_t launch_gemv(const GemvParams& p, int T, int bpr, int ntiles, hipStream_t st) {
    if (p.fmt == WF_Q6K) return launch_gemv_fmt<FmtQ6K>(p, T, bpr, ntiles, st);
    if (p.fmt == WF_Q5K) return launch_gemv_fmt<FmtQ5K>(p, T, bpr, ntiles, st);
    return launch_gemv_fmt<FmtQ4K>(p, T, bpr, ntiles, st);
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
