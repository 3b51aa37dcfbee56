// k_chain2.hip — a chain of dependent T = 1 Q4_K matvec stages in one
// persistent launch, with a one-hop exchange between stages (gfx950).
//
// Same stages and arithmetic as k_chain.hip (the dense decode layer of
// build_block_decode, desktop/engine/src/forward.cpp:2663-2856, and the
// output head, :3411-3413; each matvec ggml_vec_dot_q4_K_q8_K over Q8_K(x),
// ggml-cpu.c:1241-1439), with a different stage boundary. There, every
// stage ends in a grid barrier: results stored, the stores acknowledged, an
// arrival counter, a poll of the counters, then the next inputs loaded. Here
// a vector that a later stage reads travels through a shadow whose words
// hold CHAIN2_SENTINEL until written in this launch, and the reader polls the
// words themselves: a row's store is the only event its readers wait for.
//
// Workgroup (one per CU, cooperative launch): CHAIN2_XW exchange waves, then
// CW compute waves.
//   - Compute waves: the window of k_chain.hip (CH_D block-quarter pieces a
//     wave in flight across stage boundaries, lane mapping and per-lane
//     arithmetic of gemv_decode_kernel, row results to LDS). They issue no
//     global access but their weight loads, so the in-order vmcnt never
//     holds them behind an exchange.
//   - Exchange waves: store the workgroup's row results of the finished
//     stage (the caller's buffer with plain stores, the shadow with
//     agent-coherent ones), then gather the next stage's inputs into LDS
//     with global_load_lds -- shadows with the device-coherence bit (sc1),
//     re-loading any 16 bytes that still hold the sentinel -- add in0 + in1,
//     write this workgroup's slice of x_out, and keep x in LDS when a later
//     stage reads that x_out (the residual stream never leaves the CU).
//   - Then all waves normalise (sum of squares in double, one barrier) and
//     quantise x to Q8_K in the lane-major layout of chain_core.h.
//   Barriers a stage: B_OUT(t - 1) (row results in LDS), B_X (x staged),
//   B_NORM (norm stages), B_Q8 (activations ready).
//
// Memory ordering. Every exchanged word is written once per launch by an
// aligned 32-bit agent-scope store (global_store_dword sc1) and read with
// agent-coherent 32-bit accesses (global_load_lds ... sc1 moves each dword
// as one access). Coherence order on a word is: sentinel (stored by the
// previous launch, or at creation), then this launch's value; the previous
// launch's stores happen before this launch (kernel boundary), so a read
// returns the sentinel or the value, and a word that is not the sentinel is
// the value. No ordering between different words is needed: each is checked
// on its own. A result whose bits equal the sentinel (one NaN pattern) is
// passed on as CHAIN2_SUBST (another NaN). The launch after uses the other
// set; each launch refills the set its predecessor used. The last workgroup
// to finish (an acq_rel counter) flips the set for the next launch.
//
// Every wait is bounded: after CH_SPIN polls it sets the error word, which
// releases every other wait, and spq4k_chain_status reports -ETIMEDOUT.
#include "chain_core.h"

namespace spq4k {

namespace {

typedef __attribute__((address_space(1))) uint32_t gu32w;
typedef __attribute__((address_space(1))) f32x4 gf32x4;
typedef __attribute__((address_space(1))) uint64_t gu64;
typedef __attribute__((address_space(3))) float lfloat;
typedef __attribute__((address_space(3))) f32x4 lf32x4;

__device__ __forceinline__ void st_agent_u32(float* p, uint32_t v) {
    __hip_atomic_store((gu32w*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t shadow_bits(float v) {
    const uint32_t b = __float_as_uint(v);
    return b == CHAIN2_SENTINEL ? CHAIN2_SUBST : b;
}

// 1 KB of consecutive floats from global memory into LDS, 16 bytes a lane;
// COH: with the device-coherence bit (sc1) for shadows
template <bool COH>
__device__ __forceinline__ void gather_1k(const float* src, float* dst, int lane) {
    __builtin_amdgcn_global_load_lds((const void*)(src + 4 * lane), (lds_void*)dst, 16, 0, COH ? 16 : 0);
}

__device__ __forceinline__ bool lds4_has_sentinel(const float* p) {
    const f32x4 v = *(const lf32x4*)p;
    return __float_as_uint(v.x) == CHAIN2_SENTINEL || __float_as_uint(v.y) == CHAIN2_SENTINEL ||
           __float_as_uint(v.z) == CHAIN2_SENTINEL || __float_as_uint(v.w) == CHAIN2_SENTINEL;
}

// Normalise (optional) and quantise x = xs[0 .. K) of stage S to the
// lane-major Q8_K of chain_core.h. All NW waves of the workgroup: wave v
// takes blocks 4 v + (lane >> 4) (+ 4 NW ...), 16 lanes a block. The sum of
// squares (fp32 squares added in double, ops.cpp:3757-3761) is reduced in a
// fixed order, so every workgroup computes the same scale.
template <int NW>
__device__ __forceinline__ void norm_quant(const Chain2Stage& S, int v, float eps, const float* xs_gen, char* q8s,
                                           double* ssq) {
    const lfloat* xs = (const lfloat*)xs_gen;
    const int lane = threadIdx.x & 63;
    const int nb = S.nb, K = nb * QK;
    const bool norm = S.norm_w != nullptr;
    const lfloat* nw = xs + (S.kind[1] != CH2_NONE ? 2 * K : K);
    const int e = lane & 15;
    // waves 0 .. nqw - 1 own blocks (four each; wave v runs on SIMD v % 4, so
    // the work spreads evenly); the others only keep the barrier count
    const int nqw = (nb + 3) / 4;
    static_assert(4 * NW >= CHAIN_MAX_NB, "one pass of the workgroup's waves covers every block");
    const bool active = v < nqw;
    float scale = 1.0f;
    if (norm) {
        double sq = 0.0;
        if (active) {
            const int b = v * 4 + (lane >> 4);
            if (b < nb) {
                const lf32x4* s0 = (const lf32x4*)(xs + b * QK + 16 * e);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const f32x4 x = s0[k];
                    sq += (double)(x.x * x.x);
                    sq += (double)(x.y * x.y);
                    sq += (double)(x.z * x.z);
                    sq += (double)(x.w * x.w);
                }
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 64);
            if (lane == 0) ssq[v] = sq;
        }
        barrier_lds();   // B_NORM
        if (!active) return;
        double tot = 0.0;
        for (int w = 0; w < nqw; ++w) tot += ssq[w];
        const float mean = (float)(tot / (double)K);
        scale = 1.0f / sqrtf(mean + eps);
    }
    if (!active) return;
    {
        const int b1 = v * 4 + (lane >> 4);
        const bool valid = b1 < nb;
        const int b = valid ? b1 : nb - 1;
        XRegs r;
        const lf32x4* s0 = (const lf32x4*)(xs + b * QK + 16 * e);
        const lf32x4* sw = (const lf32x4*)(nw + b * QK + 16 * e);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            f32x4 x = s0[k];
            if (norm) {
                const f32x4 w = sw[k];
                x.x = x.x * scale * w.x; x.y = x.y * scale * w.y;
                x.z = x.z * scale * w.z; x.w = x.w * scale * w.w;
            }
            r.x[4 * k] = x.x; r.x[4 * k + 1] = x.y; r.x[4 * k + 2] = x.z; r.x[4 * k + 3] = x.w;
        }
        q8l_store_block(r, valid, b, q8s);
    }
}

// ---------------------------------------------------------------------------
// exchange waves (threads 0 .. 64 CHAIN2_XW - 1)
template <int CW>
__device__ void chain2_exchange(const Chain2Stage* __restrict__ st, const Chain2Params& p, float* xs_gen,
                                float* xl_gen, char* q8s, const float* ys, double* ssq) {
    constexpr int NX = 64 * CHAIN2_XW;
    lfloat* xs = (lfloat*)xs_gen;
    lfloat* xl = (lfloat*)xl_gen;
    const int xt = threadIdx.x;           // 0 .. NX - 1
    const int xw = xt >> 6, lane = xt & 63;
    const int nwg = gridDim.x, wg = blockIdx.x;
    const int G = nwg * CW;
    const int N = p.nstages;
    Chain2Sync* sy = p.sync;
    const uint32_t P = ld_agent(&sy->parity) & 1u;
    float* const sh = p.sh + (P ? p.sh_half : 0);
    {
        // refill the set the previous launch used: this workgroup's slice
        float* const old = p.sh + (P ? 0 : p.sh_half);
        const int64_t chunk = (p.sh_half + 4 * (int64_t)nwg - 1) / (4 * (int64_t)nwg) * 4;
        const int64_t lo = (int64_t)wg * chunk;
        const int64_t hi = lo + chunk < p.sh_half ? lo + chunk : p.sh_half;
        for (int64_t i = lo + 4 * xt; i < hi; i += 4 * NX) {
#pragma unroll
            for (int k = 0; k < 4; ++k) st_agent_u32(old + i + k, CHAIN2_SENTINEL);
        }
    }
    uint64_t* const stamps = p.stamps;
    auto stamp = [&](int t, int k) {
        if (stamps && xt == 0)
            *(gu64*)(stamps + ((size_t)wg * N + t) * CHAIN2_NSTAMP + k) = __builtin_amdgcn_s_memrealtime();
    };
    bool failed = false;

    // the workgroup's row results of stage t (ys[i * CW + c] is row wg * CW + c + i * G)
    auto store_results = [&](int t_) {
        // the stage's fields as wave-uniform scalars, read once (read inside
        // the per-lane loop they become vector loads, waited for with vmcnt)
        const Chain2Stage& S = st[ufl(t_)];
        const int rows = S.rows, rb1 = S.row_begin[1], rb2 = S.row_begin[2], rb3 = S.row_begin[3];
        float* const y0 = S.Y[0];
        float* const y1 = S.Y[1];
        float* const y2 = S.Y[2];
        float* const y3 = S.Y[3];
        const int64_t h0 = S.ysh[0], h1 = S.ysh[1], h2 = S.ysh[2], h3 = S.ysh[3];
        const int nr = (rows + G - 1) / G;
        for (int idx = xt; idx < nr * CW; idx += NX) {
            const int i = idx / CW, c = idx - i * CW;
            const int r = wg * CW + c + i * G;
            if (r < rows) {
                float* y = y0;
                int64_t h = h0;
                int row = r;
                if (r >= rb3) { y = y3; h = h3; row = r - rb3; }
                else if (r >= rb2) { y = y2; h = h2; row = r - rb2; }
                else if (r >= rb1) { y = y1; h = h1; row = r - rb1; }
                const float v = ys[idx];
                *(gfloat*)(y + row) = v;   // global stores: a flat one would count against lgkmcnt
                if (h >= 0) st_agent_u32(sh + h + row, shadow_bits(v));
            }
        }
    };

    for (int t = 0; t < N; ++t) {
        const Chain2Stage& S = st[ufl(t)];
        if (t > 0) {
            __builtin_amdgcn_s_barrier();   // B_OUT(t - 1)
            stamp(t - 1, 2);
            store_results(t - 1);
        }
        const int K = S.nb * QK;
        const int ninst = K / 256;         // 1 KB pieces a vector
        const int k0 = S.kind[0], k1 = S.kind[1];
        const bool has1 = k1 != CH2_NONE;
        // issue every gather: external inputs and the norm weights through
        // the caches, shadows with the coherence bit
        for (int q = xw; q < ninst; q += CHAIN2_XW) {
            if (k0 == CH2_EXT) gather_1k<false>(S.ext[0] + q * 256, xs_gen + q * 256, lane);
            else if (k0 == CH2_SHADOW) gather_1k<true>(sh + S.insh[0] + q * 256, xs_gen + q * 256, lane);
            if (k1 == CH2_EXT) gather_1k<false>(S.ext[1] + q * 256, xs_gen + K + q * 256, lane);
            else if (k1 == CH2_SHADOW) gather_1k<true>(sh + S.insh[1] + q * 256, xs_gen + K + q * 256, lane);
            if (S.norm_w) gather_1k<false>(S.norm_w + q * 256, xs_gen + (has1 ? 2 * K : K) + q * 256, lane);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
        // poll: re-load every 16 bytes that still hold the sentinel
        if (k0 == CH2_SHADOW || k1 == CH2_SHADOW) {
            for (unsigned it = 0;; ++it) {
                bool stale = false;
                for (int q = xw; q < ninst; q += CHAIN2_XW) {
                    if (k0 == CH2_SHADOW && lds4_has_sentinel(xs_gen + q * 256 + 4 * lane)) {
                        stale = true;
                        if (!failed) gather_1k<true>(sh + S.insh[0] + q * 256, xs_gen + q * 256, lane);
                    }
                    if (k1 == CH2_SHADOW && lds4_has_sentinel(xs_gen + K + q * 256 + 4 * lane)) {
                        stale = true;
                        if (!failed) gather_1k<true>(sh + S.insh[1] + q * 256, xs_gen + K + q * 256, lane);
                    }
                }
                if (!__any(stale) || failed) break;
                const bool bad = ld_agent(&sy->err) != 0;
                __builtin_amdgcn_s_waitcnt(0x0F70);
                if (__any(bad)) failed = true;
                else if (it >= CH_SPIN) {
                    if (lane == 0) __hip_atomic_store(&sy->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    failed = true;
                }
            }
        }
        stamp(t, 0);
        // x = in0 (+ in1) into xs[0 .. K); this workgroup's slice of x_out;
        // the kept copy for a later CH2_LOCAL input
        const int64_t c4 = ((int64_t)K / 4 + nwg - 1) / nwg * 4;
        const int xo_lo = (int)((int64_t)wg * c4 < K ? (int64_t)wg * c4 : K);
        const int xo_hi = (int)(xo_lo + c4 < K ? xo_lo + c4 : K);
        for (int e = 4 * xt; e < K; e += 4 * NX) {
            f32x4 a = k0 == CH2_LOCAL ? *(const lf32x4*)(xl + e) : *(const lf32x4*)(xs + e);
            if (has1) {
                const f32x4 b = k1 == CH2_LOCAL ? *(const lf32x4*)(xl + e) : *(const lf32x4*)(xs + K + e);
                a.x = a.x + b.x; a.y = a.y + b.y; a.z = a.z + b.z; a.w = a.w + b.w;
            }
            *(lf32x4*)(xs + e) = a;
            if (S.keep) *(lf32x4*)(xl + e) = a;
            if (S.xout && e >= xo_lo && e < xo_hi) {
                *(gf32x4*)(S.xout + e) = a;
                if (S.xosh >= 0) {
                    float* d = sh + S.xosh + e;
                    st_agent_u32(d, shadow_bits(a.x));
                    st_agent_u32(d + 1, shadow_bits(a.y));
                    st_agent_u32(d + 2, shadow_bits(a.z));
                    st_agent_u32(d + 3, shadow_bits(a.w));
                }
            }
        }
        barrier_lds();   // B_X(t)
        stamp(t, 3);
        norm_quant<CW + CHAIN2_XW>(S, ufl(xw), p.eps, xs_gen, q8s, ssq);
        barrier_lds();   // B_Q8(t)
        stamp(t, 1);
    }
    __builtin_amdgcn_s_barrier();   // B_OUT(N - 1)
    stamp(N - 1, 2);
    store_results(N - 1);
    // the last workgroup to finish flips the shadow set for the next launch
    // (every workgroup read the parity before its arrival)
    if (xt == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&sy->cnt, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == (uint32_t)nwg - 1) {
            __hip_atomic_store(&sy->cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&sy->parity, P ^ 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------------------
// compute waves (threads 64 CHAIN2_XW ..)
//
// Each compute wave walks its rows of every stage (rows g, g + G, ... of the
// stage's segments, G compute waves in the grid) as pieces: one Q4_K
// block-quarter a lane over 16 blocks (the lane mapping and per-lane
// arithmetic of gemv_decode_kernel; a row of nb blocks is ceil(nb / 16)
// pieces, a gate / up pair twice that). CH_D pieces are in flight in named
// register slots; the issue cursor runs CH_D pieces ahead of the consume
// cursor across stage boundaries, so the next stage's weights stream while
// the workgroup waits for its inputs. Both cursors are wave-uniform
// (scalar) state advanced by additions: a piece costs a few scalar
// instructions besides its loads and dot product.

// a wave-uniform pointer kept in scalar registers (readfirstlane of each half)
__device__ __forceinline__ const uint8_t* uflp(const uint8_t* p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = (uint32_t)ufl((int)(uint32_t)v), hi = (uint32_t)ufl((int)(uint32_t)(v >> 32));
    return (const uint8_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// address of row r of stage S (segment by segment; with glu the gate row)
__device__ __forceinline__ const uint8_t* stage_row(const Chain2Stage& S, int r) {
    const size_t rowb = (size_t)S.nb * Q4K_BYTES;
    int j = 0, b = 0;
    if (!S.glu) {
        if (r >= S.row_begin[3]) { j = 3; b = S.row_begin[3]; }
        else if (r >= S.row_begin[2]) { j = 2; b = S.row_begin[2]; }
        else if (r >= S.row_begin[1]) { j = 1; b = S.row_begin[1]; }
    }
    const uint8_t* w = j == 0 ? S.W[0] : j == 1 ? S.W[1] : j == 2 ? S.W[2] : S.W[3];
    return uflp(w + (size_t)(r - b) * rowb);
}

template <int CH_CW, int CH_D>
__device__ void chain2_compute(const Chain2Stage* __restrict__ st, int N, float eps, const float* xs_gen,
                               char* q8s, float* ys, double* ssq) {
    const int lane = threadIdx.x & 63;
    const int cw = ufl((int)(threadIdx.x >> 6) - CHAIN2_XW);
    const int l4 = lane & 3;
    const int bsub = lane >> 2;
    const int G = gridDim.x * CH_CW;
    const int g = ufl((int)blockIdx.x * CH_CW + cw);
    // this lane's byte offsets in a piece: header dword l4 and the 32 qs
    // bytes of quarter l4 of block bsub of the piece's 16 blocks
    const uint32_t off_h = (uint32_t)(bsub * Q4K_BYTES + 4 * l4);
    const uint32_t off_q = (uint32_t)(bsub * Q4K_BYTES + 16 + 32 * l4);

    // The issue cursor (the stage, the row iteration and the piece in the
    // row, the stage's geometry and the current row's address) and the
    // consume cursor (the geometry only): wave-uniform plain locals, so they
    // stay in scalar registers. Both read the stage table when they move to
    // another row or stage.
    int is = 0, inrow = 0, iii = 0, iip = 0, init = 1, ippr = 1, inb = 1, iglu = 0;
    const uint8_t* irow = nullptr;   // the current row (the gate row with glu)
    const uint8_t* iup = nullptr;    // the up row (glu)
    // the issue cursor at the first row of stage t or of the first later
    // stage with rows for this wave (is = N past the end)
    // (Every path assigns every variable: stores of different variables on
    // the two sides of a branch get merged into one store through a selected
    // address, and the variables then live in scratch memory.)
    auto issue_enter = [&](int t) {
        t = ufl(t);
        while (t < N && rows_of(st[t].rows, g, G) == 0) t = ufl(t + 1);
        const Chain2Stage& S = st[t < N ? t : 0];
        is = t;
        inrow = t < N ? ufl(rows_of(S.rows, g, G)) : 0;
        iii = 0;
        iip = 0;
        inb = S.nb;
        init = (S.nb + 15) >> 4;
        iglu = S.glu;
        ippr = S.glu ? 2 * init : init;
        irow = stage_row(S, g);
        iup = uflp(S.W[1] + (size_t)g * S.nb * Q4K_BYTES);
    };
    auto issue_next_row = [&]() {
        iip = 0;
        if (++iii < inrow) {
            const Chain2Stage& S = st[is];
            const int r = g + iii * G;
            irow = stage_row(S, r);
            iup = uflp(S.W[1] + (size_t)r * S.nb * Q4K_BYTES);
        } else {
            issue_enter(is + 1);
        }
    };
    int cs = 0, cnrow = 0, cii = 0, cip = 0, cnit = 1, cppr = 1, cnb = 1, cglu = 0;
    // the consume cursor at stage t (a stage without rows for this wave still
    // has its boundary run)
    auto consume_enter = [&](int t) {
        cs = ufl(t);
        cii = 0;
        cip = 0;
        const Chain2Stage& S = st[cs < N ? cs : 0];
        cnrow = cs < N ? ufl(rows_of(S.rows, g, G)) : 0;
        cnb = S.nb;
        cnit = (S.nb + 15) >> 4;
        cglu = S.glu;
        cppr = S.glu ? 2 * cnit : cnit;
    };
    issue_enter(0);
    consume_enter(0);
    while (cs < N && cnrow == 0) consume_enter(cs + 1);

    // a wave with no rows at all streams a valid address
    const uint8_t* last = st[0].W[0];
    typedef __attribute__((address_space(1))) const uint32_t gu32;
    typedef __attribute__((address_space(1))) const u32x4 gu32x4;
    // the issue cursor's piece into SLOT, then advance it; past the chain's
    // end the window re-reads the last address (the empty asm keeps the
    // compiler from replacing that load by a copy of an earlier slot, a copy
    // that would wait for its load)
    auto fill = [&](Piece& slot) {
        const uint8_t* base;
        uint32_t oh = off_h, oq = off_q;
        if (is < N) {
            const int half = (iglu && iip >= init) ? 1 : 0;
            const int it = iip - half * init;
            base = uflp((half ? iup : irow) + (size_t)it * (16 * Q4K_BYTES));
            // a partial last pass: lanes past the row re-read its last block
            const bool past = bsub + 16 * it >= inb;
            const uint32_t lb = (uint32_t)((inb - 1 - 16 * it) * Q4K_BYTES);
            oh = past ? lb + 4 * l4 : oh;
            oq = past ? lb + 16 + 32 * l4 : oq;
            last = base;
            if (++iip == ippr) issue_next_row();
        } else {
            base = last;
        }
        asm volatile("" : "+v"(oh), "+v"(oq));
        slot.h = *(gu32*)(base + oh);
        const gu32x4* q = (gu32x4*)(base + oq);
        slot.qa = q[0];
        slot.qb = q[1];
    };

    Piece slot0, slot1, slot2, slot3, slot4, slot5, slot6, slot7;
    fill(slot0);
    fill(slot1);
    if constexpr (CH_D > 2) fill(slot2);
    if constexpr (CH_D > 3) fill(slot3);
    if constexpr (CH_D > 4) fill(slot4);
    if constexpr (CH_D > 5) fill(slot5);
    if constexpr (CH_D > 6) fill(slot6);
    if constexpr (CH_D > 7) fill(slot7);

    // ---- stage boundary: the exchange waves have staged x; all waves
    // normalise and quantise it (norm_quant), then read the Q8_K from LDS
    int loaded = -1;   // stage whose activations are in LDS
    auto boundary = [&](int t) {
        if (t > 0) barrier_lds();                                   // B_OUT(t - 1)
        __builtin_amdgcn_s_barrier();                               // B_X(t)
        norm_quant<CH_CW + CHAIN2_XW>(st[t], ufl((int)(threadIdx.x >> 6)), eps, xs_gen, q8s, ssq);
        barrier_lds();                                              // B_Q8(t)
    };
    float acc0 = 0.0f, acc1 = 0.0f;
    // One consume step on window slot SLOT: the piece under the consume
    // cursor (running the boundaries of the stages it enters), then the slot
    // refilled. The loop body below is the slots written out (every slot a
    // named register set; an indexed one would be placed in scratch) and the
    // loads stay in issue order, so the compiler waits for one slot's loads
    // at a time (CH_D - 1 pieces stay in flight).
    auto step = [&](Piece& slot) {
        if (cs < N) {
            while (loaded < cs) boundary(++loaded);
            const int half = (cglu && cip >= cnit) ? 1 : 0;
            const int it = cip - half * cnit;
            float a = half ? acc1 : acc0;
            Q8Reg qx;
            q8l_read(q8s, it, lane, qx);
            const float na = piece_dot(slot, l4, qx, a);
            a = bsub + 16 * it < cnb ? na : a;
            if (half) acc1 = a;
            else acc0 = a;
            if (cip + 1 == cppr) {
                const float s0 = group_sum_last<64>(acc0);
                float v = s0;
                if (cglu) v = chain_silu(s0) * group_sum_last<64>(acc1);
                // lane 63 holds the row's sum; every lane stores it (one value,
                // one address), so no branch on the lane splits the step
                ys[cii * CH_CW + cw] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
                acc0 = 0.0f;
                acc1 = 0.0f;
                cip = 0;
                if (++cii == cnrow) {
                    // the next stage with rows for this wave; the boundaries of
                    // the stages between run when its first piece is consumed
                    do consume_enter(cs + 1);
                    while (cs < N && cnrow == 0);
                }
            } else {
                ++cip;
            }
        }
        fill(slot);
    };
    static_assert(CH_D >= 2 && CH_D <= 8, "the window steps below are written out for two to eight slots");
    // The one exit is at the top of the loop: an exit from inside a step
    // would give the loop header a path on which the latest loads are an
    // earlier slot's, and the compiler would then drain the whole window
    // (vmcnt(0)) at every pass. Steps past the chain's end consume nothing
    // and re-load the last address.
    while (cs < N) {
        step(slot0);
        step(slot1);
        if constexpr (CH_D > 2) step(slot2);
        if constexpr (CH_D > 3) step(slot3);
        if constexpr (CH_D > 4) step(slot4);
        if constexpr (CH_D > 5) step(slot5);
        if constexpr (CH_D > 6) step(slot6);
        if constexpr (CH_D > 7) step(slot7);
    }
    // the boundaries of the stages after this wave's last row
    while (loaded < N - 1) boundary(++loaded);
    barrier_lds();   // B_OUT(N - 1)
    __builtin_amdgcn_s_waitcnt(0x0F70);   // the window's trailing loads
}

template <int CW, int CH_D>
__global__ __launch_bounds__((CW + CHAIN2_XW) * 64, 1) void chain2_kernel(const Chain2Stage* __restrict__ st,
                                                                          Chain2Params p) {
    extern __shared__ __align__(16) float chain2_smem[];   // xs[CHAIN_MAX_K], then xl[CHAIN_MAX_K]
    __shared__ __align__(16) char q8s[CH_MAXIT * CH_Q8L_PASS];
    __shared__ __align__(16) float ys[CHAIN_YCAP];
    __shared__ double ssq[CW + CHAIN2_XW];
    // the role by the wave-uniform wave index (a test on threadIdx.x would be
    // a divergent branch to the compiler, and every cursor in the roles'
    // loops would then live in vector registers)
    if (ufl((int)(threadIdx.x >> 6)) < CHAIN2_XW)
        chain2_exchange<CW>(st, p, chain2_smem, chain2_smem + CHAIN_MAX_K, q8s, ys, ssq);
    else
        chain2_compute<CW, CH_D>(st, p.nstages, p.eps, chain2_smem, q8s, ys, ssq);
}

constexpr int CH2_CW = 12;

}  // namespace

int chain2_compute_waves() { return CH2_CW; }

hipError_t launch_chain2(const Chain2Stage* st, const Chain2Params& p, int grid, int depth, hipStream_t stream) {
    const size_t smem = 2 * (size_t)CHAIN_MAX_K * sizeof(float);
    const void* fn;
    switch (depth) {
        case 2: fn = (const void*)chain2_kernel<CH2_CW, 2>; break;
        case 3: fn = (const void*)chain2_kernel<CH2_CW, 3>; break;
        case 4: fn = (const void*)chain2_kernel<CH2_CW, 4>; break;
        case 6: fn = (const void*)chain2_kernel<CH2_CW, 6>; break;
        default: return hipErrorInvalidValue;
    }
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) return e;
    const Chain2Stage* a0 = st;
    Chain2Params a1 = p;
    void* args[] = {(void*)&a0, (void*)&a1};
    return hipLaunchCooperativeKernel(fn, dim3(grid), dim3((CH2_CW + CHAIN2_XW) * 64), args, smem, stream);
}

}  // namespace spq4k
