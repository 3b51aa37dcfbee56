// k_chain.hip — a chain of dependent T = 1 Q4_K matvec stages in one
// persistent launch on gfx950.
//
// The dense decode layer of the reference (build_block_decode,
// desktop/engine/src/forward.cpp:2663-2856) is, around its attention core,
//     xa = rms_norm(x) * attn_norm;  q, k, v = Wq xa, Wk xa, Wv xa
//     x  = x + Wo attn
//     xb = rms_norm(x) * ffn_norm;   h = silu(Wgate xb) * (Wup xb)
//     x  = x + Wdown h
// and the step ends with logits = Wout (rms_norm(x) * output_norm)
// (:3411-3413). Each matvec there is a ggml MUL_MAT node whose CPU kernel
// quantises its input to Q8_K and runs ggml_vec_dot_q4_K_q8_K per row
// (ggml-cpu.c:1241-1439). As separate launches, every node pays a launch gap
// and the ramp and drain of its load stream (about 2 us a node at decode
// sizes). Here one cooperative launch runs the whole chain:
//
//   stage s:  x = in0 (+ in1)              ggml_add (fp32, exact)
//             xout = x                     the residual, when asked for
//             x = rms_norm(x) * norm_w     when norm_w is given (the CPU's arithmetic)
//             x8 = Q8_K(x)                 quantize_row_q8_K_ref, bit-exact
//             y_j = W_j . x8  (j < 4)      q/k/v style: matrices sharing x
//             or y = silu(Wg . x8) * (Wu . x8)   the gate/up pair (GLU)
//
// Workgroup (one per CU): wave 0 is the control wave, waves 1..8 compute.
//   - Compute waves only ever have weight loads in flight. Wave g (of the
//     grid's G compute waves) takes rows g, g + G, ... of every stage; a row
//     is processed as pieces of one Q4_K block-quarter a lane (the lane
//     mapping and per-lane arithmetic of gemv_decode_kernel: lane (bsub, l4)
//     takes quarter l4 of blocks bsub, bsub + 16, bsub + 32), and CH_D
//     pieces are in flight per wave in a register window that runs across
//     stage boundaries: the weights of the next stage stream while the grid
//     waits for the current one. Row results go to LDS.
//   - The control wave does everything that would otherwise drain the
//     compute waves' in-order load counters: it stores the workgroup's row
//     results (agent-coherent stores), waits for them, arrives at the grid
//     barrier, waits for the other workgroups, then fetches the next
//     stage's inputs straight into LDS with agent-coherent loads.
//   - Inside the workgroup the stages are separated by four s_barriers:
//     B_IN (inputs staged), B_NORM (sum-of-squares partials, norm stages
//     only), B_Q8 (Q8_K activations in LDS), B_OUT (row results in LDS).
//
// Grid barrier: CH_NCTR counters 256 B apart; workgroup w adds 1 to counter
// w % CH_NCTR (agent-scope atomic), and the control wave's lanes 0..15 poll
// all counters (a single counter serialises 256 same-address atomics, about
// 4 us a stage against 1.7 us for 16). Counters only grow: a launch's
// targets start from gen * nstages * (grid / CH_NCTR), where gen counts the
// chain's earlier launches (read by every workgroup before its first
// arrival, advanced by workgroup 0 once all have arrived once). Every wait
// is bounded: after CH_SPIN polls it sets the error word, and a set error
// word releases every wait, so the grid always drains.
//
// Memory ordering. The exchanged vectors (row results, residuals) are
// written only with agent-scope atomic stores (global_store sc1) and read
// only with agent-scope loads (global_load_lds sc1), never with plain
// accesses. The writer's control wave waits for its stores to complete
// (s_waitcnt vmcnt(0)) before its arrival RMW; a reader's control wave
// issues the next stage's loads only after its poll has returned every
// arrival (the loads follow a completed s_waitcnt on the poll and a branch
// on its value). An agent-scope release RMW compiles on gfx950 to
// buffer_wbl2 sc1 + s_waitcnt vmcnt(0) before the RMW, and an acquire to
// buffer_inv sc1 after the load: the write-back and the invalidate serve
// plain accesses that may sit in a non-coherent L2 or L1, which this
// exchange does not make; the completion wait, which is what orders
// agent-scope atomic stores, is here. So the sequence is the compiler's own
// release / acquire for agent-scope atomic data minus the cache maintenance
// that only plain data needs. In the HIP (C++) model the relaxed accesses
// alone do not order different locations; the order rests on the ISA's
// completion and in-order issue. With the formal release / acquire pair the
// 8B step runs 1.96 ms instead of 1.56 ms (the write-back and invalidate at
// every stage boundary).
#include "chain_core.h"

namespace spq4k {

namespace {

// ---------------------------------------------------------------------------
// control wave
template <int CH_CW>
__device__ void chain_control(const ChainStage* __restrict__ st, ChainSync* __restrict__ sy, int N, float eps,
                              float* xs, const float* ys) {
    (void)eps;
    const int lane = threadIdx.x & 63;
    const int nwg = gridDim.x;
    const int G = nwg * CH_CW;
    const uint32_t per_ctr = (uint32_t)(nwg / CHAIN_NCTR);
    const uint32_t gen = ld_agent(&sy->gen);
    const uint32_t base = gen * (uint32_t)N * per_ctr;
    bool gen_done = blockIdx.x != 0;

    // until every workgroup has arrived for stages 0..s (or the error word is set)
    auto grid_wait = [&](int s) {
        const uint32_t tgt = base + (uint32_t)(s + 1) * per_ctr;
        for (uint32_t it = 0;; ++it) {
            bool ok = true, bad = false;
            if (lane < CHAIN_NCTR) ok = (int32_t)(ld_agent(&sy->ctr[lane * 64]) - tgt) >= 0;
            else if (lane == CHAIN_NCTR) bad = ld_agent(&sy->err) != 0;
            if (__all(ok) || __any(bad)) break;
            if (it >= CH_SPIN) {
                if (lane == 0) __hip_atomic_store(&sy->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    };
    auto bump_gen = [&]() {
        if (lane == 0) __hip_atomic_fetch_add(&sy->gen, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        gen_done = true;
    };

    for (int s = 0; s < N; ++s) {
        const ChainStage& S = st[s];
        const int K = S.nb * QK;
        if (s > 0) {
            grid_wait(s - 1);
            if (!gen_done) bump_gen();   // every workgroup has read gen by now
        }
        stage_vec_lds(S.in0, xs, K);
        if (S.in1) stage_vec_lds(S.in1, xs + K, K);
        if (S.norm_w) stage_vec_lds(S.norm_w, xs + (S.in1 ? 2 * K : K), K);
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the inputs are in LDS
        __builtin_amdgcn_s_barrier();         // B_IN
        if (S.xout) {
            for (int e = blockIdx.x * 64 + lane; e < K; e += nwg * 64) {
                const float v = S.in1 ? xs[e] + xs[K + e] : xs[e];
                st_agent(S.xout + e, v);
            }
        }
        if (S.norm_w) __builtin_amdgcn_s_barrier();   // B_NORM
        __builtin_amdgcn_s_barrier();                 // B_Q8
        __builtin_amdgcn_s_barrier();                 // B_OUT: the stage's row results are in LDS
        // the workgroup's rows r = (blockIdx * CH_CW + c) + i * G, result ys[i * CH_CW + c]
        const int nr = (S.rows + G - 1) / G;
        for (int idx = lane; idx < nr * CH_CW; idx += 64) {
            const int i = idx / CH_CW, c = idx - i * CH_CW;
            const int r = blockIdx.x * CH_CW + c + i * G;
            if (r < S.rows) {
                float* y;
                int row;
                if (r >= S.row_begin[3]) { y = S.Y[3]; row = r - S.row_begin[3]; }
                else if (r >= S.row_begin[2]) { y = S.Y[2]; row = r - S.row_begin[2]; }
                else if (r >= S.row_begin[1]) { y = S.Y[1]; row = r - S.row_begin[1]; }
                else { y = S.Y[0]; row = r; }
                st_agent(y + row, ys[idx]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): results and residual stored
        if (lane == 0)
            __hip_atomic_fetch_add(&sy->ctr[(blockIdx.x % CHAIN_NCTR) * 64], 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!gen_done) {
        grid_wait(N - 1);
        bump_gen();
    }
}


template <int CH_CW, int CH_D>
__device__ void chain_compute(const ChainStage* __restrict__ st, int N, float eps, const float* xs_gen, char* q8s,
                              float* ys, double* ssq) {
    // the staged inputs through an LDS-typed pointer: a generic one would
    // compile to flat loads, which count against vmcnt as well
    const __attribute__((address_space(3))) float* xs = (const __attribute__((address_space(3))) float*)xs_gen;
    const int lane = threadIdx.x & 63;
    const int cw = ufl((int)(threadIdx.x >> 6) - 1);
    const int l4 = lane & 3;
    const int bsub = lane >> 2;
    const int G = gridDim.x * CH_CW;
    const int g = ufl((int)blockIdx.x * CH_CW + cw);

    // ---- issue cursor: stage, row iteration, piece of the row, and the
    // stage's geometry and matrices (wave-uniform scalars)
    int is = 0, ii = 0, ip = 0, i_nrow = 0, i_nit = 1, i_ppr = 1, i_nb = 1, i_glu = 0;
    int i_R1 = 0, i_R2 = 0, i_R3 = 0;
    const uint8_t *i_W0 = nullptr, *i_W1 = nullptr, *i_W2 = nullptr, *i_W3 = nullptr;
#define SPQ_I_ENTER(S_)                                                                  \
    {                                                                                    \
        is = ufl(S_);                                                                    \
        ii = 0;                                                                          \
        ip = 0;                                                                          \
        if (is < N) {                                                                    \
            const ChainStage& S = st[is];                                                \
            i_nrow = ufl(rows_of(S.rows, g, G));                                              \
            i_nb = S.nb;                                                                 \
            i_nit = (i_nb + 15) >> 4;                                                    \
            i_glu = S.glu;                                                               \
            i_ppr = i_glu ? 2 * i_nit : i_nit;                                           \
            i_W0 = S.W[0]; i_W1 = S.W[1]; i_W2 = S.W[2]; i_W3 = S.W[3];                  \
            i_R1 = S.row_begin[1]; i_R2 = S.row_begin[2]; i_R3 = S.row_begin[3];         \
        } else {                                                                         \
            i_nrow = 0;                                                                  \
        }                                                                                \
    }
#define SPQ_I_SETTLE() { while (is < N && ii >= i_nrow) SPQ_I_ENTER(is + 1) }
#define SPQ_I_STEP()                                                                     \
    {                                                                                    \
        if (++ip == i_ppr) { ip = 0; ++ii; }                                             \
        SPQ_I_SETTLE()                                                                   \
    }
    SPQ_I_ENTER(0)
    SPQ_I_SETTLE()
    // a wave with no rows at all still streams a valid address
    const uint8_t* last = st[0].W[0];
    // block address of the issue cursor's piece (clamped in bounds), or the
    // previous one once the chain is exhausted
    auto issue_addr = [&]() -> const uint8_t* {
        if (is >= N) return last;
        const int half = (i_glu && ip >= i_nit) ? 1 : 0;
        const int it = ip - half * i_nit;
        int r = g + ii * G;
        const uint8_t* w;
        if (i_glu) {
            w = half ? i_W1 : i_W0;
        } else if (r >= i_R3) { w = i_W3; r -= i_R3; }
        else if (r >= i_R2) { w = i_W2; r -= i_R2; }
        else if (r >= i_R1) { w = i_W1; r -= i_R1; }
        else { w = i_W0; }
        const int b = bsub + 16 * it;
        return w + ((size_t)r * i_nb + (b < i_nb ? b : i_nb - 1)) * Q4K_BYTES;
    };

    // the window: six named slots (an array would be merged into one
    // dynamically indexed copy of the step and placed in scratch)
    Piece slot0, slot1, slot2, slot3, slot4, slot5, slot6, slot7;
    // Past the chain's end the window re-reads the last address; the empty
    // asm hides that from the compiler, which would otherwise replace the
    // load by a copy of the earlier slot -- a copy that waits for its load.
#define SPQ_FILL(SLOT)                                                                   \
    {                                                                                    \
        const uint8_t* a_ = issue_addr();                                                \
        last = a_;                                                                       \
        asm volatile("" : "+v"(a_));                                                     \
        SLOT = load_piece(a_, l4);                                                       \
        if (is < N) SPQ_I_STEP()                                                         \
    }
    SPQ_FILL(slot0) SPQ_FILL(slot1) SPQ_FILL(slot2) SPQ_FILL(slot3)
    if constexpr (CH_D > 4) SPQ_FILL(slot4)
    if constexpr (CH_D > 5) SPQ_FILL(slot5)
    if constexpr (CH_D > 6) SPQ_FILL(slot6)
    if constexpr (CH_D > 7) SPQ_FILL(slot7)

    // ---- stage boundary: inputs of stage t -> Q8_K in LDS -> this lane's registers
    int loaded = -1;   // stage whose activations are in LDS
    auto boundary = [&](int t) {
        const ChainStage& S = st[t];
        const int nb = S.nb, K = nb * QK;
        const bool has1 = S.in1 != nullptr, norm = S.norm_w != nullptr;
        const __attribute__((address_space(3))) float* x1 = xs + K;
        const __attribute__((address_space(3))) float* nw = xs + (has1 ? 2 * K : K);
        if (t > 0) barrier_lds();            // B_OUT(t - 1)
        __builtin_amdgcn_s_barrier();        // B_IN(t)
        const int e = lane & 15;
        float scale = 1.0f;
        if (norm) {
            double sq = 0.0;
            for (int b0 = 0; b0 < nb; b0 += 4 * CH_CW) {
                const int b = b0 + cw * 4 + (lane >> 4);
                if (b < nb) {
                    lfloat4* s0 = (lfloat4*)(xs + b * QK + 16 * e);
                    lfloat4* s1 = (lfloat4*)(x1 + b * QK + 16 * e);
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        f32x4 v = s0[k];
                        if (has1) {
                            const f32x4 w = s1[k];
                            v.x = v.x + w.x; v.y = v.y + w.y; v.z = v.z + w.z; v.w = v.w + w.w;
                        }
                        sq += (double)(v.x * v.x);
                        sq += (double)(v.y * v.y);
                        sq += (double)(v.z * v.z);
                        sq += (double)(v.w * v.w);
                    }
                }
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 64);
            if (lane == 0) ssq[cw] = sq;
            barrier_lds();                    // B_NORM
            double tot = 0.0;
#pragma unroll
            for (int w = 0; w < CH_CW; ++w) tot += ssq[w];
            const float mean = (float)(tot / (double)K);
            scale = 1.0f / sqrtf(mean + eps);
        }
        for (int b0 = 0; b0 < nb; b0 += 4 * CH_CW) {
            const int b1 = b0 + cw * 4 + (lane >> 4);
            const bool valid = b1 < nb;
            const int b = valid ? b1 : nb - 1;
            XRegs r;
            lfloat4* s0 = (lfloat4*)(xs + b * QK + 16 * e);
            lfloat4* s1 = (lfloat4*)(x1 + b * QK + 16 * e);
            lfloat4* sw = (lfloat4*)(nw + b * QK + 16 * e);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                f32x4 v = s0[k];
                if (has1) {
                    const f32x4 w = s1[k];
                    v.x = v.x + w.x; v.y = v.y + w.y; v.z = v.z + w.z; v.w = v.w + w.w;
                }
                if (norm) {
                    const f32x4 w = sw[k];
                    v.x = v.x * scale * w.x; v.y = v.y * scale * w.y;
                    v.z = v.z * scale * w.z; v.w = v.w * scale * w.w;
                }
                r.x[4 * k] = v.x; r.x[4 * k + 1] = v.y; r.x[4 * k + 2] = v.z; r.x[4 * k + 3] = v.w;
            }
            q8l_store_block(r, valid, b, q8s);
        }
        barrier_lds();                        // B_Q8(t)
    };

    // ---- consume cursor (does not skip stages: a stage without rows for
    // this wave still runs its boundary, whose barriers the workgroup shares)
    int cs = 0, ci = 0, cp = 0, c_nrow = 0, c_nit = 1, c_ppr = 1, c_nb = 1, c_glu = 0;
#define SPQ_C_ENTER(S_)                                                                  \
    {                                                                                    \
        cs = ufl(S_);                                                                    \
        ci = 0;                                                                          \
        cp = 0;                                                                          \
        if (cs < N) {                                                                    \
            const ChainStage& S = st[cs];                                                \
            c_nrow = ufl(rows_of(S.rows, g, G));                                              \
            c_nb = S.nb;                                                                 \
            c_nit = (c_nb + 15) >> 4;                                                    \
            c_glu = S.glu;                                                               \
            c_ppr = c_glu ? 2 * c_nit : c_nit;                                           \
        } else {                                                                         \
            c_nrow = 0;                                                                  \
        }                                                                                \
    }
    SPQ_C_ENTER(0)
    float acc0 = 0.0f, acc1 = 0.0f;
    // One consume step on window slot SLOT. The loop body below is the
    // window's slots 0, 1, .., CH_D - 1 written out: every slot is a named
    // register set (an indexed one would be placed in scratch), and the
    // loads stay in issue order on every path, so the compiler's vmcnt
    // waits are exact (CH_D - 1 pieces stay in flight). Crossing into a
    // stage runs its boundary in place; that code is inlined once per slot
    // but runs once per stage.
#define SPQ_CHAIN_STEP(SLOT)                                                             \
    {                                                                                    \
        while (cs < N && ci >= c_nrow) SPQ_C_ENTER(cs + 1)                               \
        if (cs < N) {                                                                    \
        while (loaded < cs) {                                                            \
            ++loaded;                                                                    \
            boundary(loaded);                                                            \
        }                                                                                \
        const int half = (c_glu && cp >= c_nit) ? 1 : 0;                                 \
        const int it = cp - half * c_nit;                                                \
        const bool live = bsub + 16 * it < c_nb;                                         \
        float a = half ? acc1 : acc0;                                                    \
        Q8Reg qx;                                                                        \
        q8l_read(q8s, it, lane, qx);                                                     \
        const float na = piece_dot(SLOT, l4, qx, a);                                     \
        a = live ? na : a;                                                               \
        if (half) acc1 = a;                                                              \
        else acc0 = a;                                                                   \
        if (cp + 1 == c_ppr) {                                                           \
            const float s0 = group_sum_last<64>(acc0);                                   \
            float v = s0;                                                                \
            if (c_glu) v = chain_silu(s0) * group_sum_last<64>(acc1);                    \
            if (lane == 63) ys[ci * CH_CW + cw] = v;                                     \
            acc0 = 0.0f;                                                                 \
            acc1 = 0.0f;                                                                 \
        }                                                                                \
        if (++cp == c_ppr) { cp = 0; ++ci; }                                             \
        }                                                                                \
        SPQ_FILL(SLOT)                                                                   \
    }
    static_assert(CH_D >= 4 && CH_D <= 8, "the window steps below are written out for four to eight slots");
    // The one exit is at the top of the loop: an exit from inside a step
    // would give the loop header a path on which the latest loads are an
    // earlier slot's, and the compiler would then drain the whole window
    // (vmcnt(0)) at every pass. Steps past the chain's end consume nothing
    // and re-load the last address.
    for (;;) {
        while (cs < N && ci >= c_nrow) SPQ_C_ENTER(cs + 1)
        if (cs >= N) break;
        SPQ_CHAIN_STEP(slot0)
        SPQ_CHAIN_STEP(slot1)
        SPQ_CHAIN_STEP(slot2)
        SPQ_CHAIN_STEP(slot3)
        if constexpr (CH_D > 4) SPQ_CHAIN_STEP(slot4)
        if constexpr (CH_D > 5) SPQ_CHAIN_STEP(slot5)
        if constexpr (CH_D > 6) SPQ_CHAIN_STEP(slot6)
        if constexpr (CH_D > 7) SPQ_CHAIN_STEP(slot7)
    }
#undef SPQ_CHAIN_STEP
#undef SPQ_FILL
#undef SPQ_C_ENTER
#undef SPQ_I_STEP
#undef SPQ_I_SETTLE
#undef SPQ_I_ENTER
    while (loaded < N - 1) {
        ++loaded;
        boundary(loaded);
    }
    barrier_lds();   // B_OUT(N - 1)
    __builtin_amdgcn_s_waitcnt(0x0F70);   // the window's trailing loads
}

// The stage table is a separate __restrict__ argument so that its reads are
// scalar loads: a vector load in a compute wave would have to wait for the
// whole weight window ahead of it (vmcnt counts in issue order).
template <int CH_CW, int CH_D>
__global__ __launch_bounds__((CH_CW + 1) * 64, 1) void chain_kernel(const ChainStage* __restrict__ st,
                                                                    ChainSync* __restrict__ sync, int nstages,
                                                                    float eps) {
    extern __shared__ __align__(16) float chain_xs[];        // CHAIN_MAX_K fp32: the staged inputs
    __shared__ __align__(16) char q8s[CH_MAXIT * CH_Q8L_PASS];
    __shared__ __align__(16) float ys[CHAIN_YCAP];
    __shared__ double ssq[CH_CW];
    if (threadIdx.x < 64) chain_control<CH_CW>(st, sync, nstages, eps, chain_xs, ys);
    else chain_compute<CH_CW, CH_D>(st, nstages, eps, chain_xs, q8s, ys, ssq);
}

}  // namespace

int chain_grid(int num_cus) { return (num_cus / CHAIN_NCTR) * CHAIN_NCTR; }

template <int CW, int D>
static hipError_t launch_chain_t(const ChainParams& p, int grid, hipStream_t st) {
    const size_t smem = (size_t)CHAIN_MAX_K * sizeof(float);
    const void* fn = (const void*)chain_kernel<CW, D>;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) return e;
    const ChainStage* a0 = p.st;
    ChainSync* a1 = p.sync;
    int a2 = p.nstages;
    float a3 = p.eps;
    void* args[] = {(void*)&a0, (void*)&a1, (void*)&a2, (void*)&a3};
    return hipLaunchCooperativeKernel(fn, dim3(grid), dim3((CW + 1) * 64), args, smem, st);
}

int chain_compute_waves(int shape) { return shape == 2 ? 7 : 8; }

hipError_t launch_chain(const ChainParams& p, int grid, int shape, hipStream_t st) {
    switch (shape) {
        case 0: return launch_chain_t<8, 8>(p, grid, st);
        case 1: return launch_chain_t<8, 6>(p, grid, st);
        case 2: return launch_chain_t<7, 8>(p, grid, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace spq4k
