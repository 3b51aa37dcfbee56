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
//      the compacted list of active experts and, per expert, its pairs.
//      Out-of-range ids are not routed (their outputs are left untouched; the
//      host entry points reject them).
//   2. quantize_q8k_planes_kernel: the T*ne11 input rows to Q8_K planes.
//   3. moe_gemv_kernel: workgroup (a, tile) takes active expert a and a tile
//      of its rows; its pairs are processed TC at a time, each chunk staged
//      from the Q8_K planes into LDS and streamed with the dense GEMV's code.
// Calls with at most MOE_FUSED_MAX_PAIRS pairs use moe_fused_kernel instead,
// which does all three steps in one launch. The sdot4 kernels (moe_gemv,
// moe_fused, moe_decode) are templates over the weight format and also run
// Q6_K and Q5_K expert banks (FmtQ6K, FmtQ5K); the matrix-core ring runs
// Q4_K and Q6_K (F = 1).
#include "gemv_core.h"
#include "launch.h"
#include "q5k_core.h"
#include "q6k_core.h"
#include "ring_core.h"

namespace spq4k {

// Routing tables of one call, built by one workgroup of 256 threads: the ids
// pass through LDS in chunks; per-expert counts by LDS atomics; a parallel
// scan gives each expert's first pair and the compacted list of active
// experts (ascending); the pairs are then placed by LDS atomics (their order
// inside an expert is not fixed, and no output depends on it: every pair's
// result is computed from its own input row and expert alone).
// LDS: cnt[E], pos[E], ids[ROUTE_CHUNK], partial[2 * 256] ints.
constexpr int ROUTE_CHUNK = 2048;
size_t moe_route_lds_bytes(int E) { return ((size_t)2 * E + ROUTE_CHUNK + 512) * sizeof(int); }

__device__ void route_block(const int32_t* __restrict__ ids, int n_pairs, int E, const MoeRoute& r, int* sh) {
    int* cnt = sh;
    int* pos = sh + E;
    int* idl = sh + 2 * E;
    int* part = idl + ROUTE_CHUNK;   // [256] pairs, [256] active experts
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += 256) cnt[e] = 0;
    __syncthreads();
    for (int base = 0; base < n_pairs; base += ROUTE_CHUNK) {
        const int n = min(ROUTE_CHUNK, n_pairs - base);
        for (int i = tid; i < n; i += 256) idl[i] = ids[base + i];
        __syncthreads();
        for (int i = tid; i < n; i += 256) {
            const int e = idl[i];
            if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
        }
        __syncthreads();
    }
    // thread t scans experts [t * per, (t + 1) * per)
    const int per = (E + 255) / 256;
    const int e0 = min(tid * per, E), e1 = min(e0 + per, E);
    int sp = 0, sa = 0;
    for (int e = e0; e < e1; ++e) {
        sp += cnt[e];
        sa += cnt[e] > 0;
    }
    // exclusive scan of (sp, sa) over the 256 threads: within each wave by
    // shuffles, then the four wave totals
    const int lane = tid & 63, wv = tid >> 6;
    int ip = sp, ia = sa;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int tp = __shfl_up(ip, o), ta = __shfl_up(ia, o);
        if (lane >= o) {
            ip += tp;
            ia += ta;
        }
    }
    if (lane == 63) {
        part[wv] = ip;
        part[256 + wv] = ia;
    }
    __syncthreads();
    int rp = ip - sp, ra = ia - sa;
    for (int w = 0; w < wv; ++w) {
        rp += part[w];
        ra += part[256 + w];
    }
    if (tid == 255) *r.n_act = ra + sa;
    for (int e = e0; e < e1; ++e) {
        pos[e] = rp;
        if (cnt[e] > 0) {
            r.act[ra] = e;
            r.act_off[ra] = rp;
            r.act_cnt[ra] = cnt[e];
            ++ra;
        }
        rp += cnt[e];
    }
    __syncthreads();
    for (int base = 0; base < n_pairs; base += ROUTE_CHUNK) {
        const int n = min(ROUTE_CHUNK, n_pairs - base);
        for (int i = tid; i < n; i += 256) idl[i] = ids[base + i];
        __syncthreads();
        for (int i = tid; i < n; i += 256) {
            const int e = idl[i];
            if (e >= 0 && e < E) r.pairs[atomicAdd(&pos[e], 1)] = base + i;
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void moe_route_kernel(const int32_t* __restrict__ ids, int n_pairs, int E,
                                                        MoeRoute r) {
    extern __shared__ int sh[];
    route_block(ids, n_pairs, E, r, sh);
}

template <typename Fmt, int TC, int BPR, int WAVES, int U>
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
    const size_t row_bytes = (size_t)nb * Fmt::BYTES;
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
        stream_row<Fmt, TC, BPR, U>(wrow, row_ok, l4, bsub, nb, CB, L, acc, [&](int, int) { return 0; },
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
// Single-launch form (n_pairs <= MOE_FUSED_MAX_PAIRS): workgroup (e, tile)
// lists the (token, slot) pairs routed to expert e itself (wave 0 scans ids
// with a ballot compaction that keeps pair order), returns at once when e is
// unused, and quantises the routed input rows from fp32 into LDS as it
// streams its rows: no routing pass, no Q8_K planes, one launch per call.
template <typename Fmt, int TC, int BPR, int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void moe_fused_kernel(MoeFusedParams p) {
    extern __shared__ __align__(16) char smem[];
    constexpr int LPR = 4 * BPR;
    constexpr int RPW = 64 / LPR;
    constexpr int ROWS = WAVES * RPW;
    __shared__ int s_cnt;
    __shared__ int s_pairs[MOE_FUSED_MAX_PAIRS];
    __shared__ int s_xrow[TC];
    __shared__ int s_pair[TC];

    const int e = blockIdx.x / p.tiles_per_expert;
    const int tile = blockIdx.x - e * p.tiles_per_expert;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;

    if (wave == 0) {
        int cnt = 0;
        for (int base = 0; base < p.n_pairs; base += 64) {
            const int i = base + lane;
            const bool hit = i < p.n_pairs && p.ids[i] == e;
            const uint64_t m = __ballot(hit);
            const int before = __popcll(m & ((1ull << lane) - 1ull));
            if (hit) s_pairs[cnt + before] = i;
            cnt += __popcll(m);
        }
        if (lane == 0) s_cnt = cnt;
    }
    __syncthreads();
    const int pcnt = s_cnt;
    if (pcnt == 0) return;   // uniform over the workgroup

    const int l4 = lane & 3;
    const int bsub = (lane >> 2) & (BPR - 1);
    const int M = p.M;
    const int row = tile * ROWS + wave * RPW + lane / LPR;
    const bool row_ok = row < M;
    const int nb = p.nb;
    const uint8_t* __restrict__ wrow =
        p.bank + (size_t)e * p.expert_bytes + (size_t)(row_ok ? row : M - 1) * ((size_t)nb * Fmt::BYTES);
    const int CB = p.chunk_blocks;
    const Q8Lds L = q8lds_carve(smem, TC * CB);

    for (int c = 0; c < pcnt; c += TC) {
        const int nt = min(TC, pcnt - c);
        __syncthreads();   // the previous chunk's readers of s_pair / s_xrow are done
        if (threadIdx.x < TC) {
            const int i = min((int)threadIdx.x, nt - 1);   // clamp: duplicate slots are computed, not stored
            const int pair = s_pairs[c + i];
            const int t = pair / p.n_used;
            const int sl = pair - t * p.n_used;
            s_pair[threadIdx.x] = pair;
            s_xrow[threadIdx.x] = t * p.ne11 + (sl % p.ne11);
        }
        __syncthreads();
        float acc[TC];
#pragma unroll
        for (int t = 0; t < TC; ++t) acc[t] = 0.0f;
        stream_row<Fmt, TC, BPR, U>(wrow, row_ok, l4, bsub, nb, CB, L, acc, [&](int, int) { return 0; },
                               [&](int c0, int nblk, int) {
            // quantise block c0 + b of each routed input row into slot t * CB + b
            const int nitems = TC * nblk;
            for (int base = 0; base < nitems; base += 4 * WAVES) {
                const int item0 = base + wave * 4 + (lane >> 4);
                const bool valid = item0 < nitems;
                const int item = valid ? item0 : nitems - 1;
                const int t = item / nblk;
                const int b = item - t * nblk;
                const XRegs r = load_x16(p.X, p.K, s_xrow[t], c0 + b);
                store_q8_item(r, valid, t * CB + b, L);
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
// Small-batch form (n_pairs <= MOE_DEC_MAX_PAIRS): the decode mapping. The
// rows of all routed (token, slot) pairs form one sweep, pair p owning rows
// [p M, (p + 1) M) of expert ids[p] with input row t * ne11 + s % ne11. Every
// workgroup quantises the routed input rows once into LDS; LPR = 4 * BSL lanes
// work on one row (quarter l4 of blocks bsub, bsub + BSL, ...) and waves walk
// rows g, g + G, ... of the sweep. An expert chosen by several pairs is
// streamed once per pair, which is why this form is kept to small batches.
// An id outside [0, E) leaves that pair's outputs untouched. With a second
// bank (p.M1 > 0: the up projection beside the gate, the same ids and input)
// pair p owns rows [p (M + M1), (p + 1)(M + M1)): M rows of the first bank,
// then M1 of the second, so both go in one launch and one quantisation.
// silu(x) = x / (1 + e^-x) (ggml_silu_f32, ggml-cpu/vec.h:1064-1066), as the
// dense kernels' SwiGLU epilogue and swiglu_kernel compute it
__device__ __forceinline__ float moe_silu(float x) { return x / (1.0f + expf(-x)); }

// GLU: the gate / up pair of a MoE layer (bank, bank1 of equal M): sweep row
// (pair, r) streams gate row r and up row r of the pair's expert and stores
// silu(gate . x) * (up . x) (ggml_silu then ggml_mul, forward.cpp:1102-1103).
template <typename Fmt, int NB, int BSL, int WAVES, bool GLU>
__global__ __launch_bounds__(WAVES * 64) void moe_decode_kernel(MoeFusedParams p) {
    using W = typename Fmt::W;
    extern __shared__ __align__(16) char smem[];
    constexpr int LPR = 4 * BSL;
    constexpr int RPW = 64 / LPR;
    constexpr int RPG = WAVES * RPW;             // rows of one pass of the workgroup
    constexpr int NIT = (NB + BSL - 1) / BSL;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int l4 = lane & 3;
    const int bsub = (lane & (LPR - 1)) >> 2;
    // a pair's sweep rows: the M rows of the bank, then the M1 rows of the
    // second bank when there is one (same expert, same input row)
    const int M = p.M, MV = GLU ? p.M : p.M + p.M1;
    const int total = p.n_pairs * MV;
    // this workgroup's rows of the sweep: one contiguous run (one or two
    // pairs), so it quantises only the input rows those pairs read
    const int r0 = blockIdx.x * p.rows_per_wg;
    if (r0 >= total) return;                     // uniform over the workgroup
    const int r1 = min(total, r0 + p.rows_per_wg);
    auto xrow = [&](int r) {                     // input row of sweep row r (non-decreasing in r)
        const int pr = r / MV;
        const int t = pr / p.n_used;
        return t * p.ne11 + (pr - t * p.n_used) % p.ne11;
    };
    const int xlo = xrow(r0);
    const int nitems = (xrow(r1 - 1) - xlo + 1) * NB;
    const Q8Lds L = q8lds_carve(smem, p.xwin_rows * NB);
    const int g0 = r0 + wave * RPW + lane / LPR;

    // where row r of the sweep lives: expert (or -1), its weights and output,
    // its input window slot
    struct Loc {
        const uint8_t* w;
        const uint8_t* w1;   // GLU: the up row beside the gate row
        float* y;
        int e, xs;
    };
    auto locate = [&](int r) {
        Loc l;
        const int rc = r < r1 ? r : r1 - 1;
        const int pr = rc / MV;
        const int v = rc - pr * MV;
        const bool second = !GLU && v >= M;
        const int lr = second ? v - M : v;
        const int e = p.ids[pr];
        l.e = (r < r1 && e >= 0 && e < p.E) ? e : -1;
        l.xs = (xrow(rc) - xlo) * NB;
        const size_t eo = (size_t)(l.e >= 0 ? l.e : 0);
        l.w = (second ? p.bank1 + eo * p.expert_bytes1 : p.bank + eo * p.expert_bytes) +
              (size_t)lr * ((size_t)NB * Fmt::BYTES);
        l.w1 = GLU ? p.bank1 + eo * p.expert_bytes1 + (size_t)lr * ((size_t)NB * Fmt::BYTES) : l.w;
        l.y = second ? p.Y1 + (int64_t)pr * p.M1 + lr : p.Y + (int64_t)pr * M + lr;
        return l;
    };
    auto load = [&](const Loc& l, W (&w)[NIT], W (&w1)[GLU ? NIT : 1]) {
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int bb = bsub + BSL * it;
            w[it] = Fmt::load(l.w + (size_t)(bb < NB ? bb : NB - 1) * Fmt::BYTES, l4);
        }
        if constexpr (GLU) {
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int bb = bsub + BSL * it;
                w1[it] = Fmt::load(l.w1 + (size_t)(bb < NB ? bb : NB - 1) * Fmt::BYTES, l4);
            }
        }
    };
    // order of the loads (they complete in order): the expert ids of the
    // call (for the LDS copy the later passes read), the expert id of the
    // first row, the first pass of input rows, then the first passes'
    // weights, so that the quantisation waits only for x while the weights
    // are in flight
    __shared__ int32_t ids_s[MOE_DEC_MAX_PAIRS];
    auto locate_s = [&](int r) {                 // locate with the expert id from LDS
        Loc l;
        const int rc = r < r1 ? r : r1 - 1;
        const int pr = rc / MV;
        const int v = rc - pr * MV;
        const bool second = !GLU && v >= M;
        const int lr = second ? v - M : v;
        const int e = ids_s[pr];
        l.e = (r < r1 && e >= 0 && e < p.E) ? e : -1;
        l.xs = (xrow(rc) - xlo) * NB;
        const size_t eo = (size_t)(l.e >= 0 ? l.e : 0);
        l.w = (second ? p.bank1 + eo * p.expert_bytes1 : p.bank + eo * p.expert_bytes) +
              (size_t)lr * ((size_t)NB * Fmt::BYTES);
        l.w1 = GLU ? p.bank1 + eo * p.expert_bytes1 + (size_t)lr * ((size_t)NB * Fmt::BYTES) : l.w;
        l.y = second ? p.Y1 + (int64_t)pr * p.M1 + lr : p.Y + (int64_t)pr * M + lr;
        return l;
    };
    const int item_a = wave * 4 + (lane >> 4);
    const int ci_a = item_a < nitems ? item_a : nitems - 1;
    // passes of the workgroup's rows, DP at a time in register slots. With
    // more passes than slots, each slot is reloaded with the pass DP ahead as
    // soon as it is computed, every reload unconditional (a lane whose row
    // lies past r1 loads row r1 - 1 again and drops it) and its expert id
    // read from LDS, so the next passes' weights are in flight while these
    // are computed and the compiler's waits stay exact (a load under a
    // branch, or one whose address waits for an id load, would make it wait
    // for every load in flight). One slot for the GLU sweep, whose gate and
    // up rows already double the loads of a pass (two slots: T = 4 26.9
    // against 25.3 us for the routed-expert block), and for the down bank's
    // short rows (3 blocks: measured no faster, one token slower).
    constexpr int DP = (GLU || NB < 8) ? 1 : 2;
    const int npass = (r1 - r0 + RPG - 1) / RPG;
    Loc cur[DP];
    W w[DP][NIT];
    W w1[DP][GLU ? NIT : 1];
    // the rest of the staging (the first pass of x already loaded) and, for
    // the multi-pass form, the LDS copy of the expert ids
    auto stage_rest = [&](const XRegs& xa, bool copy_ids, int32_t id_mine) {
        store_q8_item(xa, item_a < nitems, ci_a, L);
        for (int base = 4 * WAVES; base < nitems; base += 4 * WAVES) {
            const int item0 = base + item_a;
            const bool valid = item0 < nitems;
            const int item = valid ? item0 : nitems - 1;
            const XRegs r = load_x16(p.X, p.K, xlo + item / NB, item % NB);
            store_q8_item(r, valid, item, L);
        }
        if (copy_ids && (int)threadIdx.x < p.n_pairs) ids_s[threadIdx.x] = id_mine;
        __syncthreads();
    };
    // the sweep row r (pass pd of this lane) with the weights in wv / wv1
    auto compute = [&](int pd, const Loc& l, const W (&wv)[NIT], const W (&wv1)[GLU ? NIT : 1]) {
        const int r = g0 + pd * RPG;
        float acc[1] = {0.0f};
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int bb = bsub + BSL * it;
            Fmt::template dot<1>(wv[it], l4, L, l.xs + (bb < NB ? bb : NB - 1), 0, bb < NB && l.e >= 0, acc);
        }
        float sum = group_sum_last<LPR>(acc[0]);
        if constexpr (GLU) {
            float acc1[1] = {0.0f};
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int bb = bsub + BSL * it;
                Fmt::template dot<1>(wv1[it], l4, L, l.xs + (bb < NB ? bb : NB - 1), 0, bb < NB && l.e >= 0, acc1);
            }
            sum = moe_silu(sum) * group_sum_last<LPR>(acc1[0]);
        }
        if (r < r1 && l.e >= 0 && (lane & (LPR - 1)) == LPR - 1) *l.y = sum;
    };
    if (npass > DP) {   // uniform over the workgroup
        // the call's expert ids (copied to LDS with the staging), every
        // slot's expert id, then x, then every slot's weights: a weight load
        // then waits only for its own id, and at the loop header the slots'
        // loads are in flight in slot order, as on every pass
        const int32_t id_mine = p.ids[(int)threadIdx.x < p.n_pairs ? threadIdx.x : 0];
#pragma unroll
        for (int d = 0; d < DP; ++d) cur[d] = locate(g0 + d * RPG);
        const XRegs xa = load_x16(p.X, p.K, xlo + ci_a / NB, ci_a % NB);
#pragma unroll
        for (int d = 0; d < DP; ++d) load(cur[d], w[d], w1[d]);
        stage_rest(xa, true, id_mine);
        int pass = 0;
        for (; pass + 2 * DP <= npass; pass += DP) {
#pragma unroll
            for (int d = 0; d < DP; ++d) {
                compute(pass + d, cur[d], w[d], w1[d]);
                cur[d] = locate_s(g0 + (pass + DP + d) * RPG);
                load(cur[d], w[d], w1[d]);
            }
        }
        // the last one or two rounds, written out, reloading only real passes
#pragma unroll
        for (int d = 0; d < DP; ++d) {
            if (pass + d < npass) {
                compute(pass + d, cur[d], w[d], w1[d]);
                if (pass + DP + d < npass) {
                    cur[d] = locate_s(g0 + (pass + DP + d) * RPG);
                    load(cur[d], w[d], w1[d]);
                }
            }
        }
        pass += DP;
#pragma unroll
        for (int d = 0; d < DP; ++d)
            if (pass + d < npass) compute(pass + d, cur[d], w[d], w1[d]);
    } else {
        cur[0] = locate(g0);
        const XRegs xa = load_x16(p.X, p.K, xlo + ci_a / NB, ci_a % NB);
#pragma unroll
        for (int d = 0; d < DP; ++d) {
            if (d > 0) {
                cur[d] = locate(g0 + d * RPG);
                if (d < npass) load(cur[d], w[d], w1[d]);   // uniform
            } else {
                load(cur[d], w[d], w1[d]);
            }
        }
        stage_rest(xa, false, 0);
#pragma unroll
        for (int d = 0; d < DP; ++d)
            if (d < npass) compute(d, cur[d], w[d], w1[d]);
    }
}


// The routed-expert block's down projection with the weighted sum over the
// slots as its epilogue (small batches, n_used <= 8): one wave per output
// element (t, r). Lane group grp (LPR = 4 * BSL lanes, the decode mapping of
// moe_decode_kernel) computes the dots of slots grp, grp + GPW, ...: row r of
// expert ids[t][s] against the Q8_K-quantised hidden row t * n_used + s. The
// wave then adds the fp32 products D_s * w[t][s] in double over s in slot
// order and stores their sum rounded to fp32 -- moe_combine_kernel's
// arithmetic (ggml_mul, then ggml_sum_rows' double sum, forward.cpp:1107-1116),
// so Y equals that of the separate down and combine launches bit for bit. A
// workgroup owns p.rows_per_wg consecutive elements of Y [T][M] and quantises
// the hidden rows of the tokens they belong to. An id outside [0, E)
// contributes nothing.
template <typename Fmt, int NB, int BSL, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void moe_down_sum_kernel(MoeFusedParams p, const float* __restrict__ cw,
                                                                  float* __restrict__ Yc) {
    using W = typename Fmt::W;
    extern __shared__ __align__(16) char smem[];
    constexpr int LPR = 4 * BSL, GPW = 64 / LPR, SPG = (MOE_SUM_MAX_USED + GPW - 1) / GPW;
    constexpr int NIT = (NB + BSL - 1) / BSL;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int l4 = lane & 3;
    const int bsub = (lane & (LPR - 1)) >> 2;
    const int grp = lane / LPR;
    const int M = p.M, nu = p.n_used;
    const int total = (p.n_pairs / nu) * M;
    const int u0 = blockIdx.x * p.rows_per_wg;
    if (u0 >= total) return;                     // uniform over the workgroup
    const int u1 = min(total, u0 + p.rows_per_wg);
    const int tlo = u0 / M;
    const int nitems = ((u1 - 1) / M - tlo + 1) * nu * NB;
    const Q8Lds L = q8lds_carve(smem, p.xwin_rows * NB);
    const float* __restrict__ X = p.X + (int64_t)tlo * nu * p.K;
    const size_t row_bytes = (size_t)NB * Fmt::BYTES;
    // a unit's expert ids and router weights, every load unconditional (a
    // slot past n_used reads the last one and is dropped, a unit past u1 the
    // last unit), so that no load waits behind another's branch
    auto fetch_ids = [&](int u, int (&ev)[SPG], float (&cws)[SPG * GPW]) {
        const int tu = __builtin_amdgcn_readfirstlane((u < u1 ? u : u1 - 1) / M);
#pragma unroll
        for (int k = 0; k < SPG; ++k) {
            const int s = grp + GPW * k;
            ev[k] = p.ids[tu * nu + (s < nu ? s : nu - 1)];
        }
#pragma unroll
        for (int s = 0; s < SPG * GPW; ++s) cws[s] = cw[tu * nu + (s < nu ? s : nu - 1)];
    };
    auto fetch_w = [&](int u, const int (&ev)[SPG], W (&w)[SPG][NIT], bool (&live)[SPG]) {
        const int uc = u < u1 ? u : u1 - 1;
        const int r = uc - (uc / M) * M;
#pragma unroll
        for (int k = 0; k < SPG; ++k) {
            const int s = grp + GPW * k;
            const int e = s < nu ? ev[k] : -1;
            live[k] = e >= 0 && e < p.E;
            const uint8_t* wr = p.bank + (size_t)(live[k] ? e : 0) * p.expert_bytes + (size_t)r * row_bytes;
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int bb = bsub + BSL * it;
                w[k][it] = Fmt::load(wr + (size_t)(bb < NB ? bb : NB - 1) * Fmt::BYTES, l4);
            }
        }
    };
    // order of the loads (they complete in order): the first unit's ids, the
    // first pass of hidden rows, then the unit's weights, so that the
    // quantisation waits only for x while the weights are in flight
    int u = u0 + wave;
    int ev[SPG];
    float cws[SPG * GPW];
    W w[SPG][NIT];
    bool live[SPG];
    fetch_ids(u, ev, cws);
    {
        const int item0 = wave * 4 + (lane >> 4);
        const int item = item0 < nitems ? item0 : nitems - 1;
        const XRegs xr = load_x16(X, p.K, item / NB, item % NB);
        fetch_w(u, ev, w, live);
        store_q8_item(xr, item0 < nitems, item, L);
    }
    for (int base = 4 * WAVES; base < nitems; base += 4 * WAVES) {
        const int item0 = base + wave * 4 + (lane >> 4);
        const bool valid = item0 < nitems;
        const int item = valid ? item0 : nitems - 1;
        const XRegs r = load_x16(X, p.K, item / NB, item % NB);
        store_q8_item(r, valid, item, L);
    }
    __syncthreads();
    for (; u < u1; u += WAVES) {
        const int t = u / M;
        const int r = u - t * M;
        // the wave's next unit (u is uniform over the wave) in flight while
        // this one is computed
        int evn[SPG];
        float cwn[SPG * GPW];
        W wn[SPG][NIT];
        bool liven[SPG];
        const bool more = u + WAVES < u1;
        if (more) {
            fetch_ids(u + WAVES, evn, cwn);
            fetch_w(u + WAVES, evn, wn, liven);
        }
        __builtin_amdgcn_sched_barrier(0);
        float d[SPG];
#pragma unroll
        for (int k = 0; k < SPG; ++k) {
            const int s = grp + GPW * k;
            const int xs = ((t - tlo) * nu + (s < nu ? s : 0)) * NB;
            float acc[1] = {0.0f};
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int bb = bsub + BSL * it;
                Fmt::template dot<1>(w[k][it], l4, L, xs + (bb < NB ? bb : NB - 1), 0, bb < NB && live[k], acc);
            }
            d[k] = group_sum_last<LPR>(acc[0]);
        }
        // slot s = k * GPW + g sits in lane g * LPR + LPR - 1 of dot k
        double sum = 0.0;
#pragma unroll
        for (int k = 0; k < SPG; ++k)
#pragma unroll
            for (int g = 0; g < GPW; ++g) {
                const int s = k * GPW + g;
                const float ds = __shfl(d[k], g * LPR + LPR - 1, 64);
                if (s < nu) {
                    const float prod = ds * cws[s];
                    sum += (double)prod;
                }
            }
        if (lane == 63) Yc[(int64_t)t * M + r] = (float)sum;
        if (more) {
#pragma unroll
            for (int k = 0; k < SPG; ++k) {
                ev[k] = evn[k];
                live[k] = liven[k];
#pragma unroll
                for (int it = 0; it < NIT; ++it) w[k][it] = wn[k][it];
            }
#pragma unroll
            for (int s2 = 0; s2 < SPG * GPW; ++s2) cws[s2] = cwn[s2];
        }
    }
}

template <typename Fmt, int NB, int BSL>
static hipError_t launch_mdsum(const MoeFusedParams& p, const float* cw, float* Yc, int grid, hipStream_t st) {
    constexpr int WAVES = 8;
    const size_t lds = (size_t)q8lds_bytes(p.xwin_rows * NB);
    hipLaunchKernelGGL((moe_down_sum_kernel<Fmt, NB, BSL, WAVES>), dim3(grid), dim3(WAVES * 64), lds, st, p, cw, Yc);
    return hipGetLastError();
}

template <typename Fmt>
static hipError_t launch_moe_down_sum_fmt(const MoeFusedParams& p, const float* cw, float* Yc, int grid,
                                          hipStream_t st) {
    switch (p.nb) {
        case 3: return launch_mdsum<Fmt, 3, 4>(p, cw, Yc, grid, st);
        case 8: return launch_mdsum<Fmt, 8, 8>(p, cw, Yc, grid, st);
        case 16: return launch_mdsum<Fmt, 16, 16>(p, cw, Yc, grid, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_down_sum(const MoeFusedParams& p, const float* cw, float* Yc, int grid, hipStream_t st) {
    if (p.n_used < 1 || p.n_used > MOE_SUM_MAX_USED || p.n_pairs % p.n_used) return hipErrorInvalidValue;
    if (p.fmt == WF_Q6K) return launch_moe_down_sum_fmt<FmtQ6K>(p, cw, Yc, grid, st);
    if (p.fmt == WF_Q5K) return launch_moe_down_sum_fmt<FmtQ5K>(p, cw, Yc, grid, st);
    if (p.fmt == WF_Q4K) return launch_moe_down_sum_fmt<FmtQ4K>(p, cw, Yc, grid, st);
    return hipErrorInvalidValue;
}

template <typename Fmt, int NB, int BSL>
static hipError_t launch_mdec(const MoeFusedParams& p, int grid, hipStream_t st) {
    const size_t lds = (size_t)q8lds_bytes(p.xwin_rows * NB);
    if (p.glu && p.waves == 12)
        hipLaunchKernelGGL((moe_decode_kernel<Fmt, NB, BSL, 12, true>), dim3(grid), dim3(12 * 64), lds, st, p);
    else if (p.glu)
        hipLaunchKernelGGL((moe_decode_kernel<Fmt, NB, BSL, 8, true>), dim3(grid), dim3(8 * 64), lds, st, p);
    else
        hipLaunchKernelGGL((moe_decode_kernel<Fmt, NB, BSL, 8, false>), dim3(grid), dim3(8 * 64), lds, st, p);
    return hipGetLastError();
}

bool moe_decode_supported(int nb) { return nb == 3 || nb == 8 || nb == 16; }

// rows of the sweep per workgroup pass: waves * 64 / (4 * BSL), BSL = 4, 8, 16
// for rows of 3, 8 and 16 blocks
int moe_decode_rows_per_wg(int nb, int waves) { return waves * (nb == 3 ? 4 : (nb == 8 ? 2 : 1)); }

// rows per workgroup (a whole number of passes) and the input rows the
// largest run of that many sweep rows can read
void moe_decode_plan(const MoeFusedParams& p, int grid, int32_t* rows_per_wg, int32_t* xwin_rows) {
    const int64_t MV = p.glu ? (int64_t)p.M : (int64_t)p.M + p.M1;
    const int64_t total = (int64_t)p.n_pairs * MV;
    const int64_t pass = moe_decode_rows_per_wg(p.nb, p.waves ? p.waves : 8);
    int64_t rw = (total + grid - 1) / grid;
    rw = (rw + pass - 1) / pass * pass;
    *rows_per_wg = (int32_t)rw;
    // a run of rw rows touches at most rw / MV + 2 pairs, so as many input rows
    const int64_t w = rw / MV + 2;
    *xwin_rows = (int32_t)(w < p.n_xrows ? w : p.n_xrows);
}

template <typename Fmt>
static hipError_t launch_moe_decode_fmt(const MoeFusedParams& p, int grid, hipStream_t st) {
    switch (p.nb) {
        case 3: return launch_mdec<Fmt, 3, 4>(p, grid, st);
        case 8: return launch_mdec<Fmt, 8, 8>(p, grid, st);
        case 16: return launch_mdec<Fmt, 16, 16>(p, grid, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_decode(const MoeFusedParams& p, int grid, hipStream_t st) {
    if (p.fmt == WF_Q6K) return launch_moe_decode_fmt<FmtQ6K>(p, grid, st);
    if (p.fmt == WF_Q5K) return launch_moe_decode_fmt<FmtQ5K>(p, grid, st);
    return launch_moe_decode_fmt<FmtQ4K>(p, grid, st);
}

template <typename Fmt, int TC, int BPR>
static hipError_t launch_fused_tb(const MoeFusedParams& p, int grid, hipStream_t st) {
    constexpr int WAVES = 4, U = 2;
    const size_t lds = (size_t)q8lds_bytes(TC * p.chunk_blocks);
    hipLaunchKernelGGL((moe_fused_kernel<Fmt, TC, BPR, WAVES, U>), dim3(grid), dim3(WAVES * 64), lds, st, p);
    return hipGetLastError();
}

template <typename Fmt, int TC>
static hipError_t launch_fused_t(const MoeFusedParams& p, int bpr, int grid, hipStream_t st) {
    switch (bpr) {
        case 1: return launch_fused_tb<Fmt, TC, 1>(p, grid, st);
        case 2: return launch_fused_tb<Fmt, TC, 2>(p, grid, st);
        case 4: return launch_fused_tb<Fmt, TC, 4>(p, grid, st);
        case 8: return launch_fused_tb<Fmt, TC, 8>(p, grid, st);
        default: return hipErrorInvalidValue;
    }
}

template <typename Fmt>
static hipError_t launch_moe_fused_fmt(const MoeFusedParams& p, int tc, int bpr, int grid, hipStream_t st) {
    switch (tc) {
        case 1: return launch_fused_t<Fmt, 1>(p, bpr, grid, st);
        case 2: return launch_fused_t<Fmt, 2>(p, bpr, grid, st);
        case 4: return launch_fused_t<Fmt, 4>(p, bpr, grid, st);
        case 8: return launch_fused_t<Fmt, 8>(p, bpr, grid, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_fused(const MoeFusedParams& p, int tc, int bpr, int grid, hipStream_t st) {
    if (p.fmt == WF_Q6K) return launch_moe_fused_fmt<FmtQ6K>(p, tc, bpr, grid, st);
    if (p.fmt == WF_Q5K) return launch_moe_fused_fmt<FmtQ5K>(p, tc, bpr, grid, st);
    return launch_moe_fused_fmt<FmtQ4K>(p, tc, bpr, grid, st);
}

// ---------------------------------------------------------------------------
hipError_t launch_moe_route(const int32_t* ids, int n_pairs, int E, const MoeRoute& r, hipStream_t st) {
    hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(256), moe_route_lds_bytes(E), st, ids, n_pairs, E, r);
    return hipGetLastError();
}

template <typename Fmt, int TC, int BPR>
static hipError_t launch_moe_tb(const MoeParams& p, int grid, hipStream_t st) {
    constexpr int WAVES = 4, U = 2;
    const size_t lds = (size_t)q8lds_bytes(TC * p.chunk_blocks);
    hipLaunchKernelGGL((moe_gemv_kernel<Fmt, TC, BPR, WAVES, U>), dim3(grid), dim3(WAVES * 64), lds, st, p);
    return hipGetLastError();
}

template <typename Fmt, int TC>
static hipError_t launch_moe_t(const MoeParams& p, int bpr, int grid, hipStream_t st) {
    switch (bpr) {
        case 1: return launch_moe_tb<Fmt, TC, 1>(p, grid, st);
        case 2: return launch_moe_tb<Fmt, TC, 2>(p, grid, st);
        case 4: return launch_moe_tb<Fmt, TC, 4>(p, grid, st);
        case 8: return launch_moe_tb<Fmt, TC, 8>(p, grid, st);
        default: return hipErrorInvalidValue;
    }
}

template <typename Fmt>
static hipError_t launch_moe_gemv_fmt(const MoeParams& p, int tc, int bpr, int grid, hipStream_t st) {
    switch (tc) {
        case 1: return launch_moe_t<Fmt, 1>(p, bpr, grid, st);
        case 2: return launch_moe_t<Fmt, 2>(p, bpr, grid, st);
        case 4: return launch_moe_t<Fmt, 4>(p, bpr, grid, st);
        case 8: return launch_moe_t<Fmt, 8>(p, bpr, grid, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_gemv(const MoeParams& p, int tc, int bpr, int grid, hipStream_t st) {
    if (p.fmt == WF_Q6K) return launch_moe_gemv_fmt<FmtQ6K>(p, tc, bpr, grid, st);
    if (p.fmt == WF_Q5K) return launch_moe_gemv_fmt<FmtQ5K>(p, tc, bpr, grid, st);
    return launch_moe_gemv_fmt<FmtQ4K>(p, tc, bpr, grid, st);
}


// Matrix-core form for batches whose experts receive several pairs.
//   moe_prep_kernel: workgroup 0 builds the routing tables (route_block), the
//   others quantise the input rows into permuted Q8_K planes.
//   moe_ring_kernel: workgroup (a, g) takes active expert a and its 128-row
//   tiles g*ring_rt .. +ring_rt; the expert's pairs are gathered 16 at a time
//   as the tokens of the LDS ring of gemm_ring_kernel (eight waves, one
//   16-row tile each, direct global -> LDS loads S - 1 super-blocks ahead)
//   and the row tiles follow each other in one stream, so the ring stays full
//   across them; each pair's outputs are scattered to Y[pair].
__global__ __launch_bounds__(256) void moe_prep_kernel(const int32_t* __restrict__ ids, int n_pairs, int E,
                                                       MoeRoute r, const float* __restrict__ x, int64_t x_tstride,
                                                       int n_xrows, int nb, Q8Planes Q) {
    extern __shared__ int sh[];
    if (blockIdx.x == 0) {
        route_block(ids, n_pairs, E, r, sh);
        return;
    }
    quantize_planes_items(x, x_tstride, n_xrows, nb, const_cast<int8_t*>(Q.qs), const_cast<int16_t*>(Q.bs),
                          const_cast<float*>(Q.d), const_cast<uint8_t*>(Q.mn), 1, blockIdx.x - 1);
}

// F = 1: Q6_K banks (14 slots a row, the last re-reading block bytes
// 194..209; ring_block_q6); F = 2: Q5_K banks (11 slots, ring_block_q5);
// F = 3: Q8_0 banks with K a multiple of 256 (17 slots: eight 34-byte
// blocks; Q8_0 planes, the token's eight scales in its min-term slots;
// ring_block_q80); as in gemm_ring_kernel.
template <int S, int F = 0, int NW = 8>
__global__ __launch_bounds__(NW * 64) void moe_ring_kernel(MoeParams p) {
    constexpr int ROWS = 16 * NW, TOK = 16;   // a wave's 16 rows of each row tile
    constexpr int WSL = F == 1 ? 14 : F == 2 ? 11 : F == 3 ? 17 : 9;
    constexpr int BB = F == 1 ? Q6K_BYTES : F == 2 ? Q5K_BYTES : F == 3 ? Q80_RING_ROW : Q4K_BYTES;
    constexpr int ROWB = 16 * WSL;
    constexpr int W_SLOTS = ROWS * WSL, Q_SLOTS = TOK * 17, M_SLOTS = TOK * 3;
    constexpr int W_LOADS = W_SLOTS / 64, Q_LOADS = (Q_SLOTS + 63) / 64, M_LOADS = (M_SLOTS + 63) / 64;
    constexpr int NLOAD = W_LOADS + Q_LOADS + M_LOADS;
    constexpr int NPW = (NLOAD + NW - 1) / NW;
    constexpr int STAGE = NPW * NW * 1024;
    constexpr int Q_OFF = W_LOADS * 1024, M_OFF = Q_OFF + Q_LOADS * 1024;
    __shared__ __align__(1024) uint8_t lds[S][STAGE];

    // workgroups of the second bank (if any) follow the first bank's
    const int half = p.max_act * p.tiles_per_expert;
    const bool second = p.nbank > 1 && (int)blockIdx.x >= half;
    const int bid = (int)blockIdx.x - (second ? half : 0);
    const int a = bid / p.tiles_per_expert;
    const int g = bid - a * p.tiles_per_expert;
    if (a >= *p.route.n_act) return;           // uniform over the workgroup
    const int e = p.route.act[a];
    const int poff = p.route.act_off[a];
    const int pcnt = p.route.act_cnt[a];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c16 = lane & 15;
    const int q = lane >> 4;
    const int M = p.M, nb = p.nb;
    const int rt0 = g * p.ring_rt;
    const int nrt = min(p.ring_rt, (M + ROWS - 1) / ROWS - rt0);
    const int len = nrt * nb;                  // super-blocks streamed per token tile
    const uint8_t* __restrict__ W = (second ? p.bank1 : p.bank) + (size_t)e * p.expert_bytes;
    float* __restrict__ Yb = second ? p.Y1 : p.Y;
    const size_t row_bytes = (size_t)nb * BB;

    for (int tile0 = 0; tile0 < pcnt; tile0 += TOK) {
        // per load: weight slot (row within the tile, 16-byte chunk), or the
        // activation source of super-block 0 and its stride
        const uint8_t* src[NPW];
        uint32_t stride[NPW];
        int wrow[NPW];
#pragma unroll
        for (int i = 0; i < NPW; ++i) {
            const int J = NW * i + wave;
            const int slot = J * 64 + lane;
            // surplus and padding: any valid address (Q8_0 planes have no min-term plane)
            src[i] = F == 3 ? reinterpret_cast<const uint8_t*>(p.Q.qs) : p.Q.mn;
            stride[i] = 0;
            wrow[i] = -1;
            if (J < W_LOADS) {
                wrow[i] = slot / WSL;
                const int sub = slot % WSL;
                src[i] = W + (F == 1 && sub == 13 ? 194 : 16 * sub);
            } else if (J < NLOAD) {
                const bool isq = J < W_LOADS + Q_LOADS;
                const int sl = slot - (isq ? W_LOADS : W_LOADS + Q_LOADS) * 64;
                const int per = isq ? 17 : 3;
                if (sl < TOK * per) {
                    const int pid = p.route.pairs[poff + min(tile0 + sl / per, pcnt - 1)];
                    const int xr = p.ne11 == 1 ? pid / p.n_used : pid;   // input row of the pair
                    if (isq) {
                        src[i] = reinterpret_cast<const uint8_t*>(p.Q.qs) + (size_t)xr * nb * 256 + 16 * min(sl % 17, 15);
                        stride[i] = 256;
                    } else if (F == 3) {
                        src[i] = reinterpret_cast<const uint8_t*>(p.Q.d) + (size_t)xr * nb * 32 + 16 * min(sl % 3, 1);
                        stride[i] = 32;
                    } else {
                        src[i] = p.Q.mn + (size_t)xr * nb * Q8MN_BYTES + 16 * (sl % 3);
                        stride[i] = Q8MN_BYTES;
                    }
                }
            }
        }
        auto issue = [&](int sp, int buf) {
            const int rt = rt0 + sp / nb, b = sp - (sp / nb) * nb;
#pragma unroll
            for (int i = 0; i < NPW; ++i) {
                const uint8_t* a_ = (NW * i + wave) < W_LOADS
                                        ? src[i] + (size_t)min(rt * ROWS + wrow[i], M - 1) * row_bytes + (size_t)b * BB
                                        : src[i] + (size_t)b * stride[i];
                __builtin_amdgcn_global_load_lds(
                    (const void*)a_, (__attribute__((address_space(3))) void*)(lds[buf] + (NW * i + wave) * 1024), 16, 0, 0);
            }
        };
        v4f acc[1][1] = {{v4f{0, 0, 0, 0}}};
        // the previous token tile's readers are done with every buffer
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
        for (int k = 0; k < S - 1; ++k) issue(min(k, len - 1), k);
        for (int sp = 0; sp < len; ++sp) {
            const int buf = sp % S;
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((S - 2) * NPW) : "memory");
            issue(min(sp + S - 1, len - 1), (sp + S - 1) % S);
            if constexpr (F == 1)
                ring_block_q6<1, 1>(lds[buf] + (wave * 16) * ROWB, lds[buf] + Q_OFF, lds[buf] + M_OFF, c16, q, acc);
            else if constexpr (F == 2)
                ring_block_q5<1, 1>(lds[buf] + (wave * 16) * ROWB, lds[buf] + Q_OFF, lds[buf] + M_OFF, c16, q, acc);
            else if constexpr (F == 3)
                ring_block_q80<1, 1>(lds[buf] + (wave * 16) * ROWB, lds[buf] + Q_OFF, lds[buf] + M_OFF, c16, q, acc);
            else
                ring_block<1, 1>(lds[buf] + (wave * 16) * Q4K_BYTES, lds[buf] + Q_OFF, lds[buf] + M_OFF, c16, q, acc);
            if (sp - (sp / nb) * nb == nb - 1) {
                // row tile done: lane has rows 4q .. 4q+3 of the wave's 16, pair tile0 + c16
                if (tile0 + c16 < pcnt) {
                    const int pid = p.route.pairs[poff + tile0 + c16];
                    const int rq = (rt0 + sp / nb) * ROWS + wave * 16 + 4 * q;
                    float* y = Yb + (int64_t)pid * M + rq;
                    if ((M & 3) == 0 && rq + 3 < M) {
                        *reinterpret_cast<v4f*>(y) = acc[0][0];
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (rq + i < M) y[i] = acc[0][0][i];
                    }
                }
                acc[0][0] = v4f{0, 0, 0, 0};
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
}

// Q8_0 banks: the routing tables and Q8_0 planes are already in place
// (launch_moe_route, the Q8_0 planes quantiser); the ring alone.
hipError_t launch_moe_ring_q80(const MoeParams& p, int max_act, int nw, hipStream_t st) {
    if (p.fmt != WF_Q80 || (nw != 4 && nw != 8)) return hipErrorInvalidValue;
    const int64_t grid = (int64_t)max_act * p.tiles_per_expert * (p.nbank > 1 ? 2 : 1);
    if (nw == 4)
        hipLaunchKernelGGL((moe_ring_kernel<2, 3, 4>), dim3((unsigned)grid), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL((moe_ring_kernel<2, 3, 8>), dim3((unsigned)grid), dim3(512), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_moe_ring(const MoeParams& p, const int32_t* ids, int n_pairs, int E, const float* X,
                           int64_t x_tstride, int n_xrows, int max_act, int nw, hipStream_t st) {
    if (nw != 4 && nw != 8) return hipErrorInvalidValue;
    const int64_t items = (int64_t)n_xrows * p.nb;
    hipLaunchKernelGGL(moe_prep_kernel, dim3((unsigned)(1 + (items + 15) / 16)), dim3(256), moe_route_lds_bytes(E), st,
                       ids, n_pairs, E, p.route, X, x_tstride, n_xrows, p.nb, p.Q);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t grid = (int64_t)max_act * p.tiles_per_expert * (p.nbank > 1 ? 2 : 1);
    if (nw == 4) {
        if (p.fmt == WF_Q6K)
            hipLaunchKernelGGL((moe_ring_kernel<3, 1, 4>), dim3((unsigned)grid), dim3(256), 0, st, p);
        else if (p.fmt == WF_Q5K)
            hipLaunchKernelGGL((moe_ring_kernel<3, 2, 4>), dim3((unsigned)grid), dim3(256), 0, st, p);
        else
            hipLaunchKernelGGL((moe_ring_kernel<3, 0, 4>), dim3((unsigned)grid), dim3(256), 0, st, p);
    } else if (p.fmt == WF_Q6K) {
        hipLaunchKernelGGL((moe_ring_kernel<3, 1, 8>), dim3((unsigned)grid), dim3(512), 0, st, p);
    } else if (p.fmt == WF_Q5K) {
        hipLaunchKernelGGL((moe_ring_kernel<3, 2, 8>), dim3((unsigned)grid), dim3(512), 0, st, p);
    } else {
        hipLaunchKernelGGL((moe_ring_kernel<3, 0, 8>), dim3((unsigned)grid), dim3(512), 0, st, p);
    }
    return hipGetLastError();
}

// The weighted sum over the routed experts that ends a MoE FFN block
// (desktop/engine/src/forward.cpp:1107-1116): ggml_mul of the down outputs
// [n, n_used, T] by the router weights [1, n_used, T] (one fp32 product an
// element), then ggml_sum_rows over the slot axis, whose ggml_vec_sum_f32
// (ggml-cpu/vec.h:1513-1519) adds the products in double in slot order and
// rounds once. One thread per output element; a wave reads 64 consecutive
// elements of one slot row at a time.
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ D, const float* __restrict__ w,
                                                          float* __restrict__ Y, int T, int n_used, int n) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)T * n) return;
    const int t = (int)(idx / n);
    const int i = (int)(idx - (int64_t)t * n);
    const float* row = D + (int64_t)t * n_used * n + i;
    const float* wt = w + (int64_t)t * n_used;
    double acc = 0.0;
    for (int s = 0; s < n_used; ++s) {
        const float prod = row[(int64_t)s * n] * wt[s];
        acc += (double)prod;
    }
    Y[idx] = (float)acc;
}

hipError_t launch_moe_combine(const float* D, const float* w, float* Y, int T, int n_used, int n, hipStream_t st) {
    const int64_t total = (int64_t)T * n;
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, D, w, Y, T,
                       n_used, n);
    return hipGetLastError();
}

}  // namespace spq4k
