// launch.h — host-side launch interfaces of the gfx950 kernels (internal to
// libspq4k; the public C ABI is include/spq4k.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_core.h"

namespace spq4k {

constexpr int GEMV_MAX_SEG = 4;

// weight formats of the matvec kernels
enum WFmt : int32_t {
    WF_Q4K = 0,   // GGML_TYPE_Q4_K, 144-byte blocks
    WF_Q6K = 1,   // GGML_TYPE_Q6_K, 210-byte blocks
    WF_Q5K = 2,   // GGML_TYPE_Q5_K, 176-byte blocks (sdot4 kernels only)
    WF_Q80 = 3,   // GGML_TYPE_Q8_0, 34-byte blocks of 32 (kernels of k_q8_0.hip)
};

struct GemvSeg {
    const uint8_t* W;     // [M][nb] blocks of the format, row-major
    float* Y;             // y[t * y_tstride + r]
    int64_t y_tstride;
    int32_t M;
    int32_t tile_begin;   // first tile index of this segment (generic kernel)
    int32_t row_begin;    // first row of this segment in the concatenation (decode kernel)
};

struct GemvParams {
    GemvSeg seg[GEMV_MAX_SEG];
    int32_t nseg;
    int32_t nb;           // Q4_K blocks per row (K / 256)
    const float* X;       // x[t * x_tstride + k], 16-byte aligned rows
    int64_t x_tstride;
    Q8Planes Q;           // pre-quantised activations (Q.qs != nullptr) instead of X
    int32_t chunk_blocks; // blocks staged in LDS at a time
    int32_t total_rows;   // sum of the segments' M
    int32_t fmt;          // WFmt of every segment
    // fusions of the T = 1 decode kernel (DecodeCfg.norm / .glu)
    const float* norm_w;  // x -> (x * 1/sqrt(mean(x^2) + eps)) * norm_w before quantisation
    float eps;
    // wave timestamps of the T = 1 decode kernel (spq4k_set_decode_stamps):
    // 4 uint64 a wave, or null
    uint64_t* stamps;
};

// Launch shape of the T = 1 decode kernel (gemv_decode_kernel).
struct DecodeCfg {
    int waves;    // waves per workgroup: 8, 12 or 16
    int depth;    // rows of loads in flight per wave: 1 or 2
    bool xfirst;  // quantising waves fetch and quantise x before their weight loads
    int grid;     // workgroups
    bool norm;    // RMS-normalise x (p.norm_w, p.eps) before quantising it (xfirst)
    bool glu;     // segments 0 and 1 are gate and up: y0 = silu(gate . x) * (up . x) (depth 2, xfirst)
};

// rows per workgroup for a lanes-per-row choice of 4*bpr (bpr in 1, 2, 4, 8)
int gemv_rows_per_tile(int bpr);
hipError_t launch_gemv(const GemvParams& p, int T, int bpr, int ntiles, hipStream_t st);
bool decode_supported(int fmt, int nb);
// the row length (in blocks) the decode kernel instance for nb is compiled for:
// nb itself for the exact instances, else the next multiple of 16 (the
// runtime-length instances, up to DEC_MAX_NB for Q4_K, 32 for Q6_K / Q5_K); 0 if none
constexpr int DEC_MAX_NB = 112;
int decode_bucket(int fmt, int nb);
hipError_t launch_gemv_decode(const GemvParams& p, const DecodeCfg& c, hipStream_t st);
// whether the decode kernel has a timestamped instance (p.stamps) for this
// shape: the unfused Q4_K launch shapes of rows of 4096 and 12288
bool decode_stamps_supported(int fmt, int nb, const DecodeCfg& c);
// whether the decode kernel has the fused form c (norm / glu) for this format and row length
bool decode_fused_supported(int fmt, int nb, const DecodeCfg& c);
// ggml_rms_norm then ggml_mul by w (ggml-cpu/ops.cpp:3724-3784): y[t] = (x[t] * s_t) * w,
// s_t = 1 / sqrt(mean(x[t]^2) + eps), one workgroup a row
hipError_t launch_rms_norm(const float* x, int64_t x_tstride, int T, int K, const float* w, float eps, float* y,
                           hipStream_t st);
// y = silu(g) * u element-wise (ggml_silu then ggml_mul, ggml_vec_swiglu_f32)
hipError_t launch_swiglu(const float* g, const float* u, float* y, int64_t n, hipStream_t st);
hipError_t launch_subblock_sums(const uint8_t* W, int M, int nb, const float* X, int32_t* S, hipStream_t st);

// expert-gathered matvec (k_moe.hip)
struct MoeRoute {
    int32_t* n_act;     // [1] number of experts with at least one pair
    int32_t* act;       // [E] active expert ids, ascending
    int32_t* act_off;   // [E] first pair of active expert a in `pairs`
    int32_t* act_cnt;   // [E] pairs of active expert a
    int32_t* pairs;     // [T * n_used] pair index t * n_used + s, grouped by expert
};

struct MoeParams {
    MoeRoute route;
    int32_t ring_rt;         // moe_ring_kernel: 128-row tiles a workgroup streams (tiles_per_expert = groups)
    const uint8_t* bank;     // E experts of [M][nb] Q4_K blocks
    size_t expert_bytes;
    float* Y;                // [T][n_used][M]
    Q8Planes Q;              // Q8_K of the T * ne11 input rows
    int32_t M, nb, n_used, ne11;
    int32_t tiles_per_expert;
    int32_t chunk_blocks;
    int32_t fmt;             // WFmt of the bank
    // moe_ring_kernel: a second bank of the same type, K, E and M sharing the
    // routing and planes (gate and up); its workgroups follow the first
    // bank's max_act * tiles_per_expert. nbank 0 or 1: one bank.
    const uint8_t* bank1;
    float* Y1;
    int32_t nbank, max_act;
};

hipError_t launch_moe_route(const int32_t* ids, int n_pairs, int E, const MoeRoute& r, hipStream_t st);
// Y[t][i] = sum over s < n_used of D[t][s][i] * w[t][s]: fp32 products added
// in double in slot order, rounded once (ggml_mul then ggml_sum_rows)
hipError_t launch_moe_combine(const float* D, const float* w, float* Y, int T, int n_used, int n, hipStream_t st);

// single-launch MoE (routing and Q8_K quantisation inside the matvec kernel)
constexpr int MOE_FUSED_MAX_PAIRS = 2048;
struct MoeFusedParams {
    const int32_t* ids;      // [n_pairs] = [T][n_used]
    const float* X;          // [T * ne11][K] fp32, 16-byte aligned rows
    const uint8_t* bank;     // E experts of [M][nb] Q4_K blocks
    size_t expert_bytes;
    float* Y;                // [T][n_used][M]
    int32_t n_pairs, n_used, ne11, K, M, nb;
    int32_t tiles_per_expert;
    int32_t chunk_blocks;
    int32_t E;          // experts in the bank (moe_decode_kernel)
    int32_t n_xrows;    // input rows T * ne11 (moe_decode_kernel)
    int32_t rows_per_wg;   // moe_decode_kernel: contiguous sweep rows a workgroup (moe_decode_plan)
    int32_t xwin_rows;     // moe_decode_kernel: input rows quantised by a workgroup at most
    int32_t fmt;           // WFmt of the bank
    // moe_decode_kernel only: a second bank of the same type, K and E (the up
    // projection beside the gate) swept in the same launch; M1 = 0 for none
    const uint8_t* bank1;
    size_t expert_bytes1;
    float* Y1;               // [T][n_used][M1]
    int32_t M1;
    // moe_decode_kernel only: bank1 is the up bank beside the gate bank (same
    // M); Y[pair][r] = silu(gate row r . x) * (up row r . x), Y1 unused
    int32_t glu;
    // moe_decode_kernel: waves a workgroup, 8, or 12 for a GLU sweep (0 = 8)
    int32_t waves;
};
hipError_t launch_moe_fused(const MoeFusedParams& p, int tc, int bpr, int grid, hipStream_t st);

// small-batch MoE in the decode mapping (one sweep over the rows of all pairs)
constexpr int MOE_DEC_MAX_PAIRS = 64;
constexpr int MOE_DEC_MAX_XROWS = 64;
bool moe_decode_supported(int nb);
int moe_decode_rows_per_wg(int nb, int waves = 8);
void moe_decode_plan(const MoeFusedParams& p, int grid, int32_t* rows_per_wg, int32_t* xwin_rows);
hipError_t launch_moe_decode(const MoeFusedParams& p, int grid, hipStream_t st);
// the routed-expert block's down projection with the weighted slot sum as its
// epilogue (moe_down_sum_kernel): Yc [T][M] = sum over s of (bank row of ids[t][s]
// . X[t * n_used + s]) * cw[t][s]; p.rows_per_wg elements of Yc a workgroup,
// p.xwin_rows the hidden rows one quantises at most; n_used <= MOE_SUM_MAX_USED
constexpr int MOE_SUM_MAX_USED = 8;
hipError_t launch_moe_down_sum(const MoeFusedParams& p, const float* cw, float* Yc, int grid, hipStream_t st);
hipError_t launch_moe_gemv(const MoeParams& p, int tc, int bpr, int grid, hipStream_t st);
// matrix-core form: moe_prep_kernel (routing in workgroup 0, permuted Q8_K
// planes of the n_xrows input rows X in the others), then the ring kernel
// over max_act experts x p.tiles_per_expert groups of p.ring_rt row tiles
// nw: waves of a workgroup, 4 or 8 (row tiles of 16 * nw rows)
hipError_t launch_moe_ring(const MoeParams& p, const int32_t* ids, int n_pairs, int E, const float* X,
                           int64_t x_tstride, int n_xrows, int max_act, int nw, hipStream_t st);
// Q8_0 banks (K a multiple of 256; p.Q.qs / p.Q.d the Q8_0 planes, p.route
// filled): the ring kernel only
hipError_t launch_moe_ring_q80(const MoeParams& p, int max_act, int nw, hipStream_t st);

// prefill matmul on matrix cores (k_gemm.hip)
constexpr int GEMM_MAX_SEG = 4;
struct GemmSeg {
    const uint8_t* W;     // [M][nb] Q4_K
    float* Y;             // [T][M]
    int32_t M;
    int32_t tile_begin;   // first row tile of this segment (set by the launcher)
    int32_t row_begin;    // first row of this segment in the concatenation of all segments
};
struct GemmParams {
    Q8Planes Q;         // Q8_K of the T input rows
    int32_t T, nb;
    int32_t mode;       // 0 auto, 1 skinny kernel at any T, 2 tiled kernels only
    int32_t cfg;        // tiled launch shape (0 .. gemm_tiled_shapes() - 1), -1 automatic
    GemmSeg seg[GEMM_MAX_SEG];   // up to four matrices sharing the input
    int32_t nseg;
    int32_t total_tiles;
    int32_t rows;       // sum of the segments' M
    int32_t ksplit;     // K ranges (ring kernels): 1, or partial sums in P then a reduction
    int32_t kchunk;     // super-blocks per K range
    float* P;           // [ksplit][T][rows] partial plane when ksplit > 1
    int32_t fmt;        // WFmt of every segment (shapes are per format)
};
// Launch plan of the tiled / ring kernels for a GemmParams (T, nb, segments,
// cfg): shape, K split and the scratch the partial plane needs.
struct GemmPlan {
    int cfg;
    int ksplit, kchunk;
    bool perm;                 // reads the permuted Q8_K values
    size_t partial_bytes;      // ksplit * T * rows * 4 when ksplit > 1
};
bool gemm_use_skinny(int T, int mode);
int gemm_tiled_shapes();
GemmPlan gemm_plan(const GemmParams& p, int num_cus, size_t max_partial_bytes);
// p.cfg / p.ksplit / p.kchunk / p.P as planned; launches the reduction too
hipError_t launch_gemm(const GemmParams& p, hipStream_t st);
hipError_t launch_gemm_skinny(const GemmParams& p, hipStream_t st);   // skinny, all segments

// element-wise conversions (k_convert.hip)
hipError_t launch_quantize_q8k(const float* x, uint8_t* y, int64_t nblocks, hipStream_t st);
// fp32 rows x[t * x_tstride + k] -> Q8_K planes (T rows of nb blocks); perm
// stores qs in the order of the ring GEMM kernel
hipError_t launch_quantize_q8k_planes(const float* x, int64_t x_tstride, int T, int nb, int8_t* qs, int16_t* bs,
                                      float* d, uint8_t* mn, bool perm, hipStream_t st);
hipError_t launch_dequant_q4k(const uint8_t* x, float* y, int64_t nblocks, hipStream_t st);
hipError_t launch_quantize_q4k(const float* x, uint8_t* y, int64_t nblocks, hipStream_t st);
hipError_t launch_synth(float* out, int64_t n, uint64_t seed, int dist, int64_t cols, float mean, float std,
                        float outlier_mult, int64_t offset, hipStream_t st);
hipError_t launch_vec_dot_q8(const uint8_t* wx, const uint8_t* q8, int nb, float* out, hipStream_t st);
// one streaming read of `bytes` (a multiple of 16) at p by at most max_grid
// workgroups; sink: max_grid words of scratch
hipError_t launch_stream_read(const void* p, size_t bytes, int max_grid, uint32_t* sink, hipStream_t st);

// Q6_K conversions (k_q6k.hip); the Q6_K matvecs are the FmtQ6K instances of
// launch_gemv / launch_gemv_decode / launch_moe_* (fmt = WF_Q6K)
hipError_t launch_dequant_q6k(const uint8_t* x, float* y, int64_t nblocks, hipStream_t st);
hipError_t launch_quantize_q6k(const float* x, uint8_t* y, int64_t nblocks, hipStream_t st);
hipError_t launch_vec_dot_q6k(const uint8_t* wx, const uint8_t* q8, int nb, float* out, hipStream_t st);
hipError_t launch_subblock_sums_q6k(const uint8_t* W, int M, int nb, const float* X, int32_t* S, hipStream_t st);

// Q5_K conversions (k_convert.hip); the Q5_K matvecs are the FmtQ5K instances
// of launch_gemv / launch_gemv_decode / launch_moe_decode / _fused / _gemv
hipError_t launch_quantize_q5k(const float* x, uint8_t* y, int64_t nblocks, hipStream_t st);
hipError_t launch_dequant_q5k(const uint8_t* x, float* y, int64_t nblocks, hipStream_t st);
hipError_t launch_vec_dot_q5k(const uint8_t* wx, const uint8_t* q8, int nb, float* out, hipStream_t st);
hipError_t launch_subblock_sums_q5k(const uint8_t* W, int M, int nb, const float* X, int32_t* S, hipStream_t st);

// Q8_0 weights (k_q8_0.hip): Q8_0 activations, one group of lanes per row
constexpr size_t Q80_LDS_MAX = 160 * 1024;   // LDS of one workgroup on gfx950
struct Q80Params {
    GemvSeg seg[GEMV_MAX_SEG];   // dense: matrices sharing the input (W, Y, y_tstride, row_begin)
    int32_t nseg;
    int32_t nb;                  // Q8_0 blocks per row (K / 32)
    int32_t total_rows;          // dense: rows of all segments; sweep: n_pairs * M
    // activations: p.X quantised into LDS, or Q8_0 planes Aq [row][K], Ad [row][nb]
    const float* X;              // fp32 rows x[r * x_tstride + k], 16-byte aligned
    int64_t x_tstride;
    int32_t n_xrows;             // activation rows the kernel stages in LDS
    const int8_t* Aq;
    const float* Ad;
    // expert-gathered forms
    const uint8_t* bank;         // E experts of [M][nb] blocks
    size_t expert_bytes;
    float* Y;                    // [T][n_used][M]
    const int32_t* ids;          // sweep: [T][n_used]
    int32_t E, M, n_used, ne11;
    MoeRoute route;              // grouped: routing tables (launch_moe_route)
    int32_t groups;              // grouped: workgroups per active expert
    int32_t rows_per_wg;         // grouped: rows of the expert a workgroup takes
};
size_t q80_lds_bytes(int xrows, int nb);
// the weight-staging matvec (K a multiple of 256, activations in LDS):
// whether T tokens of nb blocks fit, its LDS, and its launch
bool q80_staged_fits(int T, int nb);
size_t q80_staged_lds_bytes(int T, int nb);
int q80_staged_grid(int64_t rows, int T, int nb, int num_cus, size_t lds_max);
hipError_t launch_gemv_q8_0_staged(const Q80Params& p, int T, int grid, hipStream_t st);
int q80_lanes_per_row(int nb);
int q80_rows_per_wg(int nb);
hipError_t launch_quantize_q8_0(const float* x, uint8_t* y, int64_t nblocks, bool ref_encoder, hipStream_t st);
hipError_t launch_dequant_q8_0(const uint8_t* x, float* y, int64_t nblocks, hipStream_t st);
hipError_t launch_quantize_q8_0_planes(const float* x, int64_t x_tstride, int rows, int nb, int8_t* q, float* d,
                                       hipStream_t st);
hipError_t launch_block_sums_q8_0(const uint8_t* W, int M, int nb, const float* x, int32_t* S, hipStream_t st);
hipError_t launch_vec_dot_q8_0(const uint8_t* wx, const uint8_t* a, int nb, float* out, hipStream_t st);
// T tokens (p.n_xrows == T), LDS-staged activations, or with global_acts
// (T = 1) read from p.Aq / p.Ad
hipError_t launch_gemv_q8_0(const Q80Params& p, int T, bool global_acts, int grid, hipStream_t st);
hipError_t launch_moe_q8_0_sweep(const Q80Params& p, int grid, hipStream_t st);
hipError_t launch_moe_q8_0_grouped(const Q80Params& p, int tc, int grid, hipStream_t st);

// Q4_K dequant-then-dot with fp32 activations (k_dqdot.hip, beast_matvec's
// arithmetic): Y[t * y_tstride + r] = sum_j dequant(W[r])[j] * X[t * x_tstride + j],
// T <= DQ_MATVEC_MAX_T tokens whose x (staged in LDS) fits DQ_MATVEC_LDS_MAX
constexpr int DQ_MATVEC_MAX_T = 8;
constexpr size_t DQ_MATVEC_LDS_MAX = 128 * 1024;
// the BurnHard MoE forward (k_dqdot.hip): routing of E <= BEAST_MAX_EXPERTS
// logits to top_k <= BEAST_MAX_TOPK experts (ids, scores), H [top_k][n_ff]
// the silu(gate) * up rows, out [n_embd]; Q4_K banks, n_embd and n_ff
// multiples of 256 whose rows fit the x staging. Its parts: the routing
// alone; routing + gate / up -> H; down and the weighted sum from H.
constexpr int BEAST_MAX_EXPERTS = 4096;
constexpr int BEAST_MAX_TOPK = 16;
constexpr int BEAST_DOWN_RPW = 8;
hipError_t launch_beast_route(const float* logits, int E, int top_k, int32_t* ids, float* scores, hipStream_t st);
hipError_t launch_beast_route_gate_up(const uint8_t* gate, const uint8_t* up, int E, int n_embd, int n_ff,
                                      const float* logits, int top_k, const float* hidden, int32_t* ids,
                                      float* scores, float* H, int num_cus, hipStream_t st);
hipError_t launch_beast_down(const uint8_t* down, int E, int n_embd, int n_ff, const int32_t* ids,
                             const float* scores, int top_k, const float* H, float* out, int num_cus,
                             hipStream_t st);
size_t dequant_matvec_lds_bytes(int T, int nb);
hipError_t launch_dequant_matvec(const uint8_t* W, int M, int nb, const float* X, int64_t x_tstride, float* Y,
                                 int64_t y_tstride, int T, int num_cus, hipStream_t st);

// The same dequant-then-dot for rows of any library type (k_dqdot_x.hip;
// type = SPQ4K_TYPE_Q4_K, _Q5_K, _Q6_K or _Q8_0; K a multiple of the type's
// block): dense rows (T <= DQ_MATVEC_MAX_T tokens), the selected experts'
// rows against one hidden row (mode 0: H[s][r] = the dot of bank's row;
// mode 1: H[s][r] = silu(H[s][r]) * the dot; mode 2: H[s][r] = silu(bank
// row . x) * (bank1 row . x), both banks of `type`), and the down rows'
// score-weighted sum out[i] over the selected experts in rank order.
size_t dqx_lds_bytes(int type, int64_t K, int T);
hipError_t launch_dqx_matvec(int type, const uint8_t* W, int M, int64_t K, const float* X, int64_t x_tstride,
                             float* Y, int64_t y_tstride, int T, int num_cus, hipStream_t st);
hipError_t launch_dqx_experts(int type, int mode, const uint8_t* bank, const uint8_t* bank1, int E, int rows,
                              int64_t K, const int32_t* ids, int top_k, const float* hidden, float* H, int num_cus,
                              hipStream_t st);
hipError_t launch_dqx_down(int type, const uint8_t* down, int E, int n_embd, int64_t n_ff, const int32_t* ids,
                           const float* scores, int top_k, const float* H, float* out, int num_cus, hipStream_t st);

// A chain of dependent T = 1 Q4_K matvec stages in one persistent launch
// (k_chain.hip). Stage s: x = in0 (+ in1); xout = x when set; x = rms_norm(x)
// * norm_w when set; Q8_K(x); then either the matrices W[j] (rows of segment
// j at row_begin[j] .. row_begin[j + 1]) or, with glu, y = silu(W[0] . x) *
// (W[1] . x) into Y[0].
constexpr int CHAIN_MAX_NB = 48;                 // K <= 12288
constexpr int CHAIN_MAX_K = CHAIN_MAX_NB * 256;  // fp32 input staging (LDS)
constexpr int CHAIN_NCTR = 16;                   // grid-barrier counters
constexpr int CHAIN_YCAP = 1024;                 // row results a workgroup holds per stage

struct ChainStage {
    const uint8_t* W[4];
    float* Y[4];
    int32_t row_begin[4];   // [0] = 0; segments not used start at INT32_MAX
    int32_t rows;           // total rows (glu: rows of the gate, = up)
    int32_t nb;             // Q4_K blocks per row
    int32_t glu;
    int32_t pad;
    const float* in0;       // [nb * 256]
    const float* in1;       // optional, added to in0
    float* xout;            // optional: in0 (+ in1) written here
    const float* norm_w;    // optional: RMS norm weights
};

struct ChainSync {
    uint32_t ctr[CHAIN_NCTR * 64];   // arrival counters, 256 B apart
    uint32_t gen;                    // launches completed past their first grid wait
    uint32_t pad0[63];
    uint32_t err;                    // set when a wait gave up
    uint32_t pad1[63];
};

struct ChainParams {
    const ChainStage* st;   // device table of nstages stages
    ChainSync* sync;        // zeroed before the chain's first launch
    int32_t nstages;
    float eps;
};
// The same chain with a one-hop exchange between stages (k_chain2.hip).
// Every vector a stage produces and a later stage reads (y[j], x_out) is
// also written to a shadow in a chain-owned arena whose words hold
// CHAIN2_SENTINEL until written in the current launch: a reader polls the
// words themselves, so no barrier, counter or fence sits between a row's
// store and its consumers. The arena has two sets: launch n uses set
// parity(n) and refills the other with the sentinel for launch n + 1.
constexpr uint32_t CHAIN2_SENTINEL = 0xFFFFFFFFu;   // a NaN; a result with these bits
constexpr uint32_t CHAIN2_SUBST = 0xFFFFFFFEu;      // is passed on as this NaN
enum : int32_t { CH2_NONE = 0, CH2_EXT = 1, CH2_SHADOW = 2, CH2_LOCAL = 3 };
struct Chain2Stage {
    const uint8_t* W[4];
    float* Y[4];
    int64_t ysh[4];          // shadow offset (floats) of output j, or -1 (no later reader)
    int32_t row_begin[4];    // as ChainStage
    int32_t rows;
    int32_t nb;
    int32_t glu;
    int32_t keep;            // keep x = in0 (+ in1) in the workgroup's LDS (a later CH2_LOCAL input)
    int32_t kind[2];         // in0, in1: CH2_*
    const float* ext[2];     // CH2_EXT input
    int64_t insh[2];         // CH2_SHADOW input: shadow offset of its first value
    float* xout;             // optional
    int64_t xosh;            // shadow offset of x_out, or -1
    const float* norm_w;     // optional
};
struct Chain2Sync {
    uint32_t cnt;            // workgroups of the current launch that have finished
    uint32_t pad0[63];
    uint32_t parity;         // shadow set of the next launch
    uint32_t pad1[63];
    uint32_t err;            // set when a wait gave up
    uint32_t pad2[63];
};
struct Chain2Params {
    Chain2Sync* sync;        // zeroed, arena filled with the sentinel, before the first launch
    float* sh;               // shadow arena: set 0, then set 1 at sh + sh_half
    int64_t sh_half;         // floats per set (a multiple of 4)
    uint64_t* stamps;        // optional: s_memrealtime per workgroup and stage (CHAIN2_NSTAMP each)
    int32_t nstages;
    float eps;
};
constexpr int CHAIN2_XW = 4;         // exchange waves a workgroup
constexpr int CHAIN2_NSTAMP = 4;     // stamps per workgroup and stage
// compute waves of the v2 kernel
int chain2_compute_waves();
// depth: pieces in flight a compute wave (2, 3, 4 or 6)
hipError_t launch_chain2(const Chain2Stage* st, const Chain2Params& p, int grid, int depth, hipStream_t stream);

// workgroups of a chain launch on a device with num_cus CUs (a multiple of CHAIN_NCTR)
int chain_grid(int num_cus);
// launch shapes (compute waves x pieces in flight each): 0 = 8 x 8, 1 = 8 x 6, 2 = 7 x 8
int chain_compute_waves(int shape);
hipError_t launch_chain(const ChainParams& p, int grid, int shape, hipStream_t st);

}  // namespace spq4k
