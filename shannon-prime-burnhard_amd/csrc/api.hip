// api.hip — the C ABI of libspq4k (include/spq4k.h, include/spq4k_synth.h).
//
// Host-side planning for the gfx950 kernels: argument checks, tile and
// K-split choice, scratch management, host<->device staging for the *_host
// entry points. There is no CPU compute path: every result comes from a HIP
// kernel, and a missing or failing device is an error.
#include <errno.h>
#include <limits.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <vector>
#include <algorithm>

#include <hip/hip_runtime.h>

#include "launch.h"
#include "spq4k.h"
#include "spq4k_diag.h"
#include "spq4k_synth.h"

using namespace spq4k;

// The partial-sum plane of a K-split matmul is held to a fixed budget, so the
// split (and with it the order of the fp32 sums) depends on the shape alone:
// not on how much scratch a context happens to hold, and not on whether the
// call runs on the no-allocation scratch (whose activation planes leave it
// exactly this much, SPQ4K_NOALLOC_SCRATCH_BYTES - SPQ4K_NOALLOC_PLANES_MAX).
constexpr size_t KSPLIT_PARTIAL_BYTES = (size_t)8 << 20;
static_assert(SPQ4K_NOALLOC_SCRATCH_BYTES - SPQ4K_NOALLOC_PLANES_MAX == KSPLIT_PARTIAL_BYTES,
              "the no-allocation scratch leaves a K split its whole budget");


struct spq4k_ctx {
    int device = 0;
    int num_cus = 256;
    size_t lds_max = 64 * 1024;  // LDS a workgroup may allocate (the device's limit, at most Q80_LDS_MAX)
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    // generic device scratch (Q8_K activations, routing tables)
    uint8_t* scratch = nullptr;
    size_t scratch_cap = 0;
    // intermediates of the fused entry points (normalised rows, gate / up outputs)
    uint8_t* scratch2 = nullptr;
    size_t scratch2_cap = 0;
    // scratch buffers replaced by larger ones, freed by spq4k_free
    std::vector<void*> retired;
    // set while a call runs on the no-allocation scratch (spq4k_mul_mat_noalloc):
    // a call that needs more than it holds fails instead of allocating
    bool no_alloc = false;
    int force_bpr = 0;           // tuning override (SPQ4K_GEMV_BPR = 1, 2, 4 or 8)
    int preq_mode = 0;           // SPQ4K_GEMV_PREQ: 0 auto, 1 always, 2 never
    int gemv_mfma_min_t = 4;     // SPQ4K_GEMV_MFMA_MIN_T: batches of at least this many tokens use matrix cores
    int no_decode = 0;           // SPQ4K_GEMV_GENERIC=1: T = 1 also uses the generic kernel
    int moe_unfused = 0;         // SPQ4K_MOE_UNFUSED=1: routing pass + Q8_K planes + matvec (3 launches)
    // SPQ4K_MOE_DEC_MAX_T: largest batch of the K-quant MoE decode sweep (1..8);
    // at T = 8 the sweep streams an expert once per pair, about a quarter more
    // bytes than the ring, but skips its prep launch: the 128-expert Q4_K layer
    // takes 49.0 us against 56.5 on the ring
    int moe_dec_max_t = 8;
    int moe_ring_waves = 0;      // SPQ4K_MOE_RING_WAVES: 4 or 8 waves (64- or 128-row tiles) in the expert ring kernel, 0 by format
    int moe_dec_waves = 0;       // SPQ4K_MOE_DEC_WAVES: 8 or 12 waves in a GLU expert sweep, 0 by grid
    uint64_t* dec_stamps = nullptr;   // spq4k_set_decode_stamps: the decode kernel's wave timestamps
    size_t dec_stamps_n = 0;
    int moe_mode = 0;            // SPQ4K_MOE_MODE: 2 skips the small-batch decode mapping, 3 takes the single-launch sdot4 kernel
    int gemm_mode = 0;           // SPQ4K_GEMM_MODE: 0 auto, 1 skinny kernel, 2 tiled kernel
    int gemm_cfg = -1;           // SPQ4K_GEMM_CFG: tiled launch shape, -1 automatic
    DecodeCfg dec_force = {0, 0, false, 0};   // SPQ4K_DEC_{WAVES,DEPTH,XFIRST,GRID} overrides
    int dec_xfirst_set = 0;
    int q80_grid = 0;            // SPQ4K_Q80_GRID: workgroups of the Q8_0 matvec, 0 automatic
    int q80_preq = 0;            // SPQ4K_Q80_PREQ: 0 auto, 1 always quantise x once up front, 2 never
    int q80_staged = 1;          // SPQ4K_Q80_STAGED: 0 direct block loads only, 1 staging where it measured faster, 2 staging wherever it fits
    char err[256] = {0};
};

struct spq4k_weights {
    int device = 0;              // weights may outlive the context that made them
    uint8_t* data = nullptr;
    bool owned = false;
    int type = SPQ4K_TYPE_Q4_K;  // ggml type id
    int fmt = WF_Q4K;            // kernel format of that type
    int64_t M = 0, K = 0, E = 0;
    size_t nbytes = 0;
};

namespace {

int set_err(spq4k_ctx* c, int code, const char* fmt, ...) {
    if (c) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(c->err, sizeof c->err, fmt, ap);
        va_end(ap);
    }
    return code;
}

int hip_fail(spq4k_ctx* c, hipError_t e, const char* what) {
    return set_err(c, -EIO, "%s: %s", what, hipGetErrorString(e));
}

#define SPQ_HIP(ctx, call)                                            \
    do {                                                              \
        hipError_t _e = (call);                                       \
        if (_e != hipSuccess) return hip_fail((ctx), _e, #call);      \
    } while (0)

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// weight types the kernels take: kernel format and block bytes, -1 / 0 otherwise
int type_fmt(int type) {
    return type == SPQ4K_TYPE_Q4_K ? WF_Q4K
         : type == SPQ4K_TYPE_Q5_K ? WF_Q5K
         : type == SPQ4K_TYPE_Q6_K ? WF_Q6K
         : type == SPQ4K_TYPE_Q8_0 ? WF_Q80 : -1;
}
size_t type_block_bytes(int type) {
    return type == SPQ4K_TYPE_Q4_K ? SPQ4K_Q4K_BLOCK_BYTES
         : type == SPQ4K_TYPE_Q5_K ? SPQ4K_Q5K_BLOCK_BYTES
         : type == SPQ4K_TYPE_Q6_K ? SPQ4K_Q6K_BLOCK_BYTES
         : type == SPQ4K_TYPE_Q8_0 ? SPQ4K_Q8_0_BLOCK_BYTES : 0;
}
// values per block (ggml's blck_size): 32 for Q8_0, 256 for the K-quants
int64_t type_block_values(int type) { return type == SPQ4K_TYPE_Q8_0 ? SPQ4K_QK8_0 : SPQ4K_QK_K; }
// alignment the kernels need of a block pointer of the type
size_t type_align(int type) { return type == SPQ4K_TYPE_Q4_K || type == SPQ4K_TYPE_Q5_K ? 16 : 2; }
// K-quant formats whose batches run on the matrix-core ring from
// gemv_mfma_min_t tokens (Q8_0 batches take the ring through q80_dense)
bool fmt_has_mfma(int fmt) { return fmt == WF_Q4K || fmt == WF_Q6K || fmt == WF_Q5K; }
// formats of the expert-gathered ring kernel (moe_ring_kernel)
bool fmt_has_moe_ring(int fmt) { return fmt == WF_Q4K || fmt == WF_Q6K || fmt == WF_Q5K; }
// Waves of the expert ring kernel, measured on the 128-expert down bank at
// T = 32 (us, 4 / 8 waves): Q6_K 54.9 / 59.9, Q5_K 45.0 / 48.0; Q4_K (the
// MoE layer) 97.0 / 88.7 and Q8_0 70.2 / 67.6 keep 8.
int moe_ring_waves(const spq4k_ctx* c, int fmt) {
    if (c->moe_ring_waves) return c->moe_ring_waves;
    return fmt == WF_Q6K || fmt == WF_Q5K ? 4 : 8;
}

int use_device(spq4k_ctx* c) {
    if (!c) return -EINVAL;
    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) return hip_fail(c, e, "hipSetDevice");
    (void)hipGetLastError();   // launch errors below are this call's own
    return 0;
}

// Grows one of the context's scratch buffers to at least `bytes`. The buffer
// it replaces is retired, not freed: work already enqueued, and HIP graphs
// captured earlier, keep pointing at it, so it stays allocated until
// spq4k_free. Growth at least doubles the capacity, so the retired buffers
// of a context add up to less than its current one. A call that would grow
// a buffer while the stream is being captured fails with -EBUSY (nothing is
// enqueued): a graph must not depend on an allocation made during its
// capture; spq4k_reserve grows the buffers ahead of a capture.
int grow_scratch(spq4k_ctx* c, uint8_t** buf, size_t* cap, size_t bytes, size_t min_cap, const char* what) {
    if (bytes <= *cap) return 0;
    if (c->no_alloc)
        return set_err(c, -EINVAL, "%s: %zu bytes needed, beyond the %zu bytes of the no-allocation scratch", what,
                       bytes, *cap);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    SPQ_HIP(c, hipStreamIsCapturing(c->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return set_err(c, -EBUSY,
                       "%s: %zu bytes needed, %zu held, and the stream is capturing a graph (call spq4k_reserve "
                       "before the capture)", what, bytes, *cap);
    size_t ncap = 2 * *cap;
    if (ncap < bytes) ncap = bytes;
    if (ncap < min_cap) ncap = min_cap;
    void* p = nullptr;
    if (hipMalloc(&p, ncap) != hipSuccess) return set_err(c, -ENOMEM, "%s of %zu bytes", what, ncap);
    if (*buf) c->retired.push_back(*buf);
    *buf = static_cast<uint8_t*>(p);
    *cap = ncap;
    return 0;
}

int ensure_scratch(spq4k_ctx* c, size_t bytes) {
    return grow_scratch(c, &c->scratch, &c->scratch_cap, bytes, (size_t)4 << 20, "scratch");
}

int ensure_scratch2(spq4k_ctx* c, size_t bytes) {
    return grow_scratch(c, &c->scratch2, &c->scratch2_cap, bytes, (size_t)1 << 20, "fusion scratch");
}

int check_shape(spq4k_ctx* c, int64_t M, int64_t K, int64_t E, int64_t qk = SPQ4K_QK_K) {
    if (M <= 0 || K <= 0 || E <= 0) return set_err(c, -EINVAL, "non-positive shape M=%lld K=%lld E=%lld",
                                                   (long long)M, (long long)K, (long long)E);
    if (K % qk) return set_err(c, -EINVAL, "K=%lld is not a multiple of %lld", (long long)K, (long long)qk);
    if (M > (1ll << 30) || K > (1ll << 30)) return set_err(c, -EINVAL, "shape too large");
    return 0;
}

// Quantise T rows of x (row stride x_tstride) into Q8_K planes in the
// context scratch; Q receives the plane pointers.
size_t q8_planes_bytes(int T, int nb) {
    return (((size_t)T * nb * (256 + Q8MN_BYTES + 32 + 4)) + 255) & ~(size_t)255;
}

// extra: bytes of scratch wanted behind the planes (at q8_planes_bytes)
int q8_planes(spq4k_ctx* c, const float* x, int64_t x_tstride, int T, int nb, Q8Planes* Q, bool perm = false,
              size_t extra = 0) {
    const size_t items = (size_t)T * nb;
    int rc = ensure_scratch(c, q8_planes_bytes(T, nb) + extra);
    if (rc) return rc;
    int8_t* qs = (int8_t*)c->scratch;
    uint8_t* mn = c->scratch + items * 256;
    int16_t* bs = (int16_t*)(c->scratch + items * (256 + Q8MN_BYTES));
    float* d = (float*)(c->scratch + items * (256 + Q8MN_BYTES + 32));
    hipError_t e = launch_quantize_q8k_planes(x, x_tstride, T, nb, qs, bs, d, mn, perm, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "quantize_q8k_planes launch");
    Q->qs = qs;
    Q->bs = bs;
    Q->d = d;
    Q->mn = mn;
    return 0;
}

// ---- GEMV planning ---------------------------------------------------------
constexpr int LDS_BUDGET = 48 * 1024;

// Largest rows-per-workgroup (fewest activation re-quantisations) that still
// gives at least two workgroups per CU.
int pick_bpr(const spq4k_ctx* c, const int64_t* M, int n) {
    if (c->force_bpr) return c->force_bpr;
    const int64_t target = 2 * (int64_t)c->num_cus;
    for (int bpr = 1; bpr <= 8; bpr *= 2) {
        const int rows = gemv_rows_per_tile(bpr);
        int64_t tiles = 0;
        for (int i = 0; i < n; ++i) tiles += (M[i] + rows - 1) / rows;
        if (tiles >= target) return bpr;
    }
    return 8;
}

// Launch shape of the T = 1 decode kernel. One workgroup per CU, so that x is
// quantised once per CU, one wave per row; measured on MI355X for the 8B
// decode shapes (cold weights, graph replay, us a launch in the step's
// stage replay, one run against the previous choice):
//   K = 4096,  M <= 4096   : 16 waves, x-first          (o projection: 4.05
//                            against 4.11 without x-first)
//   K = 4096,  M <= 8192   : 16 waves                   (q/k/v, 6144 rows: 5.20
//                            against 5.46 with 12 waves = 2 rows a wave)
//   K = 4096,  M <= 32768  : 16 waves                   (gate/up, 24576 rows:
//                            11.11 against 11.24 x-first)
//   K = 4096,  larger M    : 8 waves, 2 rows in flight, x-first (lm_head:
//                            62.0 against 63.4 with 12 waves)
//   K = 12288, Q4_K        : 8 waves, weights first (4096 x 12288: 8.21 against
//                            8.52 us with 16 waves x-first; 1024 rows 5.25 against
//                            6.53, 28672 rows 35.7 against 36.8, 12288 rows 16.8
//                            against 16.7), two rows a wave with the second row's
//                            loads issued after the quantisation barrier (8.50-8.52
//                            against 8.61-8.63 us with one row in flight; both rows
//                            at the start 9.55), each consumed as it arrives (the
//                            one-pass form when a wave has at most two rows: 8.07
//                            in the 8B step); other formats 12 waves, x-first
//   K = 27648              : 8 waves (the registers of 7 Q8_K blocks a lane), x-first
DecodeCfg plan_decode(const spq4k_ctx* c, int fmt, int nb_rows, int64_t rows, bool fused = false) {
    DecodeCfg d{};
    // register limits follow the row length the kernel instance is compiled for
    const int nb = decode_bucket(fmt, nb_rows) > 0 ? decode_bucket(fmt, nb_rows) : nb_rows;
    if (nb > 48) {
        d.waves = 8; d.depth = 1; d.xfirst = true;
    } else if (nb >= 48 && fmt == WF_Q4K) {
        // fused forms load x first, where a second row at the start is slower
        d.waves = 8; d.depth = fused ? 1 : 2; d.xfirst = false;
    } else if (nb >= 48) {
        d.waves = 16; d.depth = 1; d.xfirst = true;
    } else if (rows <= 4096) {
        d.waves = 16; d.depth = 1; d.xfirst = true;
    } else if (rows <= 8192) {
        d.waves = 16; d.depth = 1; d.xfirst = false;
    } else if (rows <= 32768) {
        d.waves = 16; d.depth = 1; d.xfirst = false;
    } else {
        d.waves = 8; d.depth = 2; d.xfirst = true;
    }
    if (c->dec_force.waves) d.waves = c->dec_force.waves;
    if (c->dec_force.depth) d.depth = c->dec_force.depth;
    if (c->dec_xfirst_set) d.xfirst = c->dec_force.xfirst;
    // K = 12288 with two rows in flight needs more than the 128 registers a
    // 16-wave workgroup allows: one row in flight; K = 27648 runs 8 waves, one row
    if (nb >= 48 && d.waves == 16) d.depth = 1;
    if (nb > 48) {
        d.waves = 8;
        d.depth = 1;
    }
    // Q6_K and Q5_K at K = 12288 (15 + 21 and 20 + 19 registers a block):
    // 12 waves, one row in flight
    if (fmt != WF_Q4K && nb >= 48 && (d.waves == 16 || (d.waves == 12 && d.depth == 2))) {
        d.waves = 12;
        d.depth = 1;
    }
    const int64_t wgs = (rows + d.waves - 1) / d.waves;
    d.grid = (int)(wgs < c->num_cus ? wgs : c->num_cus);
    if (c->dec_force.grid) d.grid = c->dec_force.grid;
    return d;
}

int gemm_segments(spq4k_ctx* c, int n, const spq4k_weights* const* W, const float* X, float* const* Y, int64_t T,
                  int mode);

// A fusion asked of gemv_launch: the decode kernel's RMS-norm prologue
// (norm_w) and / or its gate-up SiLU epilogue (glu: W[0] gate, W[1] up, y[0]
// the output). gemv_launch returns 1 when the fused kernel does not apply
// (the caller then runs the unfused steps).
struct Fuse {
    const float* norm_w = nullptr;
    float eps = 0.0f;
    bool glu = false;
};

// ---- Q8_0 planning ------------------------------------------------------------
// Q8_0 planes of `rows` activation rows in the context scratch: values
// [rows][K] int8, then scales [rows][nb] fp32; `extra` bytes behind them.
size_t q80_planes_bytes(int64_t rows, int nb) { return (((size_t)rows * nb * 36) + 255) & ~(size_t)255; }

int q80_planes(spq4k_ctx* c, const float* x, int64_t x_tstride, int64_t rows, int nb, Q80Params* p,
               size_t extra = 0) {
    int rc = ensure_scratch(c, q80_planes_bytes(rows, nb) + extra);
    if (rc) return rc;
    int8_t* q = (int8_t*)c->scratch;
    float* d = (float*)(c->scratch + (size_t)rows * nb * 32);
    hipError_t e = launch_quantize_q8_0_planes(x, x_tstride, (int)rows, nb, q, d, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "quantize_q8_0_planes launch");
    p->Aq = q;
    p->Ad = d;
    return 0;
}

// Workgroups of a Q8_0 matvec over `rows` weight rows: one or two per CU,
// never more than there are row groups. Two when the activation rows a
// workgroup stages are small (36 KB or less), one otherwise.
int q80_grid(const spq4k_ctx* c, int64_t rows, int nb, int64_t xrows) {
    if (c->q80_grid) return c->q80_grid;
    const int64_t per_wg = q80_rows_per_wg(nb);
    const int64_t need = (rows + per_wg - 1) / per_wg;
    const int64_t cap = (q80_lds_bytes((int)xrows, nb) <= 36 * 1024 ? 2 : 1) * (int64_t)c->num_cus;
    return (int)(need < cap ? need : cap);
}

// GGML_OP_MUL_MAT for Q8_0 weights, any T: n matrices sharing the input x
// (rows of K floats). T <= 8 tokens go in one launch with the activations
// quantised in every workgroup (T = 1) or once up front into planes that the
// workgroups copy to LDS; larger T run over slices of those planes, as many
// tokens a launch as LDS holds (at most 8); a row too long for LDS reads its
// one token from the planes directly.
// Q8_0 batches on the matrix cores (gemm_ring_kernel, F = 3): the Q8_0
// planes of X in the scratch with the partial plane of a K split behind them,
// then the ring launch (and the reduction of the K ranges).
int q80_gemm(spq4k_ctx* c, int n, const spq4k_weights* const* W, const float* X, float* const* Y, int64_t T) {
    const int64_t K = W[0]->K;
    const int nb = (int)(K / SPQ4K_QK8_0);
    GemmParams p;
    memset(&p, 0, sizeof p);
    p.T = (int32_t)T;
    p.nb = (int32_t)(K / SPQ4K_QK_K);
    p.cfg = c->gemm_cfg;
    int64_t rows = 0;
    for (int i = 0; i < n; ++i) {
        p.seg[i].W = W[i]->data;
        p.seg[i].Y = Y[i];
        p.seg[i].M = (int32_t)W[i]->M;
        p.seg[i].row_begin = (int32_t)rows;
        rows += W[i]->M;
    }
    for (int i = n; i < GEMM_MAX_SEG; ++i) p.seg[i].tile_begin = p.seg[i].row_begin = INT32_MAX;
    p.nseg = n;
    p.rows = (int32_t)rows;
    p.fmt = WF_Q80;
    if ((rows + 15) / 16 * ((T + 15) / 16) > (1ll << 31) - 1 || rows > (1ll << 31) - 1)
        return set_err(c, -EINVAL, "gemm: grid too large");
    const size_t planes = q80_planes_bytes(T, nb);
    const GemmPlan g = gemm_plan(p, c->num_cus, KSPLIT_PARTIAL_BYTES);
    p.cfg = g.cfg;
    p.ksplit = g.ksplit;
    p.kchunk = g.kchunk;
    Q80Params qp;
    memset(&qp, 0, sizeof qp);
    int rc = q80_planes(c, X, K, T, nb, &qp, g.partial_bytes);
    if (rc) return rc;
    p.Q.qs = qp.Aq;
    p.Q.d = qp.Ad;
    p.Q.mn = reinterpret_cast<const uint8_t*>(qp.Aq);   // no min-term plane: a valid address for stray reads
    p.P = g.ksplit > 1 ? reinterpret_cast<float*>(c->scratch + planes) : nullptr;
    const hipError_t e = launch_gemm(p, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "gemm (Q8_0) launch");
    return 0;
}

int q80_dense(spq4k_ctx* c, int n, const spq4k_weights* const* W, const float* X, float* const* Y, int64_t T) {
    const int64_t K = W[0]->K;
    const int nb = (int)(K / SPQ4K_QK8_0);
    // batches beyond the matvec's 8 tokens, K a multiple of 256: matrix cores
    if (T > SPQ4K_GEMV_MAX_T && K % SPQ4K_QK_K == 0 && c->gemm_mode != 1) return q80_gemm(c, n, W, X, Y, T);
    Q80Params p;
    memset(&p, 0, sizeof p);
    int64_t total = 0;
    for (int i = 0; i < n; ++i) {
        p.seg[i].W = W[i]->data;
        p.seg[i].Y = Y[i];
        p.seg[i].M = (int32_t)W[i]->M;
        p.seg[i].y_tstride = W[i]->M;
        p.seg[i].row_begin = (int32_t)total;
        total += W[i]->M;
    }
    if (total > (1ll << 31) - 1) return set_err(c, -EINVAL, "gemv: too many rows");
    for (int i = n; i < GEMV_MAX_SEG; ++i) {   // unused segments: never selected
        p.seg[i] = p.seg[0];
        p.seg[i].row_begin = INT32_MAX;
    }
    p.nseg = n;
    p.nb = nb;
    p.total_rows = (int32_t)total;
    p.X = X;
    p.x_tstride = K;
    const size_t per_tok = q80_lds_bytes(1, nb);
    const int64_t fit = (int64_t)(c->lds_max / per_tok);   // tokens whose planes fit in LDS
    const int64_t tmax = fit < SPQ4K_GEMV_MAX_T ? fit : SPQ4K_GEMV_MAX_T;
    bool preq = T > 1 || tmax < 1;
    if (c->q80_preq == 1) preq = true;
    if (c->q80_preq == 2 && T <= tmax) preq = false;
    // decode, K a multiple of 256: the weight-staging kernel (contiguous
    // loads) where it measured faster on MI355X (cold, us, staged / direct):
    // 151936 x 4096 128.6 / 149.7, 1024 x 4096 6.2 / 7.5, 2048 x 4096
    // 6.7 / 7.6; not for the mid shapes (4096 x 4096 8.6 / 8.2, 12288 x 4096
    // 16.4 / 15.3, 4096 x 12288 19.3 / 18.6, 1024 x 12288 12.8 / 11.3) nor
    // T > 1 (its LDS then leaves one workgroup a CU: T = 8 15.3 / 13.8)
    const bool staged_wins = total >= 65536 || (total <= 2048 && nb <= 128);
    if (c->q80_staged && T == 1 && (staged_wins || c->q80_staged == 2) && q80_staged_fits((int)T, nb) &&
        q80_staged_lds_bytes((int)T, nb) <= c->lds_max) {
        if (preq) {
            int rc = q80_planes(c, X, K, T, nb, &p);
            if (rc) return rc;
        }
        p.n_xrows = (int32_t)T;
        const int grid = q80_staged_grid(total, (int)T, nb, c->num_cus, c->lds_max);
        hipError_t e = launch_gemv_q8_0_staged(p, (int)T, grid, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "gemv_q8_0 (staged) launch");
        return 0;
    }
    if (!preq) {
        p.n_xrows = (int32_t)T;
        hipError_t e = launch_gemv_q8_0(p, (int)T, false, q80_grid(c, total, nb, T), c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "gemv_q8_0 launch");
        return 0;
    }
    int rc = q80_planes(c, X, K, T, nb, &p);
    if (rc) return rc;
    const int8_t* q0 = p.Aq;
    const float* d0 = p.Ad;
    const int64_t step = tmax >= 1 ? tmax : 1;
    for (int64_t t0 = 0; t0 < T; t0 += step) {
        const int tc = (int)(T - t0 < step ? T - t0 : step);
        p.Aq = q0 + t0 * K;
        p.Ad = d0 + t0 * nb;
        p.n_xrows = tc;
        for (int i = 0; i < n; ++i) p.seg[i].Y = Y[i] + t0 * W[i]->M;
        for (int i = n; i < GEMV_MAX_SEG; ++i) p.seg[i].Y = p.seg[0].Y;
        hipError_t e = launch_gemv_q8_0(p, tc, tmax < 1, q80_grid(c, total, nb, tmax < 1 ? 0 : tc), c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "gemv_q8_0 launch");
    }
    return 0;
}

int gemv_launch(spq4k_ctx* c, int n, const spq4k_weights* const* W, const float* x, float* const* y, int64_t T,
                const Fuse* fuse = nullptr) {
    if (n < 1 || n > GEMV_MAX_SEG) return set_err(c, -EINVAL, "gemv: n=%d matrices (1..4)", n);
    if (T < 1 || T > SPQ4K_GEMV_MAX_T) return set_err(c, -EINVAL, "gemv: T=%lld (1..8)", (long long)T);
    if (!x || !aligned(x, 16)) return set_err(c, -EINVAL, "gemv: x null or not 16-byte aligned");
    if (!W[0]) return set_err(c, -EINVAL, "gemv: null weight");
    const int64_t K = W[0]->K;
    int64_t Ms[GEMV_MAX_SEG];
    for (int i = 0; i < n; ++i) {
        if (!W[i] || !W[i]->data || !y || !y[i]) return set_err(c, -EINVAL, "gemv: null weight or output");
        if (W[i]->K != K || W[i]->E != 1) return set_err(c, -EINVAL, "gemv: matrices must share K and have E=1");
        if (W[i]->type != W[0]->type) return set_err(c, -EINVAL, "gemv: matrices must share the weight type");
        if (!aligned(W[i]->data, type_align(W[i]->type))) return set_err(c, -EINVAL, "gemv: weights misaligned");
        if (W[i]->device != c->device) return set_err(c, -EINVAL, "gemv: weights live on another device");
        Ms[i] = W[i]->M;
    }
    if (fuse && (W[0]->fmt == WF_Q80 || T != 1)) return 1;
    if (W[0]->fmt == WF_Q80) return q80_dense(c, n, W, x, y, T);
    const int bpr = pick_bpr(c, Ms, n);
    const int rows = gemv_rows_per_tile(bpr);
    GemvParams p;
    memset(&p, 0, sizeof p);
    int64_t tiles = 0, total = 0;
    for (int i = 0; i < n; ++i) {
        p.seg[i].W = W[i]->data;
        p.seg[i].Y = y[i];
        p.seg[i].M = (int32_t)W[i]->M;
        p.seg[i].y_tstride = W[i]->M;
        p.seg[i].tile_begin = (int32_t)tiles;
        p.seg[i].row_begin = (int32_t)total;
        tiles += (W[i]->M + rows - 1) / rows;
        total += W[i]->M;
    }
    if (tiles > (1ll << 31) - 1 || total > (1ll << 31) - 1) return set_err(c, -EINVAL, "gemv: too many rows");
    p.nseg = n;
    p.nb = (int32_t)(K / SPQ4K_QK_K);
    p.X = x;
    p.x_tstride = K;
    p.total_rows = (int32_t)total;
    p.fmt = W[0]->fmt;
    for (int i = n; i < GEMV_MAX_SEG; ++i) {   // unused segments: never selected
        p.seg[i] = p.seg[0];
        p.seg[i].row_begin = INT32_MAX;
        p.seg[i].tile_begin = INT32_MAX;
    }
    if (fuse) {
        if (c->no_decode || !decode_supported(p.fmt, p.nb)) return 1;
        DecodeCfg dc = plan_decode(c, p.fmt, p.nb, fuse->glu ? W[0]->M : total, true);
        dc.norm = fuse->norm_w != nullptr;
        dc.glu = fuse->glu;
        dc.xfirst = true;
        if (dc.glu) {
            dc.depth = 2;
            if (!c->dec_force.waves)
                for (int w : {16, 12, 8}) {
                    dc.waves = w;
                    if (decode_fused_supported(p.fmt, p.nb, dc)) break;
                }
            const int64_t wgs = (W[0]->M + dc.waves - 1) / dc.waves;
            dc.grid = c->dec_force.grid ? c->dec_force.grid : (int)(wgs < c->num_cus ? wgs : c->num_cus);
        }
        if (!decode_fused_supported(p.fmt, p.nb, dc)) return 1;
        p.norm_w = fuse->norm_w;
        p.eps = fuse->eps;
        hipError_t e = launch_gemv_decode(p, dc, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "gemv decode (fused) launch");
        return 0;
    }
    if (T == 1 && !c->no_decode && c->preq_mode != 1 && decode_supported(p.fmt, p.nb)) {
        const DecodeCfg dc = plan_decode(c, p.fmt, p.nb, total);
        if (c->dec_stamps) {
            if (!decode_stamps_supported(p.fmt, p.nb, dc))
                return set_err(c, -EINVAL, "decode stamps: no timestamped instance for this launch shape");
            if ((size_t)dc.grid * dc.waves * 4 > c->dec_stamps_n)
                return set_err(c, -EINVAL, "decode stamps: buffer smaller than grid * waves * 4");
            p.stamps = c->dec_stamps;
        }
        hipError_t e = launch_gemv_decode(p, dc, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "gemv decode launch");
        return 0;
    }
    // SPQ4K_GEMM_MODE=1 keeps Q6_K and Q5_K batches on the sdot4 kernels (gemv_chunked)
    if (T >= c->gemv_mfma_min_t && c->force_bpr == 0 && fmt_has_mfma(p.fmt) &&
        !(p.fmt != WF_Q4K && c->gemm_mode == 1)) {
        // 4 <= T <= 8: the sdot4 kernel's integer work grows with T while the
        // matrix cores' 16-token tile costs the same from T = 1 to 16
        return gemm_segments(c, n, W, x, y, T, c->gemm_mode == 1 ? 1 : 0);
    }
    const int cb_max = LDS_BUDGET / ((int)T * 292);
    p.chunk_blocks = p.nb < cb_max ? p.nb : cb_max;
    // Quantise the activations once, up front, when re-quantising them in
    // every workgroup would cost more than the extra launch.
    bool preq = (int64_t)p.nb * T > 48;
    if (c->preq_mode == 1) preq = true;
    if (c->preq_mode == 2) preq = false;
    if (preq) {
        int rc = q8_planes(c, x, K, (int)T, p.nb, &p.Q);
        if (rc) return rc;
    }
    hipError_t e = launch_gemv(p, (int)T, bpr, (int)tiles, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "gemv launch");
    return 0;
}

// Batches of more than SPQ4K_GEMV_MAX_T tokens for formats without a
// matrix-core kernel (Q6_K): X is quantised once into Q8_K planes, then the
// sdot4 GEMV runs over slices of 8 tokens of those planes.
int gemv_chunked(spq4k_ctx* c, int n, const spq4k_weights* const* W, const float* X, float* const* Y, int64_t T) {
    const int64_t K = W[0]->K;
    const int nb = (int)(K / SPQ4K_QK_K);
    int64_t Ms[GEMV_MAX_SEG];
    for (int i = 0; i < n; ++i) Ms[i] = W[i]->M;
    const int bpr = pick_bpr(c, Ms, n);
    const int rows = gemv_rows_per_tile(bpr);
    GemvParams p;
    memset(&p, 0, sizeof p);
    int64_t tiles = 0, total = 0;
    for (int i = 0; i < n; ++i) {
        p.seg[i].W = W[i]->data;
        p.seg[i].M = (int32_t)W[i]->M;
        p.seg[i].y_tstride = W[i]->M;
        p.seg[i].tile_begin = (int32_t)tiles;
        p.seg[i].row_begin = (int32_t)total;
        tiles += (W[i]->M + rows - 1) / rows;
        total += W[i]->M;
    }
    if (tiles > (1ll << 31) - 1 || total > (1ll << 31) - 1) return set_err(c, -EINVAL, "gemv: too many rows");
    for (int i = n; i < GEMV_MAX_SEG; ++i) {
        p.seg[i] = p.seg[0];
        p.seg[i].row_begin = INT32_MAX;
        p.seg[i].tile_begin = INT32_MAX;
    }
    p.nseg = n;
    p.nb = nb;
    p.x_tstride = K;
    p.total_rows = (int32_t)total;
    p.fmt = W[0]->fmt;
    const int cb_max = LDS_BUDGET / (SPQ4K_GEMV_MAX_T * 292);
    p.chunk_blocks = nb < cb_max ? nb : cb_max;
    Q8Planes Q;
    int rc = q8_planes(c, X, K, (int)T, nb, &Q);
    if (rc) return rc;
    for (int64_t t0 = 0; t0 < T; t0 += SPQ4K_GEMV_MAX_T) {
        const int tc = (int)(T - t0 < SPQ4K_GEMV_MAX_T ? T - t0 : SPQ4K_GEMV_MAX_T);
        p.Q.qs = Q.qs + t0 * nb * 256;
        p.Q.bs = Q.bs + t0 * nb * 16;
        p.Q.d = Q.d + t0 * nb;
        for (int i = 0; i < n; ++i) p.seg[i].Y = Y[i] + t0 * W[i]->M;
        for (int i = n; i < GEMV_MAX_SEG; ++i) p.seg[i].Y = p.seg[0].Y;
        hipError_t e = launch_gemv(p, tc, bpr, (int)tiles, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "gemv launch");
    }
    return 0;
}

}  // namespace

// ---- the no-allocation scratch ---------------------------------------------
// Device memory of spq4k_mul_mat_noalloc: a file-scope array, so that the
// entry point needs no hipMalloc. Every GPU the library runs on holds its own
// copy (SPQ4K_NOALLOC_SCRATCH_BYTES) from the first use of the library on
// that GPU until the process ends. In host code `scratch` names a host-side
// stand-in, never the device memory: its device address is looked up once per
// device (hipGetSymbolAddress, at spq4k_init with the device current) and only
// that address is passed to kernels.
static __device__ __align__(256) uint8_t scratch[SPQ4K_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_noalloc_mu;
uint8_t* g_noalloc_ptr[NOALLOC_MAX_DEVICES] = {};

// device address of `scratch` on `device`, the current device (0 on error)
int noalloc_scratch_setup(int device) {
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) return -ENODEV;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (g_noalloc_ptr[device]) return 0;
    // SPQ4K_TEST_NOALLOC_LOOKUP_FAIL=1 makes the lookup fail (for the test
    // that a context still comes up and the entry point reports -EIO)
    if (const char* f = getenv("SPQ4K_TEST_NOALLOC_LOOKUP_FAIL"))
        if (atoi(f) == 1) return -EIO;
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return -EIO;
    g_noalloc_ptr[device] = static_cast<uint8_t*>(p);
    return 0;
}

uint8_t* noalloc_scratch_of(int device) {
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    return g_noalloc_ptr[device];
}
}  // namespace

// ============================================================================
extern "C" {

int spq4k_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int spq4k_init(int device, spq4k_ctx** out) {
    if (!out) return -EINVAL;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return -ENODEV;
    spq4k_ctx* c = new (std::nothrow) spq4k_ctx();
    if (!c) return -ENOMEM;
    c->device = device;
    if (hipSetDevice(device) != hipSuccess) { delete c; return -ENODEV; }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0) {
        c->num_cus = prop.multiProcessorCount;
        c->lds_max = prop.sharedMemPerBlock < Q80_LDS_MAX ? prop.sharedMemPerBlock : Q80_LDS_MAX;
    }
    if (hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) != hipSuccess) { delete c; return -EIO; }
    c->stream = c->own_stream;
    if (const char* f = getenv("SPQ4K_GEMV_BPR")) {
        const int v = atoi(f);
        if (v == 1 || v == 2 || v == 4 || v == 8) c->force_bpr = v;
    }
    if (const char* f = getenv("SPQ4K_GEMV_GENERIC")) c->no_decode = atoi(f) == 1;
    if (const char* f = getenv("SPQ4K_MOE_UNFUSED")) c->moe_unfused = atoi(f) == 1;
    if (const char* f = getenv("SPQ4K_MOE_MODE")) c->moe_mode = atoi(f);
    if (const char* f = getenv("SPQ4K_GEMM_MODE")) c->gemm_mode = atoi(f);
    if (const char* f = getenv("SPQ4K_GEMM_CFG")) {
        const int v = atoi(f);
        if (v >= 0 && v < gemm_tiled_shapes()) c->gemm_cfg = v;
    }
    if (const char* f = getenv("SPQ4K_DEC_WAVES")) {
        const int v = atoi(f);
        if (v == 8 || v == 12 || v == 16) c->dec_force.waves = v;
    }
    if (const char* f = getenv("SPQ4K_DEC_DEPTH")) {
        const int v = atoi(f);
        if (v == 1 || v == 2) c->dec_force.depth = v;
    }
    if (const char* f = getenv("SPQ4K_DEC_XFIRST")) {
        c->dec_force.xfirst = atoi(f) == 1;
        c->dec_xfirst_set = 1;
    }
    if (const char* f = getenv("SPQ4K_DEC_GRID")) {
        const int v = atoi(f);
        if (v > 0 && v <= 65536) c->dec_force.grid = v;
    }
    if (const char* f = getenv("SPQ4K_GEMV_PREQ")) {
        const int v = atoi(f);
        if (v == 1 || v == 2) c->preq_mode = v;
    }
    if (const char* f = getenv("SPQ4K_GEMV_MFMA_MIN_T")) {
        const int v = atoi(f);
        if (v >= 2) c->gemv_mfma_min_t = v;
    }
    if (const char* f = getenv("SPQ4K_Q80_GRID")) {
        const int v = atoi(f);
        if (v > 0 && v <= 65536) c->q80_grid = v;
    }
    if (const char* f = getenv("SPQ4K_Q80_STAGED")) {
        const int v = atoi(f);
        if (v >= 0 && v <= 2) c->q80_staged = v;
    }
    if (const char* f = getenv("SPQ4K_MOE_DEC_MAX_T")) {
        const int v = atoi(f);
        if (v >= 1 && v <= 8) c->moe_dec_max_t = v;
    }
    if (const char* f = getenv("SPQ4K_MOE_DEC_WAVES")) {
        const int v = atoi(f);
        if (v == 8 || v == 12) c->moe_dec_waves = v;
    }
    if (const char* f = getenv("SPQ4K_MOE_RING_WAVES")) {
        const int v = atoi(f);
        if (v == 4 || v == 8) c->moe_ring_waves = v;
    }
    if (const char* f = getenv("SPQ4K_Q80_PREQ")) {
        const int v = atoi(f);
        if (v == 1 || v == 2) c->q80_preq = v;
    }
    // The no-allocation scratch's address is looked up here, with the device
    // current; a failure does not fail the context (only the no-allocation
    // entry point needs it, and it tries again on its first call).
    (void)noalloc_scratch_setup(device);
    // scratch for Q8_K activation planes: sized for prefill batches up front
    // so that steady-state calls (and graph capture) never allocate
    if (ensure_scratch(c, (size_t)16 << 20) != 0 || ensure_scratch2(c, (size_t)4 << 20) != 0) {
        if (c->scratch) (void)hipFree(c->scratch);
        if (c->scratch2) (void)hipFree(c->scratch2);
        (void)hipStreamDestroy(c->own_stream);
        delete c;
        return -ENOMEM;
    }
    *out = c;
    return 0;
}

void spq4k_free(spq4k_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    if (c->scratch) (void)hipFree(c->scratch);
    if (c->scratch2) (void)hipFree(c->scratch2);
    for (void* p : c->retired) (void)hipFree(p);
    if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
    delete c;
}

int spq4k_set_stream(spq4k_ctx* c, void* s) {
    if (!c) return -EINVAL;
    c->stream = s ? (hipStream_t)s : c->own_stream;
    return 0;
}

void* spq4k_get_stream(spq4k_ctx* c) { return c ? (void*)c->stream : nullptr; }
int spq4k_get_device(const spq4k_ctx* c) { return c ? c->device : -EINVAL; }

int spq4k_synchronize(spq4k_ctx* c) {
    int rc = use_device(c);
    if (rc) return rc;
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

const char* spq4k_last_error(const spq4k_ctx* c) { return c ? c->err : "null context"; }

// ---- weights -----------------------------------------------------------------
static int weights_new(spq4k_ctx* c, int type, int64_t M, int64_t K, int64_t E, spq4k_weights** out) {
    if (!out) return set_err(c, -EINVAL, "weights: null out");
    *out = nullptr;
    if (type_fmt(type) < 0)
        return set_err(c, -EINVAL, "weights: unsupported type %d (Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14)", type);
    int rc = check_shape(c, M, K, E, type_block_values(type));
    if (rc) return rc;
    spq4k_weights* w = new (std::nothrow) spq4k_weights();
    if (!w) return -ENOMEM;
    w->device = c->device;
    w->type = type;
    w->fmt = type_fmt(type);
    w->M = M;
    w->K = K;
    w->E = E;
    w->nbytes = (size_t)E * (size_t)M * (size_t)(K / type_block_values(type)) * type_block_bytes(type);
    *out = w;
    return 0;
}

int spq4k_weights_alloc(spq4k_ctx* c, int64_t M, int64_t K, int64_t E, spq4k_weights** out) {
    return spq4k_weights_alloc_type(c, SPQ4K_TYPE_Q4_K, M, K, E, out);
}

int spq4k_weights_alloc_type(spq4k_ctx* c, int type, int64_t M, int64_t K, int64_t E, spq4k_weights** out) {
    int rc = use_device(c);
    if (rc) return rc;
    spq4k_weights* w;
    rc = weights_new(c, type, M, K, E, &w);
    if (rc) return rc;
    if (hipMalloc(&w->data, w->nbytes) != hipSuccess) {
        const size_t nbytes = w->nbytes;
        delete w;
        return set_err(c, -ENOMEM, "weights: %zu bytes", nbytes);
    }
    w->owned = true;
    *out = w;
    return 0;
}

int spq4k_weights_upload(spq4k_ctx* c, const void* host, int64_t M, int64_t K, int64_t E, spq4k_weights** out) {
    return spq4k_weights_upload_type(c, SPQ4K_TYPE_Q4_K, host, M, K, E, out);
}

int spq4k_weights_upload_type(spq4k_ctx* c, int type, const void* host, int64_t M, int64_t K, int64_t E,
                              spq4k_weights** out) {
    if (!host) return set_err(c, -EINVAL, "weights_upload: null host pointer");
    int rc = spq4k_weights_alloc_type(c, type, M, K, E, out);
    if (rc) return rc;
    hipError_t e = hipMemcpyAsync((*out)->data, host, (*out)->nbytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        spq4k_weights_free(*out);
        *out = nullptr;
        return hip_fail(c, e, "weights_upload copy");
    }
    return 0;
}

int spq4k_weights_wrap(spq4k_ctx* c, const void* dev, int64_t M, int64_t K, int64_t E, spq4k_weights** out) {
    return spq4k_weights_wrap_type(c, SPQ4K_TYPE_Q4_K, dev, M, K, E, out);
}

int spq4k_weights_wrap_type(spq4k_ctx* c, int type, const void* dev, int64_t M, int64_t K, int64_t E,
                            spq4k_weights** out) {
    if (!dev || !aligned(dev, 16)) return set_err(c, -EINVAL, "weights_wrap: null or not 16-byte aligned");
    int rc = weights_new(c, type, M, K, E, out);
    if (rc) return rc;
    (*out)->data = (uint8_t*)dev;
    (*out)->owned = false;
    return 0;
}

void spq4k_weights_free(spq4k_weights* w) {
    if (!w) return;
    if (w->owned && w->data) {
        // hipFree waits for outstanding work on the device that uses the buffer
        (void)hipSetDevice(w->device);
        (void)hipFree(w->data);
    }
    delete w;
}

void* spq4k_weights_data(const spq4k_weights* w) { return w ? (void*)w->data : nullptr; }
int spq4k_weights_type(const spq4k_weights* w) { return w ? w->type : -EINVAL; }
int spq4k_weights_shape(const spq4k_weights* w, int64_t* M, int64_t* K, int64_t* E) {
    if (!w) return -EINVAL;
    if (M) *M = w->M;
    if (K) *K = w->K;
    if (E) *E = w->E;
    return 0;
}
size_t spq4k_weights_nbytes(const spq4k_weights* w) { return w ? w->nbytes : 0; }

// ---- type traits ---------------------------------------------------------------
int spq4k_dequant(spq4k_ctx* c, const void* vx, float* y, int64_t k) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!vx || !y || k < 0 || k % SPQ4K_QK_K || !aligned(vx, 16) || !aligned(y, 16))
        return set_err(c, -EINVAL, "dequant: bad arguments");
    hipError_t e = launch_dequant_q4k((const uint8_t*)vx, y, k / SPQ4K_QK_K, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "dequant launch");
    return 0;
}

int spq4k_quantize_q8K(spq4k_ctx* c, const float* x, void* vy, int64_t k) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!x || !vy || k < 0 || k % SPQ4K_QK_K || !aligned(x, 16) || !aligned(vy, 4))
        return set_err(c, -EINVAL, "quantize_q8K: bad arguments");
    hipError_t e = launch_quantize_q8k(x, (uint8_t*)vy, k / SPQ4K_QK_K, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "quantize_q8K launch");
    return 0;
}

int spq4k_quantize_q4K(spq4k_ctx* c, const float* src, void* dst, int64_t nrow, int64_t n_per_row) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!src || !dst || nrow < 0 || n_per_row <= 0 || n_per_row % SPQ4K_QK_K || !aligned(src, 16) ||
        !aligned(dst, 16))
        return set_err(c, -EINVAL, "quantize_q4K: bad arguments");
    hipError_t e = launch_quantize_q4k(src, (uint8_t*)dst, nrow * (n_per_row / SPQ4K_QK_K), c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "quantize_q4K launch");
    return 0;
}

int spq4k_vec_dot(spq4k_ctx* c, int n, float* s, const void* vx, const void* vy) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!s || !vx || !vy || n <= 0 || n % SPQ4K_QK_K || !aligned(vx, 16) || !aligned(vy, 4))
        return set_err(c, -EINVAL, "vec_dot: bad arguments");
    hipError_t e = launch_vec_dot_q8((const uint8_t*)vx, (const uint8_t*)vy, n / SPQ4K_QK_K, s, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "vec_dot launch");
    return 0;
}

// host variants: stage through device scratch
namespace {
struct DevBuf {
    void* p = nullptr;
    ~DevBuf() { if (p) (void)hipFree(p); }
};
}  // namespace

int spq4k_dequant_host(spq4k_ctx* c, const void* vx, float* y, int64_t k) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!vx || !y || k < 0 || k % SPQ4K_QK_K) return set_err(c, -EINVAL, "dequant_host: bad arguments");
    const size_t nin = (size_t)(k / SPQ4K_QK_K) * SPQ4K_Q4K_BLOCK_BYTES, nout = (size_t)k * sizeof(float);
    DevBuf a, b;
    if (hipMalloc(&a.p, nin + 16) != hipSuccess || hipMalloc(&b.p, nout + 16) != hipSuccess)
        return set_err(c, -ENOMEM, "dequant_host");
    SPQ_HIP(c, hipMemcpyAsync(a.p, vx, nin, hipMemcpyHostToDevice, c->stream));
    rc = spq4k_dequant(c, a.p, (float*)b.p, k);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(y, b.p, nout, hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

int spq4k_quantize_q8K_host(spq4k_ctx* c, const float* x, void* vy, int64_t k) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!x || !vy || k < 0 || k % SPQ4K_QK_K) return set_err(c, -EINVAL, "quantize_q8K_host: bad arguments");
    const size_t nin = (size_t)k * sizeof(float), nout = (size_t)(k / SPQ4K_QK_K) * SPQ4K_Q8K_BLOCK_BYTES;
    DevBuf a, b;
    if (hipMalloc(&a.p, nin + 16) != hipSuccess || hipMalloc(&b.p, nout + 16) != hipSuccess)
        return set_err(c, -ENOMEM, "quantize_q8K_host");
    SPQ_HIP(c, hipMemcpyAsync(a.p, x, nin, hipMemcpyHostToDevice, c->stream));
    rc = spq4k_quantize_q8K(c, (const float*)a.p, b.p, k);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(vy, b.p, nout, hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

int spq4k_quantize_q4K_host(spq4k_ctx* c, const float* src, void* dst, int64_t nrow, int64_t n_per_row) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!src || !dst || nrow < 0 || n_per_row <= 0 || n_per_row % SPQ4K_QK_K)
        return set_err(c, -EINVAL, "quantize_q4K_host: bad arguments");
    const int64_t k = nrow * n_per_row;
    const size_t nin = (size_t)k * sizeof(float), nout = (size_t)(k / SPQ4K_QK_K) * SPQ4K_Q4K_BLOCK_BYTES;
    DevBuf a, b;
    if (hipMalloc(&a.p, nin + 16) != hipSuccess || hipMalloc(&b.p, nout + 16) != hipSuccess)
        return set_err(c, -ENOMEM, "quantize_q4K_host");
    SPQ_HIP(c, hipMemcpyAsync(a.p, src, nin, hipMemcpyHostToDevice, c->stream));
    rc = spq4k_quantize_q4K(c, (const float*)a.p, b.p, nrow, n_per_row);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(dst, b.p, nout, hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

int spq4k_vec_dot_host(spq4k_ctx* c, int n, float* s, const void* vx, const void* vy) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!s || !vx || !vy || n <= 0 || n % SPQ4K_QK_K) return set_err(c, -EINVAL, "vec_dot_host: bad arguments");
    const size_t nx = (size_t)(n / SPQ4K_QK_K) * SPQ4K_Q4K_BLOCK_BYTES;
    const size_t ny = (size_t)(n / SPQ4K_QK_K) * SPQ4K_Q8K_BLOCK_BYTES;
    DevBuf a, b, o;
    if (hipMalloc(&a.p, nx + 16) != hipSuccess || hipMalloc(&b.p, ny + 16) != hipSuccess ||
        hipMalloc(&o.p, 16) != hipSuccess)
        return set_err(c, -ENOMEM, "vec_dot_host");
    SPQ_HIP(c, hipMemcpyAsync(a.p, vx, nx, hipMemcpyHostToDevice, c->stream));
    SPQ_HIP(c, hipMemcpyAsync(b.p, vy, ny, hipMemcpyHostToDevice, c->stream));
    rc = spq4k_vec_dot(c, n, (float*)o.p, a.p, b.p);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(s, o.p, sizeof(float), hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

// ---- type traits of any supported weight type ------------------------------------
int spq4k_to_float(spq4k_ctx* c, int type, const void* vx, float* y, int64_t k) {
    if (type == SPQ4K_TYPE_Q4_K) return spq4k_dequant(c, vx, y, k);
    int rc = use_device(c);
    if (rc) return rc;
    if (type == SPQ4K_TYPE_Q8_0) {
        if (!vx || !y || k < 0 || k % SPQ4K_QK8_0 || !aligned(vx, 2) || !aligned(y, 16))
            return set_err(c, -EINVAL, "to_float: bad arguments");
        hipError_t e = launch_dequant_q8_0((const uint8_t*)vx, y, k / SPQ4K_QK8_0, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "dequant_q8_0 launch");
        return 0;
    }
    if (type != SPQ4K_TYPE_Q6_K && type != SPQ4K_TYPE_Q5_K)
        return set_err(c, -EINVAL, "to_float: unsupported type %d", type);
    if (!vx || !y || k < 0 || k % SPQ4K_QK_K || !aligned(vx, type == SPQ4K_TYPE_Q5_K ? 16 : 2) || !aligned(y, 16))
        return set_err(c, -EINVAL, "to_float: bad arguments");
    hipError_t e = type == SPQ4K_TYPE_Q5_K ? launch_dequant_q5k((const uint8_t*)vx, y, k / SPQ4K_QK_K, c->stream)
                                           : launch_dequant_q6k((const uint8_t*)vx, y, k / SPQ4K_QK_K, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "dequant_q6k launch");
    return 0;
}

int spq4k_quantize_chunk(spq4k_ctx* c, int type, const float* src, void* dst, int64_t nrow, int64_t n_per_row) {
    if (type == SPQ4K_TYPE_Q4_K) return spq4k_quantize_q4K(c, src, dst, nrow, n_per_row);
    int rc = use_device(c);
    if (rc) return rc;
    if (type == SPQ4K_TYPE_Q8_0) {
        if (!src || !dst || nrow < 0 || n_per_row <= 0 || n_per_row % SPQ4K_QK8_0 || !aligned(src, 16) ||
            !aligned(dst, 2))
            return set_err(c, -EINVAL, "quantize_chunk: bad arguments");
        hipError_t e = launch_quantize_q8_0(src, (uint8_t*)dst, nrow * (n_per_row / SPQ4K_QK8_0), true, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "quantize_q8_0 launch");
        return 0;
    }
    if (type != SPQ4K_TYPE_Q6_K && type != SPQ4K_TYPE_Q5_K)
        return set_err(c, -EINVAL, "quantize_chunk: unsupported type %d", type);
    if (!src || !dst || nrow < 0 || n_per_row <= 0 || n_per_row % SPQ4K_QK_K || !aligned(src, 16) ||
        !aligned(dst, type == SPQ4K_TYPE_Q5_K ? 16 : 2))
        return set_err(c, -EINVAL, "quantize_chunk: bad arguments");
    const int64_t nblk = nrow * (n_per_row / SPQ4K_QK_K);
    hipError_t e = type == SPQ4K_TYPE_Q5_K ? launch_quantize_q5k(src, (uint8_t*)dst, nblk, c->stream)
                                           : launch_quantize_q6k(src, (uint8_t*)dst, nblk, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "quantize_q6k launch");
    return 0;
}

int spq4k_vec_dot_q8K(spq4k_ctx* c, int type, int n, float* s, const void* vx, const void* vy) {
    if (type == SPQ4K_TYPE_Q4_K) return spq4k_vec_dot(c, n, s, vx, vy);
    int rc = use_device(c);
    if (rc) return rc;
    if (type != SPQ4K_TYPE_Q6_K && type != SPQ4K_TYPE_Q5_K)
        return set_err(c, -EINVAL, "vec_dot_q8K: unsupported type %d", type);
    if (!s || !vx || !vy || n <= 0 || n % SPQ4K_QK_K || !aligned(vx, type == SPQ4K_TYPE_Q5_K ? 16 : 2) ||
        !aligned(vy, 4))
        return set_err(c, -EINVAL, "vec_dot_q8K: bad arguments");
    hipError_t e = type == SPQ4K_TYPE_Q5_K
                       ? launch_vec_dot_q5k((const uint8_t*)vx, (const uint8_t*)vy, n / SPQ4K_QK_K, s, c->stream)
                       : launch_vec_dot_q6k((const uint8_t*)vx, (const uint8_t*)vy, n / SPQ4K_QK_K, s, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "vec_dot_q6k launch");
    return 0;
}

int spq4k_quantize_q8_0(spq4k_ctx* c, const float* x, void* vy, int64_t k) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!x || !vy || k < 0 || k % SPQ4K_QK8_0 || !aligned(x, 16) || !aligned(vy, 2))
        return set_err(c, -EINVAL, "quantize_q8_0: bad arguments");
    hipError_t e = launch_quantize_q8_0(x, (uint8_t*)vy, k / SPQ4K_QK8_0, false, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "quantize_q8_0 launch");
    return 0;
}

int spq4k_vec_dot_q8_0(spq4k_ctx* c, int n, float* s, const void* vx, const void* vy) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!s || !vx || !vy || n <= 0 || n % SPQ4K_QK8_0 || !aligned(vx, 2) || !aligned(vy, 2))
        return set_err(c, -EINVAL, "vec_dot_q8_0: bad arguments");
    hipError_t e = launch_vec_dot_q8_0((const uint8_t*)vx, (const uint8_t*)vy, n / SPQ4K_QK8_0, s, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "vec_dot_q8_0 launch");
    return 0;
}

int spq4k_quantize_q8_0_host(spq4k_ctx* c, const float* x, void* vy, int64_t k) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!x || !vy || k < 0 || k % SPQ4K_QK8_0) return set_err(c, -EINVAL, "quantize_q8_0_host: bad arguments");
    const size_t nin = (size_t)k * sizeof(float), nout = (size_t)(k / SPQ4K_QK8_0) * SPQ4K_Q8_0_BLOCK_BYTES;
    DevBuf a, b;
    if (hipMalloc(&a.p, nin + 16) != hipSuccess || hipMalloc(&b.p, nout + 16) != hipSuccess)
        return set_err(c, -ENOMEM, "quantize_q8_0_host");
    SPQ_HIP(c, hipMemcpyAsync(a.p, x, nin, hipMemcpyHostToDevice, c->stream));
    rc = spq4k_quantize_q8_0(c, (const float*)a.p, b.p, k);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(vy, b.p, nout, hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

int spq4k_vec_dot_q8_0_host(spq4k_ctx* c, int n, float* s, const void* vx, const void* vy) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!s || !vx || !vy || n <= 0 || n % SPQ4K_QK8_0) return set_err(c, -EINVAL, "vec_dot_q8_0_host: bad arguments");
    const size_t nx = (size_t)(n / SPQ4K_QK8_0) * SPQ4K_Q8_0_BLOCK_BYTES;
    DevBuf a, b, o;
    if (hipMalloc(&a.p, nx + 16) != hipSuccess || hipMalloc(&b.p, nx + 16) != hipSuccess ||
        hipMalloc(&o.p, 16) != hipSuccess)
        return set_err(c, -ENOMEM, "vec_dot_q8_0_host");
    SPQ_HIP(c, hipMemcpyAsync(a.p, vx, nx, hipMemcpyHostToDevice, c->stream));
    SPQ_HIP(c, hipMemcpyAsync(b.p, vy, nx, hipMemcpyHostToDevice, c->stream));
    rc = spq4k_vec_dot_q8_0(c, n, (float*)o.p, a.p, b.p);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(s, o.p, sizeof(float), hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

int spq4k_to_float_host(spq4k_ctx* c, int type, const void* vx, float* y, int64_t k) {
    int rc = use_device(c);
    if (rc) return rc;
    const size_t bb = type_block_bytes(type);
    const int64_t qk = type_block_values(type);
    if (!vx || !y || k < 0 || k % qk || !bb) return set_err(c, -EINVAL, "to_float_host: bad arguments");
    const size_t nin = (size_t)(k / qk) * bb, nout = (size_t)k * sizeof(float);
    DevBuf a, b;
    if (hipMalloc(&a.p, nin + 16) != hipSuccess || hipMalloc(&b.p, nout + 16) != hipSuccess)
        return set_err(c, -ENOMEM, "to_float_host");
    SPQ_HIP(c, hipMemcpyAsync(a.p, vx, nin, hipMemcpyHostToDevice, c->stream));
    rc = spq4k_to_float(c, type, a.p, (float*)b.p, k);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(y, b.p, nout, hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

int spq4k_quantize_chunk_host(spq4k_ctx* c, int type, const float* src, void* dst, int64_t nrow, int64_t n_per_row) {
    int rc = use_device(c);
    if (rc) return rc;
    const size_t bb = type_block_bytes(type);
    const int64_t qk = type_block_values(type);
    if (!src || !dst || nrow < 0 || n_per_row <= 0 || n_per_row % qk || !bb)
        return set_err(c, -EINVAL, "quantize_chunk_host: bad arguments");
    const int64_t k = nrow * n_per_row;
    const size_t nin = (size_t)k * sizeof(float), nout = (size_t)(k / qk) * bb;
    DevBuf a, b;
    if (hipMalloc(&a.p, nin + 16) != hipSuccess || hipMalloc(&b.p, nout + 16) != hipSuccess)
        return set_err(c, -ENOMEM, "quantize_chunk_host");
    SPQ_HIP(c, hipMemcpyAsync(a.p, src, nin, hipMemcpyHostToDevice, c->stream));
    rc = spq4k_quantize_chunk(c, type, (const float*)a.p, b.p, nrow, n_per_row);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(dst, b.p, nout, hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

int spq4k_vec_dot_q8K_host(spq4k_ctx* c, int type, int n, float* s, const void* vx, const void* vy) {
    int rc = use_device(c);
    if (rc) return rc;
    const size_t bb = type_block_bytes(type);
    if (!s || !vx || !vy || n <= 0 || n % SPQ4K_QK_K || !bb) return set_err(c, -EINVAL, "vec_dot_q8K_host: bad arguments");
    const size_t nx = (size_t)(n / SPQ4K_QK_K) * bb;
    const size_t ny = (size_t)(n / SPQ4K_QK_K) * SPQ4K_Q8K_BLOCK_BYTES;
    DevBuf a, b, o;
    if (hipMalloc(&a.p, nx + 16) != hipSuccess || hipMalloc(&b.p, ny + 16) != hipSuccess ||
        hipMalloc(&o.p, 16) != hipSuccess)
        return set_err(c, -ENOMEM, "vec_dot_q8K_host");
    SPQ_HIP(c, hipMemcpyAsync(a.p, vx, nx, hipMemcpyHostToDevice, c->stream));
    SPQ_HIP(c, hipMemcpyAsync(b.p, vy, ny, hipMemcpyHostToDevice, c->stream));
    rc = spq4k_vec_dot_q8K(c, type, n, (float*)o.p, a.p, b.p);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(s, o.p, sizeof(float), hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

// ---- matmul ----------------------------------------------------------------------
int spq4k_gemv(spq4k_ctx* c, const spq4k_weights* W, const float* x, float* y, int64_t T) {
    int rc = use_device(c);
    if (rc) return rc;
    const spq4k_weights* ws[1] = {W};
    float* ys[1] = {y};
    return gemv_launch(c, 1, ws, x, ys, T);
}

int spq4k_gemv_multi(spq4k_ctx* c, int n, const spq4k_weights* const* W, const float* x, float* const* y,
                     int64_t T) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!W || !y) return set_err(c, -EINVAL, "gemv_multi: null arrays");
    return gemv_launch(c, n, W, x, y, T);
}

namespace {

// Matrix-core matmul of n matrices sharing the input (shapes checked by the
// callers): plan, quantise X once into the context scratch (with the partial
// plane of a K split behind it), launch.
int gemm_segments(spq4k_ctx* c, int n, const spq4k_weights* const* W, const float* X, float* const* Y, int64_t T,
                  int mode) {
    if (W[0]->fmt == WF_Q80) return q80_dense(c, n, W, X, Y, T);
    const int64_t K = W[0]->K;
    GemmParams p;
    memset(&p, 0, sizeof p);
    p.T = (int32_t)T;
    p.nb = (int32_t)(K / SPQ4K_QK_K);
    p.mode = mode;
    p.cfg = c->gemm_cfg;
    int64_t tiles16 = 0, rows = 0;
    for (int i = 0; i < n; ++i) {
        p.seg[i].W = W[i]->data;
        p.seg[i].Y = Y[i];
        p.seg[i].M = (int32_t)W[i]->M;
        p.seg[i].tile_begin = (int32_t)tiles16;
        p.seg[i].row_begin = (int32_t)rows;
        tiles16 += (W[i]->M + 15) / 16;
        rows += W[i]->M;
    }
    for (int i = n; i < GEMM_MAX_SEG; ++i) p.seg[i].tile_begin = p.seg[i].row_begin = INT32_MAX;
    p.nseg = n;
    p.rows = (int32_t)rows;
    p.fmt = W[0]->fmt;
    if (tiles16 * ((T + 15) / 16) > (1ll << 31) - 1 || rows > (1ll << 31) - 1)
        return set_err(c, -EINVAL, "gemm: grid too large");
    if (!fmt_has_mfma(p.fmt) || (p.fmt != WF_Q4K && mode == 1)) {   // sdot4 kernels over 8-token slices
        if (T <= SPQ4K_GEMV_MAX_T) return gemv_launch(c, n, W, X, Y, T);
        return gemv_chunked(c, n, W, X, Y, T);
    }
    hipError_t e;
    if (gemm_use_skinny((int)T, mode)) {
        int rc = q8_planes(c, X, K, (int)T, p.nb, &p.Q);
        if (rc) return rc;
        p.total_tiles = (int32_t)tiles16;
        e = launch_gemm_skinny(p, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "gemm skinny launch");
        return 0;
    }
    const size_t planes = q8_planes_bytes((int)T, p.nb);
    const GemmPlan g = gemm_plan(p, c->num_cus, KSPLIT_PARTIAL_BYTES);
    p.cfg = g.cfg;
    p.ksplit = g.ksplit;
    p.kchunk = g.kchunk;
    int rc = q8_planes(c, X, K, (int)T, p.nb, &p.Q, g.perm, g.partial_bytes);
    if (rc) return rc;
    p.P = g.ksplit > 1 ? reinterpret_cast<float*>(c->scratch + planes) : nullptr;
    e = launch_gemm(p, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "gemm launch");
    return 0;
}

}  // namespace

int spq4k_gemm_multi(spq4k_ctx* c, int n, const spq4k_weights* const* W, const float* X, float* const* Y,
                     int64_t T) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!W || !Y || n < 1 || n > GEMM_MAX_SEG) return set_err(c, -EINVAL, "gemm: n=%d matrices (1..4)", n);
    if (!X || T < 1 || !aligned(X, 16)) return set_err(c, -EINVAL, "gemm: bad activations");
    if (T > (1 << 20)) return set_err(c, -EINVAL, "gemm: T too large");
    if (!W[0]) return set_err(c, -EINVAL, "gemm: null weight");
    const int64_t K = W[0]->K;
    for (int i = 0; i < n; ++i) {
        if (!W[i] || !W[i]->data || !Y[i] || W[i]->E != 1 || W[i]->K != K)
            return set_err(c, -EINVAL, "gemm: matrices must be non-null, E=1 and share K");
        if (W[i]->type != W[0]->type) return set_err(c, -EINVAL, "gemm: matrices must share the weight type");
        if (!aligned(W[i]->data, type_align(W[i]->type))) return set_err(c, -EINVAL, "gemm: misaligned weights");
        if (W[i]->device != c->device) return set_err(c, -EINVAL, "gemm: weights live on another device");
    }
    return gemm_segments(c, n, W, X, Y, T, c->gemm_mode);
}

int spq4k_gemm(spq4k_ctx* c, const spq4k_weights* W, const float* X, float* Y, int64_t T) {
    const spq4k_weights* ws[1] = {W};
    float* ys[1] = {Y};
    return spq4k_gemm_multi(c, 1, ws, X, ys, T);
}

int spq4k_mul_mat(spq4k_ctx* c, const spq4k_weights* W, const float* X, float* Y, int64_t T) {
    if (T >= 1 && T <= SPQ4K_GEMV_MAX_T) return spq4k_gemv(c, W, X, Y, T);
    return spq4k_gemm(c, W, X, Y, T);
}

int spq4k_ptr_on_device(spq4k_ctx* c, const void* p, size_t bytes) {
    if (!c || !p) return 0;
    hipPointerAttribute_t a;
    for (const char* q : {(const char*)p, (const char*)p + (bytes ? bytes - 1 : 0)}) {
        if (hipPointerGetAttributes(&a, q) != hipSuccess) {
            (void)hipGetLastError();   // an unknown pointer is an answer, not a sticky error
            return 0;
        }
        if (a.type != hipMemoryTypeDevice || a.device != c->device) return 0;
    }
    return 1;
}

int spq4k_mul_mat_noalloc(spq4k_ctx* c, const spq4k_weights* W, const float* X, float* Y, int64_t T) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!W || !W->data) return set_err(c, -EINVAL, "mul_mat_noalloc: null weight");
    uint8_t* base = noalloc_scratch_of(c->device);
    if (!base && noalloc_scratch_setup(c->device) == 0) base = noalloc_scratch_of(c->device);
    if (!base) return set_err(c, -EIO, "mul_mat_noalloc: no device address of the no-allocation scratch");
    if (T < 1 || T > (1 << 20)) return set_err(c, -EINVAL, "mul_mat_noalloc: T=%lld", (long long)T);
    // the activation planes must leave the partial plane of a K split its 8 MiB
    const size_t planes = W->fmt == WF_Q80 ? q80_planes_bytes(T, (int)(W->K / SPQ4K_QK8_0))
                                           : q8_planes_bytes((int)T, (int)(W->K / SPQ4K_QK_K));
    if (planes > SPQ4K_NOALLOC_PLANES_MAX)
        return set_err(c, -EINVAL,
                       "mul_mat_noalloc: T=%lld rows of K=%lld need %zu bytes of activation planes, more than the "
                       "%zu the no-allocation scratch holds for them", (long long)T, (long long)W->K, planes,
                       (size_t)SPQ4K_NOALLOC_PLANES_MAX);
    uint8_t* const own = c->scratch;
    const size_t own_cap = c->scratch_cap;
    c->scratch = base;
    c->scratch_cap = SPQ4K_NOALLOC_SCRATCH_BYTES;
    c->no_alloc = true;
    rc = spq4k_mul_mat(c, W, X, Y, T);
    c->scratch = own;
    c->scratch_cap = own_cap;
    c->no_alloc = false;
    return rc;
}

int spq4k_reserve(spq4k_ctx* c, size_t scratch_bytes, size_t fusion_bytes) {
    int rc = use_device(c);
    if (rc) return rc;
    rc = ensure_scratch(c, scratch_bytes);
    if (rc) return rc;
    return ensure_scratch2(c, fusion_bytes);
}

namespace {

// GGML_OP_MUL_MAT_ID for a Q8_0 bank (arguments checked by spq4k_moe).
// Small batches sweep the rows of every routed pair in one launch with the
// input rows quantised into each workgroup's LDS; larger ones quantise the
// input rows once into planes, route the pairs by expert and stream each
// active expert once, its pairs TC at a time.
int q80_moe(spq4k_ctx* c, const spq4k_weights* const* banks, int nbank, const int32_t* ids, int64_t n_used,
            int64_t ne11, int64_t T, const float* X, float* const* Ys) {
    const spq4k_weights* bank = banks[0];
    float* Y = Ys[0];
    const int E = (int)bank->E, M = (int)bank->M, nb = (int)(bank->K / SPQ4K_QK8_0);
    const int64_t rows = T * ne11, n_pairs = T * n_used;
    // two banks (gate and up of equal rows) share the planes, the routing and
    // one launch of the matrix-core expert kernel; anything else is the
    // caller's, one bank at a time
    if (nbank > 1) {
        const int64_t ma = n_pairs < E ? n_pairs : E;
        if (c->moe_unfused || bank->K % SPQ4K_QK_K != 0 || (n_pairs + ma - 1) / ma < 2 || banks[1]->M != M ||
            (T <= 4 && n_pairs <= MOE_DEC_MAX_PAIRS && q80_lds_bytes((int)rows, nb) <= 64 * 1024 &&
             c->moe_mode == 0))
            return 1;
    }
    Q80Params p;
    memset(&p, 0, sizeof p);
    p.nb = nb;
    p.bank = bank->data;
    p.expert_bytes = (size_t)M * nb * SPQ4K_Q8_0_BLOCK_BYTES;
    p.Y = Y;
    p.E = E;
    p.M = M;
    p.n_used = (int32_t)n_used;
    p.ne11 = (int32_t)ne11;
    p.X = X;
    p.x_tstride = bank->K;
    if (T <= 4 && n_pairs <= MOE_DEC_MAX_PAIRS && q80_lds_bytes((int)rows, nb) <= 64 * 1024 && c->moe_mode == 0 &&
        !c->moe_unfused && n_pairs * M <= INT32_MAX) {
        p.ids = ids;
        p.n_xrows = (int32_t)rows;
        p.total_rows = (int32_t)(n_pairs * M);
        hipError_t e = launch_moe_q8_0_sweep(p, q80_grid(c, n_pairs * M, nb, rows), c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "moe_q8_0 sweep launch");
        return 0;
    }
    if (rows * nb > INT32_MAX) return set_err(c, -EINVAL, "moe: too many input rows");
    // scratch: Q8_0 planes | routing tables
    const size_t planes = q80_planes_bytes(rows, nb);
    const size_t route_bytes = (size_t)(1 + 3 * E + n_pairs) * sizeof(int32_t);
    int rc = q80_planes(c, X, bank->K, rows, nb, &p, route_bytes);
    if (rc) return rc;
    int32_t* rt = (int32_t*)(c->scratch + planes);
    p.route.n_act = rt;
    p.route.act = rt + 1;
    p.route.act_off = rt + 1 + E;
    p.route.act_cnt = rt + 1 + 2 * E;
    p.route.pairs = rt + 1 + 3 * E;
    hipError_t e = launch_moe_route(ids, (int)n_pairs, E, p.route, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "moe route launch");
    const int64_t max_act = n_pairs < E ? n_pairs : E;
    const int64_t mean_pairs = (n_pairs + max_act - 1) / max_act;
    // matrix cores once the active experts receive two pairs on average (K a
    // multiple of 256): moe_ring_kernel streams each expert once per 16 pairs
    if (!c->moe_unfused && bank->K % SPQ4K_QK_K == 0 && mean_pairs >= 2) {
        MoeParams mp;
        memset(&mp, 0, sizeof mp);
        mp.route = p.route;
        mp.bank = bank->data;
        mp.expert_bytes = p.expert_bytes;
        mp.Y = Y;
        mp.Q.qs = p.Aq;
        mp.Q.d = p.Ad;
        mp.Q.mn = reinterpret_cast<const uint8_t*>(p.Aq);   // no min-term plane: a valid address for stray reads
        mp.M = M;
        mp.nb = (int32_t)(bank->K / SPQ4K_QK_K);
        mp.n_used = (int32_t)n_used;
        mp.ne11 = (int32_t)ne11;
        mp.fmt = WF_Q80;
        mp.nbank = nbank;
        mp.max_act = (int32_t)max_act;
        if (nbank > 1) {
            mp.bank1 = banks[1]->data;
            mp.Y1 = Ys[1];
        }
        const int nw = moe_ring_waves(c, WF_Q80);
        const int64_t ntiles = (M + 16 * nw - 1) / (16 * nw);
        int64_t rtw = ntiles * max_act * nbank / (2 * (int64_t)c->num_cus);
        if (rtw < 1) rtw = 1;
        if (rtw > ntiles) rtw = ntiles;
        mp.ring_rt = (int32_t)rtw;
        mp.tiles_per_expert = (int32_t)((ntiles + rtw - 1) / rtw);
        if (max_act * mp.tiles_per_expert * nbank > (1ll << 31) - 1) return set_err(c, -EINVAL, "moe: grid too large");
        e = launch_moe_ring_q80(mp, (int)max_act, nw, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "moe ring (Q8_0) launch");
        return 0;
    }
    if (nbank > 1) return 1;   // the grouped matvec takes one bank (the caller runs each)
    // pairs a row is dotted with at a time: about twice the mean an active
    // expert receives, at most 8
    int tc = 1;
    while (tc < 8 && tc < 2 * mean_pairs) tc *= 2;
    // rows of an expert a workgroup takes: whole passes of its waves, as few
    // as still give two workgroups per CU over the experts that can be active
    const int64_t pass = q80_rows_per_wg(nb);
    const int64_t passes = (M + pass - 1) / pass;
    int64_t groups = (2 * (int64_t)c->num_cus + max_act - 1) / max_act;
    if (groups > passes) groups = passes;
    const int64_t per_wg = (passes + groups - 1) / groups * pass;
    p.rows_per_wg = (int32_t)per_wg;
    p.groups = (int32_t)((M + per_wg - 1) / per_wg);
    if (max_act * p.groups > INT32_MAX) return set_err(c, -EINVAL, "moe: grid too large");
    e = launch_moe_q8_0_grouped(p, tc, (int)(max_act * p.groups), c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "moe_q8_0 grouped launch");
    return 0;
}

}  // namespace

// ---- the operations fused around the matvec -------------------------------------
int spq4k_rms_norm(spq4k_ctx* c, const float* x, const float* w, float eps, float* y, int64_t K, int64_t T) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!x || !w || !y || K <= 0 || K > (1 << 30) || T < 1 || T > (1 << 24) || !(eps >= 0.0f) || !aligned(x, 4) ||
        !aligned(y, 4) || !aligned(w, 4))
        return set_err(c, -EINVAL, "rms_norm: bad arguments");
    hipError_t e = launch_rms_norm(x, K, (int)T, (int)K, w, eps, y, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "rms_norm launch");
    return 0;
}

int spq4k_swiglu(spq4k_ctx* c, const float* g, const float* u, float* y, int64_t n) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!g || !u || !y || n < 0 || !aligned(g, 4) || !aligned(u, 4) || !aligned(y, 4))
        return set_err(c, -EINVAL, "swiglu: bad arguments");
    hipError_t e = launch_swiglu(g, u, y, n, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "swiglu launch");
    return 0;
}

namespace {

// matmul of n matrices sharing X, any T (spq4k_mul_mat's dispatch)
int mul_mat_n(spq4k_ctx* c, int n, const spq4k_weights* const* W, const float* X, float* const* Y, int64_t T) {
    if (T <= SPQ4K_GEMV_MAX_T) return gemv_launch(c, n, W, X, Y, T);
    return gemm_segments(c, n, W, X, Y, T, c->gemm_mode);
}

int check_fused_args(spq4k_ctx* c, const char* what, int n, const spq4k_weights* const* W, const float* x,
                     const float* norm_w, float eps, int64_t T) {
    if (!W || n < 1 || n > GEMV_MAX_SEG || !W[0]) return set_err(c, -EINVAL, "%s: bad matrices", what);
    if (!x || !aligned(x, 16) || T < 1 || T > (1 << 20)) return set_err(c, -EINVAL, "%s: bad activations", what);
    if (norm_w && (!aligned(norm_w, 16) || !(eps >= 0.0f))) return set_err(c, -EINVAL, "%s: bad norm weights", what);
    for (int i = 0; i < n; ++i) {
        if (!W[i] || !W[i]->data || W[i]->E != 1 || W[i]->K != W[0]->K || W[i]->type != W[0]->type)
            return set_err(c, -EINVAL, "%s: matrices must be non-null, E = 1, and share K and type", what);
        if (!aligned(W[i]->data, type_align(W[i]->type))) return set_err(c, -EINVAL, "%s: misaligned weights", what);
        if (W[i]->device != c->device) return set_err(c, -EINVAL, "%s: weights live on another device", what);
    }
    return 0;
}

}  // namespace

int spq4k_mul_mat_rms_norm(spq4k_ctx* c, int n, const spq4k_weights* const* W, const float* x, const float* norm_w,
                           float eps, float* const* y, int64_t T) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!norm_w) return set_err(c, -EINVAL, "mul_mat_rms_norm: null norm weights");
    rc = check_fused_args(c, "mul_mat_rms_norm", n, W, x, norm_w, eps, T);
    if (rc) return rc;
    if (!y) return set_err(c, -EINVAL, "mul_mat_rms_norm: null outputs");
    for (int i = 0; i < n; ++i)
        if (!y[i]) return set_err(c, -EINVAL, "mul_mat_rms_norm: null output");
    if (T == 1) {
        Fuse f;
        f.norm_w = norm_w;
        f.eps = eps;
        rc = gemv_launch(c, n, W, x, y, T, &f);
        if (rc <= 0) return rc;
    }
    // unfused: the normalised rows, then the matmul on them
    const int64_t K = W[0]->K;
    rc = ensure_scratch2(c, (size_t)T * K * sizeof(float));
    if (rc) return rc;
    float* xn = reinterpret_cast<float*>(c->scratch2);
    hipError_t e = launch_rms_norm(x, K, (int)T, (int)K, norm_w, eps, xn, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "rms_norm launch");
    return mul_mat_n(c, n, W, xn, y, T);
}

int spq4k_mul_mat_swiglu(spq4k_ctx* c, const spq4k_weights* Wg, const spq4k_weights* Wu, const float* x,
                         const float* norm_w, float eps, float* y, int64_t T) {
    int rc = use_device(c);
    if (rc) return rc;
    const spq4k_weights* W[2] = {Wg, Wu};
    rc = check_fused_args(c, "mul_mat_swiglu", 2, W, x, norm_w, eps, T);
    if (rc) return rc;
    if (!y || Wg->M != Wu->M) return set_err(c, -EINVAL, "mul_mat_swiglu: null output or gate / up rows differ");
    if (T == 1) {
        Fuse f;
        f.norm_w = norm_w;
        f.eps = eps;
        f.glu = true;
        float* ys[2] = {y, y};
        rc = gemv_launch(c, 2, W, x, ys, T, &f);
        if (rc <= 0) return rc;
    }
    // unfused: [normalised rows], gate and up, then silu(gate) * up
    const int64_t K = Wg->K, M = Wg->M;
    const size_t xb = norm_w ? (((size_t)T * K * sizeof(float) + 255) & ~(size_t)255) : 0;
    const size_t gb = (((size_t)T * M * sizeof(float)) + 255) & ~(size_t)255;
    rc = ensure_scratch2(c, xb + 2 * gb);
    if (rc) return rc;
    const float* xin = x;
    hipError_t e;
    if (norm_w) {
        float* xn = reinterpret_cast<float*>(c->scratch2);
        e = launch_rms_norm(x, K, (int)T, (int)K, norm_w, eps, xn, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "rms_norm launch");
        xin = xn;
    }
    float* G = reinterpret_cast<float*>(c->scratch2 + xb);
    float* U = reinterpret_cast<float*>(c->scratch2 + xb + gb);
    float* gu[2] = {G, U};
    rc = mul_mat_n(c, 2, W, xin, gu, T);
    if (rc) return rc;
    e = launch_swiglu(G, U, y, T * M, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "swiglu launch");
    return 0;
}

namespace {

int moe_check(spq4k_ctx* c, const spq4k_weights* bank, const int32_t* ids, int64_t n_used, int64_t ne11,
              int64_t T, const float* X, const float* Y) {
    if (!bank || !bank->data || !ids || !X || !Y) return set_err(c, -EINVAL, "moe: null argument");
    if (T < 1 || n_used < 1 || n_used > bank->E || (ne11 != 1 && ne11 != n_used))
        return set_err(c, -EINVAL, "moe: T=%lld n_used=%lld ne11=%lld", (long long)T, (long long)n_used,
                       (long long)ne11);
    if (!aligned(X, 16) || !aligned(bank->data, type_align(bank->type)) || !aligned(ids, 4))
        return set_err(c, -EINVAL, "moe: misaligned pointer");
    if (bank->E > 4096 || T * n_used > (1 << 24)) return set_err(c, -EINVAL, "moe: too many experts or pairs");
    return 0;
}

// Small batches of a K-quant bank, or of two banks of one type, K and E
// sharing ids and X (gate and up): the decode mapping, every routed pair's
// rows (of both banks) in one sweep and one launch. An expert chosen twice
// is streamed twice, so only for small batches (T <= moe_dec_max_t).
// Returns 1 when it does not apply.
// glu (nbank 2, banks of equal M: gate then up): Y[0] = silu(gate . x) * (up . x)
// in the same launch, the SwiGLU epilogue of the pair
int moe_decode_try(spq4k_ctx* c, const spq4k_weights* const* banks, int nbank, const int32_t* ids,
                   int64_t n_used, int64_t ne11, int64_t T, const float* X, float* const* Y, bool glu = false) {
    const spq4k_weights* bank = banks[0];
    const int E = (int)bank->E, nb = (int)(bank->K / SPQ4K_QK_K), M = (int)bank->M;
    const int M1 = nbank > 1 ? (int)banks[1]->M : 0;
    if (glu && (nbank != 2 || M1 != M)) return 1;
    const int64_t MV = glu ? M : (int64_t)M + M1;   // sweep rows a pair
    const size_t bb = type_block_bytes(bank->type);
    const int64_t rows = T * ne11, n_pairs = T * n_used;
    if (!(T <= c->moe_dec_max_t && n_pairs <= MOE_DEC_MAX_PAIRS && rows <= MOE_DEC_MAX_XROWS && moe_decode_supported(nb) &&
          !c->moe_unfused && c->moe_mode == 0 && n_pairs * MV <= INT32_MAX))
        return 1;
    MoeFusedParams f;
    memset(&f, 0, sizeof f);
    f.ids = ids;
    f.X = X;
    f.bank = bank->data;
    f.expert_bytes = (size_t)M * nb * bb;
    f.fmt = bank->fmt;
    f.Y = Y[0];
    f.n_pairs = (int32_t)n_pairs;
    f.n_used = (int32_t)n_used;
    f.ne11 = (int32_t)ne11;
    f.K = (int32_t)bank->K;
    f.M = M;
    f.nb = nb;
    f.E = E;
    f.n_xrows = (int32_t)rows;
    if (nbank > 1) {
        f.bank1 = banks[1]->data;
        f.expert_bytes1 = (size_t)M1 * nb * bb;
        f.Y1 = glu ? nullptr : Y[1];
        f.M1 = glu ? 0 : M1;
        f.glu = glu ? 1 : 0;
    }
    // a GLU sweep that 12-wave workgroups cover in one workgroup a CU runs
    // so: these 8-wave workgroups start one a CU (their registers), so a
    // grid above the CU count runs in two rounds (the 30B-A3B block at T = 1:
    // 384 workgroups of 8 waves, the last 128 starting when the first end)
    int waves = 8;
    if (glu) {
        const int64_t pw12 = moe_decode_rows_per_wg(nb, 12);
        if ((n_pairs * MV + pw12 - 1) / pw12 <= c->num_cus) waves = 12;
        if (c->moe_dec_waves) waves = c->moe_dec_waves;
    }
    f.waves = waves;
    const int64_t per_wg = moe_decode_rows_per_wg(nb, waves);
    const int64_t need = (n_pairs * MV + per_wg - 1) / per_wg;
    const int grid = (int)(need < 2 * c->num_cus ? need : 2 * c->num_cus);
    moe_decode_plan(f, grid, &f.rows_per_wg, &f.xwin_rows);
    // the input rows a workgroup quantises must fit its LDS
    if ((size_t)q8lds_bytes(f.xwin_rows * nb) > (size_t)LDS_BUDGET) return 1;
    hipError_t e = launch_moe_decode(f, grid, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "moe decode launch");
    return 0;
}

// The routed-expert block's down projection and weighted slot sum in one
// launch (moe_down_sum_kernel), for n_used <= MOE_SUM_MAX_USED and exactly
// when spq4k_moe(down, ne11 = n_used) takes the decode mapping
// (moe_decode_try's conditions), whose per-row arithmetic it shares: the
// result is then that of the down launch and the combine launch bit for bit.
// H holds the T * n_used hidden rows. Returns 1 when it does not apply.
int moe_down_sum_try(spq4k_ctx* c, const spq4k_weights* down, const int32_t* ids, int64_t n_used, int64_t T,
                     const float* H, const float* w, float* Y) {
    const int nb = (int)(down->K / SPQ4K_QK_K), M = (int)down->M;
    const int64_t n_pairs = T * n_used, total = T * down->M;
    if (!(T <= c->moe_dec_max_t && n_pairs <= MOE_DEC_MAX_PAIRS && n_pairs <= MOE_DEC_MAX_XROWS &&
          n_used <= MOE_SUM_MAX_USED && moe_decode_supported(nb) && !c->moe_unfused && c->moe_mode == 0 &&
          down->fmt != WF_Q80 && total <= INT32_MAX))
        return 1;
    {
        // moe_decode_try's window rule for the same call
        MoeFusedParams d;
        memset(&d, 0, sizeof d);
        d.M = M;
        d.n_pairs = (int32_t)n_pairs;
        d.nb = nb;
        d.n_xrows = (int32_t)n_pairs;
        const int64_t pw = moe_decode_rows_per_wg(nb), need = (n_pairs * M + pw - 1) / pw;
        int32_t rw, xw;
        moe_decode_plan(d, (int)(need < 2 * c->num_cus ? need : 2 * c->num_cus), &rw, &xw);
        if ((size_t)q8lds_bytes(xw * nb) > (size_t)LDS_BUDGET) return 1;
    }
    MoeFusedParams f;
    memset(&f, 0, sizeof f);
    f.ids = ids;
    f.X = H;
    f.bank = down->data;
    f.expert_bytes = (size_t)M * nb * type_block_bytes(down->type);
    f.fmt = down->fmt;
    f.n_pairs = (int32_t)n_pairs;
    f.n_used = (int32_t)n_used;
    f.ne11 = (int32_t)n_used;
    f.K = (int32_t)down->K;
    f.M = M;
    f.nb = nb;
    f.E = (int32_t)down->E;
    f.n_xrows = (int32_t)n_pairs;
    // one output element a wave at a time, about two workgroups of 8 waves a CU
    const int64_t waves = 2 * (int64_t)c->num_cus * 8;
    int64_t per_wg = 8 * ((total + waves - 1) / waves);
    const int grid = (int)((total + per_wg - 1) / per_wg);
    // a run of per_wg elements spans at most per_wg / M + 2 tokens
    int64_t toks = per_wg / M + 2;
    if (toks > T) toks = T;
    f.rows_per_wg = (int32_t)per_wg;
    f.xwin_rows = (int32_t)(toks * n_used);
    if ((size_t)q8lds_bytes(f.xwin_rows * nb) > (size_t)LDS_BUDGET) return 1;
    hipError_t e = launch_moe_down_sum(f, w, Y, grid, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "moe down-sum launch");
    return 0;
}

bool moe_ring_chosen(const spq4k_ctx* c, const spq4k_weights* bank, int64_t mean_pairs) {
    return !c->moe_unfused && fmt_has_moe_ring(bank->fmt) && (bank->fmt == WF_Q4K || mean_pairs >= 2);
}

// The matrix-core expert kernel over one bank, or two of one type, K, E and M
// sharing ids and X (gate and up): one prep launch (routing and the permuted
// Q8_K planes), then one ring launch whose grid covers every bank.
int moe_ring_run(spq4k_ctx* c, const spq4k_weights* const* banks, int nbank, const int32_t* ids, int64_t n_used,
                 int64_t ne11, int64_t T, const float* X, float* const* Y) {
    const spq4k_weights* bank = banks[0];
    const int E = (int)bank->E, nb = (int)(bank->K / SPQ4K_QK_K), M = (int)bank->M;
    const size_t bb = type_block_bytes(bank->type);
    const int64_t rows = T * ne11, n_pairs = T * n_used;
    const int64_t max_act = n_pairs < E ? n_pairs : E;
    // scratch: Q8_K planes | routing tables
    const size_t items = (size_t)rows * nb;
    const size_t q8_bytes = (items * (256 + Q8MN_BYTES + 32 + 4) + 255) & ~(size_t)255;
    const size_t route_bytes = (size_t)(1 + 3 * E + n_pairs) * sizeof(int32_t);
    int rc = ensure_scratch(c, q8_bytes + route_bytes);
    if (rc) return rc;
    MoeParams p;
    memset(&p, 0, sizeof p);
    int32_t* rt = (int32_t*)(c->scratch + q8_bytes);
    p.route.n_act = rt;
    p.route.act = rt + 1;
    p.route.act_off = rt + 1 + E;
    p.route.act_cnt = rt + 1 + 2 * E;
    p.route.pairs = rt + 1 + 3 * E;
    p.bank = bank->data;
    p.expert_bytes = (size_t)M * nb * bb;
    p.fmt = bank->fmt;
    p.Y = Y[0];
    p.Q.qs = (int8_t*)c->scratch;
    p.Q.mn = c->scratch + items * 256;
    p.Q.bs = (int16_t*)(c->scratch + items * (256 + Q8MN_BYTES));
    p.Q.d = (float*)(c->scratch + items * (256 + Q8MN_BYTES + 32));
    p.M = M;
    p.nb = nb;
    p.n_used = (int)n_used;
    p.ne11 = (int)ne11;
    p.nbank = nbank;
    p.max_act = (int32_t)max_act;
    if (nbank > 1) {
        p.bank1 = banks[1]->data;
        p.Y1 = Y[1];
    }
    // row tiles a workgroup streams: as many as still leave two workgroups
    // per CU over the experts (of every bank) that can be active
    const int nw = moe_ring_waves(c, bank->fmt);
    const int64_t ntiles = (M + 16 * nw - 1) / (16 * nw);
    int64_t rtw = ntiles * max_act * nbank / (2 * (int64_t)c->num_cus);
    if (rtw < 1) rtw = 1;
    if (rtw > ntiles) rtw = ntiles;
    p.ring_rt = (int32_t)rtw;
    p.tiles_per_expert = (int32_t)((ntiles + rtw - 1) / rtw);
    if (max_act * p.tiles_per_expert * nbank > (1ll << 31) - 1 || rows * nb / 16 > (1ll << 31) - 2)
        return set_err(c, -EINVAL, "moe: grid too large");
    const hipError_t e = launch_moe_ring(p, ids, (int)n_pairs, E, X, bank->K, (int)rows, (int)max_act, nw,
                                         c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "moe ring launch");
    return 0;
}

}  // namespace

int spq4k_moe_multi(spq4k_ctx* c, int n, const spq4k_weights* const* banks, const int32_t* ids, int64_t n_used,
                    int64_t ne11, int64_t T, const float* X, float* const* Y) {
    int rc = use_device(c);
    if (rc) return rc;
    if (n < 1 || n > 2 || !banks || !Y) return set_err(c, -EINVAL, "moe_multi: n=%d banks (1..2)", n);
    for (int i = 0; i < n; ++i) {
        rc = moe_check(c, banks[i], ids, n_used, ne11, T, X, Y[i]);
        if (rc) return rc;
        if (banks[i]->type != banks[0]->type || banks[i]->K != banks[0]->K || banks[i]->E != banks[0]->E)
            return set_err(c, -EINVAL, "moe_multi: banks must share type, K and E");
    }
    if (n == 2 && banks[0]->fmt == WF_Q80) {
        rc = q80_moe(c, banks, 2, ids, n_used, ne11, T, X, Y);
        if (rc <= 0) return rc;
    }
    if (n == 2 && banks[0]->fmt != WF_Q80) {
        rc = moe_decode_try(c, banks, 2, ids, n_used, ne11, T, X, Y);
        if (rc <= 0) return rc;
        const int64_t n_pairs = T * n_used, max_act = n_pairs < banks[0]->E ? n_pairs : banks[0]->E;
        if (banks[1]->M == banks[0]->M && c->moe_mode != 3 &&
            moe_ring_chosen(c, banks[0], (n_pairs + max_act - 1) / max_act))
            return moe_ring_run(c, banks, 2, ids, n_used, ne11, T, X, Y);
    }
    for (int i = 0; i < n; ++i) {
        rc = spq4k_moe(c, banks[i], ids, n_used, ne11, T, X, Y[i]);
        if (rc) return rc;
    }
    return 0;
}

int spq4k_moe(spq4k_ctx* c, const spq4k_weights* bank, const int32_t* ids, int64_t n_used, int64_t ne11,
              int64_t T, const float* X, float* Y) {
    int rc = use_device(c);
    if (rc) return rc;
    rc = moe_check(c, bank, ids, n_used, ne11, T, X, Y);
    if (rc) return rc;
    if (bank->fmt == WF_Q80) {
        const spq4k_weights* b1[1] = {bank};
        float* y1[1] = {Y};
        return q80_moe(c, b1, 1, ids, n_used, ne11, T, X, y1);
    }
    const int E = (int)bank->E, nb = (int)(bank->K / SPQ4K_QK_K), M = (int)bank->M;
    const size_t bb = type_block_bytes(bank->type);
    const int64_t rows = T * ne11, n_pairs = T * n_used;
    // chunk width TC of the sdot4 expert kernels: about twice the mean number
    // of pairs an active expert receives (they are uneven), at most 8; every
    // pair of a chunk costs its integer work even when the chunk is not full
    const int64_t max_act = n_pairs < E ? n_pairs : E;
    const int64_t mean_pairs = (n_pairs + max_act - 1) / max_act;
    int tc = 1;
    while (tc < 8 && tc < 2 * mean_pairs) tc *= 2;
    int64_t Mtot[1] = {(int64_t)M * max_act};
    const int bpr = pick_bpr(c, Mtot, 1);
    const int rows_per_tile = gemv_rows_per_tile(bpr);
    const int tiles_per_expert = (M + rows_per_tile - 1) / rows_per_tile;
    const int cb_max = LDS_BUDGET / (tc * 292);
    const int chunk_blocks = nb < cb_max ? nb : cb_max;
    // small batches: the decode mapping
    {
        const spq4k_weights* b1[1] = {bank};
        float* y1[1] = {Y};
        rc = moe_decode_try(c, b1, 1, ids, n_used, ne11, T, X, y1);
        if (rc <= 0) return rc;
    }
    if (c->moe_mode == 3 && n_pairs <= MOE_FUSED_MAX_PAIRS && !c->moe_unfused) {
        MoeFusedParams f;
        memset(&f, 0, sizeof f);
        f.ids = ids;
        f.X = X;
        f.bank = bank->data;
        f.expert_bytes = (size_t)M * nb * bb;
        f.fmt = bank->fmt;
        f.Y = Y;
        f.n_pairs = (int32_t)n_pairs;
        f.n_used = (int32_t)n_used;
        f.ne11 = (int32_t)ne11;
        f.K = (int32_t)bank->K;
        f.M = M;
        f.nb = nb;
        f.tiles_per_expert = tiles_per_expert;
        f.chunk_blocks = chunk_blocks;
        const int64_t grid = (int64_t)E * tiles_per_expert;
        if (grid > (1ll << 31) - 1) return set_err(c, -EINVAL, "moe: grid too large");
        hipError_t e = launch_moe_fused(f, tc, bpr, (int)grid, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "moe fused launch");
        return 0;
    }
    // matrix cores unless the sdot4 kernels are asked for (SPQ4K_MOE_UNFUSED);
    // a Q6_K or Q5_K bank's operand preparation costs more, so its experts go
    // to the matrix cores only once they receive two pairs on average
    // (measured on the Q6_K 2048 x 768 down bank: T = 8 sdot4 31 us against
    // 36, T = 32 65 against 61)
    if (moe_ring_chosen(c, bank, mean_pairs)) {
        const spq4k_weights* b1[1] = {bank};
        float* y1[1] = {Y};
        return moe_ring_run(c, b1, 1, ids, n_used, ne11, T, X, y1);
    }
    // scratch: Q8_K planes | routing tables
    const size_t items = (size_t)rows * nb;
    const size_t q8_bytes = (items * (256 + Q8MN_BYTES + 32 + 4) + 255) & ~(size_t)255;
    const size_t route_bytes = (size_t)(1 + 3 * E + n_pairs) * sizeof(int32_t);
    rc = ensure_scratch(c, q8_bytes + route_bytes);
    if (rc) return rc;
    MoeParams p;
    memset(&p, 0, sizeof p);
    int8_t* qs = (int8_t*)c->scratch;
    uint8_t* mn = c->scratch + items * 256;
    int16_t* bs = (int16_t*)(c->scratch + items * (256 + Q8MN_BYTES));
    float* d = (float*)(c->scratch + items * (256 + Q8MN_BYTES + 32));
    int32_t* rt = (int32_t*)(c->scratch + q8_bytes);
    p.route.n_act = rt;
    p.route.act = rt + 1;
    p.route.act_off = rt + 1 + E;
    p.route.act_cnt = rt + 1 + 2 * E;
    p.route.pairs = rt + 1 + 3 * E;
    hipError_t e = launch_quantize_q8k_planes(X, bank->K, (int)rows, nb, qs, bs, d, mn, false, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "moe quantize launch");
    e = launch_moe_route(ids, (int)n_pairs, E, p.route, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "moe route launch");
    p.bank = bank->data;
    p.expert_bytes = (size_t)M * nb * bb;
    p.fmt = bank->fmt;
    p.Y = Y;
    p.Q.qs = qs;
    p.Q.bs = bs;
    p.Q.d = d;
    p.Q.mn = mn;
    p.M = M;
    p.nb = nb;
    p.n_used = (int)n_used;
    p.ne11 = (int)ne11;
    p.tiles_per_expert = tiles_per_expert;
    p.chunk_blocks = chunk_blocks;
    const int64_t grid = max_act * p.tiles_per_expert;
    if (grid > (1ll << 31) - 1) return set_err(c, -EINVAL, "moe: grid too large");
    e = launch_moe_gemv(p, tc, bpr, (int)grid, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "moe gemv launch");
    return 0;
}

int spq4k_mul_mat_host(spq4k_ctx* c, const spq4k_weights* W, const float* X, float* Y, int64_t T) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!W || !X || !Y || T < 1) return set_err(c, -EINVAL, "mul_mat_host: bad arguments");
    const size_t nx = (size_t)T * W->K * sizeof(float), ny = (size_t)T * W->M * sizeof(float);
    DevBuf a, b;
    if (hipMalloc(&a.p, nx + 16) != hipSuccess || hipMalloc(&b.p, ny + 16) != hipSuccess)
        return set_err(c, -ENOMEM, "mul_mat_host");
    SPQ_HIP(c, hipMemcpyAsync(a.p, X, nx, hipMemcpyHostToDevice, c->stream));
    rc = spq4k_mul_mat(c, W, (const float*)a.p, (float*)b.p, T);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(Y, b.p, ny, hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

int spq4k_moe_host(spq4k_ctx* c, const spq4k_weights* bank, const int32_t* ids, int64_t n_used, int64_t ne11,
                   int64_t T, const float* X, float* Y) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!bank || !ids || !X || !Y || T < 1 || n_used < 1 || (ne11 != 1 && ne11 != n_used))
        return set_err(c, -EINVAL, "moe_host: bad arguments");
    for (int64_t i = 0; i < T * n_used; ++i)
        if (ids[i] < 0 || ids[i] >= bank->E) return set_err(c, -EINVAL, "moe_host: expert id %d out of range", ids[i]);
    const size_t ni = (size_t)T * n_used * sizeof(int32_t);
    const size_t nx = (size_t)T * ne11 * bank->K * sizeof(float);
    const size_t ny = (size_t)T * n_used * bank->M * sizeof(float);
    DevBuf a, b, d;
    if (hipMalloc(&a.p, ni + 16) != hipSuccess || hipMalloc(&b.p, nx + 16) != hipSuccess ||
        hipMalloc(&d.p, ny + 16) != hipSuccess)
        return set_err(c, -ENOMEM, "moe_host");
    SPQ_HIP(c, hipMemcpyAsync(a.p, ids, ni, hipMemcpyHostToDevice, c->stream));
    SPQ_HIP(c, hipMemcpyAsync(b.p, X, nx, hipMemcpyHostToDevice, c->stream));
    rc = spq4k_moe(c, bank, (const int32_t*)a.p, n_used, ne11, T, (const float*)b.p, (float*)d.p);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(Y, d.p, ny, hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

// ---- fp32-activation dequant-then-dot (beast_matvec) ----------------------------------
int spq4k_dequant_matvec(spq4k_ctx* c, const spq4k_weights* W, const float* X, float* Y, int64_t T) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!W || !W->data || !X || !Y || T < 1) return set_err(c, -EINVAL, "dequant_matvec: bad arguments");
    if (W->E != 1) return set_err(c, -EINVAL, "dequant_matvec: a dense matrix is required");
    if (!aligned(X, 16) || !aligned(Y, 4)) return set_err(c, -EINVAL, "dequant_matvec: misaligned pointer");
    if (W->type != SPQ4K_TYPE_Q4_K) {
        // Q5_K / Q6_K / Q8_0 rows: the type-generic kernels, tokens in groups
        // whose x fits the staging area
        if (dqx_lds_bytes(W->type, W->K, 1) > DQ_MATVEC_LDS_MAX)
            return set_err(c, -EINVAL, "dequant_matvec: K = %lld exceeds %zu staged values", (long long)W->K,
                           DQ_MATVEC_LDS_MAX / sizeof(float));
        int tg = DQ_MATVEC_MAX_T;
        while (tg > 1 && dqx_lds_bytes(W->type, W->K, tg) > DQ_MATVEC_LDS_MAX) --tg;
        for (int64_t t0 = 0; t0 < T; t0 += tg) {
            const int n = (int)(T - t0 < tg ? T - t0 : tg);
            hipError_t e = launch_dqx_matvec(W->type, W->data, (int)W->M, W->K, X + t0 * W->K, W->K, Y + t0 * W->M,
                                             W->M, n, c->num_cus, c->stream);
            if (e != hipSuccess) return hip_fail(c, e, "dequant_matvec launch");
        }
        return 0;
    }
    const int nb = (int)(W->K / SPQ4K_QK_K);
    if (dequant_matvec_lds_bytes(1, nb) > DQ_MATVEC_LDS_MAX)
        return set_err(c, -EINVAL, "dequant_matvec: K = %lld exceeds %zu staged values", (long long)W->K,
                       DQ_MATVEC_LDS_MAX / sizeof(float));
    // tokens in groups whose x fits the staging area
    int tg = DQ_MATVEC_MAX_T;
    while (tg > 1 && dequant_matvec_lds_bytes(tg, nb) > DQ_MATVEC_LDS_MAX) --tg;
    for (int64_t t0 = 0; t0 < T; t0 += tg) {
        const int n = (int)(T - t0 < tg ? T - t0 : tg);
        hipError_t e = launch_dequant_matvec(W->data, (int)W->M, nb, X + t0 * W->K, W->K, Y + t0 * W->M, W->M, n,
                                             c->num_cus, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "dequant_matvec launch");
    }
    return 0;
}

int spq4k_dequant_matvec_host(spq4k_ctx* c, const spq4k_weights* W, const float* X, float* Y, int64_t T) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!W || !X || !Y || T < 1) return set_err(c, -EINVAL, "dequant_matvec_host: bad arguments");
    const size_t nx = (size_t)T * W->K * sizeof(float), ny = (size_t)T * W->M * sizeof(float);
    DevBuf a, b;
    if (hipMalloc(&a.p, nx + 16) != hipSuccess || hipMalloc(&b.p, ny + 16) != hipSuccess)
        return set_err(c, -ENOMEM, "dequant_matvec_host");
    SPQ_HIP(c, hipMemcpyAsync(a.p, X, nx, hipMemcpyHostToDevice, c->stream));
    rc = spq4k_dequant_matvec(c, W, (const float*)a.p, (float*)b.p, T);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(Y, b.p, ny, hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

// ---- BurnHard MoE forward (sp_beast_moe_forward) ------------------------------------
int spq4k_beast_moe_forward(spq4k_ctx* c, const spq4k_weights* gate, const spq4k_weights* up,
                            const spq4k_weights* down, const float* router_logits, int64_t top_k,
                            const float* hidden, float* output, int32_t* ids, float* scores) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!gate || !up || !down || !gate->data || !up->data || !down->data || !router_logits || !hidden || !output)
        return set_err(c, -EINVAL, "beast_moe_forward: null argument");
    const int64_t E = gate->E, n_embd = gate->K, n_ff = gate->M;
    if (up->E != E || up->K != n_embd || up->M != n_ff || down->E != E || down->K != n_ff || down->M != n_embd)
        return set_err(c, -EINVAL, "beast_moe_forward: gate [%lld x %lld x %lld], up and down banks do not match",
                       (long long)n_ff, (long long)n_embd, (long long)E);
    if (E > BEAST_MAX_EXPERTS) return set_err(c, -EINVAL, "beast_moe_forward: E = %lld experts", (long long)E);
    // sp_beast_route_experts (sp_beast_canyon.c:389-392): 2 by default, at most E
    if (top_k <= 0) top_k = 2;
    if (top_k > E) top_k = E;
    if (top_k > BEAST_MAX_TOPK) return set_err(c, -EINVAL, "beast_moe_forward: top_k = %lld", (long long)top_k);
    const bool q4_gu = gate->type == SPQ4K_TYPE_Q4_K && up->type == SPQ4K_TYPE_Q4_K;
    const bool q4_dn = down->type == SPQ4K_TYPE_Q4_K;
    // every bank's rows staged whole: the Q4_K kernels' layout for Q4_K
    // gate / up pairs and Q4_K down banks, the type-generic one otherwise
    const size_t lds_e = q4_gu ? dequant_matvec_lds_bytes(1, (int)(n_embd / SPQ4K_QK_K))
                               : std::max(dqx_lds_bytes(gate->type, n_embd, 1), dqx_lds_bytes(up->type, n_embd, 1));
    const size_t lds_f = q4_dn ? dequant_matvec_lds_bytes(1, (int)(n_ff / SPQ4K_QK_K))
                               : dqx_lds_bytes(down->type, n_ff, 1);
    if (lds_e > DQ_MATVEC_LDS_MAX || lds_f > DQ_MATVEC_LDS_MAX)
        return set_err(c, -EINVAL, "beast_moe_forward: rows longer than %zu values", DQ_MATVEC_LDS_MAX / sizeof(float));
    if (!aligned(hidden, 16) || !aligned(router_logits, 4) || !aligned(output, 4) || !aligned(ids, 4) ||
        !aligned(scores, 4))
        return set_err(c, -EINVAL, "beast_moe_forward: misaligned pointer");
    // routing, then the hidden rows, in the fusion scratch
    const size_t rb = 256;
    rc = ensure_scratch2(c, rb + (size_t)top_k * n_ff * sizeof(float));
    if (rc) return rc;
    int32_t* rid = reinterpret_cast<int32_t*>(c->scratch2);
    float* rsc = reinterpret_cast<float*>(c->scratch2 + 128);
    float* H = reinterpret_cast<float*>(c->scratch2 + rb);
    // routing and H = silu(gate . x) * (up . x): the fused Q4_K launch, or
    // the routing alone, then the gate rows into H and the up rows finishing it
    hipError_t e;
    if (q4_gu) {
        e = launch_beast_route_gate_up(gate->data, up->data, (int)E, (int)n_embd, (int)n_ff, router_logits, (int)top_k,
                                       hidden, rid, rsc, H, c->num_cus, c->stream);
    } else {
        // gate and up in one launch when they share a type, else the gate
        // rows into H and the up rows finishing it
        e = launch_beast_route(router_logits, (int)E, (int)top_k, rid, rsc, c->stream);
        if (e == hipSuccess && gate->type == up->type) {
            e = launch_dqx_experts(gate->type, 2, gate->data, up->data, (int)E, (int)n_ff, n_embd, rid, (int)top_k,
                                   hidden, H, c->num_cus, c->stream);
        } else if (e == hipSuccess) {
            e = launch_dqx_experts(gate->type, 0, gate->data, nullptr, (int)E, (int)n_ff, n_embd, rid, (int)top_k,
                                   hidden, H, c->num_cus, c->stream);
            if (e == hipSuccess)
                e = launch_dqx_experts(up->type, 1, up->data, nullptr, (int)E, (int)n_ff, n_embd, rid, (int)top_k,
                                       hidden, H, c->num_cus, c->stream);
        }
    }
    if (e != hipSuccess) return hip_fail(c, e, "beast moe gate / up launch");
    e = q4_dn ? launch_beast_down(down->data, (int)E, (int)n_embd, (int)n_ff, rid, rsc, (int)top_k, H, output,
                                  c->num_cus, c->stream)
              : launch_dqx_down(down->type, down->data, (int)E, (int)n_embd, n_ff, rid, rsc, (int)top_k, H, output,
                                c->num_cus, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "beast moe down launch");
    if (ids) SPQ_HIP(c, hipMemcpyAsync(ids, rid, (size_t)top_k * sizeof(int32_t), hipMemcpyDeviceToDevice, c->stream));
    if (scores)
        SPQ_HIP(c, hipMemcpyAsync(scores, rsc, (size_t)top_k * sizeof(float), hipMemcpyDeviceToDevice, c->stream));
    return 0;
}

int spq4k_beast_moe_forward_host(spq4k_ctx* c, const spq4k_weights* gate, const spq4k_weights* up,
                                 const spq4k_weights* down, const float* router_logits, int64_t top_k,
                                 const float* hidden, float* output, int32_t* ids, float* scores) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!gate || !up || !down || !router_logits || !hidden || !output)
        return set_err(c, -EINVAL, "beast_moe_forward_host: null argument");
    const int64_t E = gate->E, n_embd = gate->K;
    int64_t k = top_k <= 0 ? 2 : top_k;
    if (k > E) k = E;
    if (k > BEAST_MAX_TOPK) return set_err(c, -EINVAL, "beast_moe_forward_host: top_k = %lld", (long long)top_k);
    DevBuf l, h, o, r;
    if (hipMalloc(&l.p, (size_t)E * sizeof(float) + 16) != hipSuccess ||
        hipMalloc(&h.p, (size_t)n_embd * sizeof(float) + 16) != hipSuccess ||
        hipMalloc(&o.p, (size_t)n_embd * sizeof(float) + 16) != hipSuccess ||
        hipMalloc(&r.p, 2 * BEAST_MAX_TOPK * sizeof(float)) != hipSuccess)
        return set_err(c, -ENOMEM, "beast_moe_forward_host");
    SPQ_HIP(c, hipMemcpyAsync(l.p, router_logits, (size_t)E * sizeof(float), hipMemcpyHostToDevice, c->stream));
    SPQ_HIP(c, hipMemcpyAsync(h.p, hidden, (size_t)n_embd * sizeof(float), hipMemcpyHostToDevice, c->stream));
    int32_t* di = reinterpret_cast<int32_t*>(r.p);
    float* ds = reinterpret_cast<float*>(r.p) + BEAST_MAX_TOPK;
    rc = spq4k_beast_moe_forward(c, gate, up, down, (const float*)l.p, top_k, (const float*)h.p, (float*)o.p, di, ds);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(output, o.p, (size_t)n_embd * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    if (ids) SPQ_HIP(c, hipMemcpyAsync(ids, di, (size_t)k * sizeof(int32_t), hipMemcpyDeviceToHost, c->stream));
    if (scores) SPQ_HIP(c, hipMemcpyAsync(scores, ds, (size_t)k * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

// ---- routed-expert FFN block (BURN_MOE) --------------------------------------------
int spq4k_moe_ffn(spq4k_ctx* c, const spq4k_weights* gate, const spq4k_weights* up, const spq4k_weights* down,
                  const int32_t* ids, const float* weights, int64_t n_used, int64_t T, const float* X, float* Y) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!gate || !up || !down || !weights || !Y) return set_err(c, -EINVAL, "moe_ffn: null argument");
    if (gate->type != up->type || gate->K != up->K || gate->M != up->M || gate->E != up->E)
        return set_err(c, -EINVAL, "moe_ffn: gate and up banks differ in type or shape");
    if (down->K != gate->M || down->M != gate->K || down->E != gate->E)
        return set_err(c, -EINVAL, "moe_ffn: down bank [%lld x %lld x %lld] does not match gate [%lld x %lld x %lld]",
                       (long long)down->K, (long long)down->M, (long long)down->E, (long long)gate->K,
                       (long long)gate->M, (long long)gate->E);
    rc = moe_check(c, gate, ids, n_used, 1, T, X, Y);
    if (rc) return rc;
    if (!aligned(weights, 4) || !aligned(Y, 4)) return set_err(c, -EINVAL, "moe_ffn: misaligned pointer");
    const int64_t n_embd = gate->K, n_ff = gate->M, pairs = T * n_used;
    // fusion scratch: gate and up outputs, their SwiGLU (down's input rows, 16-byte
    // aligned for the matvec), down outputs
    const size_t fb = (((size_t)pairs * n_ff * sizeof(float)) + 255) & ~(size_t)255;
    const size_t db = (((size_t)pairs * n_embd * sizeof(float)) + 255) & ~(size_t)255;
    rc = ensure_scratch2(c, 3 * fb + db);
    if (rc) return rc;
    float* G = reinterpret_cast<float*>(c->scratch2);
    float* U = reinterpret_cast<float*>(c->scratch2 + fb);
    float* H = reinterpret_cast<float*>(c->scratch2 + 2 * fb);
    float* D = reinterpret_cast<float*>(c->scratch2 + 3 * fb);
    // up and gate of every routed pair (forward.cpp:1100-1101) and silu(gate)
    // * up (:1102-1103): small batches of K-quant banks in one sweep with the
    // SwiGLU epilogue, otherwise one spq4k_moe_multi call and swiglu_kernel
    const spq4k_weights* gu[2] = {gate, up};
    float* hy[1] = {H};
    hipError_t e;
    rc = gate->fmt == WF_Q80 ? 1 : moe_decode_try(c, gu, 2, ids, n_used, 1, T, X, hy, true);
    if (rc < 0) return rc;
    if (rc > 0) {
        float* gy[2] = {G, U};
        rc = spq4k_moe_multi(c, 2, gu, ids, n_used, 1, T, X, gy);
        if (rc) return rc;
        e = launch_swiglu(G, U, H, pairs * n_ff, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "swiglu launch");
    }
    // down of each pair's own hidden row (forward.cpp:1104: b = par [n_ff, n_used, T], ne11 = n_used)
    // with the weights and the sum over the slots (:1107-1116) as its epilogue
    // for small batches; otherwise down, then the combine launch
    rc = moe_down_sum_try(c, down, ids, n_used, T, H, weights, Y);
    if (rc <= 0) return rc;
    rc = spq4k_moe(c, down, ids, n_used, n_used, T, H, D);
    if (rc) return rc;
    // weights and the sum over the slots (forward.cpp:1107-1116)
    e = launch_moe_combine(D, weights, Y, (int)T, (int)n_used, (int)n_embd, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "moe_combine launch");
    return 0;
}

int spq4k_moe_ffn_host(spq4k_ctx* c, const spq4k_weights* gate, const spq4k_weights* up, const spq4k_weights* down,
                       const int32_t* ids, const float* weights, int64_t n_used, int64_t T, const float* X,
                       float* Y) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!gate || !up || !down || !ids || !weights || !X || !Y || T < 1 || n_used < 1 || n_used > gate->E)
        return set_err(c, -EINVAL, "moe_ffn_host: bad arguments");
    for (int64_t i = 0; i < T * n_used; ++i)
        if (ids[i] < 0 || ids[i] >= gate->E)
            return set_err(c, -EINVAL, "moe_ffn_host: expert id %d out of range", ids[i]);
    const size_t ni = (size_t)T * n_used * sizeof(int32_t);
    const size_t nw = (size_t)T * n_used * sizeof(float);
    const size_t nx = (size_t)T * gate->K * sizeof(float);
    DevBuf a, w, b, d;
    if (hipMalloc(&a.p, ni + 16) != hipSuccess || hipMalloc(&w.p, nw + 16) != hipSuccess ||
        hipMalloc(&b.p, nx + 16) != hipSuccess || hipMalloc(&d.p, nx + 16) != hipSuccess)
        return set_err(c, -ENOMEM, "moe_ffn_host");
    SPQ_HIP(c, hipMemcpyAsync(a.p, ids, ni, hipMemcpyHostToDevice, c->stream));
    SPQ_HIP(c, hipMemcpyAsync(w.p, weights, nw, hipMemcpyHostToDevice, c->stream));
    SPQ_HIP(c, hipMemcpyAsync(b.p, X, nx, hipMemcpyHostToDevice, c->stream));
    rc = spq4k_moe_ffn(c, gate, up, down, (const int32_t*)a.p, (const float*)w.p, n_used, T, (const float*)b.p,
                       (float*)d.p);
    if (rc) return rc;
    SPQ_HIP(c, hipMemcpyAsync(Y, d.p, nx, hipMemcpyDeviceToHost, c->stream));
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    return 0;
}

// ---- diagnostics / synth -------------------------------------------------------------
int spq4k_stream_read(spq4k_ctx* c, const void* p, size_t bytes) {
    int rc = use_device(c);
    if (rc) return rc;
    if ((bytes && !p) || !aligned(p, 16) || bytes % 16) return set_err(c, -EINVAL, "stream_read: bad arguments");
    // four workgroups a CU unless SPQ4K_STREAM_GRID sets the largest grid
    int max_grid = 4 * c->num_cus;
    if (const char* g = getenv("SPQ4K_STREAM_GRID")) {
        const int v = atoi(g);
        if (v > 0 && v <= (1 << 16)) max_grid = v;
    }
    rc = ensure_scratch(c, (size_t)max_grid * sizeof(uint32_t));
    if (rc) return rc;
    hipError_t e = launch_stream_read(p, bytes, max_grid, reinterpret_cast<uint32_t*>(c->scratch), c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "stream_read launch");
    return 0;
}

int spq4k_subblock_sums(spq4k_ctx* c, const void* W, int64_t M, int64_t K, const float* x, int32_t* S) {
    int rc = use_device(c);
    if (rc) return rc;
    rc = check_shape(c, M, K, 1);
    if (rc) return rc;
    if (!W || !x || !S || !aligned(W, 16) || !aligned(x, 16)) return set_err(c, -EINVAL, "subblock_sums: bad pointers");
    hipError_t e = launch_subblock_sums((const uint8_t*)W, (int)M, (int)(K / SPQ4K_QK_K), x, S, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "subblock_sums launch");
    return 0;
}

int spq4k_subblock_sums_type(spq4k_ctx* c, int type, const void* W, int64_t M, int64_t K, const float* x,
                             int32_t* S) {
    if (type == SPQ4K_TYPE_Q4_K) return spq4k_subblock_sums(c, W, M, K, x, S);
    int rc = use_device(c);
    if (rc) return rc;
    if (type == SPQ4K_TYPE_Q8_0) {
        rc = check_shape(c, M, K, 1, SPQ4K_QK8_0);
        if (rc) return rc;
        if (!W || !x || !S || !aligned(W, 2) || !aligned(x, 16)) return set_err(c, -EINVAL, "subblock_sums: bad pointers");
        hipError_t e = launch_block_sums_q8_0((const uint8_t*)W, (int)M, (int)(K / SPQ4K_QK8_0), x, S, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "block_sums_q8_0 launch");
        return 0;
    }
    if (type != SPQ4K_TYPE_Q6_K && type != SPQ4K_TYPE_Q5_K)
        return set_err(c, -EINVAL, "subblock_sums: unsupported type %d", type);
    rc = check_shape(c, M, K, 1);
    if (rc) return rc;
    if (!W || !x || !S || !aligned(W, type == SPQ4K_TYPE_Q5_K ? 16 : 2) || !aligned(x, 16))
        return set_err(c, -EINVAL, "subblock_sums: bad pointers");
    hipError_t e = type == SPQ4K_TYPE_Q5_K
                       ? launch_subblock_sums_q5k((const uint8_t*)W, (int)M, (int)(K / SPQ4K_QK_K), x, S, c->stream)
                       : launch_subblock_sums_q6k((const uint8_t*)W, (int)M, (int)(K / SPQ4K_QK_K), x, S, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "subblock_sums_q6k launch");
    return 0;
}

int spq4k_synth_fill(spq4k_ctx* c, float* out, int64_t n, uint64_t seed, int dist, int64_t cols, float mean,
                     float std, float outlier_mult, int64_t offset) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!out || n < 0 || (dist != SPQ4K_DIST_NORMAL && dist != SPQ4K_DIST_STUDENT_T4) || cols < 0)
        return set_err(c, -EINVAL, "synth_fill: bad arguments");
    hipError_t e = launch_synth(out, n, seed, dist, cols, mean, std, outlier_mult, offset, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "synth launch");
    return 0;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// decode chains (k_chain.hip)
struct spq4k_chain {
    int device = 0;
    int version = 1;                   // 1: grid barrier a stage (k_chain.hip); 2: one-hop exchange (k_chain2.hip)
    ChainStage* d_st = nullptr;
    ChainSync* d_sync = nullptr;
    Chain2Stage* d_st2 = nullptr;
    Chain2Sync* d_sync2 = nullptr;
    float* d_sh = nullptr;             // v2 shadow arena, two sets of sh_half floats
    int64_t sh_half = 0;
    uint64_t* stamps = nullptr;        // v2 diagnostics (caller's buffer) or null
    int nstages = 0;
    float eps = 0.0f;
    int grid = 0;
    int shape = 0;
};

namespace {
bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
    if (!a || !b) return false;
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + nb && y < x + na;
}

// The v2 form of a chain (k_chain2.hip) when its data flow allows it: every
// vector a stage writes (y[j], x_out) lies apart from every other one, and an
// input is either one of them or a part of one written by an earlier stage
// (read through its shadow, or from LDS when it is the x_out of the latest
// stage with one) or touches none of them (read as it is). Then no stage
// writes memory an earlier stage reads or writes, which the loosely ordered
// stages of v2 need. Returns false (use v1) otherwise.
bool chain2_plan(const std::vector<ChainStage>& tab, int grid, std::vector<Chain2Stage>& out, int64_t& sh_half) {
    struct Prod {
        uintptr_t p;
        size_t bytes;
        int stage, which;   // which: 0..3 = y[j], 4 = x_out
        int64_t sh;
    };
    const int n = (int)tab.size();
    const int64_t G = (int64_t)grid * chain2_compute_waves();
    std::vector<Prod> prods;
    for (int s = 0; s < n; ++s) {
        const ChainStage& t = tab[(size_t)s];
        if ((t.rows + G - 1) / G * chain2_compute_waves() > CHAIN_YCAP) return false;
        const int nout = t.glu ? 1 : 4;
        for (int j = 0; j < nout; ++j) {
            if (!t.Y[j]) continue;
            const int64_t end = j + 1 < 4 && t.row_begin[j + 1] != INT32_MAX ? t.row_begin[j + 1] : t.rows;
            prods.push_back({(uintptr_t)t.Y[j], (size_t)(end - t.row_begin[j]) * sizeof(float), s, j, -1});
        }
        if (t.xout) prods.push_back({(uintptr_t)t.xout, (size_t)t.nb * QK * sizeof(float), s, 4, -1});
    }
    std::vector<size_t> ord(prods.size());
    for (size_t i = 0; i < ord.size(); ++i) ord[i] = i;
    std::sort(ord.begin(), ord.end(), [&](size_t a, size_t b) { return prods[a].p < prods[b].p; });
    for (size_t i = 1; i < ord.size(); ++i)
        if (prods[ord[i - 1]].p + prods[ord[i - 1]].bytes > prods[ord[i]].p) return false;
    // the produced vector holding [p, p + bytes), -1 if none touches it, -2 on a partial overlap
    auto find = [&](const void* pp, size_t bytes) -> int {
        const uintptr_t p = (uintptr_t)pp;
        size_t lo = 0, hi = ord.size();
        while (lo < hi) {   // first produced range starting past p
            const size_t mid = (lo + hi) / 2;
            if (prods[ord[mid]].p <= p) lo = mid + 1; else hi = mid;
        }
        if (lo > 0) {
            const Prod& q = prods[ord[lo - 1]];
            if (p < q.p + q.bytes) return p + bytes <= q.p + q.bytes ? (int)ord[lo - 1] : -2;
        }
        if (lo < ord.size() && prods[ord[lo]].p < p + bytes) return -2;
        return -1;
    };
    out.assign((size_t)n, Chain2Stage{});
    std::vector<int> in_prod((size_t)n * 2, -1);
    int last_xout = -1;
    for (int s = 0; s < n; ++s) {
        const ChainStage& t = tab[(size_t)s];
        Chain2Stage& o = out[(size_t)s];
        for (int j = 0; j < 4; ++j) {
            o.W[j] = t.W[j];
            o.Y[j] = t.Y[j];
            o.ysh[j] = -1;
            o.row_begin[j] = t.row_begin[j];
        }
        o.rows = t.rows;
        o.nb = t.nb;
        o.glu = t.glu;
        o.xout = t.xout;
        o.xosh = -1;
        o.norm_w = t.norm_w;
        const size_t xb = (size_t)t.nb * QK * sizeof(float);
        if (t.norm_w && find(t.norm_w, xb) != -1) return false;
        const float* in[2] = {t.in0, t.in1};
        for (int i = 0; i < 2; ++i) {
            o.kind[i] = CH2_NONE;
            if (!in[i]) continue;
            const int f = find(in[i], xb);
            if (f == -2) return false;
            if (f == -1) {
                o.kind[i] = CH2_EXT;
                o.ext[i] = in[i];
                continue;
            }
            const Prod& q = prods[(size_t)f];
            if (q.stage >= s) return false;
            if (q.which == 4 && q.stage == last_xout && q.p == (uintptr_t)in[i] && q.bytes == xb) {
                o.kind[i] = CH2_LOCAL;
                out[(size_t)q.stage].keep = 1;
            } else {
                o.kind[i] = CH2_SHADOW;
                in_prod[(size_t)s * 2 + i] = f;
            }
        }
        if (t.xout) last_xout = s;
    }
    // shadows for the vectors read through one, 256-byte aligned
    int64_t off = 0;
    for (int s = 0; s < n; ++s)
        for (int i = 0; i < 2; ++i) {
            const int f = in_prod[(size_t)s * 2 + i];
            if (f < 0 || prods[(size_t)f].sh >= 0) continue;
            prods[(size_t)f].sh = off;
            off += ((int64_t)(prods[(size_t)f].bytes / sizeof(float)) + 63) / 64 * 64;
        }
    for (const Prod& q : prods) {
        if (q.sh < 0) continue;
        if (q.which == 4) out[(size_t)q.stage].xosh = q.sh;
        else out[(size_t)q.stage].ysh[q.which] = q.sh;
    }
    for (int s = 0; s < n; ++s)
        for (int i = 0; i < 2; ++i) {
            const int f = in_prod[(size_t)s * 2 + i];
            if (f < 0) continue;
            const Prod& q = prods[(size_t)f];
            const float* in = i ? tab[(size_t)s].in1 : tab[(size_t)s].in0;
            out[(size_t)s].insh[i] = q.sh + (int64_t)(((uintptr_t)in - q.p) / sizeof(float));
        }
    sh_half = off;
    return true;
}
}  // namespace

extern "C" {

void spq4k_chain_free(spq4k_chain* ch) {
    if (!ch) return;
    int prev = -1;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(ch->device);
    if (ch->d_st) (void)hipFree(ch->d_st);
    if (ch->d_sync) (void)hipFree(ch->d_sync);
    if (ch->d_st2) (void)hipFree(ch->d_st2);
    if (ch->d_sync2) (void)hipFree(ch->d_sync2);
    if (ch->d_sh) (void)hipFree(ch->d_sh);
    if (prev >= 0) (void)hipSetDevice(prev);
    delete ch;
}

int spq4k_chain_create(spq4k_ctx* c, const spq4k_chain_stage* stages, int n, float eps, spq4k_chain** out) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!out) return set_err(c, -EINVAL, "chain_create: null output");
    *out = nullptr;
    if (!stages || n <= 0 || n > (1 << 20)) return set_err(c, -EINVAL, "chain_create: bad stage count %d", n);
    if (!(eps >= 0.0f)) return set_err(c, -EINVAL, "chain_create: bad eps");
    int shape = 0;
    if (const char* f = getenv("SPQ4K_CHAIN_SHAPE")) {
        const int v = atoi(f);
        if (v >= 0 && v <= 2) shape = v;
    }
    const int grid = chain_grid(c->num_cus);
    if (grid <= 0) return set_err(c, -ENODEV, "chain_create: %d CUs is too few", c->num_cus);
    const int cw = chain_compute_waves(shape);
    const int64_t G = (int64_t)grid * cw;
    std::vector<ChainStage> tab((size_t)n);
    for (int s = 0; s < n; ++s) {
        const spq4k_chain_stage& in = stages[s];
        ChainStage& o = tab[(size_t)s];
        memset(&o, 0, sizeof o);
        if (in.n < 1 || in.n > 4 || (in.glu && in.n != 2))
            return set_err(c, -EINVAL, "chain stage %d: %d matrices%s", s, in.n, in.glu ? " with glu (needs 2)" : "");
        const int64_t K = in.W[0] ? in.W[0]->K : 0;
        int64_t rows = 0;
        for (int j = 0; j < in.n; ++j) {
            const spq4k_weights* w = in.W[j];
            const bool need_y = !(in.glu && j == 1);   // with glu the product goes to y[0]
            if (!w || (need_y && !in.y[j])) return set_err(c, -EINVAL, "chain stage %d: null matrix or output %d", s, j);
            if (w->device != c->device) return set_err(c, -EINVAL, "chain stage %d: weights on another device", s);
            if (w->type != SPQ4K_TYPE_Q4_K || w->E != 1)
                return set_err(c, -EINVAL, "chain stage %d: matrix %d is not a dense Q4_K matrix", s, j);
            if (w->K != K) return set_err(c, -EINVAL, "chain stage %d: matrices differ in K", s);
            if (need_y && !aligned(in.y[j], 16))
                return set_err(c, -EINVAL, "chain stage %d: output %d not 16-byte aligned", s, j);
            o.W[j] = w->data;
            o.Y[j] = in.y[j];
            if (!in.glu) {
                o.row_begin[j] = (int32_t)rows;
                rows += w->M;
            }
        }
        if (in.glu) {
            if (in.W[0]->M != in.W[1]->M) return set_err(c, -EINVAL, "chain stage %d: gate and up rows differ", s);
            rows = in.W[0]->M;
            o.row_begin[0] = 0;
            o.Y[1] = nullptr;
        }
        for (int j = in.glu ? 1 : in.n; j < 4; ++j) o.row_begin[j] = INT32_MAX;
        if (K <= 0 || K % SPQ4K_QK_K || K / SPQ4K_QK_K > CHAIN_MAX_NB)
            return set_err(c, -EINVAL, "chain stage %d: K = %lld (a multiple of 256 up to %d)", s, (long long)K,
                           CHAIN_MAX_K);
        if (rows <= 0 || rows > INT32_MAX / 2 || (rows + G - 1) / G * cw > CHAIN_YCAP)
            return set_err(c, -EINVAL, "chain stage %d: %lld rows", s, (long long)rows);
        const int nvec = 1 + (in.in1 ? 1 : 0) + (in.norm_w ? 1 : 0);
        if (nvec * K > CHAIN_MAX_K)
            return set_err(c, -EINVAL, "chain stage %d: %d input vectors of %lld exceed %d values", s, nvec,
                           (long long)K, CHAIN_MAX_K);
        if (!in.in0 || !aligned(in.in0, 16) || !aligned(in.in1, 16) || !aligned(in.x_out, 16) ||
            !aligned(in.norm_w, 16))
            return set_err(c, -EINVAL, "chain stage %d: null or misaligned input", s);
        // A stage's outputs (y[j], x_out) overlap none of its inputs (in0,
        // in1, norm_w) nor each other: the stage's rows and its residual
        // store run concurrently with the reads of every input.
        const size_t xb = (size_t)K * sizeof(float);
        const int ny = in.glu ? 1 : in.n;
        for (int j = 0; j < ny; ++j) {
            const size_t yb = (size_t)(in.glu ? rows : in.W[j]->M) * sizeof(float);
            if (overlaps(in.y[j], yb, in.in0, xb) || overlaps(in.y[j], yb, in.in1, xb) ||
                overlaps(in.y[j], yb, in.norm_w, xb))
                return set_err(c, -EINVAL, "chain stage %d: output %d overlaps the stage's inputs", s, j);
            if (overlaps(in.y[j], yb, in.x_out, xb))
                return set_err(c, -EINVAL, "chain stage %d: output %d overlaps x_out", s, j);
            for (int k = 0; k < j; ++k)
                if (overlaps(in.y[j], yb, in.y[k], (size_t)in.W[k]->M * sizeof(float)))
                    return set_err(c, -EINVAL, "chain stage %d: outputs %d and %d overlap", s, k, j);
        }
        if (overlaps(in.x_out, xb, in.in0, xb) || overlaps(in.x_out, xb, in.in1, xb) ||
            overlaps(in.x_out, xb, in.norm_w, xb))
            return set_err(c, -EINVAL, "chain stage %d: x_out overlaps the stage's inputs", s);
        o.rows = (int32_t)rows;
        o.nb = (int32_t)(K / SPQ4K_QK_K);
        o.glu = in.glu ? 1 : 0;
        o.in0 = in.in0;
        o.in1 = in.in1;
        o.xout = in.x_out;
        o.norm_w = in.norm_w;
    }
    spq4k_chain* ch = new (std::nothrow) spq4k_chain();
    if (!ch) return set_err(c, -ENOMEM, "chain_create: out of host memory");
    ch->device = c->device;
    ch->nstages = n;
    ch->eps = eps;
    ch->grid = grid;
    ch->shape = shape;
    // Form 1 (a grid barrier every stage) unless SPQ4K_CHAIN_V=2 asks for
    // form 2 (the one-hop exchange) and the chain's data flow allows it. On
    // the 8B decode step form 1 measures faster (1.56 against 1.69 ms): both
    // are bound by their compute waves' instruction issue, and form 2 gives
    // four waves of each workgroup to the exchange.
    std::vector<Chain2Stage> tab2;
    int64_t sh_half = 0;
    const char* fv = getenv("SPQ4K_CHAIN_V");
    const bool want2 = fv && atoi(fv) == 2;
    if (want2 && chain2_plan(tab, grid, tab2, sh_half)) ch->version = 2;
    hipError_t e = hipSuccess;
    if (ch->version == 2) {
        ch->sh_half = sh_half;
        e = hipMalloc(&ch->d_st2, sizeof(Chain2Stage) * (size_t)n);
        if (e == hipSuccess) e = hipMalloc(&ch->d_sync2, sizeof(Chain2Sync));
        if (e == hipSuccess) e = hipMalloc(&ch->d_sh, sizeof(float) * (size_t)(2 * sh_half + 64));
        if (e == hipSuccess)
            e = hipMemcpy(ch->d_st2, tab2.data(), sizeof(Chain2Stage) * (size_t)n, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemset(ch->d_sync2, 0, sizeof(Chain2Sync));
        if (e == hipSuccess) e = hipMemset(ch->d_sh, 0xFF, sizeof(float) * (size_t)(2 * sh_half + 64));
    } else {
        e = hipMalloc(&ch->d_st, sizeof(ChainStage) * (size_t)n);
        if (e == hipSuccess) e = hipMalloc(&ch->d_sync, sizeof(ChainSync));
        if (e == hipSuccess) e = hipMemcpy(ch->d_st, tab.data(), sizeof(ChainStage) * (size_t)n, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemset(ch->d_sync, 0, sizeof(ChainSync));
    }
    if (e != hipSuccess) {
        spq4k_chain_free(ch);
        return e == hipErrorOutOfMemory ? set_err(c, -ENOMEM, "chain_create: out of device memory")
                                        : hip_fail(c, e, "chain_create");
    }
    *out = ch;
    return 0;
}

int spq4k_chain_run(spq4k_ctx* c, spq4k_chain* ch) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!ch || ch->device != c->device) return set_err(c, -EINVAL, "chain_run: no chain for this device");
    if (ch->version == 2) {
        Chain2Params p;
        p.sync = ch->d_sync2;
        p.sh = ch->d_sh;
        p.sh_half = ch->sh_half;
        p.stamps = ch->stamps;
        p.nstages = ch->nstages;
        p.eps = ch->eps;
        int depth = 4;
        if (const char* f = getenv("SPQ4K_CHAIN2_D")) depth = atoi(f);
        if (depth != 2 && depth != 3 && depth != 6) depth = 4;
        hipError_t e = launch_chain2(ch->d_st2, p, ch->grid, depth, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "chain launch");
        return 0;
    }
    ChainParams p;
    p.st = ch->d_st;
    p.sync = ch->d_sync;
    p.nstages = ch->nstages;
    p.eps = ch->eps;
    hipError_t e = launch_chain(p, ch->grid, ch->shape, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "chain launch");
    return 0;
}

int spq4k_chain_info(const spq4k_chain* ch, int* version, int* grid, int* n_stages) {
    if (!ch) return -EINVAL;
    if (version) *version = ch->version;
    if (grid) *grid = ch->grid;
    if (n_stages) *n_stages = ch->nstages;
    return 0;
}

int spq4k_set_decode_stamps(spq4k_ctx* c, uint64_t* stamps, size_t n) {
    if (!c) return -EINVAL;
    if (stamps && (!aligned(stamps, 8) || n == 0))
        return set_err(c, -EINVAL, "set_decode_stamps: misaligned or empty buffer");
    c->dec_stamps = stamps;
    c->dec_stamps_n = stamps ? n : 0;
    return 0;
}

int spq4k_chain_set_stamps(spq4k_ctx* c, spq4k_chain* ch, uint64_t* stamps) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!ch || ch->device != c->device) return set_err(c, -EINVAL, "chain_set_stamps: no chain for this device");
    if (ch->version != 2) return set_err(c, -EINVAL, "chain_set_stamps: the chain runs in form 1");
    if (!aligned(stamps, 8)) return set_err(c, -EINVAL, "chain_set_stamps: misaligned buffer");
    ch->stamps = stamps;
    return 0;
}

int spq4k_chain_status(spq4k_ctx* c, spq4k_chain* ch) {
    int rc = use_device(c);
    if (rc) return rc;
    if (!ch || ch->device != c->device) return set_err(c, -EINVAL, "chain_status: no chain for this device");
    SPQ_HIP(c, hipStreamSynchronize(c->stream));
    uint32_t err = 0;
    if (ch->version == 2) {
        SPQ_HIP(c, hipMemcpy(&err, &ch->d_sync2->err, sizeof err, hipMemcpyDeviceToHost));
        if (err) {
            SPQ_HIP(c, hipMemset(ch->d_sync2, 0, sizeof(Chain2Sync)));
            SPQ_HIP(c, hipMemset(ch->d_sh, 0xFF, sizeof(float) * (size_t)(2 * ch->sh_half + 64)));
            return set_err(c, -ETIMEDOUT, "chain: a stage wait gave up; outputs invalid, chain reset");
        }
        return 0;
    }
    SPQ_HIP(c, hipMemcpy(&err, &ch->d_sync->err, sizeof err, hipMemcpyDeviceToHost));
    if (err) {
        SPQ_HIP(c, hipMemset(ch->d_sync, 0, sizeof(ChainSync)));
        return set_err(c, -ETIMEDOUT, "chain: a stage wait gave up; outputs invalid, chain reset");
    }
    return 0;
}

}  // extern "C"
