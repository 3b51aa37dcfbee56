/*
 * q4k_oracle.h — CPU restatement of the reference's Q4_K x Q8_K arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP kernels
 * in shannon-prime-burnhard_amd/csrc. Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load it. No product code path may
 * call it, link it, or fall back to it.
 *
 * Every function restates a function of the vendored ggml in the reference
 * (vendor/ggml/src/...), cited at its definition in q4k_oracle.c. It is
 * compiled with -ffp-contract=off so that each floating-point operation is
 * rounded exactly once, as in ggml-base (which is built without FMA flags).
 *
 * q6k_oracle.c, q5k_oracle.c and q8_0_oracle.c restate the Q6_K, Q5_K and
 * Q8_0 functions the same way.
 *
 * Parity pins (see tests/): golden fixtures written by tests/golden/gen_golden.py
 * from the reference compiled in oracle/_ref, exhaustive and closed-form checks
 * of the scale unpacker, dequantiser and Q8_K quantiser, and brute-force
 * integer sub-block sums.
 */
#ifndef Q4K_ORACLE_H
#define Q4K_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_QK_K 256
#define OR_Q4K_BLOCK_BYTES 144   /* d, dmin (fp16), scales[12], qs[128] */
#define OR_Q8K_BLOCK_BYTES 292   /* d (f32), qs[256] (i8), bsums[16] (i16) */

typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t  scales[12];
    uint8_t  qs[128];
} or_block_q4K;

typedef struct {
    float   d;
    int8_t  qs[256];
    int16_t bsums[16];
} or_block_q8K;

#define OR_Q6K_BLOCK_BYTES 210   /* ql[128], qh[64], scales[16] (i8), d (fp16) */
typedef struct {
    uint8_t  ql[128];
    uint8_t  qh[64];
    int8_t   scales[16];
    uint16_t d;
} or_block_q6K;

#define OR_Q5K_BLOCK_BYTES 176   /* d, dmin (fp16), scales[12], qh[32], qs[128] */
typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t  scales[12];
    uint8_t  qh[32];
    uint8_t  qs[128];
} or_block_q5K;

#define OR_QK8_0 32
#define OR_Q8_0_BLOCK_BYTES 34   /* d (fp16), qs[32] (i8) */
typedef struct {
    uint16_t d;
    int8_t   qs[32];
} or_block_q8_0;

/* weight types, numbered as ggml.h:392-404 numbers them */
#define OR_TYPE_Q8_0 8
#define OR_TYPE_Q4_K 12
#define OR_TYPE_Q5_K 13
#define OR_TYPE_Q6_K 14

/* scalar helpers */
float    or_fp16_to_fp32(uint16_t h);
uint16_t or_fp32_to_fp16(float f);
int      or_nearest_int(float v);
void     or_scale_min_k4(int j, const uint8_t *scales, uint8_t *sc, uint8_t *m);

/* type traits (ggml_to_float_t / ggml_from_float_t shapes) */
void or_quantize_row_q4K(const float *x, void *y, int64_t k);
size_t or_quantize_q4K(const float *src, void *dst, int64_t nrow, int64_t n_per_row);
void or_dequantize_row_q4K(const void *x, float *y, int64_t k);
void or_quantize_row_q8K(const float *x, void *y, int64_t k);

/* dot products (ggml_vec_dot_t semantics, nrc == 1) */
float  or_vec_dot_generic(int n, const void *vx, const void *vy);
float  or_vec_dot_avx2order(int n, const void *vx, const void *vy);
double or_vec_dot_exact(int n, const void *vx, const void *vy);
/* S[b*8 + j] = sum over the 32 weights of sub-block j of block b of q4*q8 */
void   or_subblock_sums(int n, const void *vx, const void *vy, int32_t *S);

/* drivers: ggml_compute_forward_mul_mat / _mul_mat_id numerics.
 * W: M rows of K/256 Q4_K blocks; X: T rows of K fp32; Y: T rows of M fp32.
 * order: 0 = generic float order, 1 = x86 AVX2 float order. */
void or_mul_mat(const void *W, int64_t M, int64_t K, const float *X, int64_t T,
                float *Y, int order);
/* as: E experts of [M x K]; X: [T][ne11][K] with ne11 in {1, k};
 * ids: [T][k] int32; Y: [T][k][M]. Returns 0, or -22 on a bad expert id. */
int  or_mul_mat_id(const void *as, int64_t M, int64_t K, int64_t E,
                   const float *X, int64_t ne11, const int32_t *ids, int64_t k,
                   int64_t T, float *Y, int order);
/* dequant-then-dot in double with the fp32 activations as given (the exact
 * value of an fp32-activation dequant-then-dot: beast_matvec's semantics) */
void or_mul_mat_dequant_f64(const void *W, int64_t M, int64_t K, const float *X,
                            int64_t T, double *Y);

/* Q6_K (q6k_oracle.c) */
void   or_quantize_row_q6K(const float *x, void *y, int64_t k);
size_t or_quantize_q6K(const float *src, void *dst, int64_t nrow, int64_t n_per_row);
void   or_dequantize_row_q6K(const void *x, float *y, int64_t k);
float  or_vec_dot_q6K_generic(int n, const void *vx, const void *vy);
float  or_vec_dot_q6K_avx2order(int n, const void *vx, const void *vy);
double or_vec_dot_q6K_exact(int n, const void *vx, const void *vy);
/* S[b*16 + j] = sum over the 16 weights of sub-block j of block b of (q-32)*q8 */
void   or_subblock_sums_q6K(int n, const void *vx, const void *vy, int32_t *S);

/* Q5_K (q5k_oracle.c) */
void   or_quantize_row_q5K(const float *x, void *y, int64_t k);
size_t or_quantize_q5K(const float *src, void *dst, int64_t nrow, int64_t n_per_row);
void   or_dequantize_row_q5K(const void *x, float *y, int64_t k);
float  or_vec_dot_q5K_generic(int n, const void *vx, const void *vy);
float  or_vec_dot_q5K_avx2order(int n, const void *vx, const void *vy);
double or_vec_dot_q5K_exact(int n, const void *vx, const void *vy);
/* S[b*8 + j] = sum over the 32 weights of sub-block j of block b of q5*q8 */
void   or_subblock_sums_q5K(int n, const void *vx, const void *vy, int32_t *S);

/* Q8_0 (q8_0_oracle.c): weights and their Q8_0 activations, 32 values a block */
void   or_quantize_row_q8_0(const float *x, void *y, int64_t k);        /* activations: x86 CPU backend */
void   or_quantize_row_q8_0_ref(const float *x, void *y, int64_t k);    /* weights: model-file encoder */
void   or_dequantize_row_q8_0(const void *x, float *y, int64_t k);
float  or_vec_dot_q8_0_generic(int n, const void *vx, const void *vy);
float  or_vec_dot_q8_0_avx2order(int n, const void *vx, const void *vy);
double or_vec_dot_q8_0_exact(int n, const void *vx, const void *vy);
void   or_block_sums_q8_0(int n, const void *vx, const void *vy, int32_t *S);
int    or_mul_mat_q8_0(const void *W, int64_t M, int64_t K, const float *X, int64_t T, float *Y, int order);
int    or_mul_mat_id_q8_0(const void *as, int64_t M, int64_t K, int64_t E, const float *X, int64_t ne11,
                          const int32_t *ids, int64_t k, int64_t T, float *Y, int order);

/* make_qkx2_quants (q4k_oracle.c), shared by the Q4_K and Q5_K encoders */
float or_qkx2_fit(int n, int nmax, const float *x, const float *w, uint8_t *L,
                  float *neg_min, uint8_t *Laux, float rmin, float rdelta, int nstep);

/* the drivers above for a weight type (OR_TYPE_Q4_K, _Q5_K or _Q6_K);
 * return -22 for another type or a bad expert id */
int or_mul_mat_type(int type, const void *W, int64_t M, int64_t K, const float *X, int64_t T,
                    float *Y, int order);
int or_mul_mat_id_type(int type, const void *as, int64_t M, int64_t K, int64_t E,
                       const float *X, int64_t ne11, const int32_t *ids, int64_t k,
                       int64_t T, float *Y, int order);
int or_mul_mat_dequant_f64_type(int type, const void *W, int64_t M, int64_t K, const float *X,
                                int64_t T, double *Y);
/* dequantize_row_q8_K (ggml-quants.c:2731-2740) */
void or_dequantize_row_q8K(const void *x, float *y, int64_t k);
/* the parity bar's second form for the matmuls: sum of dequant(W) *
 * dequant(Q(x)) in double, Q the type's activation quantiser (Q8_K, or
 * Q8_0 for Q8_0 weights); types Q4_K, Q5_K, Q6_K, Q8_0 */
int or_mul_mat_dq_f64_type(int type, const void *W, int64_t M, int64_t K, const float *X,
                           int64_t T, double *Y);
/* beast_matvec (sp_beast_canyon.c:1122-1134) as the reference's build
 * evaluates it (fp32 products summed in index order), for one fp32 input x;
 * Q4_K and Q8_0 with the reference's dequantisers, Q5_K and Q6_K with the
 * format's (the reference's read other bits). or_beast_moe_routed: the MoE
 * forward's per-expert loop (:486-545) over a given routing, a type per bank */
int or_beast_matvec_type(int type, const void *W, int64_t M, int64_t K, const float *x, float *y);
int or_beast_moe_routed(int tg, const void *gate, int tu, const void *up, int td, const void *down, int64_t E,
                        int64_t n_embd, int64_t n_ff, const int32_t *ids, const float *scores, int64_t k,
                        const float *hidden, float *out);

/* synthetic data, bit-identical with the device generator */
void or_synth_fill(float *out, int64_t n, uint64_t seed, int dist, int64_t cols,
                   float mean, float std, float outlier_mult, int64_t offset);

/* fused neighbours of the matvec (fusion_oracle.c) */
void or_rms_norm(const float *x, int64_t K, int64_t T, const float *w, float eps, float *y);
void or_swiglu(const float *g, const float *u, int64_t n, float *y);

#ifdef __cplusplus
}
#endif

#endif /* Q4K_ORACLE_H */
