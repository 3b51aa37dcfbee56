/* spq4k_diag.h — diagnostics and measurement entry points of libspq4k.
 *
 * None of these has a counterpart in the reference, and a drop-in caller of
 * the Q4_K path (include/spq4k.h) needs none of them: they expose internal
 * integer sums for the parity tests, a read-only streaming probe for the
 * HBM floor measurement, and the stage timestamps of a decode chain. They
 * live in the same library and use the same context and error codes
 * (spq4k_last_error). */
#ifndef SPQ4K_DIAG_H
#define SPQ4K_DIAG_H

#include "spq4k.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- integer sums and the streaming probe --------------------------------
 * Exact integer sub-block sums S[r][b][j] = sum_{l<32} q4 * q8 over
 * sub-block j of block b of row r, against Q8_K(x), formed by the same lane
 * code as the GEMV. No reference function returns them; they are the integer
 * core of ggml_vec_dot_q4_K_q8_K (ggml-cpu/quants.c:645-718). */
int spq4k_subblock_sums(spq4k_ctx *ctx, const void *W, int64_t M, int64_t K, const float *x, int32_t *S);
/* The same for a weight type: Q4_K as above; Q5_K gives S[r][b][j], j < 8,
 * the sum of q5 * q8 over sub-block j (ggml-cpu/quants.c:720-798); Q6_K gives
 * S[r][b][j], j < 16, the sum over the 16 weights of sub-block j of
 * (q - 32) * q8, the integer core of ggml_vec_dot_q6_K_q8_K
 * (ggml-cpu/quants.c:800-852); Q8_0 gives S[r][b], b < K/32, the sum of
 * qw * qx over block b against spq4k_quantize_q8_0(x), the integer core of
 * ggml_vec_dot_q8_0_q8_0 (ggml-cpu/quants.c:400-428). */
int spq4k_subblock_sums_type(spq4k_ctx *ctx, int type, const void *W, int64_t M, int64_t K, const float *x,
                             int32_t *S);
/* A read of `bytes` of device memory at p (16-byte aligned, a multiple of
 * 16 bytes; 0 launches a kernel that reads nothing) by one launch on the
 * context stream: each wave reads 4 KB of consecutive bytes per step as four
 * coalesced 16-byte-a-lane loads, four workgroups a CU (SPQ4K_STREAM_GRID
 * sets another largest grid), no other work -- the HBM floor of a launch of
 * the same bytes. No reference counterpart; for measurement (bench.py
 * --config floor). */
int spq4k_stream_read(spq4k_ctx *ctx, const void *p, size_t bytes);

/* ---- decode-chain stage timestamps --------------------------------------
 * spq4k_chain_info reports the form a chain runs in (1: a grid barrier at
 * every stage; 2: the one-hop exchange of csrc/k_chain2.hip), its
 * workgroups and its stages. spq4k_chain_set_stamps gives a form-2 chain a
 * device buffer of grid * n_stages * 4 uint64 (NULL stops it): every later
 * run writes, per workgroup w and stage t at [(w * n_stages + t) * 4 + k],
 * the device's constant 100 MHz clock (s_memrealtime) when
 *   k = 0  the first exchange wave's share of the stage's inputs was
 *          gathered (every shadow word current),
 *   k = 3  every exchange wave's share was, and x = in0 (+ in1) formed,
 *   k = 1  its Q8_K activations were ready (the rows start),
 *   k = 2  the workgroup's rows of the stage were done.
 * -EINVAL for a form-1 chain. */
int spq4k_chain_info(const spq4k_chain *chain, int *version, int *grid, int *n_stages);
int spq4k_chain_set_stamps(spq4k_ctx *ctx, spq4k_chain *chain, uint64_t *stamps);

/* ---- decode-kernel wave timestamps -------------------------------------
 * spq4k_set_decode_stamps gives ctx a device buffer of n uint64 (NULL stops
 * it). While it is set, every T = 1 matvec on ctx that runs the decode
 * kernel unfused writes, for wave v of workgroup w at [(w * waves + v) * 4 + k],
 * the device's constant 100 MHz clock (s_memrealtime) when
 *   k = 0  the wave started,
 *   k = 1  it passed the barrier that publishes the workgroup's Q8_K
 *          activations in LDS,
 *   k = 2  its first row's dot product was done and, in the forms that
 *          store each row at once, its store issued (0: a wave without rows),
 *   k = 3  it had issued the store of its last row (every row's store, in
 *          the forms that collect a wave's results for one store at the end).
 * Each launch overwrites the buffer. Only the Q4_K launch shapes the planner
 * picks for rows of K = 4096 and K = 12288 (the 8B step's) have a
 * timestamped instance: another shape, or a launch whose grid * waves * 4
 * exceeds n, fails with -EINVAL while stamps are set. */
int spq4k_set_decode_stamps(spq4k_ctx *ctx, uint64_t *stamps, size_t n);

#ifdef __cplusplus
}
#endif

#endif /* SPQ4K_DIAG_H */
