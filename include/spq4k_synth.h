/*
 * spq4k_synth.h — seeded synthetic inputs on the device.
 *
 * Counterpart of the seeded generators in the reference's tests
 * (tests/desktop/test_sp_quant_q5k.cpp:32-34: std::mt19937 +
 * std::normal_distribution(0, 0.02)), which are implementation-defined. Here
 * value i of a fill is a pure function of (seed, offset + i) computed with
 * IEEE basic operations only, so the host checker regenerates any slice
 * bit-identically. Used by bench.py and the tests to synthesise the BASELINE
 * workloads (weights N(0, 0.02) or Student-t(4) * 0.02 with outlier columns,
 * activations N(0, 1)) directly in HBM.
 */
#ifndef SPQ4K_SYNTH_H
#define SPQ4K_SYNTH_H

#include <stdint.h>
#include "spq4k.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SPQ4K_DIST_NORMAL 0
#define SPQ4K_DIST_STUDENT_T4 1

/* out[i] = mean + std * X_{offset+i} (X ~ N(0,1) or t(4)), multiplied by
 * outlier_mult when column (offset+i) % cols is an outlier column (about 1%
 * of columns; outlier_mult = 1 disables it). out is a device pointer;
 * asynchronous on the context stream. */
int spq4k_synth_fill(spq4k_ctx *ctx, float *out, int64_t n, uint64_t seed, int dist, int64_t cols,
                     float mean, float std, float outlier_mult, int64_t offset);

#ifdef __cplusplus
}
#endif

#endif /* SPQ4K_SYNTH_H */
