/*
 * synth_math.h — deterministic, counter-based synthetic data for the Q4_K path.
 *
 * The reference's own seeded tests draw N(0, 0.02) weights with
 * std::mt19937 + std::normal_distribution
 * (tests/desktop/test_sp_quant_q5k.cpp:32-34). normal_distribution is
 * implementation-defined, and a GPU cannot run it, so this file defines a
 * generator whose every value is a pure function of (seed, index) and is
 * computed with IEEE-754 basic operations only (+, -, *, /, exact bit
 * manipulation). The host (gcc) and device (hipcc) builds therefore produce
 * bit-identical streams, which lets a 4.26 GB weight set be synthesised on
 * the GPU while the CPU checker regenerates any slice of it exactly.
 *
 *   uniform:  SplitMix64 finaliser of (seed, index) -> 53-bit u in (0, 1)
 *   normal:   Box-Muller on the pair (2p, 2p+1); ln, sin, cos evaluated by
 *             the fixed series below in double, then rounded to fp32
 *   student-t(nu=4): Z / sqrt(V/4), V = -2 ln(U3 U4) ~ chi^2(4)
 *
 * This header is C (gcc) and HIP (hipcc) compatible. It must be compiled
 * with floating-point contraction disabled (-ffp-contract=off) on both
 * sides so that no a*b+c is fused differently on one of them.
 */
#ifndef SPQ4K_SYNTH_MATH_H
#define SPQ4K_SYNTH_MATH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define SPQ_HD __host__ __device__ static inline
#else
#define SPQ_HD static inline
#endif

/* ---- bit casts -------------------------------------------------------- */
SPQ_HD double spq_u64_as_f64(uint64_t u) { union { uint64_t u; double d; } c; c.u = u; return c.d; }
SPQ_HD uint64_t spq_f64_as_u64(double d) { union { uint64_t u; double d; } c; c.d = d; return c.u; }
SPQ_HD uint32_t spq_f32_as_u32(float f) { union { uint32_t u; float f; } c; c.f = f; return c.u; }
SPQ_HD float spq_u32_as_f32(uint32_t u) { union { uint32_t u; float f; } c; c.u = u; return c.f; }

/* ---- counter-based uniform -------------------------------------------- */
SPQ_HD uint64_t spq_mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* 64-bit hash of (seed, index): two rounds so that nearby seeds decorrelate. */
SPQ_HD uint64_t spq_hash2(uint64_t seed, uint64_t idx) {
    return spq_mix64(spq_mix64(seed) ^ (idx * 0xD1B54A32D192ED03ull));
}

/* u in (0, 1), never 0 or 1: (top 53 bits + 0.5) * 2^-53. */
SPQ_HD double spq_uniform(uint64_t seed, uint64_t idx) {
    uint64_t h = spq_hash2(seed, idx);
    return ((double)(h >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

/* ---- natural log on (0, inf), double, basic ops only --------------------
 * x = m * 2^e with m in [sqrt(1/2), sqrt(2)); ln m = 2 atanh(s), s=(m-1)/(m+1),
 * |s| <= 0.1716; the odd series to s^27 leaves a truncation error < 1e-21. */
SPQ_HD double spq_ln(double x) {
    uint64_t b = spq_f64_as_u64(x);
    int e = (int)((b >> 52) & 0x7FF) - 1023;
    double m = spq_u64_as_f64((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull); /* [1,2) */
    if (m > 1.4142135623730951) { m = m * 0.5; e += 1; }
    double s = (m - 1.0) / (m + 1.0);
    double s2 = s * s;
    double t = 1.0 / 27.0;
    t = t * s2 + 1.0 / 25.0;
    t = t * s2 + 1.0 / 23.0;
    t = t * s2 + 1.0 / 21.0;
    t = t * s2 + 1.0 / 19.0;
    t = t * s2 + 1.0 / 17.0;
    t = t * s2 + 1.0 / 15.0;
    t = t * s2 + 1.0 / 13.0;
    t = t * s2 + 1.0 / 11.0;
    t = t * s2 + 1.0 / 9.0;
    t = t * s2 + 1.0 / 7.0;
    t = t * s2 + 1.0 / 5.0;
    t = t * s2 + 1.0 / 3.0;
    t = t * s2 + 1.0;
    return (double)e * 0.69314718055994530942 + 2.0 * s * t;
}

/* ---- square root for x > 0, double ---------------------------------------
 * Newton's iteration y <- (y + x/y)/2 from an exponent-halved first guess
 * (relative error < 0.42), six steps. Only +, *, / are used, so the value is
 * the same on every IEEE-754 machine; it is within 1 ulp, not necessarily
 * correctly rounded, which does not matter for data synthesis. */
SPQ_HD double spq_sqrt(double x) {
    uint64_t b = spq_f64_as_u64(x);
    int e = (int)((b >> 52) & 0x7FF) - 1023;
    int h = e >> 1;                               /* floor(e/2) */
    double y = spq_u64_as_f64((uint64_t)(h + 1023) << 52);
    if (e & 1) y = y * 1.4142135623730951;
    for (int i = 0; i < 6; ++i) y = 0.5 * (y + x / y);
    return y;
}

/* ---- sin and cos of 2*pi*u for u in [0, 1) ------------------------------
 * Quadrant q = floor(4u); theta = (4u - q) * pi/2 in [0, pi/2); Taylor series
 * to theta^23 / theta^22 (error < 1e-17 on that interval). */
SPQ_HD void spq_sincos_2pi(double u, double *s_out, double *c_out) {
    double f4 = u * 4.0;
    int q = (int)f4;
    if (q > 3) q = 3;
    double th = (f4 - (double)q) * 1.57079632679489661923;
    double t2 = th * th;
    /* sin(th) = th * (1 - t2/3! + t2^2/5! - ...) */
    double sp = -1.0 / 25852016738884976640000.0;    /* -1/23! */
    sp = sp * t2 + 1.0 / 51090942171709440000.0;     /* 1/21! */
    sp = sp * t2 - 1.0 / 121645100408832000.0;       /* 1/19! */
    sp = sp * t2 + 1.0 / 355687428096000.0;          /* 1/17! */
    sp = sp * t2 - 1.0 / 1307674368000.0;            /* 1/15! */
    sp = sp * t2 + 1.0 / 6227020800.0;               /* 1/13! */
    sp = sp * t2 - 1.0 / 39916800.0;                 /* 1/11! */
    sp = sp * t2 + 1.0 / 362880.0;                   /* 1/9! */
    sp = sp * t2 - 1.0 / 5040.0;                     /* 1/7! */
    sp = sp * t2 + 1.0 / 120.0;                      /* 1/5! */
    sp = sp * t2 - 1.0 / 6.0;                        /* 1/3! */
    sp = sp * t2 + 1.0;
    double sn = th * sp;
    double cp = 1.0 / 1124000727777607680000.0;      /* 1/22! */
    cp = cp * t2 - 1.0 / 2432902008176640000.0;      /* 1/20! */
    cp = cp * t2 + 1.0 / 6402373705728000.0;         /* 1/18! */
    cp = cp * t2 - 1.0 / 20922789888000.0;           /* 1/16! */
    cp = cp * t2 + 1.0 / 87178291200.0;              /* 1/14! */
    cp = cp * t2 - 1.0 / 479001600.0;                /* 1/12! */
    cp = cp * t2 + 1.0 / 3628800.0;                  /* 1/10! */
    cp = cp * t2 - 1.0 / 40320.0;                    /* 1/8! */
    cp = cp * t2 + 1.0 / 720.0;                      /* 1/6! */
    cp = cp * t2 - 1.0 / 24.0;                       /* 1/4! */
    cp = cp * t2 + 1.0 / 2.0;                        /* 1/2! */
    double cs = 1.0 - t2 * cp;
    /* rotate by q quarter turns */
    double s = sn, c = cs;
    if (q == 1) { s = cs;  c = -sn; }
    if (q == 2) { s = -sn; c = -cs; }
    if (q == 3) { s = -cs; c = sn; }
    *s_out = s;
    *c_out = c;
}

/* Standard normal number idx of stream `seed` (double). Pair p = idx/2 uses
 * uniforms 2p and 2p+1; even idx takes the cosine branch, odd the sine. */
SPQ_HD double spq_normal(uint64_t seed, uint64_t idx) {
    uint64_t p = idx >> 1;
    double u1 = spq_uniform(seed, 2 * p);
    double u2 = spq_uniform(seed, 2 * p + 1);
    double r2 = -2.0 * spq_ln(u1);
    double r = spq_sqrt(r2);
    double s, c;
    spq_sincos_2pi(u2, &s, &c);
    return (idx & 1) ? r * s : r * c;
}

/* Student-t with nu = 4 degrees of freedom. */
SPQ_HD double spq_student_t4(uint64_t seed, uint64_t idx) {
    double z = spq_normal(seed, idx);
    uint64_t s2 = spq_mix64(seed ^ 0x5851F42D4C957F2Dull);
    double u3 = spq_uniform(s2, 2 * idx);
    double u4 = spq_uniform(s2, 2 * idx + 1);
    double v = -2.0 * (spq_ln(u3) + spq_ln(u4));   /* chi^2 with 4 dof */
    return z / spq_sqrt(v * 0.25);
}

/* Outlier-column selector for the skewed large-K workload: column c is an
 * outlier when the hash of (seed, c) falls in the lowest 1/100 of its range. */
SPQ_HD int spq_is_outlier_col(uint64_t seed, uint64_t col) {
    return (spq_hash2(seed ^ 0xA0761D6478BD642Full, col) % 100ull) == 0ull;
}

/* Distribution selectors shared by the host and device fill routines. */
enum { SPQ_DIST_NORMAL = 0, SPQ_DIST_STUDENT_T4 = 1 };

/* Value idx of a [rows x cols] row-major fill (col = idx % cols):
 *   mean + std * X,  X ~ N(0,1) or t(4); times outlier_mult on outlier columns
 *   when outlier_mult != 1. Rounded once to fp32. */
SPQ_HD float spq_synth_value(uint64_t seed, int dist, uint64_t idx, uint64_t cols,
                             float mean, float std, float outlier_mult) {
    double x = (dist == SPQ_DIST_STUDENT_T4) ? spq_student_t4(seed, idx) : spq_normal(seed, idx);
    double v = (double)mean + (double)std * x;
    if (outlier_mult != 1.0f && cols != 0 && spq_is_outlier_col(seed, idx % cols)) {
        v = v * (double)outlier_mult;
    }
    return (float)v;
}

#endif /* SPQ4K_SYNTH_MATH_H */
