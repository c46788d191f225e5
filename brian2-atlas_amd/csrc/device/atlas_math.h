/*
 * Shared f64 exponential functions of the Brian2-Atlas engines.
 *
 * One source, compiled three ways: into the hiprtc tick kernels (device), into
 * libatlas_sim_hip.so (host evaluation of per-tick scalar statements) and into
 * the CPU oracle.  Every operation is an IEEE binary64 add, multiply, fma, rint
 * or ldexp, all correctly rounded on both gfx950 and x86-64, and every build
 * uses -ffp-contract=off, so the CPU and the GPU produce identical bits.
 *
 * The reference evaluates Rust's f64::exp / f64::exp_m1 (executor.rs:5957-5967),
 * i.e. the host libm.  These functions aim at the correctly rounded result: a
 * double-double evaluation with relative error below 2^-95, rounded once, which
 * is the correctly rounded value except when the exact value lies within 2^-95
 * of a rounding midpoint (probability about 2^-42 per call).  Where the host
 * libm is also correctly rounded the two agree; the tests measure the agreement.
 *
 * Method (Tang's table-driven exponential, in double-double arithmetic):
 *   x = k ln2/64 + r,  k = rint(64 x / ln2),  |r| <= ln2/128,
 *   ln2/64 = C1 + C2 + C3 with C1 of 36 bits (k C1 exact for |k| < 2^17);
 *   exp(x) = 2^(k div 64) * T[k mod 64] * (1 + p(r)),  T[j] = 2^(j/64) double-double,
 *   p(r) = r + r^2 (1/2 + r (1/6 + r (1/24 + r (1/120 + r q(r))))) with the
 *   coefficients to 1/5! in double-double and q (1/6! .. 1/11!) in double;
 *   the truncated term r^12/12! < 2^-105.
 * expm1 uses p(x) directly for |x| <= ln2/128 (relative accuracy near 0) and
 * otherwise subtracts 1 from the double-double exponential before rounding.
 *
 * Results in the subnormal range are rounded twice (once to double, once by
 * ldexp); those arguments (x < -708.4) do not occur in the supported models.
 */
#ifndef ATLAS_MATH_H
#define ATLAS_MATH_H

#if defined(__HIPCC_RTC__)
#define ATLAS_MATH_FN __device__ __forceinline__
#define ATLAS_MATH_TABLE __device__ const
#elif defined(__HIPCC__)
#define ATLAS_MATH_FN __host__ __device__ static inline
#define ATLAS_MATH_TABLE static constexpr
#else
#include <math.h>
#define ATLAS_MATH_FN static inline
#define ATLAS_MATH_TABLE static const
#endif

#ifndef ATLAS_MATH_TABLES_INLINED
#include "atlas_math_tables.h"
#endif

ATLAS_MATH_TABLE double atlas_exp_table[128] = {ATLAS_EXP_TABLE_DATA};

typedef struct {
    double hi, lo;
} atlas_dd;

/* s + e == a + b exactly (Knuth's TwoSum). */
ATLAS_MATH_FN atlas_dd atlas_two_sum(double a, double b) {
    atlas_dd r;
    r.hi = a + b;
    double bb = r.hi - a;
    r.lo = (a - (r.hi - bb)) + (b - bb);
    return r;
}

/* s + e == a + b exactly, for |a| >= |b| or a == 0 (Dekker's FastTwoSum). */
ATLAS_MATH_FN atlas_dd atlas_fast_two_sum(double a, double b) {
    atlas_dd r;
    r.hi = a + b;
    r.lo = b - (r.hi - a);
    return r;
}

ATLAS_MATH_FN atlas_dd atlas_dd_mul(atlas_dd a, atlas_dd b) {
    double p = a.hi * b.hi;
    double e = fma(a.hi, b.hi, -p);
    e = e + (a.hi * b.lo + a.lo * b.hi);
    return atlas_fast_two_sum(p, e);
}

ATLAS_MATH_FN atlas_dd atlas_dd_mul_d(atlas_dd a, double b) {
    double p = a.hi * b;
    double e = fma(a.hi, b, -p);
    e = e + a.lo * b;
    return atlas_fast_two_sum(p, e);
}

ATLAS_MATH_FN atlas_dd atlas_dd_add(atlas_dd a, atlas_dd b) {
    atlas_dd s = atlas_two_sum(a.hi, b.hi);
    double e = s.lo + (a.lo + b.lo);
    return atlas_fast_two_sum(s.hi, e);
}

ATLAS_MATH_FN atlas_dd atlas_dd_make(double hi, double lo) {
    atlas_dd r;
    r.hi = hi;
    r.lo = lo;
    return r;
}

/* p(r) = exp(r) - 1 for |r| <= ln2/128, r given as a double-double. */
ATLAS_MATH_FN atlas_dd atlas_expm1_poly(atlas_dd r) {
    const double rh = r.hi;
    double q = ATLAS_INV_FACT11;
    q = fma(q, rh, ATLAS_INV_FACT10);
    q = fma(q, rh, ATLAS_INV_FACT9);
    q = fma(q, rh, ATLAS_INV_FACT8);
    q = fma(q, rh, ATLAS_INV_FACT7);
    q = fma(q, rh, ATLAS_INV_FACT6);
    atlas_dd acc = atlas_dd_add(atlas_dd_make(ATLAS_INV_FACT5_HI, ATLAS_INV_FACT5_LO), atlas_dd_mul_d(r, q));
    acc = atlas_dd_add(atlas_dd_make(ATLAS_INV_FACT4_HI, ATLAS_INV_FACT4_LO), atlas_dd_mul(r, acc));
    acc = atlas_dd_add(atlas_dd_make(ATLAS_INV_FACT3_HI, ATLAS_INV_FACT3_LO), atlas_dd_mul(r, acc));
    acc = atlas_dd_add(atlas_dd_make(0.5, 0.0), atlas_dd_mul(r, acc));
    return atlas_dd_add(r, atlas_dd_mul(atlas_dd_mul(r, r), acc));
}

/* exp(x) = 2^m * T_j * (1 + p), T_j = 2^(j/64) from the table as double-double and
 * p = exp(r) - 1 with r = x - (64 m + j) ln2/64; for |x| <= ln2/128 (k = 0) r is x exactly. */
ATLAS_MATH_FN atlas_dd atlas_exp_parts(double x, int* m, int* jo) {
    const double kd = rint(x * ATLAS_INV_LN2_64);
    const int k = (int)kd;
    const int j = k & 63;
    *m = (k - j) / 64;
    *jo = j;
    /* r = x - k (C1 + C2 + C3): k C1 is exact, the other products are split exactly */
    const double r1 = x - kd * ATLAS_LN2_64_C1;
    const double p2 = kd * ATLAS_LN2_64_C2;
    const double e2 = fma(kd, ATLAS_LN2_64_C2, -p2);
    atlas_dd r = atlas_two_sum(r1, -p2);
    r.lo = r.lo - e2 - kd * ATLAS_LN2_64_C3;
    r = atlas_fast_two_sum(r.hi, r.lo);
    return atlas_expm1_poly(r);
}

ATLAS_MATH_FN atlas_dd atlas_exp_from_parts(atlas_dd p, int j) {
    const atlas_dd t = atlas_dd_make(atlas_exp_table[2 * j], atlas_exp_table[2 * j + 1]);
    return atlas_dd_add(t, atlas_dd_mul(t, p));
}

/* exp(x) = 2^m * (hi + lo), hi + lo in [2^-1/128, 2^(1+1/128)) as double-double. */
ATLAS_MATH_FN atlas_dd atlas_exp_dd(double x, int* m) {
    int j;
    const atlas_dd p = atlas_exp_parts(x, m, &j);
    return atlas_exp_from_parts(p, j);
}

/* Branch-free: the main path always runs, on the argument clamped to its range, and the special
 * cases are selected afterwards, so that independent calls can be interleaved by the compiler
 * (a call site's exponentials are one basic block).  The results are those of the main path
 * inside the range, and NaN, +inf or 0 outside it. */
ATLAS_MATH_FN double atlas_exp(double x) {
    const double xc = x > 709.79 ? 709.79 : (x < -745.2 ? -745.2 : (x == x ? x : 0.0));
    int m;
    const atlas_dd y = atlas_exp_dd(xc, &m);
    const double r = ldexp(y.hi + y.lo, m);
    return x != x ? x : (x > 709.79 ? __builtin_huge_val() : (x < -745.2 ? 0.0 : r));
}

/* Branch-free like atlas_exp.  For |x| <= 0.0054 (k = 0 in the reduction, r = x exactly) the
 * result is the polynomial p = exp(x) - 1 itself, which the exp path has already formed; the
 * other arguments go through exp(x) - 1 = 2^m T_j (1 + p) - 1. */
ATLAS_MATH_FN double atlas_expm1(double x) {
    const double xc = x > 709.79 ? 709.79 : (x < -745.2 ? -745.2 : (x == x ? x : 0.0));
    int m, j;
    const atlas_dd p = atlas_exp_parts(xc, &m, &j);
    const atlas_dd y = atlas_exp_from_parts(p, j);
    const double big = ldexp(y.hi, m);
    const atlas_dd s = atlas_two_sum(big, -1.0);
    const double r = big == __builtin_huge_val() ? big : s.hi + (s.lo + ldexp(y.lo, m));
    return (x != x || x == 0.0) ? x
         : (x > 709.79 ? __builtin_huge_val()
         : (x < -745.2 ? -1.0 : (fabs(x) <= 0.0054 ? p.hi + p.lo : r)));
}

/* Natural logarithm, table-driven in double-double (Tang's method for log):
 *   x = 2^e m,  m in [sqrt(1/2), sqrt(2)),  F = 1 + j/128 nearest to m (j = rint(128 (m - 1))),
 *   f = m - F (exact),  r = f / F as double-double (the fma remainder gives the low part),
 *   log x = e ln2 + log F + log1p(r),  |r| <= 2^-7.49,
 *   log1p(r) = r + r^2 A(r),  A(r) = sum_k (-1)^(k+1) r^k / (k+2): the terms to k = 4 in
 *   double-double, k = 5..12 in double (the first term left out is below 2^-108 of r);
 *   e ln2 from a three-part split whose first two parts make e L1 and e L2 exact.
 * The sum is formed in double-double (relative error below about 2^-95) and rounded once,
 * so the result is the correctly rounded logarithm except within about 2^-95 of a rounding
 * midpoint.  Near x = 1 (e = 0, j = 0) r = m - 1 exactly and the result keeps its full
 * relative accuracy. */
ATLAS_MATH_TABLE double atlas_log_table[186] = {ATLAS_LOG_TABLE_DATA};

ATLAS_MATH_FN double atlas_log(double x) {
    if (x != x || x < 0.0) return __builtin_nan("");
    if (x == 0.0) return -__builtin_huge_val();
    if (x == __builtin_huge_val()) return x;
    int e;
    double m = frexp(x, &e);          /* m in [1/2, 1), exact for subnormal x too */
    if (m < 0x1.6a09e667f3bcdp-1) {   /* sqrt(1/2) rounded up: m in [sqrt(1/2), sqrt(2)) below */
        m = m * 2.0;
        e = e - 1;
    }
    const double d = m - 1.0;         /* exact (Sterbenz) */
    const double jd = rint(d * 128.0);
    const int j = (int)jd;
    const double F = 1.0 + jd * 0.0078125;
    const double f = d - jd * 0.0078125;  /* exact: both are multiples of 2^-53, |f| <= 2^-8 */
    const double rh = f / F;
    const double rl = fma(-rh, F, f) / F;
    const atlas_dd r = atlas_fast_two_sum(rh, rl);
    double q = ATLAS_LOG1P_C12;
    q = fma(q, r.hi, ATLAS_LOG1P_C11);
    q = fma(q, r.hi, ATLAS_LOG1P_C10);
    q = fma(q, r.hi, ATLAS_LOG1P_C9);
    q = fma(q, r.hi, ATLAS_LOG1P_C8);
    q = fma(q, r.hi, ATLAS_LOG1P_C7);
    q = fma(q, r.hi, ATLAS_LOG1P_C6);
    q = fma(q, r.hi, ATLAS_LOG1P_C5);
    atlas_dd a = atlas_dd_add(atlas_dd_make(ATLAS_LOG1P_C4_HI, ATLAS_LOG1P_C4_LO), atlas_dd_mul_d(r, q));
    a = atlas_dd_add(atlas_dd_make(ATLAS_LOG1P_C3_HI, ATLAS_LOG1P_C3_LO), atlas_dd_mul(r, a));
    a = atlas_dd_add(atlas_dd_make(ATLAS_LOG1P_C2_HI, ATLAS_LOG1P_C2_LO), atlas_dd_mul(r, a));
    a = atlas_dd_add(atlas_dd_make(ATLAS_LOG1P_C1_HI, ATLAS_LOG1P_C1_LO), atlas_dd_mul(r, a));
    a = atlas_dd_add(atlas_dd_make(ATLAS_LOG1P_C0_HI, ATLAS_LOG1P_C0_LO), atlas_dd_mul(r, a));
    const atlas_dd p = atlas_dd_add(r, atlas_dd_mul(atlas_dd_mul(r, r), a));
    const int t = 2 * (j - ATLAS_LOG_TABLE_FIRST);
    atlas_dd s = atlas_dd_add(atlas_dd_make(atlas_log_table[t], atlas_log_table[t + 1]), p);
    if (e != 0) {
        const double ed = (double)e;
        atlas_dd l = atlas_two_sum(ed * ATLAS_LN2_L1, ed * ATLAS_LN2_L2);
        l.lo = l.lo + ed * ATLAS_LN2_L3;
        s = atlas_dd_add(atlas_fast_two_sum(l.hi, l.lo), s);
    }
    return s.hi + s.lo;
}

ATLAS_MATH_FN float atlas_expf(float x) { return (float)atlas_exp((double)x); }
ATLAS_MATH_FN float atlas_logf(float x) { return (float)atlas_log((double)x); }

/* Brian2's exprel as the reference evaluates it (executor.rs:5959-5967). */
ATLAS_MATH_FN double atlas_exprel(double x) {
    const double q = atlas_expm1(x) / x;
    return fabs(x) < 1e-16 ? 1.0 : (x > 717.0 ? __builtin_huge_val() : q);
}

#endif /* ATLAS_MATH_H */
