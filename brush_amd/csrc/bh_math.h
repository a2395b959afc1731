/*
 * bh_math.h — reproducible scalar float primitives shared by the gfx950
 * kernels and the CPU restatement.
 *
 * Why this exists: the rasterizer's integer outputs (visibility, per-splat
 * tile counts, tile ids, sort keys, tile offsets) are decided by float
 * comparisons that sit downstream of exp() and log() (sigmoid of the raw
 * opacity, exp of the log-scales, ln(255 * opacity) power threshold,
 * brush-render/src/kernels/project_forward.rs:82-133,
 * brush-render/src/kernels/helpers.rs:87-97,241-280).  Vendor libm and the
 * device math library each round exp/log their own way, so the only way for a
 * CPU checker and the GPU to agree bit for bit is to evaluate both functions
 * with the same sequence of correctly rounded IEEE-754 operations
 * (+, -, *, /, fma).  Every function here uses only those, plus integer bit
 * manipulation, and the translation units that include this header are
 * compiled without floating-point contraction (-ffp-contract=off), so gcc on
 * x86-64 (SSE, FLT_EVAL_METHOD == 0) and hipcc for gfx950 (IEEE mode,
 * f32 denormals kept, correctly rounded division) produce identical bits.
 *
 * Methods:
 *   bh_expf — Cody & Waite argument reduction x = n ln2 + r with a two-part
 *             ln2 (hi part with 15 significant bits, so n*ln2_hi is exact for
 *             |n| <= 2^8), then the degree-7 Taylor polynomial of e^r on
 *             |r| <= ln2/2 (truncation error < 0.05 ulp), scaled by 2^n.
 *   bh_logf — x = 2^e m with m in [sqrt(1/2), sqrt(2)), f = m - 1,
 *             s = f / (2 + f), log(1+f) = 2 atanh(s) = f - s (f - R) with
 *             R = sum_{k>=1} 2 s^{2k} / (2k+1) truncated after s^8 (the
 *             rearrangement used by the classic BSD/fdlibm logf), plus e ln2.
 *   bh_atan2f — t = min(|y|,|x|) / max(|y|,|x|) in [0, 1]; with the nearest
 *             centre c = tan(k pi / 12), k = 0..3, atan(t) = atan(c) +
 *             atan((t - c) / (1 + t c)) leaves |s| <= tan(pi/24); atan(s) is
 *             the Taylor series through s^13 (truncation below 1e-13
 *             relative); atan(c) of the f32 c and the quadrant fix-ups
 *             (pi/2 - a when |y| > |x|, pi - a when x < 0) use two-part
 *             constants; sign of y.
 * All stay within 2 ulp of the correctly rounded result over all finite
 * inputs (pinned on the CPU against float64 libm by the oracle tests).
 *   bh_exp2_neg — the splat Gaussian's 2^x (see its comment): rint, a
 *             degree-5 minimax polynomial of 2^f on [-1/2, 1/2], ldexp;
 *             within 3 ulp of 2^x on [-126, 1].
 *
 * This header is plain C99 so the CPU restatement (gcc) can include it; under
 * hipcc every function is callable from host and device.
 */
#ifndef BH_MATH_H
#define BH_MATH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define BH_HD __host__ __device__ static inline
#else
#define BH_HD static inline
#include <math.h>
#endif

#define BH_INF_BITS 0x7f800000u
#define BH_NAN_BITS 0x7fc00000u

BH_HD uint32_t bh_as_uint(float x) {
    uint32_t u;
    __builtin_memcpy(&u, &x, sizeof(u));
    return u;
}

BH_HD float bh_as_float(uint32_t u) {
    float x;
    __builtin_memcpy(&x, &u, sizeof(x));
    return x;
}

/* Bit-level finiteness: NaN and +-Inf have an all-ones exponent
 * (brush-cube/src/lib.rs:626-630). */
BH_HD int bh_is_finite(float x) { return ((bh_as_uint(x) >> 23) & 0xFFu) != 0xFFu; }

/* min/max with a fixed NaN rule so both sides agree: the first operand is
 * returned unless the second compares strictly smaller (larger). */
BH_HD float bh_minf(float a, float b) { return (b < a) ? b : a; }
BH_HD float bh_maxf(float a, float b) { return (b > a) ? b : a; }
BH_HD float bh_clampf(float x, float lo, float hi) { return bh_minf(bh_maxf(x, lo), hi); }
BH_HD float bh_absf(float x) { return bh_as_float(bh_as_uint(x) & 0x7fffffffu); }

BH_HD float bh_fmaf(float a, float b, float c) {
#if defined(__HIPCC__)
    return __builtin_fmaf(a, b, c);
#else
    return fmaf(a, b, c);
#endif
}

/* Round to the nearest integer, ties to even (exact). */
BH_HD float bh_rintf(float x) {
#if defined(__HIPCC__)
    return __builtin_rintf(x);
#else
    return rintf(x);
#endif
}

/* p * 2^n (exact while the result is a normal number). */
BH_HD float bh_ldexpf(float p, int n) {
#if defined(__HIPCC__)
    return __builtin_ldexpf(p, n);
#else
    return ldexpf(p, n);
#endif
}

/* Multiply p by 2^n for n in [-150, 128] with IEEE rounding. */
BH_HD float bh_scale_pow2(float p, int n) {
    if (n > 127) {
        p = p * 2.0f;
        n -= 1;
    }
    if (n < -126) {
        p = p * bh_as_float((uint32_t)(n + 24 + 127) << 23);
        return p * 5.9604644775390625e-08f; /* 2^-24 */
    }
    return p * bh_as_float((uint32_t)(n + 127) << 23);
}

BH_HD float bh_expf(float x) {
    if (!(x == x)) return x; /* NaN propagates */
    if (x > 89.0f) return bh_as_float(BH_INF_BITS);
    if (x < -104.0f) return 0.0f;
    const float log2e = 1.44269502162933349609375f;
    const float ln2_hi = 0.693145751953125f;        /* 0x3f317200 */
    const float ln2_lo = 1.428606765330187045e-06f; /* 0x35bfbe8e */
    const float shifter = 12582912.0f;              /* 1.5 * 2^23: round to nearest even */
    float k = x * log2e;
    float kr = (k + shifter) - shifter;
    int n = (int)kr;
    float r = bh_fmaf(kr, -ln2_hi, x);
    r = bh_fmaf(kr, -ln2_lo, r);
    /* e^r = sum r^i / i!, i = 0..7, Horner form */
    float p = 1.98412698412698413e-04f; /* 1/5040 */
    p = bh_fmaf(p, r, 1.38888888888888889e-03f); /* 1/720 */
    p = bh_fmaf(p, r, 8.33333333333333333e-03f); /* 1/120 */
    p = bh_fmaf(p, r, 4.16666666666666667e-02f); /* 1/24 */
    p = bh_fmaf(p, r, 1.66666666666666667e-01f); /* 1/6 */
    p = bh_fmaf(p, r, 0.5f);
    p = bh_fmaf(p, r, 1.0f);
    p = bh_fmaf(p, r, 1.0f);
    return bh_scale_pow2(p, n);
}

BH_HD float bh_logf(float x) {
    if (!(x == x)) return x;
    if (x < 0.0f) return bh_as_float(BH_NAN_BITS);
    if (x == 0.0f) return -bh_as_float(BH_INF_BITS);
    uint32_t bits = bh_as_uint(x);
    if (bits == BH_INF_BITS) return x;
    int e = 0;
    if (bits < 0x00800000u) { /* subnormal: renormalise exactly */
        x = x * 33554432.0f;  /* 2^25 */
        bits = bh_as_uint(x);
        e = -25;
    }
    e += (int)(bits >> 23) - 127;
    float m = bh_as_float((bits & 0x007fffffu) | 0x3f800000u); /* [1, 2) */
    if (m > 1.41421353816986083984375f) {
        m = m * 0.5f;
        e += 1;
    }
    float f = m - 1.0f; /* exact */
    float s = f / (2.0f + f);
    float s2 = s * s;
    float t = 2.22222222222222222e-01f;          /* 2/9 */
    t = bh_fmaf(t, s2, 2.85714285714285714e-01f); /* 2/7 */
    t = bh_fmaf(t, s2, 4.0e-01f);                 /* 2/5 */
    t = bh_fmaf(t, s2, 6.66666666666666667e-01f); /* 2/3 */
    float R = t * s2;
    float logm = f - s * (f - R);
    const float ln2_hi = 0.693145751953125f;
    const float ln2_lo = 1.428606765330187045e-06f;
    float ef = (float)e;
    return ef * ln2_hi + (ef * ln2_lo + logm);
}

/* The splat Gaussian e^-sigma, sigma = (c00 dx^2 + c11 dy^2) / 2 + c01 dx dy
 * (brush-cube/src/lib.rs:632-638, kernels/rasterize.rs), evaluated in base 2.
 * The conic is scaled once per splat (bh_conic_log2: a = c00 log2(e) / 2,
 * b = c01 log2(e), c = c11 log2(e) / 2), so a pixel's exponent
 * sigma log2(e) = dx (a dx + b dy) + (c dy) dy costs three products and
 * two fmas (bh_power_log2), and 2^-y needs no ln 2 reduction (bh_exp2_neg): with
 * n = rint(y) and f = y - n in [-1/2, 1/2] (exact), 2^f is a degree-5
 * polynomial fitted for least maximum relative error on [-1/2, 1/2]
 * (6.9e-8 before rounding, within 3 ulp of 2^f in float), scaled by 2^n.
 * Against e^-sigma of the unscaled power this differs by the rounding of the
 * scaled conic and exponent, a few ulp of the result; the blend, its replay
 * and the CPU restatement all evaluate alpha this way, so their decisions
 * agree bit for bit. */
BH_HD void bh_conic_log2(float c00, float c01, float c11, float* a, float* b, float* c) {
    const float half_log2e = 0.72134752044448170368f; /* log2(e) / 2 */
    const float log2e = 1.44269504088896340736f;
    *a = half_log2e * c00;
    *b = log2e * c01;
    *c = half_log2e * c11;
}

BH_HD float bh_power_log2(float a, float b, float c, float dx, float dy) {
    const float q = bh_fmaf(a, dx, b * dy);
    return bh_fmaf(dx, q, (c * dy) * dy);
}

/* 2^x for x in [-126, 1] (x = -power: the power is >= 0 where it is used,
 * up to rounding); below -200 the result is 0 and NaN stays NaN. */
BH_HD float bh_exp2_neg(float x) {
#if !defined(__HIPCC__)
    /* the CPU restatement never converts an out-of-range n (on the GPU the
     * conversion saturates and ldexp gives 0 for x < -200 as well) */
    if (!(x >= -200.0f)) return x == x ? 0.0f : x;
#endif
    const float n = bh_rintf(x);
    const float f = x - n;
    float p = 1.33523193e-03f;
    p = bh_fmaf(p, f, 9.67188086e-03f);
    p = bh_fmaf(p, f, 5.55045046e-02f);
    p = bh_fmaf(p, f, 2.40222305e-01f);
    p = bh_fmaf(p, f, 6.93147242e-01f);
    p = bh_fmaf(p, f, 1.0f);
    return bh_ldexpf(p, (int)n);
}

/* 1 / (1 + e^-x)  (brush-cube/src/lib.rs:620-623) */
BH_HD float bh_sigmoidf(float x) { return 1.0f / (1.0f + bh_expf(-x)); }

/* atan2 (the fisheye camera models' theta = atan2(r, z),
 * brush-render/src/kernels/camera_model/kannala_brandt_4.rs:38 and
 * project_forward.rs:55-62), IEEE special cases included. */
BH_HD float bh_atan2f(float y, float x) {
    if (!(x == x) || !(y == y)) return x + y;
    const int xneg = (int)(bh_as_uint(x) >> 31), yneg = (int)(bh_as_uint(y) >> 31);
    const float ax = bh_absf(x), ay = bh_absf(y);
    const float pi_hi = 3.14159274101257324f, pi_lo = -8.74227766e-08f;
    const float pi2_hi = 1.57079637050628662f, pi2_lo = -4.37113883e-08f;
    const float inf = bh_as_float(BH_INF_BITS);
    float a;
    if (ay == 0.0f) {
        a = xneg ? pi_hi : 0.0f;
    } else if (ax == 0.0f) {
        a = pi2_hi;
    } else if (ax == inf || ay == inf) {
        if (ax == inf && ay == inf) a = xneg ? 2.35619449615478516f : 0.785398185253143311f;
        else if (ay == inf) a = pi2_hi;
        else a = xneg ? pi_hi : 0.0f;
    } else {
        const int swap = ay > ax;
        const float t = swap ? ax / ay : ay / ax; /* [0, 1] */
        /* nearest centre c_k = tan(k pi / 12), atan(c_k) as hi + lo for the f32 c_k */
        float c = 0.0f, at_hi = 0.0f, at_lo = 0.0f;
        if (t > 0.767327011f) {
            c = 1.0f, at_hi = 0.785398185253143311f, at_lo = -2.18556941e-08f;
        } else if (t > 0.414213568f) {
            c = 0.577350259f, at_hi = 0.523598790168762207f, at_lo = -2.23422756e-08f;
        } else if (t > 0.131652504f) {
            c = 0.267949194f, at_hi = 0.261799395084381104f, at_lo = -6.08637896e-09f;
        }
        const float s = c == 0.0f ? t : (t - c) / bh_fmaf(t, c, 1.0f); /* |s| <= tan(pi/24) */
        const float z = s * s;
        float p = 7.69230769e-02f;               /* 1/13 */
        p = bh_fmaf(p, z, -9.09090909e-02f);     /* -1/11 */
        p = bh_fmaf(p, z, 1.11111111e-01f);      /* 1/9 */
        p = bh_fmaf(p, z, -1.42857143e-01f);     /* -1/7 */
        p = bh_fmaf(p, z, 2.0e-01f);             /* 1/5 */
        p = bh_fmaf(p, z, -3.33333333e-01f);     /* -1/3 */
        const float at = bh_fmaf(s * z, p, s);
        a = at_hi + (at + at_lo);
        if (swap) a = (pi2_hi - a) + pi2_lo;
        if (xneg) a = (pi_hi - a) + pi_lo;
    }
    return yneg ? -a : a;
}

#endif /* BH_MATH_H */
