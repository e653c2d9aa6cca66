// gelu_exact.h -- the reference's GELU bit for bit.
//
// fno.cpp:41-46 evaluates 0.5f * z * (1 + std::tanh(c * (z + 0.044715f z^3)))
// with glibc's tanhf; its build (g++ -O3 -mfma) fuses the last product of the
// cubic term with the addition.  glibc's float tanhf and expm1f are the
// fdlibm algorithms (s_tanhf.c, s_expm1f.c; notice below): tanhf from
// expm1f of 2|x|, expm1f by argument reduction x = k ln2 + r and a rational
// approximation in r^2 with the published coefficients below.  This
// restatement reproduces glibc 2.35's tanhf on every one of the 2^32 float
// inputs when each float operation is rounded on its own (-ffp-contract=off,
// correctly rounded division), which both the host build and the gfx950
// build of this library do.
//
// Usable from host code (the test harness) and device code.
//
// expm1f_fdlibm and tanhf_fdlibm below follow fdlibm's s_expm1f.c and
// s_tanhf.c (their thresholds, coefficients and control flow), which carry
// this notice:
//
// ====================================================
// Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//
// Developed at SunPro, a Sun Microsystems, Inc. business.
// Permission to use, copy, modify, and distribute this
// software is freely granted, provided that this notice
// is preserved.
// ====================================================
//
// (The float versions: conversion to float by Ian Lance Taylor, Cygnus
// Support, ian@cygnus.com.)
#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIP__)
#define NFQ_HD __host__ __device__
#else
#define NFQ_HD
#endif

namespace nfq {

NFQ_HD inline uint32_t gx_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}
NFQ_HD inline float gx_float(uint32_t u) {
    float x;
    memcpy(&x, &u, 4);
    return x;
}
NFQ_HD inline float gx_fabs(float x) { return gx_float(gx_bits(x) & 0x7fffffffu); }

// fdlibm expm1f: e^x - 1.
NFQ_HD inline float expm1f_fdlibm(float x) {
    const float o_threshold = 8.8721679688e+01f, ln2_hi = 6.9313812256e-01f,
                ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
                Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
    float hi, lo, c = 0.0f, t;
    int32_t k;
    uint32_t hx = gx_bits(x);
    const uint32_t xsb = hx & 0x80000000u;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) {                 // |x| >= 27 ln2
        if (hx >= 0x42b17218u) {             // |x| >= 88.72...
            if (hx > 0x7f800000u) return x + x;                  // NaN
            if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;  // +-Inf
            if (x > o_threshold) return gx_float(0x7f800000u);  // overflow
        }
        if (xsb != 0) return -1.0f;          // x < -27 ln2
    }
    if (hx > 0x3eb17218u) {                  // |x| > 0.5 ln2
        if (hx < 0x3F851592u) {              // and < 1.5 ln2
            if (xsb == 0) {
                hi = x - ln2_hi;
                lo = ln2_lo;
                k = 1;
            } else {
                hi = x + ln2_hi;
                lo = -ln2_lo;
                k = -1;
            }
        } else {
            k = static_cast<int32_t>(invln2 * x + ((xsb == 0) ? 0.5f : -0.5f));
            t = static_cast<float>(k);
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {           // |x| < 2^-25
        return x;
    } else {
        k = 0;
    }
    const float hfx = 0.5f * x;
    const float hxs = x * hfx;
    const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    t = 3.0f - r1 * hfx;
    float e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    const float twopk = gx_float(0x3f800000u + (static_cast<uint32_t>(k) << 23));
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return 1.0f + 2.0f * (x - e);
    }
    float y;
    if (k <= -2 || k > 56) {
        y = 1.0f - (e - x);
        if (k == 128)
            y = y * 2.0f * gx_float(0x7f000000u);
        else
            y = y * twopk;
        return y - 1.0f;
    }
    if (k < 23) {
        t = gx_float(0x3f800000u - (0x1000000u >> k));  // 1 - 2^-k
        y = t - (e - x);
        y = y * twopk;
    } else {
        t = gx_float(static_cast<uint32_t>(0x7f - k) << 23);  // 2^-k
        y = x - (e + t);
        y += 1.0f;
        y = y * twopk;
    }
    return y;
}

// fdlibm tanhf.
NFQ_HD inline float tanhf_fdlibm(float x) {
    const uint32_t jx = gx_bits(x), ix = jx & 0x7fffffffu;
    float z;
    if (ix >= 0x7f800000u) {                 // Inf or NaN
        return (jx & 0x80000000u) == 0 ? 1.0f / x + 1.0f : 1.0f / x - 1.0f;
    }
    if (ix < 0x41b00000u) {                  // |x| < 22
        if (ix == 0) return x;
        if (ix < 0x24000000u) return x * (1.0f + x);  // |x| < 2^-55
        if (ix >= 0x3f800000u) {             // |x| >= 1
            const float t = expm1f_fdlibm(2.0f * gx_fabs(x));
            z = 1.0f - 2.0f / (t + 2.0f);
        } else {
            const float t = expm1f_fdlibm(-2.0f * gx_fabs(x));
            z = -t / (t + 2.0f);
        }
    } else {
        z = 1.0f;                            // 1 - tiny rounds to 1
    }
    return (jx & 0x80000000u) == 0 ? z : -z;
}

// The same tanhf as straight-line code: every branch's value is computed and
// the one the branchy form would return is selected, so a wave whose lanes
// take different branches pays for one evaluation instead of several.  Only
// +-Inf / NaN branch (a division the common path does not need).  Bit-exact
// with tanhf_fdlibm on every input (checked on the host).
NFQ_HD inline float tanhf_fdlibm_select(float x) {
    const uint32_t jx = gx_bits(x), ix = jx & 0x7fffffffu;
    if (ix >= 0x7f800000u) return (jx & 0x80000000u) == 0 ? 1.0f / x + 1.0f : 1.0f / x - 1.0f;
    const bool big = ix >= 0x3f800000u;      // |x| >= 1
    const float ax = gx_fabs(x);
    // expm1f_fdlibm(a) for a = 2|x| (|x| >= 1) or -2|x|; a is then within
    // (-2, 0] or [2, 44), so only the reduction paths below occur (|x| >= 22
    // is replaced by 1 afterwards).
    const float a = big ? 2.0f * ax : -2.0f * ax;
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
                Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
    const uint32_t ha = gx_bits(a) & 0x7fffffffu;
    const bool neg = (gx_bits(a) & 0x80000000u) != 0;
    const bool reduce = ha > 0x3eb17218u;
    const bool near1 = ha < 0x3F851592u;
    const int32_t kg = static_cast<int32_t>(invln2 * a + (neg ? -0.5f : 0.5f));
    const float tg = static_cast<float>(kg);
    const float hi = near1 ? (neg ? a + ln2_hi : a - ln2_hi) : a - tg * ln2_hi;
    const float lo = near1 ? (neg ? -ln2_lo : ln2_lo) : tg * ln2_lo;
    const int32_t k = reduce ? (near1 ? (neg ? -1 : 1) : kg) : 0;
    const float xr = reduce ? hi - lo : a;
    const float c = reduce ? (hi - xr) - lo : 0.0f;
    const float hfx = 0.5f * xr;
    const float hxs = xr * hfx;
    const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    const float tt = 3.0f - r1 * hfx;
    const float e0 = hxs * ((r1 - tt) / (6.0f - xr * tt));
    const float res_k0 = xr - (xr * e0 - hxs);
    float e = (xr * (e0 - c) - c);
    e -= hxs;
    const float res_km1 = 0.5f * (xr - e) - 0.5f;
    const float res_k1 = (xr < -0.25f) ? -2.0f * (e - (xr + 0.5f)) : 1.0f + 2.0f * (xr - e);
    const float twopk = gx_float(0x3f800000u + (static_cast<uint32_t>(k) << 23));
    const float res_far = (1.0f - (e - xr)) * twopk - 1.0f;              // k <= -2 or k > 56 (k < 128 here)
    const int kc = k < 0 ? 0 : (k > 31 ? 31 : k);
    const float res_mid = (gx_float(0x3f800000u - (0x1000000u >> kc)) - (e - xr)) * twopk;  // 2 <= k < 23
    const float res_hi = ((xr - (e + gx_float(static_cast<uint32_t>(0x7f - (k > 0x7f ? 0x7f : k)) << 23))) +
                          1.0f) * twopk;                                   // 23 <= k <= 56
    float t = k == 0 ? res_k0
            : k == -1 ? res_km1
            : k == 1 ? res_k1
            : (k <= -2 || k > 56) ? res_far
            : k < 23 ? res_mid : res_hi;
    if (ha < 0x33000000u) t = a;             // |a| < 2^-25: expm1 returns a
    const float q = (big ? 2.0f : -t) / (t + 2.0f);
    float z = big ? 1.0f - q : q;
    if (ix >= 0x41b00000u) z = 1.0f;         // |x| >= 22
    z = (jx & 0x80000000u) == 0 ? z : -z;
    return ix < 0x24000000u ? x * (1.0f + x) : z;   // |x| < 2^-55 (and +-0)
}

#if defined(__HIP__)
// n / d for the two quotients of the tanhf below, where both operands and
// the quotient are normal: r = v_rcp_f32(d) (within 1 ulp of 1/d), q = n r,
// then q + (n - d q) r with the residual n - d q exact by FMA.  REFINE = 1
// first takes r + (1 - d r) r.  Whether this rounds as n / d does on every
// argument the tanhf passes is what the exhaustive device check measures
// (tests/native/gelu_device_check.hip).
template <int REFINE>
__device__ inline float div_rcp_step(float n, float d) {
    float r = __builtin_amdgcn_rcpf(d);
    if (REFINE) r = __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
    const float q = n * r;
    return __builtin_fmaf(__builtin_fmaf(-d, q, n), r, q);
}

// tanhf_fdlibm_select with the branches its argument ranges leave out
// removed and the two common-path divisions as div_rcp_step: the expm1f
// argument a is 2|x| >= 2 or -2|x| in (-2, 0], so k = 1 (0.35 < a < 1.04)
// never occurs and the k = -1 reduction only for a < 0.  The +-Inf / NaN
// branch keeps the IEEE division.
template <int REFINE>
__device__ inline float tanhf_fdlibm_fast(float x) {
    const uint32_t jx = gx_bits(x), ix = jx & 0x7fffffffu;
    if (ix >= 0x7f800000u) return (jx & 0x80000000u) == 0 ? 1.0f / x + 1.0f : 1.0f / x - 1.0f;
    const bool big = ix >= 0x3f800000u;      // |x| >= 1: a >= 2; else a <= 0
    const float ax = gx_fabs(x);
    const float a = big ? 2.0f * ax : -2.0f * ax;
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
                Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
    const uint32_t ha = gx_bits(a) & 0x7fffffffu;
    const bool reduce = ha > 0x3eb17218u;
    const bool near1 = ha < 0x3F851592u;     // (a < 0 whenever it holds)
    const int32_t kg = static_cast<int32_t>(invln2 * a + (big ? 0.5f : -0.5f));
    const float tg = static_cast<float>(kg);
    const float hi = near1 ? a + ln2_hi : a - tg * ln2_hi;
    const float lo = near1 ? -ln2_lo : tg * ln2_lo;
    const int32_t k = reduce ? (near1 ? -1 : kg) : 0;
    const float xr = reduce ? hi - lo : a;
    const float c = reduce ? (hi - xr) - lo : 0.0f;
    const float hfx = 0.5f * xr;
    const float hxs = xr * hfx;
    const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    const float tt = 3.0f - r1 * hfx;
    const float e0 = hxs * div_rcp_step<REFINE>(r1 - tt, 6.0f - xr * tt);
    const float res_k0 = xr - (xr * e0 - hxs);
    float e = (xr * (e0 - c) - c);
    e -= hxs;
    const float res_km1 = 0.5f * (xr - e) - 0.5f;
    const float twopk = gx_float(0x3f800000u + (static_cast<uint32_t>(k) << 23));
    const float res_far = (1.0f - (e - xr)) * twopk - 1.0f;              // k = -2, -3 or k > 56
    const int kc = k < 0 ? 0 : (k > 31 ? 31 : k);
    const float res_mid = (gx_float(0x3f800000u - (0x1000000u >> kc)) - (e - xr)) * twopk;  // 3 <= k < 23
    const float res_hi = ((xr - (e + gx_float(static_cast<uint32_t>(0x7f - (k > 0x7f ? 0x7f : k)) << 23))) +
                          1.0f) * twopk;                                   // 23 <= k <= 56
    float t = k == 0 ? res_k0
            : k == -1 ? res_km1
            : (k < 0 || k > 56) ? res_far
            : k < 23 ? res_mid : res_hi;
    if (ha < 0x33000000u) t = a;             // |a| < 2^-25: expm1 returns a
    const float q = div_rcp_step<REFINE>(big ? 2.0f : -t, t + 2.0f);
    float z = big ? 1.0f - q : q;
    if (ix >= 0x41b00000u) z = 1.0f;         // |x| >= 22
    z = (jx & 0x80000000u) == 0 ? z : -z;
    return ix < 0x24000000u ? x * (1.0f + x) : z;   // |x| < 2^-55 (and +-0)
}
#endif

// c = std::sqrt(2.0f / static_cast<float>(M_PI)) (fno.cpp:42).
constexpr float kGeluC = 0x1.988452p-1f;

// fno.cpp:41-46 as the reference build computes it.
NFQ_HD inline float gelu_ref(float z) {
    const float inner = __builtin_fmaf((0.044715f * z) * z, z, z);
    return (0.5f * z) * (1.0f + tanhf_fdlibm_select(kGeluC * inner));
}

#if defined(__HIP__)
// gelu_ref over tanhf_fdlibm_fast: the form the device kernels run.  Equal
// to gelu_ref on all 2^32 inputs on gfx950 for the REFINE the kernels use
// (tests/test_gpu_gelu_device.py counts the differences on the device).
template <int REFINE>
__device__ inline float gelu_fast(float z) {
    const float inner = __builtin_fmaf((0.044715f * z) * z, z, z);
    return (0.5f * z) * (1.0f + tanhf_fdlibm_fast<REFINE>(kGeluC * inner));
}
constexpr int kGeluRefine = 0;
#endif

}  // namespace nfq
