// tanhf.hpp - the C library tanhf of the reference's hosts, restated for the device.
//
// Rust's f32::tanh is the platform tanhf; on the reference's Linux hosts (glibc 2.35) that is the
// fdlibm algorithm (Sun Microsystems; glibc sysdeps/ieee754/flt-32/s_tanhf.c and s_expm1f.c).
// fb_expm1f / fb_tanhf below are that published algorithm with the same single-precision
// operations; tanhf_select evaluates the same operations without branches. Both equal glibc's
// tanhf on every f32 input (swept over all 2^32 inputs; tests/test_tanhf_restatement.py compiles
// this header for the host and checks a sample against the host libm on every run).
// No HIP headers here, so that the host compiler can include it on its own.
//
// Notice of the restated algorithm and its constants (fdlibm s_tanhf.c and s_expm1f.c, as glibc
// ships them):
//   Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//   Developed at SunPro, a Sun Microsystems, Inc. business.
//   Permission to use, copy, modify, and distribute this software is freely granted, provided
//   that this notice is preserved.
#pragma once
#include <math.h>
#include <stdint.h>

#ifdef __HIPCC__
#define RVM_HD __host__ __device__
#else
#define RVM_HD
#endif

namespace rvm {

RVM_HD inline float fb_expm1f(float x) {
    const float one = 1.0f, huge = 1.0e+30f, tiny = 1.0e-30f;
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
                Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
    float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
    int32_t k;
    uint32_t hx = __builtin_bit_cast(uint32_t, x);
    const uint32_t xsb = hx & 0x80000000u;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) {  // |x| >= 27 ln2
        if (hx >= 0x42b17218u) {
            if (hx > 0x7f800000u) return x + x;
            if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;
            if (xsb == 0 && hx > 0x42b17217u) return huge * huge;
        }
        if (xsb != 0) return tiny - one;
    }
    if (hx > 0x3eb17218u) {  // |x| > ln2 / 2: argument reduction
        if (hx < 0x3F851592u) {
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
            k = (int32_t)(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
            t = (float)k;
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {  // |x| < 2^-25
        t = huge + x;
        return x - (t - (huge + x));
    } else {
        k = 0;
    }
    hfx = 0.5f * x;
    hxs = x * hfx;
    r1 = one + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    t = 3.0f - r1 * hfx;
    e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) return x < -0.25f ? -2.0f * (e - (x + 0.5f)) : one + 2.0f * (x - e);
    if (k <= -2 || k > 56) {
        y = one - (e - x);
        y = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, y) + ((uint32_t)k << 23));
        return y - one;
    }
    if (k < 23) {
        t = __builtin_bit_cast(float, 0x3f800000u - (0x1000000u >> k));
        y = t - (e - x);
        y = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, y) + ((uint32_t)k << 23));
    } else {
        t = __builtin_bit_cast(float, (uint32_t)(0x7f - k) << 23);
        y = x - (e + t);
        y += one;
        y = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, y) + ((uint32_t)k << 23));
    }
    return y;
}

RVM_HD inline float fb_tanhf(float x) {
    const float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
    float t, z;
    const int32_t jx = __builtin_bit_cast(int32_t, x);
    const int32_t ix = jx & 0x7fffffff;
    if (ix >= 0x7f800000) return jx >= 0 ? one / x + one : one / x - one;
    if (ix < 0x41b00000) {  // |x| < 22
        if (ix == 0) return x;
        if (ix < 0x24000000) return x * (one + x);  // |x| < 2^-55
        if (ix >= 0x3f800000) {
            t = fb_expm1f(two * fabsf(x));
            z = one - two / (t + two);
        } else {
            t = fb_expm1f(-two * fabsf(x));
            z = -t / (t + two);
        }
    } else {
        z = one - tiny;
    }
    return jx >= 0 ? z : -z;
}

// fb_tanhf without branches: every case of fb_tanhf and of the fb_expm1f call it makes is
// evaluated with the same operations and the result is selected, so that a wave whose lanes take
// different cases runs one straight sequence (one expm1f core and two divisions) instead of every
// path in turn. Equal to fb_tanhf bit for bit on every f32 input (the CPU tests compare them).
RVM_HD inline float tanhf_select(float x) {
    const float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
                Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
    const int32_t jx = __builtin_bit_cast(int32_t, x);
    const int32_t ix = jx & 0x7fffffff;
    const bool big = ix >= 0x3f800000;  // |x| >= 1: z = 1 - 2 / (expm1(2|x|) + 2)
    const bool mid = ix >= 0x24000000 && ix < 0x41b00000;  // the range that calls expm1f
    // expm1f(a) with a = +-2|x| (|a| < 44); out-of-range lanes use a = 1
    const float a = mid ? (big ? two * fabsf(x) : -two * fabsf(x)) : 1.0f;
    const uint32_t ha = __builtin_bit_cast(uint32_t, a) & 0x7fffffffu;
    const bool neg = a < 0.0f;
    const bool sat = ha >= 0x4195b844u && neg;  // a <= -27 ln2: expm1f returns tiny - one
    const bool red = ha > 0x3eb17218u;          // |a| > ln2 / 2: argument reduction
    const bool near = ha < 0x3F851592u;         // |a| < 1.5 ln2: k = +-1
    const bool tiny_a = ha < 0x33000000u;       // |a| < 2^-25: expm1f returns a
    const int32_t kf = (int32_t)(invln2 * a + (neg ? -0.5f : 0.5f));
    const float tk = (float)kf;
    const float hi_far = a - tk * ln2_hi, lo_far = tk * ln2_lo;
    const float hi_near = neg ? a + ln2_hi : a - ln2_hi, lo_near = neg ? -ln2_lo : ln2_lo;
    const float hi = near ? hi_near : hi_far, lo = near ? lo_near : lo_far;
    const int32_t kr = near ? (neg ? -1 : 1) : kf;
    const float xr_red = hi - lo;
    const float c_red = (hi - xr_red) - lo;
    const float xr = red ? xr_red : a, c = red ? c_red : 0.0f;
    const int32_t k = red ? kr : 0;
    const float hfx = 0.5f * xr;
    const float hxs = xr * hfx;
    const float r1 = one + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    const float t = 3.0f - r1 * hfx;
    float e = hxs * ((r1 - t) / (6.0f - xr * t));
    const float res_k0 = xr - (xr * e - hxs);
    e = (xr * (e - c) - c);
    e -= hxs;
    const float res_km1 = 0.5f * (xr - e) - 0.5f;
    const float res_k1 = xr < -0.25f ? -2.0f * (e - (xr + 0.5f)) : one + 2.0f * (xr - e);
    const uint32_t kbits = (uint32_t)k << 23;
    const float yb = one - (e - xr);
    const float res_out = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, yb) + kbits) - one;
    const int32_t kc = k < 0 ? 0 : (k > 31 ? 31 : k);
    const float t1 = __builtin_bit_cast(float, 0x3f800000u - (0x1000000u >> kc));
    const float y1 = t1 - (e - xr);
    const float res_lo = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, y1) + kbits);
    const float t2 = __builtin_bit_cast(float, (uint32_t)(0x7f - (k > 127 ? 127 : k)) << 23);
    float y2 = xr - (e + t2);
    y2 += one;
    const float res_hi = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, y2) + kbits);
    float em = k == 0 ? res_k0
               : k == -1 ? res_km1
               : k == 1 ? res_k1
               : (k <= -2 || k > 56) ? res_out
               : k < 23 ? res_lo : res_hi;
    em = sat ? tiny - one : (tiny_a ? a : em);
    // tanhf from t = expm1f(a): one division for both signs of the branch
    const float q = (big ? two : -em) / (em + two);
    float z = big ? one - q : q;
    z = ix >= 0x41b00000 ? one - tiny : z;
    float r = jx >= 0 ? z : -z;
    r = ix < 0x24000000 ? x * (one + x) : r;  // |x| < 2^-55, and +-0
    r = ix >= 0x7f800000 ? (ix > 0x7f800000 ? x + x : (jx >= 0 ? one : -one)) : r;
    return r;
}

}  // namespace rvm
