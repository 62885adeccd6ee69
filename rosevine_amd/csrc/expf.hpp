// expf.hpp - the C library expf of the reference's hosts, restated for the device.
//
// Rust's f32::exp is the platform expf. glibc (2.28 and later; the reference's hosts run 2.35)
// computes it with Szabolcs Nagy's method from ARM's optimized-routines (glibc
// sysdeps/ieee754/flt-32/e_expf.c, e_exp2f_data.c): x * 32/ln2 = k + r with k an integer (rounded
// by adding 1.5 * 2^52), exp(x) = 2^(k/32) * 2^(r/32), where 2^(k/32) is the correctly rounded
// double 2^((k mod 32)/32) with k/32 added to its exponent field, and 2^(r/32) - 1 is a cubic in r
// (minimax coefficients published with the method); everything in double, one rounding to float.
// On x86-64 hosts with FMA (every host the reference targets) glibc selects its FMA build, in which
// the reduction (k and r) and the three polynomial steps are fused multiply-adds; glibc_expf uses
// the same fused operations. It equals the host libm's expf on every negative f32 input (all 2^31
// swept: the softmax only exponentiates x - max <= 0); tests/test_expf_restatement.py compiles
// this header for the host and checks a sample of all inputs on every run. The 32 table entries
// are the correctly rounded doubles of 2^(i/32) minus i << 47 (checked in that test from the
// mathematics).
// No HIP headers here, so that the host compiler can include it on its own.
//
// Notice of the restated method and its constants (Arm optimized-routines math/expf.c and
// math/exp2f_data.c, by Szabolcs Nagy, which glibc ships as e_expf.c and e_exp2f_data.c):
//   Copyright (c) 2017-2018, Arm Limited.
//   SPDX-License-Identifier: MIT OR Apache-2.0 WITH LLVM-exception
#pragma once
#include <math.h>
#include <stdint.h>

#ifdef __HIPCC__
#define RVM_HD __host__ __device__
#else
#define RVM_HD
#endif

namespace rvm {

RVM_HD inline uint64_t exp2f_table(int i) {
    constexpr uint64_t T[32] = {
        0x3ff0000000000000, 0x3fefd9b0d3158574, 0x3fefb5586cf9890f, 0x3fef9301d0125b51,
        0x3fef72b83c7d517b, 0x3fef54873168b9aa, 0x3fef387a6e756238, 0x3fef1e9df51fdee1,
        0x3fef06fe0a31b715, 0x3feef1a7373aa9cb, 0x3feedea64c123422, 0x3feece086061892d,
        0x3feebfdad5362a27, 0x3feeb42b569d4f82, 0x3feeab07dd485429, 0x3feea47eb03a5585,
        0x3feea09e667f3bcd, 0x3fee9f75e8ec5f74, 0x3feea11473eb0187, 0x3feea589994cce13,
        0x3feeace5422aa0db, 0x3feeb737b0cdc5e5, 0x3feec49182a3f090, 0x3feed503b23e255d,
        0x3feee89f995ad3ad, 0x3feeff76f2fb5e47, 0x3fef199bdd85529c, 0x3fef3720dcef9069,
        0x3fef5818dcfba487, 0x3fef7c97337b9b5f, 0x3fefa4afa2a490da, 0x3fefd0765b6e4540};
    return T[i & 31];
}

RVM_HD inline float glibc_expf(float x) {
    const uint32_t ix = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ix >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88, or x is NaN
        if (ix == 0xff800000u) return 0.0f;                 // -inf
        if (abstop >= 0x7f8u) return x + x;                 // +inf, NaN
        if (x > 0x1.62e42ep6f) return __builtin_huge_valf();  // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;                // below log(2^-150): underflow to 0
        if (x < -0x1.9d1d9ep6f) return 0x1p-149f;           // below log(2^-149): the smallest subnormal
    }
    const double xd = (double)x, inv = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    double kd = fma(inv, xd, shift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = fma(inv, xd, -kd);
    const double s = __builtin_bit_cast(double, exp2f_table((int)(ki & 31)) + (ki << 47));
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double z = fma(c0, r, c1), r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return (float)y;
}

}  // namespace rvm
