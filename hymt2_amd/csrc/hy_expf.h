// hy_expf: expf with results identical to glibc's. Plain C++ so the same code compiles for the
// GPU (included by hy_common.h) and for host-side tests (compiled with g++).
#pragma once

#include <stdint.h>

#ifndef HY_HD
#if defined(__HIPCC__)
#define HY_HD __host__ __device__
#else
#define HY_HD
#endif
#endif

// expf with results identical to glibc 2.35's x86-64 expf (the FMA variant selected on CPUs
// with FMA), which the reference calls for softmax and SiLU (src/model.c:787, :875). It
// restates the published method of ARM's optimized-routines exp2f/expf (Szabolcs Nagy, 2017;
// adopted by glibc): x*N/ln2 = k + r with N = 32, 2^(k/N) from a 32-entry table with the
// exponent folded in, and a cubic in r evaluated in double precision, rounded once to float.
// The table entries are 2^(i/32) correctly rounded to double, minus i<<47. The FMA placement
// matches glibc's FMA build exactly: checked against the host libm on every float in
// [-105, 90] (tests/test_expf.py), and on the device against libm in the GPU tests.
//
// Attribution: the method, the table layout and the polynomial coefficients below are those of
// Arm's optimized-routines, math/expf.c and math/exp2f_data.c, Copyright (c) 2017-2018 Arm
// Limited, SPDX-License-Identifier: MIT OR Apache-2.0 WITH LLVM-exception; the same routine
// ships in glibc as sysdeps/ieee754/flt-32/e_expf.c and e_exp2f_data.c (LGPL-2.1-or-later,
// contributed by Arm). The code here is written for this file; only the numbers must be equal.
// The 32 table entries (2^(i/32) correctly rounded to double, minus i << 47).
#define HY_EXP2F_TABLE \
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull

// expf with the table T[32] supplied by the caller (GPU kernels pass a copy in LDS, so that a
// lookup is an LDS read rather than a load from global memory on the critical path).
HY_HD inline float hy_expf_tab(float x, const uint64_t* T) {
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
    constexpr double kShift = 0x1.8p+52;
    constexpr double kC0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88, inf or nan
        if (ux == 0xff800000u) return 0.f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.f;
    }
    const double xd = (double)x;
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    const uint64_t t = T[ki & 31u] + (ki << 47);
    const double s = __builtin_bit_cast(double, t);
    const double z = __builtin_fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

HY_HD inline float hy_expf(float x) {
    constexpr uint64_t T[32] = {HY_EXP2F_TABLE};
    return hy_expf_tab(x, T);
}

