// Bit-exact fp32 transcendentals and order keys for the sampling kernels.
//
// The reference sampler calls glibc's tanhf (softcap, src/generation.cpp:434)
// and expf (softmax, src/generation.cpp:97) through std::tanh / std::exp on
// float. Token ids depend on those exact roundings (about 5% of fp32 inputs
// in [0, 32) have a glibc tanhf result that differs from the correctly
// rounded one), so the device restates the published algorithms glibc 2.35
// uses on x86-64 rather than calling a device libm:
//
//   tanhf  — fdlibm s_tanhf.c (Sun Microsystems, 1993), as shipped in
//            glibc 2.35 sysdeps/ieee754/flt-32/s_tanhf.c:
//            |x| >= 1: 1 - 2 / (expm1(2|x|) + 2); else -t / (t + 2),
//            t = expm1(-2|x|); |x| >= 22 -> +-1.
//   expm1f — fdlibm s_expm1f.c (glibc flt-32/s_expm1f.c): argument reduction
//            by ln2 (hi/lo split), the 5-term rational correction Q1..Q5.
//   expf   — the ARM optimized-routines algorithm (Szabolcs Nagy, 2017) used
//            by glibc 2.27+ sysdeps/ieee754/flt-32/e_expf.c: x*N/ln2 = k + r,
//            N = 32, 2^(k/N) from a 32-entry table, degree-3 polynomial in
//            double, one rounding to float. glibc dispatches the FMA build of
//            it on FMA-capable x86-64 hosts, so the reduction and polynomial
//            below use fused multiply-adds exactly where that build does.
//
// The 32-entry table holds, for entry i, the bits of the IEEE double nearest
// 2^(i/32) minus (i << 47); tests/test_math.py recomputes every entry from
// 2^(i/32) in 60-digit decimal arithmetic. tests/test_math.py also checks
// every fp32 input of both functions against the host's glibc (this header
// compiled for the host by tests/cpp/math_check.hip) and digests of the
// device build's outputs on the GPU.
//
// Every function here is evaluated with floating-point contraction off; the
// fused operations are explicit fma() calls.
//
// Notices of the published sources whose algorithms and constants the
// tanhf / expm1f and expf restatements follow:
//
//   fdlibm s_tanhf.c, s_expm1f.c (float conversion by Ian Lance Taylor,
//   Cygnus Support):
//   ====================================================
//   Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//
//   Developed at SunPro, a Sun Microsystems, Inc. business.
//   Permission to use, copy, modify, and distribute this
//   software is freely granted, provided that this notice
//   is preserved.
//   ====================================================
//
//   ARM optimized-routines math/expf.c:
//   Copyright (c) 2017-2019, Arm Limited.
//   SPDX-License-Identifier: MIT
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace ge {

__host__ __device__ inline uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
__host__ __device__ inline uint64_t d2u(double d) { return __builtin_bit_cast(uint64_t, d); }
__host__ __device__ inline double u2d(uint64_t u) { return __builtin_bit_cast(double, u); }

// src/tensor.cpp:226-231: bf16 widens exactly by a 16-bit shift.
__host__ __device__ inline float bf16_to_f32(uint16_t b) { return u2f(static_cast<uint32_t>(b) << 16); }

// fdlibm expm1f, float arithmetic throughout.
__host__ __device__ inline float expm1f_fdlibm(float x) {
    const float one = 1.0f;
    const float ln2_hi = u2f(0x3f317180u);  // 6.9313812256e-01
    const float ln2_lo = u2f(0x3717f7d1u);  // 9.0580006145e-06
    const float invln2 = u2f(0x3fb8aa3bu);  // 1.4426950216e+00
    const float o_threshold = u2f(0x42b17180u);
    const float Q1 = u2f(0xbd088889u), Q2 = u2f(0x3ad00d01u), Q3 = u2f(0xb8a670cdu),
                Q4 = u2f(0x36867e54u), Q5 = u2f(0xb457edbbu);
    float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
    int32_t k;
    uint32_t hx = f2u(x);
    const uint32_t xsb = hx & 0x80000000u;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) {          // |x| >= 27 ln2
        if (hx >= 0x42b17218u) {      // |x| >= 88.72
            if (hx > 0x7f800000u) return x + x;                 // NaN
            if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;  // +-inf
            if (x > o_threshold) return u2f(0x7f800000u);        // overflow
        }
        if (xsb != 0) return 1.0e-30f - one;  // x < -27 ln2: -1 (inexact)
    }
    if (hx > 0x3eb17218u) {           // |x| > 0.5 ln2
        if (hx < 0x3F851592u) {       // and < 1.5 ln2
            if (xsb == 0) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
            else          { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
        } else {
            k = static_cast<int32_t>(invln2 * x + ((xsb == 0) ? 0.5f : -0.5f));
            t = static_cast<float>(k);
            hi = x - t * ln2_hi;      // exact
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {    // |x| < 2^-25
        return x;
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
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return one + 2.0f * (x - e);
    }
    if (k <= -2 || k > 56) {          // exp(x) - 1 ~ exp(x)
        y = one - (e - x);
        if (k == 128) y = y * 2.0f * u2f(0x7f000000u);
        else y = u2f(f2u(y) + (static_cast<uint32_t>(k) << 23));
        return y - one;
    }
    if (k < 23) {
        t = u2f(0x3f800000u - (0x1000000u >> k));  // 1 - 2^-k
        y = t - (e - x);
        y = u2f(f2u(y) + (static_cast<uint32_t>(k) << 23));
    } else {
        t = u2f(static_cast<uint32_t>(0x7f - k) << 23);  // 2^-k
        y = x - (e + t);
        y += one;
        y = u2f(f2u(y) + (static_cast<uint32_t>(k) << 23));
    }
    return y;
}

// fdlibm expm1f restricted to the arguments tanhf gives it, y = +-2|x| with
// 2^-55 <= |x| < 22, and written without branches: every case of
// expm1f_fdlibm is computed and the result selected, so a wave whose lanes
// take different cases runs the code once. The operations and their order
// are those of expm1f_fdlibm case by case:
//   * the argument reduction with k = +-1 (|y| in (ln2/2, 3 ln2/2)) uses
//     hi = y -+ ln2_hi, lo = +-ln2_lo; the general form y - t*ln2_hi, t*ln2_lo
//     with t = k = +-1 computes the same values (t*ln2_hi and t*ln2_lo are
//     exact), and with t = 0 it leaves y and c = 0 as the k = 0 case does;
//   * |y| < 2^-25 returns y; the overflow and y <= -27 ln2 cases cannot occur.
__host__ __device__ inline float expm1f_tanh(float y) {
    const float one = 1.0f;
    const float ln2_hi = u2f(0x3f317180u);
    const float ln2_lo = u2f(0x3717f7d1u);
    const float invln2 = u2f(0x3fb8aa3bu);
    const float Q1 = u2f(0xbd088889u), Q2 = u2f(0x3ad00d01u), Q3 = u2f(0xb8a670cdu),
                Q4 = u2f(0x36867e54u), Q5 = u2f(0xb457edbbu);
    const uint32_t hy = f2u(y);
    const bool neg = (hy & 0x80000000u) != 0u;
    const uint32_t hx = hy & 0x7fffffffu;
    const int32_t kg = static_cast<int32_t>(invln2 * y + (neg ? -0.5f : 0.5f));
    const int32_t k = hx <= 0x3eb17218u ? 0 : (hx < 0x3F851592u ? (neg ? -1 : 1) : kg);
    const float t = static_cast<float>(k);
    const float hi = y - t * ln2_hi;
    const float lo = t * ln2_lo;
    const float x = hi - lo;
    const float c = (hi - x) - lo;
    const float hfx = 0.5f * x;
    const float hxs = x * hfx;
    const float r1 = one + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    const float tt = 3.0f - r1 * hfx;
    const float e0 = hxs * ((r1 - tt) / (6.0f - x * tt));
    const float res0 = x - (x * e0 - hxs);                    // k == 0
    const float e = (x * (e0 - c) - c) - hxs;
    const float resm1 = 0.5f * (x - e) - 0.5f;                // k == -1
    const float resp1 = x < -0.25f ? -2.0f * (e - (x + 0.5f)) : one + 2.0f * (x - e);  // k == 1
    const uint32_t k23 = static_cast<uint32_t>(k) << 23;
    const float yb = u2f(f2u(one - (e - x)) + k23) - one;    // k <= -2 or k > 56
    const int ks = k < 0 ? 0 : (k > 31 ? 31 : k);            // shift counts used only where valid
    const float ys = u2f(f2u(u2f(0x3f800000u - (0x1000000u >> ks)) - (e - x)) + k23);  // 2 <= k < 23
    const float yl = u2f(f2u((x - (e + u2f(static_cast<uint32_t>(0x7f - k) << 23))) + one) + k23);  // 23 <= k <= 56
    float r = yl;
    if (k < 23) r = ys;
    if (k <= -2 || k > 56) r = yb;
    if (k == 1) r = resp1;
    if (k == -1) r = resm1;
    if (k == 0) r = res0;
    if (hx < 0x33000000u) r = y;                              // |y| < 2^-25
    return r;
}

// fdlibm tanhf, with the two expm1f calls merged into one on a selected
// argument and the two divisions into one on a selected numerator (the
// quotient 2/(t+2) or -t/(t+2) is the same single rounding either way).
__host__ __device__ inline float tanhf_fdlibm(float x) {
    const uint32_t jx = f2u(x);
    const uint32_t ix = jx & 0x7fffffffu;
    if (ix >= 0x7f800000u) {          // inf or NaN
        if ((jx >> 31) == 0) return 1.0f / x + 1.0f;
        return 1.0f / x - 1.0f;
    }
    // |x| >= 22 returns +-1 below; its expm1 argument is replaced by one in
    // range (the value is discarded) so the conversions stay defined.
    const float ax = ix >= 0x41b00000u ? 1.0f : u2f(ix);
    const bool big = ax >= 1.0f;                              // |x| >= 1
    const float t = expm1f_tanh(big ? 2.0f * ax : -2.0f * ax);
    const float q = (big ? 2.0f : -t) / (t + 2.0f);
    float z = big ? 1.0f - q : q;
    if (ix >= 0x41b00000u) z = 1.0f - 1.0e-30f;               // |x| >= 22: +-1
    z = (jx >> 31) ? -z : z;
    if (ix < 0x24000000u) z = x * (1.0f + x);                 // |x| < 2^-55 (and +-0)
    return z;
}

// 2^(i/32) nearest double, minus (i << 47) in the bit pattern.
#define GE_EXP2_TABLE                                                                  \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

static const uint64_t kExp2TableHost[32] = GE_EXP2_TABLE;

__host__ __device__ inline uint64_t exp2_table(uint32_t i) {
#if defined(__HIP_DEVICE_COMPILE__)
    // A local constant array: addressed PC-relative, with no load of its
    // address first (a __constant__ variable is reached through the GOT).
    static constexpr uint64_t kTab[32] = GE_EXP2_TABLE;
    return kTab[i];
#else
    return kExp2TableHost[i];
#endif
}

// ARM optimized-routines expf (glibc e_expf.c, FMA build).
// `tab(i)` returns table entry i: the constant table, or a copy of it that a
// kernel staged in LDS (same bits).
template <typename Tab>
__host__ __device__ inline float expf_glibc_tab(float x, Tab&& tab) {
    const double kInvLn2N = 0x1.71547652b82fep+5;  // 32 / ln2
    const double kShift = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-20;       // poly / N^3, N^2, N
    const double C1 = 0x1.ebfce50fac4f3p-13;
    const double C2 = 0x1.62e42ff0c52d6p-6;
    const uint32_t ux = f2u(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                         // |x| >= 88 or NaN
        if (ux == 0xff800000u) return 0.0f;         // -inf
        if (abstop >= 0x7f8u) return x + x;         // +inf or NaN
        if (x > u2f(0x42b17217u)) return u2f(0x7f800000u);  // > log(2^128)
        if (x < u2f(0xc2cff1b4u)) return 0.0f;      // < log(2^-150)
    }
    const double xd = static_cast<double>(x);
    double kd = fma(kInvLn2N, xd, kShift);          // round(x*N/ln2) in the low bits
    const uint64_t ki = d2u(kd);
    kd -= kShift;
    const double r = fma(kInvLn2N, xd, -kd);
    uint64_t t = tab(static_cast<uint32_t>(ki % 32));
    t += ki << 47;
    const double s = u2d(t);
    const double z = fma(C0, r, C1);
    const double r2 = r * r;
    double y = fma(C2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return static_cast<float>(y);
}

__host__ __device__ inline float expf_glibc(float x) {
    return expf_glibc_tab(x, [](uint32_t i) { return exp2_table(i); });
}

// Final-logit softcap, src/generation.cpp:431-437: c * tanh(l / c) when c > 0.
__host__ __device__ inline float softcap(float l, float c) {
    return (c > 0.0f) ? c * tanhf_fdlibm(l / c) : l;
}

// Repetition penalty (CTRL rule): v > 0 ? v / r : v * r.
__host__ __device__ inline float penalize(float v, float r) { return v > 0.0f ? v / r : v * r; }

// Order key: larger key <=> larger value; -0 and +0 share a key; NaN maps to
// kKeyNaN, below every number. Key 0 marks "not a candidate".
constexpr uint32_t kKeyNone = 0u;
constexpr uint32_t kKeyNaN = 1u;
constexpr uint32_t kKeyNegInf = 0x007fffffu;
constexpr uint32_t kKeyPosInf = 0xff800000u;

__host__ __device__ inline uint32_t order_key(float f) {
    uint32_t b = f2u(f);
    if ((b & 0x7fffffffu) > 0x7f800000u) return kKeyNaN;
    if ((b & 0x7fffffffu) == 0u) b = 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__host__ __device__ inline float key_value(uint32_t key) {
    return u2f((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// Composite sort key: value descending, then index ascending.
__host__ __device__ inline uint64_t composite(uint32_t key, uint32_t index) {
    return (static_cast<uint64_t>(key) << 32) | static_cast<uint64_t>(0xffffffffu - index);
}
__host__ __device__ inline uint32_t composite_index(uint64_t c) {
    return 0xffffffffu - static_cast<uint32_t>(c);
}
__host__ __device__ inline uint32_t composite_key(uint64_t c) { return static_cast<uint32_t>(c >> 32); }

}  // namespace ge
