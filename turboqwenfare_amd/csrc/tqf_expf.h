// tqf_expf.h -- binary32 exp, bit-identical to the host C library's expf.
//
// The reference's stochastic sampler exponentiates with f32::exp
// (sampling/mod.rs:166-190), which on Linux is glibc's expf.  glibc (2.28
// and later) computes expf with the table-driven method of Szabolcs Nagy
// (ARM optimized-routines, "exp2f_data"): with N = 32,
//
//   x * N / ln 2 = k + r,  k = round-to-nearest-even integer, |r| <= 1/2,
//   exp(x) = 2^(k/N) * 2^(r/N) ~= s * (C0 r^3 + C1 r^2 + C2 r + 1),
//
// evaluated in binary64 and rounded to binary32 once.  s = 2^(k/N) is the
// correctly rounded binary64 value of 2^((k mod N)/N) (the table below,
// stored with (k mod N) << 47 subtracted so that adding k << 47 scales it by
// 2^(k div N)), and C0..C2 are the method's minimax coefficients for
// 2^(r/N), scaled by N^-3, N^-2, N^-1.  The rounding of k uses the 1.5 * 2^52
// shift (an add and a subtract in binary64).
//
// glibc's x86-64 build selects a variant compiled with fused multiply-add;
// this is that evaluation order, every fusion written out as fma():
//   kd = fma(N/ln2, x, shift);  r = fma(N/ln2, x, -(kd - shift));
//   y = fma(fma(C0, r, C1), r*r, fma(C2, r, 1)) * s.
// No operation is left for a compiler to contract, so host and device builds
// evaluate the same binary64 operations.  tests/test_expf.py compares this
// function with the host's expf on every binary32 input the sampler's
// softmax can reach (-inf, all negative values, -0, +0 and NaN: the
// arguments (l - max) / T are never positive).
//
// The device code and the host test (built with hipcc, run on the CPU)
// compile the same definition.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

namespace tqf {

namespace expf_detail {
// 2^(i/32) rounded to binary64, minus i << 47 (i = 0..31).
constexpr uint64_t kTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;  // 32 / ln 2
constexpr double kShift = 0x1.8p+52;
constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32;

__host__ __device__ inline uint32_t bits32(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
__host__ __device__ inline uint64_t bits64(double d) {
    uint64_t u;
    memcpy(&u, &d, 8);
    return u;
}
__host__ __device__ inline double from64(uint64_t u) {
    double d;
    memcpy(&d, &u, 8);
    return d;
}
}  // namespace expf_detail

__host__ __device__ inline float ref_expf(float x) {
    using namespace expf_detail;
    const uint32_t abstop = (bits32(x) >> 20) & 0x7ffu;
    if (abstop >= (0x42b00000u >> 20)) {  // |x| >= 88, or not finite
        if (bits32(x) == 0xff800000u) return 0.0f;         // -inf
        if (abstop >= (0x7f800000u >> 20)) return x + x;  // +inf, NaN
        if (x > 0x1.62e42ep6f) return x * 0x1p127f * 0x1p127f;  // overflow: +inf
        if (x < -0x1.9fe368p6f) return 0.0f;                  // underflow
    }
    const double xd = (double)x;
    double kd = fma(kInvLn2N, xd, kShift);
    const uint64_t ki = bits64(kd);
    kd -= kShift;
    const double r = fma(kInvLn2N, xd, -kd);
    const double s = from64(kTab[ki % 32] + (ki << 47));
    const double z = fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = fma(kC2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

}  // namespace tqf
