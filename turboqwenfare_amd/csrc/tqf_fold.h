// tqf_fold.h -- the grid rule of the exact parallel f32 fold (tqf_sample.hip).
//
// A sequential f32 sum of terms t >= +0 never decreases.  While the running
// sum s lies in one binade [2^(eg-127), 2^(eg-126)) (eg >= 2), or below
// 2^-125 (eg = 1: the subnormals and the lowest binade share one spacing),
// its values are the multiples of g = 2^(eg - 150), and for a term t with
// s + t below the binade's top
//   fl(s + t) = s + g * rne(t / g)
// unless t / g is an odd multiple of 1/2 (a tie, whose rounding depends on the
// parity of s / g).  s is kept as (eg, n = s / g); a run of terms without a
// tie that keeps n below 2^24 adds integer counts, in any order.
//
// The device code and the host check (tests/native/fold_check.cpp, built with
// hipcc, run on the CPU) compile the same definitions.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

namespace tqf {

constexpr uint32_t kTie = 1u << 8;   // a term lies halfway between two grid points
constexpr uint32_t kNan = 1u << 9;   // a term is NaN
constexpr uint32_t kInf = 1u << 10;  // a term is +inf
constexpr uint32_t kNeg = 1u << 11;  // a term has the sign bit set (-0, negative, -inf)
constexpr uint32_t kTop = 1u << 24;  // grid units at which the sum reaches its binade's top
constexpr uint32_t kSat = 1u << 25;  // saturation of a chunk's count (any count >= kTop crosses)

__host__ __device__ inline uint32_t sat_add(uint32_t x, uint32_t y) {
    const uint32_t s = x + y;  // x, y <= kSat: no wrap
    return s < kSat ? s : kSat;
}

__host__ __device__ inline uint32_t term_flags(uint32_t tb) {
    if ((tb & 0x7fffffffu) > 0x7f800000u) return kNan;
    if (tb >> 31) return kNeg;
    return tb == 0x7f800000u ? kInf : 0u;
}

// t / g rounded to nearest for a finite t >= +0 on the grid of exponent eg
// (1 <= eg <= 254).  tie: t / g is an odd multiple of 1/2 (the returned count
// is then immaterial).  t is first clamped to the binade's top 2^(eg - 126),
// so a term that alone reaches the top counts 2^24; the scaling by
// 2^(150 - eg) is then exact (a power of two, no overflow; a result below
// the normal range is far below 1/2 and rounds to a count of 0 either way).
__host__ __device__ inline uint32_t grid_units(float t, uint32_t eg, bool &tie) {
    float top;
    const uint32_t tb = (eg + 1u) << 23;
    memcpy(&top, &tb, 4);
    const float x = ldexpf(fminf(t, top), 150 - (int)eg);
    const float r = rintf(x);
    tie = x - floorf(x) == 0.5f;
    return (uint32_t)r;
}

// The running sum on its grid: value bits = ((eg - 1) << 23) + n, n < 2^24
// (n >= 2^23 for eg >= 2).
struct Grid {
    uint32_t eg, n;
};
__host__ __device__ inline Grid grid_of(uint32_t bits) {
    const uint32_t e = bits >> 23, eg = e > 1u ? e : 1u;
    return {eg, bits - ((eg - 1u) << 23)};
}
__host__ __device__ inline uint32_t grid_bits(uint32_t eg, uint32_t n) { return ((eg - 1u) << 23) + n; }

}  // namespace tqf
