// Exhaustive host-side check of tqf::ref_expf (turboqwenfare_amd/csrc/tqf_expf.h)
// against the host C library's expf over every binary32 input the sampler's
// softmax reaches: all negative values from -0 to -inf (2^31 - 2^23 + 1
// patterns), +0, and quiet / signalling NaNs of both signs.  Built with hipcc
// (the header's __host__ __device__ function, compiled for the host), run on
// the CPU with one thread per core.
//
// usage: expf_sweep [control]
//   control: also sweep a copy of the evaluation whose reduction computes
//   r = z - kd from a rounded z = (N / ln 2) * x instead of the fused form --
//   a plausible slip that must show up as a mismatch (negative control).
// Prints "checked <n> mismatches <m> control_mismatches <c>"; exit 0.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <thread>
#include <vector>

#include "tqf_expf.h"

static float control_expf(float x) {
    using namespace tqf::expf_detail;
    const uint32_t abstop = (bits32(x) >> 20) & 0x7ffu;
    if (abstop >= (0x42b00000u >> 20)) return tqf::ref_expf(x);
    const double xd = (double)x;
    const double z = kInvLn2N * xd;
    double kd = fma(kInvLn2N, xd, kShift);
    const uint64_t ki = bits64(kd);
    kd -= kShift;
    const double r = z - kd;  // the slip: z rounded before the subtraction
    const double s = from64(kTab[ki % 32] + (ki << 47));
    double y = fma(kC2, r, 1.0);
    y = fma(fma(kC0, r, kC1), r * r, y);
    return (float)(y * s);
}

static uint32_t bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static float from(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

int main(int argc, char **argv) {
    const bool control = argc > 1;
    std::vector<uint32_t> extra = {0x00000000u, 0x7fc00000u, 0xffc00000u, 0x7f800001u, 0xff800001u, 0x7fffffffu};
    const uint64_t lo = 0x80000000ull, hi = 0xff800000ull;  // -0 .. -inf
    const unsigned nt = std::thread::hardware_concurrency() ? std::thread::hardware_concurrency() : 8;
    std::atomic<uint64_t> mism{0}, cmism{0};
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; ++t) {
        th.emplace_back([&, t]() {
            uint64_t m = 0, c = 0;
            for (uint64_t u = lo + t; u <= hi; u += nt) {
                const float x = from((uint32_t)u);
                const uint32_t want = bits(expf(x));
                if (bits(tqf::ref_expf(x)) != want) {
                    if (m < 3) printf("mismatch x=%a libm=%a ref=%a\n", x, expf(x), tqf::ref_expf(x));
                    ++m;
                }
                if (control && bits(control_expf(x)) != want) ++c;
            }
            mism += m;
            cmism += c;
        });
    }
    for (auto &t : th) t.join();
    uint64_t n = hi - lo + 1;
    for (uint32_t u : extra) {
        const float x = from(u);
        ++n;
        if (bits(tqf::ref_expf(x)) != bits(expf(x))) {
            printf("mismatch x=0x%08x\n", u);
            ++mism;
        }
    }
    printf("checked %llu mismatches %llu control_mismatches %llu\n", (unsigned long long)n,
           (unsigned long long)mism.load(), (unsigned long long)cmism.load());
    return 0;
}
