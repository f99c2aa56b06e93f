// Host-side check of the persistent stack kernel's partial-word tags
// (turboqwenfare_amd/csrc/tqf_tags.h): a mixed-depth sequence of launches,
// each tagging layer l with stack_part_tag(base, l) and advancing base with
// stack_next_base at its exit.  Every partial word is rewritten at every
// layer, so one simulated word stands for all of them: before layer l of a
// launch writes it, it must not already carry that layer's tag (a reader
// polling for the tag would take the stale value).
//
// usage: stack_tags_check <scheme> <start> <launches> <seed>
//   seed 0: depths alternate 40, 1, 40, 1, ... (target, draft); otherwise a
//   seeded random mix
//   scheme 0: the layer-step tags of tqf_tags.h
//   scheme 1: launch-count tags, seq * n_layers + l (the earlier definition,
//             kept as a negative control: it collides for mixed depths)
// Prints "ok <launches>" or "collision <launch> <layer> <tag>" and exits 0 / 1.
#include <cstdio>
#include <cstdlib>
#include <cstdint>

#include "tqf_tags.h"

static uint32_t launch_count_tag(uint32_t seq, uint32_t n, uint32_t l) {
    return 0x80000000u | ((seq * n + l) & 0x7FFFFFFFu);
}

int main(int argc, char **argv) {
    if (argc != 5) return 2;
    const int scheme = std::atoi(argv[1]);
    uint32_t state = (uint32_t)std::strtoul(argv[2], nullptr, 0);  // base (0) or seq (1)
    const long launches = std::atol(argv[3]);
    const bool seed0 = std::strtoull(argv[4], nullptr, 0) == 0;
    uint64_t rng = std::strtoull(argv[4], nullptr, 0) * 0x9E3779B97F4A7C15ull + 1;
    uint32_t word = 0;  // the zeroed allocation
    for (long j = 0; j < launches; ++j) {
        rng ^= rng << 13;
        rng ^= rng >> 7;
        rng ^= rng << 17;
        // depths as the MTP loop mixes them: a 1-layer draft stack, the
        // 40-layer target, and an occasional other depth
        const uint32_t r = (uint32_t)(rng >> 33) % 8;
        const uint32_t n = seed0 ? (j % 2 == 0 ? 40u : 1u)
                                 : r < 3 ? 1u : r < 7 ? 40u : 1u + (uint32_t)(rng >> 45) % 64;
        for (uint32_t l = 0; l < n; ++l) {
            const uint32_t tag = scheme == 0 ? tqf::stack_part_tag(state, l) : launch_count_tag(state, n, l);
            if (word == tag) {
                std::printf("collision %ld %u %u\n", j, l, tag);
                return 1;
            }
            word = tag;
        }
        state = scheme == 0 ? tqf::stack_next_base(state, n) : state + 1;
    }
    std::printf("ok %ld\n", launches);
    return 0;
}
