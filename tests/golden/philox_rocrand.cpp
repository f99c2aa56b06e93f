// Known-answer vectors for Philox4x32-10 from ROCm's open-source rocRAND
// device/host header (rocrand_philox4x32_10.h, philox4x32_10_engine::
// ten_rounds).  Built and run on the host by make_golden.py; prints one line
// per (counter, key): c0 c1 c2 c3 k0 k1 -> r0 r1 r2 r3 (hex).
#include <cstdio>
#include <cstdint>

#include <rocrand/rocrand_philox4x32_10.h>

struct Engine : rocrand_device::philox4x32_10_engine {
    uint4 run(uint4 c, uint2 k) { return ten_rounds(c, k); }
};

int main() {
    Engine e;
    const uint32_t cases[][6] = {
        {0u, 0u, 0u, 0u, 0u, 0u},
        {0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu},
        {0x243f6a88u, 0x85a308d3u, 0x13198a2eu, 0x03707344u, 0xa4093822u, 0x299f31d0u},
        {1u, 0u, 0u, 0u, 0u, 0x243F6A88u},
        {7u, 3u, 0u, 0u, 12345u, 0x243F6A88u},
        {123456u, 0u, 1u, 0u, 1000003u, 0u},
        {0x89abcdefu, 0x01234567u, 0u, 0u, 42u, 7u},
        {5u, 0u, 0u, 0u, 0u, 0x243F6A88u},
    };
    for (const auto &c : cases) {
        const uint4 r = e.run(uint4{c[0], c[1], c[2], c[3]}, uint2{c[4], c[5]});
        std::printf("%08x %08x %08x %08x %08x %08x -> %08x %08x %08x %08x\n", c[0], c[1], c[2],
                    c[3], c[4], c[5], r.x, r.y, r.z, r.w);
    }
    return 0;
}
