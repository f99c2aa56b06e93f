// tqf_synth.hip -- seeded synthetic Q4_0 weights generated directly in HBM.
//
// No reference counterpart: the benchmark configurations name synthetic
// weights from a seeded Philox stream, and writing 18 GB from the host would
// cost minutes.  The definition is shared with the host generator in
// turboqwenfare_amd/synth.py (tests compare the two byte for byte):
//   key = (tensor_id, seed); block b (row-major) of the matrix:
//   Philox4x32-10(ctr = (b_lo, b_hi, 0, 0)) -> 4 words = the 16 nibble bytes
//     (little-endian), i.e. nibbles uniform on 0..15;
//   Philox4x32-10(ctr = (b_lo, b_hi, 1, 0)) word 0 -> u = (w >> 8) 2^-24,
//     d = 0.005 + 0.015 u in binary32 (no fused multiply-add), stored as
//     binary16 rounded to nearest even.
// Recipe TQF_HIP_SYNTH_ZERO_MEAN then maps every nibble 0 to 8, so that
// q - 8 is symmetric on [-7, 7]: uniform nibbles give E[q - 8] = -0.5, a
// rank-one component common to every matrix that, through SwiGLU and the
// residual stream, drives the rows of a stack towards one direction.
#include <hip/hip_runtime.h>

#include "../../include/tqf_hip_synth.h"
#include "tqf_internal.h"

#pragma clang fp contract(off)

namespace tqf {

__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int round = 0; round < 10; ++round) {
        if (round) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
        c[1] = (uint32_t)p1;
        c[3] = (uint32_t)p0;
        c[0] = n0;
        c[2] = n2;
    }
}

// Nibble 0 -> 8 in every nibble of w: bit 4j of t is the OR of nibble j's
// four bits (no bit of another nibble reaches it).
__device__ __forceinline__ uint32_t zero_mean_nibbles(uint32_t w) {
    uint32_t t = w | (w >> 1);
    t |= t >> 2;
    return w | ((~t & 0x11111111u) << 3);
}

__global__ __launch_bounds__(256) void synth_q4_0_kernel(MatrixDims dims, uint32_t key0,
                                                         uint32_t key1, uint32_t recipe,
                                                         uint8_t *__restrict__ tiles) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)dims.rows * dims.blocks) return;
    const uint32_t r = (uint32_t)(idx / dims.blocks), b = (uint32_t)(idx % dims.blocks);
    uint32_t q[4] = {(uint32_t)idx, (uint32_t)(idx >> 32), 0u, 0u};
    philox4x32_10(q, key0, key1);
    if (recipe == TQF_HIP_SYNTH_ZERO_MEAN)
        for (int i = 0; i < 4; ++i) q[i] = zero_mean_nibbles(q[i]);
    uint32_t s[4] = {(uint32_t)idx, (uint32_t)(idx >> 32), 1u, 0u};
    philox4x32_10(s, key0, key1);
    const float u = (float)(s[0] >> 8) * 0x1p-24f;
    const float d = 0.005f + 0.015f * u;
    const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)d);
    *reinterpret_cast<uint4 *>(tiles + nibble_offset(dims, r, b)) = make_uint4(q[0], q[1], q[2], q[3]);
    *reinterpret_cast<uint16_t *>(tiles + scale_offset(dims, r, b)) = h;
}

hipError_t launch_synth_q4_0(hipStream_t s, const MatrixDims &d, uint32_t tensor_id,
                             uint32_t seed, uint32_t recipe, uint8_t *tiles) {
    const uint64_t n = (uint64_t)d.rows * (d.cols / 32);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(synth_q4_0_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s,
                       d, tensor_id, seed, recipe, tiles);
    return hipGetLastError();
}

}  // namespace tqf
