// tqf_loop.hip -- the two row kernels the MTP decode loop needs around the
// stack, the LM head and the acceptance:
//
//   * embedding rows: token ids -> f32 rows of a Q4_0 [V x hidden] matrix in
//     the row-lane layout (Qwen36Runtime::decode_step's embedding.row,
//     model/qwen36/runtime.rs:403, decoded per the row's dtype as
//     LoadedQwen36Tensor::row does, model/qwen36/weights.rs:346-379), with an
//     optional row added element-wise (the draft head's input, see
//     turboqwenfare_amd/mtp_loop.py);
//   * RMSNorm rows: the final norm before the LM head (runtime.rs:430-431,
//     Qwen36Activation::qwen_rmsnorm: x * (1 / sqrt(mean(x^2) + 1e-6)) * w).
//
// Both are HBM-light (one row per workgroup; the decode is exact: the f16
// scale times a small integer).
#include <hip/hip_runtime.h>

#include "tqf_device.h"
#include "tqf_internal.h"

namespace tqf {

// One wavefront per row, one lane per 32-element block (looping for rows of
// more than 64 blocks).  Element j < 16 of a block is the low nibble of byte
// j, element j + 16 its high nibble, each (q - 8) * d.  `add` may be `out`
// (the draft head adds its embedding in place): element c is read and then
// written by the same thread, so neither pointer is declared __restrict__.
__global__ __launch_bounds__(64) void embed_rows_kernel(const uint8_t *__restrict__ tiles, MatrixDims d,
                                                        const int32_t *__restrict__ tokens,
                                                        const float *add, float *out,
                                                        int32_t *__restrict__ status) {
    const uint32_t t = blockIdx.x;
    const int32_t tok = tokens[t];
    const bool ok = tok >= 0 && (uint32_t)tok < d.rows;
    if (!ok && threadIdx.x == 0 && status) *status = TQF_HIP_ERR_INVALID;
    float *y = out + (size_t)t * d.cols;
    const float *a = add ? add + (size_t)t * d.cols : nullptr;
    for (uint32_t b = threadIdx.x; b < d.blocks; b += 64) {
        float v[32];
        if (ok) {
            const uint8_t *sc = tiles + scale_offset(d, (size_t)tok, b);
            const float dd = f16_to_f32((uint32_t)sc[0] | ((uint32_t)sc[1] << 8));
            const uint4 q = *reinterpret_cast<const uint4 *>(tiles + nibble_offset(d, (size_t)tok, b));
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t byte = (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
                v[j] = (float)((int)(byte & 0x0Fu) - 8) * dd;
                v[j + 16] = (float)((int)(byte >> 4) - 8) * dd;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 32; ++j) v[j] = __int_as_float(0x7FC00000);
        }
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const size_t c = (size_t)b * 32 + j;
            y[c] = a ? a[c] + v[j] : v[j];
        }
    }
}

hipError_t launch_embed_rows(hipStream_t s, const uint8_t *tiles, const MatrixDims &d, const int32_t *tokens,
                             uint32_t n, const float *add, float *out, int32_t *status) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(embed_rows_kernel, dim3(n), dim3(64), 0, s, tiles, d, tokens, add, out, status);
    return hipGetLastError();
}

// One workgroup of 256 threads per row: per-thread partial sums of squares
// over a strided slice, a block reduction, then x * inv_rms * w element-wise.
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float *__restrict__ x, uint32_t cols,
                                                           const float *__restrict__ w,
                                                           float *__restrict__ out) {
    __shared__ float s_part[4];
    const uint32_t t = blockIdx.x;
    const float *xr = x + (size_t)t * cols;
    float ss = 0.0f;
    for (uint32_t c = threadIdx.x; c < cols; c += 256) ss = __builtin_fmaf(xr[c], xr[c], ss);
    ss = group_reduce<64>(ss, AddOp());
    if ((threadIdx.x & 63) == 0) s_part[threadIdx.x / 64] = ss;
    __syncthreads();
    const float total = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
    const float inv = 1.0f / sqrtf(total / (float)cols + 1e-6f);
    float *yr = out + (size_t)t * cols;
    for (uint32_t c = threadIdx.x; c < cols; c += 256) yr[c] = xr[c] * inv * w[c];
}

hipError_t launch_rmsnorm_rows(hipStream_t s, const float *x, uint32_t n, uint32_t cols, const float *w,
                               float *out) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(n), dim3(256), 0, s, x, cols, w, out);
    return hipGetLastError();
}

}  // namespace tqf
