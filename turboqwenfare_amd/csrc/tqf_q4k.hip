// tqf_q4k.hip -- canonical Q4_K matrices (GGML super-blocks of 256 elements,
// 144 bytes: f16 d, f16 dmin, 12 bytes of packed 6-bit sub-block scales and
// mins, 128 nibble bytes; format/quant/dequant.rs:139-184) on gfx950.
//
//   * the lossless repack into the Q4_K row-lane layout (tqf_internal.h);
//   * the fp32-semantics GEMV of backend::reference::q4k_gemv (reference.rs:
//     49-67): sum_i (d sc q_i - dmin m) x_i, evaluated as
//       d sc * sum_i (q_i - 8) x_i  +  (8 d sc - dmin m) * sum_i x_i
//     per 32-element sub-block with the exact int4 activation-record dot of
//     the Q4_0 path (the record carries sum_i X_i in its spare dword 25);
//   * the Q8_K integer path of matvec_payload (weights.rs:680-735):
//     quantize_q8_k (weights.rs:898-931) and q4_k_dot_pre (weights.rs:
//     944-1021), bit-identical to the scalar loop: the integer lane sums are
//     exact, and the f32 combine runs in the reference's order (per output
//     row, super-block after super-block, no fused multiply-adds).
//
// Every kernel is HBM-bound on the weight bytes; the layout gives each lane
// one 32-element sub-block of eight rows, so a wavefront reads a contiguous
// stretch per row octet exactly as the Q4_0 GEMV does.
#include <hip/hip_runtime.h>

#include "tqf_device.h"
#include "tqf_internal.h"

namespace tqf {

// Scale and min (6 bits each) of sub-block j of one super-block's 12 packed
// bytes (q4_k_scale_min, weights.rs:933-942; the same split as dequant.rs:
// 154-184).
__device__ __forceinline__ void q4k_scale_min(const uint8_t *p, int j, uint32_t &sc, uint32_t &mn) {
    if (j < 4) {
        sc = p[j] & 63u;
        mn = p[j + 4] & 63u;
    } else {
        sc = (p[j + 4] & 0xFu) | ((uint32_t)(p[j - 4] >> 6) << 4);
        mn = (uint32_t)(p[j + 4] >> 4) | ((uint32_t)(p[j] >> 6) << 4);
    }
}

// ---------------------------------------------------------------------------
// Repack: GGML Q4_K (rows x cols/256 x 144 bytes) -> Q4_K row-lane layout.
// One thread per (row, sub-block); the destination was zero-filled, so
// padding rows and sub-blocks decode to exactly 0.  Sub-block j of a
// super-block holds elements 32j..32j+31: the low nibbles of qs[32(j/2) ..
// +32) for even j, the high nibbles for odd j.  They are stored in class
// order: byte 4i + t holds element 2i + 8t (low nibble) and 2i + 1 + 8t
// (high nibble), so that the low (high) nibbles of nibble dword i are the
// four elements of class 2i (2i + 1), where class c = {c, c+8, c+16, c+24}.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void q4k_repack_kernel(const uint8_t *__restrict__ aos,
                                                         MatrixDims d, uint8_t *__restrict__ dst) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)d.rows * d.blocks) return;
    const uint32_t r = (uint32_t)(idx / d.blocks), b = (uint32_t)(idx % d.blocks);
    const uint32_t s = b >> 3;
    const int j = (int)(b & 7);
    const uint8_t *src = aos + ((size_t)r * (d.blocks >> 3) + s) * kQ4KBlock;
    uint32_t sc, mn;
    q4k_scale_min(src + 4, j, sc, mn);
    const uint8_t *qs = src + 16 + 32 * (j >> 1);
    const int shift = 4 * (j & 1);
    uint8_t *nib = dst + nibble_offset(d, q4k_slot_row(r, b), b);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t lo = (qs[2 * i + 8 * t] >> shift) & 15u;
            const uint32_t hi = (qs[2 * i + 1 + 8 * t] >> shift) & 15u;
            nib[4 * i + t] = (uint8_t)(lo | (hi << 4));
        }
    uint8_t *scp = dst + scale_offset(d, q4k_slot_row(r, b), b);
    scp[0] = (uint8_t)sc;
    scp[1] = (uint8_t)mn;
    if (j == 0) {
        uint8_t *dm = dst + q4k_dm_offset(d, r, s);
#pragma unroll
        for (int i = 0; i < 4; ++i) dm[i] = src[i];
    }
}

hipError_t launch_q4k_repack(hipStream_t s, const uint8_t *d_aos, const MatrixDims &d,
                             uint8_t *dst) {
    const uint64_t n = (uint64_t)d.rows * d.blocks;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(q4k_repack_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s,
                       d_aos, d, dst);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Activation records for the fp32-semantics GEMV: the Q4_0 record format
// (tqf_internal.h) with the digit nibbles in class order (element j at dword
// (j mod 8) / 2, bit 4 (2 (j / 8) + j mod 2), pairing with the class-ordered
// weight nibbles) and dword 25 = sum_j X_j (int32, |sum| <= 2^27).  One
// thread per element, 32 lanes per sub-block.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void q4k_prep_kernel(const float *__restrict__ x, uint32_t cols,
                                                       uint32_t bp, uint32_t *__restrict__ xprep) {
    const uint32_t t = blockIdx.y;
    const uint32_t kb = (blockIdx.x * blockDim.x + threadIdx.x) / 32;
    if (kb >= bp) return;  // whole 32-lane groups
    const int j = (int)(threadIdx.x & 31);
    const uint32_t col = kb * 32 + j;
    const float v = col < cols ? x[(size_t)t * cols + col] : 0.0f;
    const float a = fabsf(v);
    const bool bad = !(a <= 3.402823466e38f);
    const float amax = group_reduce<32>(bad ? 0.0f : a, MaxOp());
    const int badi = group_reduce<32>(bad ? 1 : 0, MaxOp());
    int e;
    const float scale = block_scale(amax, badi != 0, e);
    int dg[6];
    split_digits16(v, e, scale, dg);
    const int X = scale > 0.0f ? (int)__builtin_rintf(__builtin_ldexpf(v, -e)) : 0;
    const int sum_x = group_reduce<32>(X, AddOp());
    const int dw = (j & 7) >> 1, sh = 4 * (2 * (j >> 3) + (j & 1));
    uint32_t *row = xprep + (size_t)t * bp * kXprepDwords;
#pragma unroll
    for (int k = 0; k < 6; ++k)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            int part = (q == dw) ? (int)(((uint32_t)dg[k] & 15u) << sh) : 0;
            part = group_reduce<32>(part, OrOp());
            if (j == 0) *rec_dw(row, bp, kb, 4 * k + q) = (uint32_t)part;
        }
    if (j == 0) {
        *rec_dw(row, bp, kb, 24) = __float_as_uint(scale);
        *rec_dw(row, bp, kb, 25) = (uint32_t)sum_x;
    }
}

hipError_t launch_q4k_prep(hipStream_t s, const float *x, uint32_t m, uint32_t cols, uint32_t bp,
                           uint32_t *xprep) {
    const uint32_t grid = (bp * 32 + 255) / 256;
    hipLaunchKernelGGL(q4k_prep_kernel, dim3(grid, m), dim3(256), 0, s, x, cols, bp, xprep);
    return hipGetLastError();
}

// Sub-block scale and min of the eight rows of one lane's octet: the 16-byte
// scale vector holds (sc, m) as two bytes per row.
__device__ __forceinline__ void octet_sc_m(const uint4 v, int n, uint32_t &sc, uint32_t &mn) {
    const uint32_t sv[4] = {v.x, v.y, v.z, v.w};
    const uint32_t h = sv[n >> 1] >> (16 * (n & 1));
    sc = h & 0xFFu;
    mn = (h >> 8) & 0xFFu;
}

constexpr int kDppRowRor8 = 0x128;  // row_ror:8: lane i <- lane i ^ 8 within 16

// Slots 4 (k & 4), 2 (k & 2) and 1 (k & 1) apart swapped: the bits of k
// that dm0/dm1's load addresses have not already applied (k & 4 there).
__device__ __forceinline__ void xor_permute8(uint32_t (&v)[8], int k) {
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        if ((p & 2) == 0) {
            const uint32_t a = v[p], b = v[p + 2];
            v[p] = (k & 2) ? b : a;
            v[p + 2] = (k & 2) ? a : b;
        }
    }
#pragma unroll
    for (int p = 0; p < 8; p += 2) {
        const uint32_t a = v[p], b = v[p + 1];
        v[p] = (k & 1) ? b : a;
        v[p + 1] = (k & 1) ? a : b;
    }
}

// Row sums of a lane group: register slot p of lane k (k = lane mod 8)
// holds a partial of row p ^ k.  Three select-free butterfly stages over the
// eight lanes leave row k's sum over them in slot 0 (each stage adds the
// partner's slot p ^ mask to slot p), then the LPR / 8 groups of a lane
// group are added (lanes k, k + 8, ...).  Valid in the first eight lanes.
template <int LPR>
__device__ __forceinline__ float xor_reduce_rows(float (&v)[8]) {
#pragma unroll
    for (int p = 0; p < 4; ++p) v[p] += dpp_f<kDppHalfMirror>(v[p ^ 7]);
#pragma unroll
    for (int p = 0; p < 2; ++p) v[p] += dpp_f<kDppQuadRev>(v[p ^ 3]);
    v[0] += dpp_f<kDppXor1>(v[1]);
    if constexpr (LPR >= 16) v[0] += dpp_f<kDppRowRor8>(v[0]);
    if constexpr (LPR >= 32) permlane16_stage<1>(v);
    if constexpr (LPR >= 64) permlane32_stage<1>(v);
    return v[0];
}

// ---------------------------------------------------------------------------
// fp32-semantics GEMV / small-M GEMM: the Q4_0 GEMV's geometry (lane group
// of LPR lanes per row octet, lane b owns sub-block b of each chunk, every
// load issued before any arithmetic), plus the octet's (d, dmin) pairs of
// the lane's super-block (32 bytes shared by the eight lanes of that
// super-block).
// ---------------------------------------------------------------------------
constexpr int kQ4KWaves = 8;

template <int LPR, int TG>
__global__ __launch_bounds__(kQ4KWaves * kWave) void q4k_gemv_kernel(
    const uint8_t *const *__restrict__ tables, MatrixDims d, const uint32_t *__restrict__ xprep,
    uint32_t m, float *__restrict__ y) {
    constexpr int G = kWave / LPR;
    constexpr int RW = 8 * G;
    constexpr int NL = 8;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const uint32_t jg = (uint32_t)lane / LPR, b = (uint32_t)lane % LPR;
    const uint32_t mat = blockIdx.y;
    const uint32_t r0 = (blockIdx.x * kQ4KWaves + wave) * RW;
    if (r0 >= d.rows_padded) return;
    const uint8_t *base = tables[mat];
    const RowLane W = row_lane(base, d.blocks_padded);
    const uint32_t rl = r0 + jg * NL;
    const int k = (int)(b & 7);  // register slot p holds row rl + (p ^ k)
    const uint32_t row = rl + k;
    const bool writer = b < 8 && row < d.rows;
    const uint32_t chunks = d.blocks_padded / LPR;
    const size_t xstride = (size_t)d.blocks_padded * kXprepDwords;
    const uint8_t *dm_octet = base + q4k_dm_offset(d, rl, 0);
    for (uint32_t t0 = 0; t0 < m; t0 += TG) {
        float acc[TG][NL];
#pragma unroll
        for (int t = 0; t < TG; ++t)
#pragma unroll
            for (int n = 0; n < NL; ++n) acc[t][n] = 0.0f;
        for (uint32_t c = 0; c < chunks; ++c) {
            const uint32_t blk = c * LPR + b;
            uint4 nib[NL];
#pragma unroll
            for (int n = 0; n < NL; ++n) nib[n] = q4_signed(load_nibbles(W, rl + n, blk));
            const uint4 scm = load_scales(W, rl / 8, blk);
            const uint8_t *dmp = dm_octet + (size_t)(blk >> 3) * 32;
            const uint4 dm0 = load_global_u4(dmp + ((k & 4) ? 16 : 0));  // rows 0..3 ^ (k & 4)
            const uint4 dm1 = load_global_u4(dmp + ((k & 4) ? 0 : 16));
            uint32_t x[TG][28];
#pragma unroll
            for (int t = 0; t < TG; ++t) {
                const uint32_t tt = t0 + t < m ? t0 + t : 0;  // loads stay unconditional
                load_xrec(xprep + tt * xstride, d.blocks_padded, blk, x[t]);
                if (blk >= d.blocks) x[t][24] = 0;  // padding: exactly 0 whatever it holds
            }
            __builtin_amdgcn_sched_barrier(0);  // every load in flight before any math
            uint32_t dmv[8] = {dm0.x, dm0.y, dm0.z, dm0.w, dm1.x, dm1.y, dm1.z, dm1.w};
            xor_permute8(dmv, k);  // (d, dmin) of row p ^ k in slot p
            float dsc[NL], bias[NL];
#pragma unroll
            for (int n = 0; n < NL; ++n) {
                uint32_t sc, mn;
                octet_sc_m(scm, n, sc, mn);
                dsc[n] = f16_to_f32(dmv[n]) * (float)sc;                         // exact (17 bits)
                bias[n] = 8.0f * dsc[n] - f16_to_f32(dmv[n] >> 16) * (float)mn;  // one rounding
            }
#pragma unroll
            for (int t = 0; t < TG; ++t) {
                const float sx = (float)(int)x[t][25] * __uint_as_float(x[t][24]);
#pragma unroll
                for (int n = 0; n < NL; ++n)
                    acc[t][n] = fmaf(dsc[n], q4_block_dot(nib[n], x[t]), fmaf(bias[n], sx, acc[t][n]));
            }
        }
#pragma unroll
        for (int t = 0; t < TG; ++t) {
            const float s = xor_reduce_rows<LPR>(acc[t]);
            if (writer && t0 + t < m) y[((size_t)mat * m + t0 + t) * d.rows + row] = s;
        }
    }
}

template <int LPR>
hipError_t launch_q4k_gemv_lpr(hipStream_t s, const uint8_t *const *tables, uint32_t count,
                               const MatrixDims &d, const uint32_t *xprep, uint32_t m, float *y) {
    constexpr uint32_t rows_per_group = kQ4KWaves * 8 * (kWave / LPR);
    const dim3 grid((d.rows_padded + rows_per_group - 1) / rows_per_group, count);
    const dim3 block(kQ4KWaves * kWave);
    if (m <= 1) hipLaunchKernelGGL((q4k_gemv_kernel<LPR, 1>), grid, block, 0, s, tables, d, xprep, m, y);
    else if (m <= 2) hipLaunchKernelGGL((q4k_gemv_kernel<LPR, 2>), grid, block, 0, s, tables, d, xprep, m, y);
    else hipLaunchKernelGGL((q4k_gemv_kernel<LPR, 4>), grid, block, 0, s, tables, d, xprep, m, y);
    return hipGetLastError();
}

hipError_t launch_q4k_gemv(hipStream_t s, const uint8_t *const *tables, uint32_t count,
                           const MatrixDims &d, const uint32_t *xprep, uint32_t m, float *y) {
    if (d.lpr == 16) return launch_q4k_gemv_lpr<16>(s, tables, count, d, xprep, m, y);
    if (d.lpr == 32) return launch_q4k_gemv_lpr<32>(s, tables, count, d, xprep, m, y);
    return launch_q4k_gemv_lpr<64>(s, tables, count, d, xprep, m, y);
}

// ---------------------------------------------------------------------------
// Q8_K activation quantization, quantize_q8_k (weights.rs:898-931), one
// wavefront per (token, 256-element chunk).  Lane 8k + c owns class c of
// sub-block k (elements 32k + c + 8t, t = 0..3), so its four int8 values
// form one class-ordered dword of the record.  Records: per (token,
// sub-block) 12 dwords in three 16-byte planes of the token row,
//   plane 0, 1  q8 class dwords 0..3, 4..7 (byte t of class c = element c+8t)
//   plane 2     dword 0: sum of the sub-block's 32 values (int32, the
//               reference's sums[2k] + sums[2k+1]); dword 1: the chunk's
//               scale (f32); dwords 2, 3 unused
// Row stride 12 Bp dwords.  Chunks past cols are not written.
//   signed maximum: the first element of largest |v| (NaN never compares
//   greater); all-zero chunks give zeros and scale 0; inverse = -127 / that
//   maximum and scale = 1 / inverse, both correctly rounded; each value is
//   round_ties_even(v * inverse), then f32::min(127) (NaN -> 127) and the
//   saturating cast to i8.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void q8k_quantize_kernel(const float *__restrict__ x,
                                                           uint32_t cols, uint32_t bp,
                                                           uint32_t *__restrict__ q8) {
    const uint32_t t = blockIdx.y;
    const uint32_t chunk = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    if (chunk >= cols / 256) return;  // whole wavefronts
    const int lane = threadIdx.x & 63, k = lane >> 3, c = lane & 7;
    const float *src = x + (size_t)t * cols + (size_t)chunk * 256 + 32 * k + c;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = src[8 * i];
    q8k_quantize_values(v, q8 + (size_t)t * bp * kQ8KRecDwords, bp, chunk);
}

// SwiGLU fused into the quantization of h: h = (g / (1 + exp(-g))) * u per
// element (Qwen36Activation::silu_mul, weights.rs:241-260), g and u the
// gate and up rows of row t (gu = [gate rows | up rows], up_offset floats
// apart), then quantize_q8_k of h as above.
__global__ __launch_bounds__(256) void q8k_swiglu_quantize_kernel(const float *__restrict__ gu,
                                                                  size_t up_offset, uint32_t cols,
                                                                  uint32_t bp,
                                                                  uint32_t *__restrict__ q8) {
    const uint32_t t = blockIdx.y;
    const uint32_t chunk = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    if (chunk >= cols / 256) return;  // whole wavefronts
    const int lane = threadIdx.x & 63, k = lane >> 3, c = lane & 7;
    const size_t e0 = (size_t)t * cols + (size_t)chunk * 256 + 32 * k + c;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float g = gu[e0 + 8 * i], u = gu[up_offset + e0 + 8 * i];
        v[i] = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u);
    }
    q8k_quantize_values(v, q8 + (size_t)t * bp * kQ8KRecDwords, bp, chunk);
}

hipError_t launch_q8k_quantize(hipStream_t s, const float *x, uint32_t m, uint32_t cols,
                               uint32_t bp, uint32_t *q8) {
    const uint32_t waves = cols / 256;
    hipLaunchKernelGGL(q8k_quantize_kernel, dim3((waves + 3) / 4, m), dim3(256), 0, s, x, cols, bp,
                       q8);
    return hipGetLastError();
}

hipError_t launch_q8k_swiglu_quantize(hipStream_t s, const float *gu, uint32_t m, uint32_t cols,
                                      uint32_t bp, uint32_t *q8) {
    const uint32_t waves = cols / 256;
    hipLaunchKernelGGL(q8k_swiglu_quantize_kernel, dim3((waves + 3) / 4, m), dim3(256), 0, s, gu,
                       (size_t)m * cols, cols, bp, q8);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Q8_K integer matvec, q4_k_dot_pre per row (weights.rs:944-1021).
//
// Integer phase.  Lane b of a lane group owns sub-block b of the chunk for
// the octet's eight rows.  Its partial lane sums are sc * dot4(q, q8) per
// class (the reference's lane = index mod 8 is the class), exact int32.
// The eight lanes of one super-block are summed with a butterfly that needs
// no selects: lane k of the eight keeps row k, and it holds the values of
// row p ^ k in register slot p from the start (the layout stores them in
// that order), so each halving stage adds the partner's slot p ^ mask to
// slot p.
// After it, lane 8g + k holds row k's eight class sums and its
// block_minimum_sum for super-block g of the chunk.
//
// Combine phase (f32, the reference's order).  Each lane forms the nine
// products (d q8scale) lane_sum and (dmin q8scale) block_minimum_sum; the
// nine running sums of a row (lane_acc[0..8) and minimum_sum) are dealt to
// the row's lanes of the lane group (chain ch to super-block lane ch mod
// LPR/8) and advanced super-block after super-block through LDS.  The last
// step, minimum_sum + (-0.0 + lane_acc[0] + ... + lane_acc[7]), is taken by
// the row's first lane.  Super-blocks past cols (padding) do not enter.
//
// SRC says where workgroup row blockIdx.y takes its matrix and records:
// kSrcTables -- tables[blockIdx.y], the m rows of q8; kSrcSlotGateUp --
// matrix blockIdx.y / S (0 gate, 1 up) of plan slot blockIdx.y % S (S =
// gridDim.y / 2), the records of the slot's token; kSrcSlotDown -- the down
// matrix of slot blockIdx.y, the slot's own records.  The slot forms run one
// row of records (m = 1) and skip slots without work (routing failed).
// kSrcSlotDownSwiglu -- as kSrcSlotDown, but the workgroup first makes the
// slot's records itself, in LDS: quantize_q8_k of h = silu_mul(gate, up) from
// gu ([gate rows | up rows] of every slot, gridDim.y slots, d.cols each),
// the arithmetic of q8k_swiglu_quantize_kernel.
// With fold.out set (kSrcSlotDownSwiglu only; every wavefront of a
// workgroup has rows), the layer's combine is folded in: each slot
// workgroup writes its rows of y with device-coherent stores and arrives on
// the counter of (its token, its row tile); the last of the token's nine
// slots to arrive sums them for the tile in q4k_moe_combine_kernel's order
// and arithmetic, adds the residual, writes fold.out, and resets the counter.
// ---------------------------------------------------------------------------
constexpr int kSrcTables = 0, kSrcSlotGateUp = 1, kSrcSlotDown = 2, kSrcSlotDownSwiglu = 3;
constexpr int kMaxRecBp = 64;  // padded sub-blocks of a record row made in LDS (cols <= 2048)

struct Fold {
    float *out;             // [M x rows] layer output (may alias resid)
    const float *resid;     // [M x rows] or null
    uint32_t *counters;     // [M x tiles], zero between launches
};

template <int LPR, int TG, int SRC>
__global__ __launch_bounds__(kQ4KWaves * kWave) void q4k_q8k_gemv_kernel(
    const uint8_t *const *__restrict__ tables, const Plan *__restrict__ plan, MatrixDims d,
    const uint32_t *__restrict__ q8, uint32_t m, float *__restrict__ y, const float *__restrict__ gu,
    Fold fold) {
    constexpr int G = kWave / LPR;         // row octets per wavefront
    constexpr int SB = LPR / 8;            // super-blocks per lane group and chunk
    constexpr int NCH = (9 + SB - 1) / SB; // running sums per lane
    __shared__ float lds[kQ4KWaves][kWave][9];
    __shared__ uint4 s_rec[SRC == kSrcSlotDownSwiglu ? 3 * kMaxRecBp : 1];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int jg = lane / LPR, b = lane % LPR, k = b & 7, g = b >> 3;
    const uint32_t mat = blockIdx.y;
    if constexpr (SRC == kSrcSlotDownSwiglu) {
        // before any wavefront can leave: every wavefront reaches the barrier
        if (plan->slots[mat].token >= 0) {
            const uint32_t cols = d.cols, S = gridDim.y;
            const int kk = lane >> 3, cc = lane & 7;
            for (uint32_t ch = (uint32_t)wave; ch < cols / 256; ch += kQ4KWaves) {
                const size_t e0 = (size_t)mat * cols + (size_t)ch * 256 + 32 * kk + cc;
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float gv = gu[e0 + 8 * i], uv = gu[(size_t)S * cols + e0 + 8 * i];
                    v[i] = __fmul_rn(__fdiv_rn(gv, __fadd_rn(1.0f, expf(-gv))), uv);
                }
                q8k_quantize_values(v, reinterpret_cast<uint32_t *>(s_rec), d.blocks_padded, ch);
            }
        }
        __syncthreads();
    }
    const uint32_t r0 = (blockIdx.x * kQ4KWaves + wave) * 8 * G;
    if (r0 >= d.rows_padded) return;  // no workgroup barrier below
    const uint8_t *base;
    if constexpr (SRC == kSrcTables) {
        base = tables[mat];
    } else {
        const uint32_t S = SRC == kSrcSlotGateUp ? gridDim.y / 2 : gridDim.y;
        const uint32_t slot = mat % S;
        const SlotRec rec = load_slot(&plan->slots[slot]);
        if (rec.token < 0) return;  // routing failed: no work
        // a select, not an index: a dynamic index would move the record to LDS
        base = SRC == kSrcSlotGateUp ? (mat < S ? rec.mat[0] : rec.mat[1]) : rec.mat[2];
        if constexpr (SRC != kSrcSlotDownSwiglu)
            q8 += (size_t)(SRC == kSrcSlotGateUp ? (uint32_t)rec.token : slot) * d.blocks_padded *
                  kQ8KRecDwords;
    }
    const RowLane W = row_lane(base, d.blocks_padded);
    const uint32_t rl = r0 + jg * 8;
    const uint32_t nb = d.blocks >> 3;
    const uint32_t chunks = d.blocks_padded / LPR;
    const size_t rstride = (size_t)d.blocks_padded * kQ8KRecDwords;
    const uint32_t bp = d.blocks_padded;
    const uint8_t *dm_row = base + q4k_dm_offset(d, rl + k, 0);
    float(*my)[9] = lds[wave];
    const int gbase = jg * LPR;
    for (uint32_t t0 = 0; t0 < m; t0 += TG) {
        float acc[TG][NCH];
#pragma unroll
        for (int t = 0; t < TG; ++t)
#pragma unroll
            for (int q = 0; q < NCH; ++q) acc[t][q] = 0.0f;
        for (uint32_t c = 0; c < chunks; ++c) {
            const uint32_t blk = c * LPR + b;
            uint4 nib[8];
#pragma unroll
            for (int p = 0; p < 8; ++p) nib[p] = load_nibbles(W, rl + p, blk);  // row rl + (p ^ k)
            const uint4 scm = load_scales(W, rl / 8, blk);
            const uint32_t dmw = *(const __attribute__((address_space(1))) uint32_t *)(dm_row + (size_t)(blk >> 3) * 32);
            uint4 xa[TG], xb[TG], xc[TG];
#pragma unroll
            for (int t = 0; t < TG; ++t) {
                if constexpr (SRC == kSrcSlotDownSwiglu) {
                    xa[t] = s_rec[blk];
                    xb[t] = s_rec[bp + blk];
                    xc[t] = s_rec[2 * bp + blk];
                } else {
                    const uint32_t tt = t0 + t < m ? t0 + t : 0;
                    const uint32_t *xr = q8 + tt * rstride + 4 * blk;
                    xa[t] = load_global_u4(xr);
                    xb[t] = load_global_u4(xr + 4 * bp);
                    xc[t] = load_global_u4(xr + 8 * bp);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            uint32_t scp[8], mnp[8];  // (sc, m) of row p ^ k, stored in position p
#pragma unroll
            for (int p = 0; p < 8; ++p) octet_sc_m(scm, p, scp[p], mnp[p]);
            const float ws = f16_to_f32(dmw), ms = f16_to_f32(dmw >> 16);
#pragma unroll
            for (int t = 0; t < TG; ++t) {
                const int qd[8] = {(int)xa[t].x, (int)xa[t].y, (int)xa[t].z, (int)xa[t].w,
                                   (int)xb[t].x, (int)xb[t].y, (int)xb[t].z, (int)xb[t].w};
                const int s32 = (int)xc[t].x;
                const float qscale = __uint_as_float(xc[t].y);
                // class dots of every slot; slots 4..7 are scaled and handed
                // to the half-mirror partner, whose slots 0..3 take them in
                // the same multiply-add as their own scaling (the first
                // butterfly stage)
                int D[64], L[32], bm[8];
#pragma unroll
                for (int p = 0; p < 8; ++p) {
                    const uint32_t wv[4] = {nib[p].x, nib[p].y, nib[p].z, nib[p].w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int lo = (int)(wv[i] & 0x0F0F0F0Fu), hi = (int)((wv[i] >> 4) & 0x0F0F0F0Fu);
                        D[8 * p + 2 * i] = __builtin_amdgcn_sdot4(lo, qd[2 * i], 0, false);
                        D[8 * p + 2 * i + 1] = __builtin_amdgcn_sdot4(hi, qd[2 * i + 1], 0, false);
                    }
                    bm[p] = __mul24((int)mnp[p], s32);
                }
#pragma unroll
                for (int p = 0; p < 4; ++p)
#pragma unroll
                    for (int cc = 0; cc < 8; ++cc) {
                        const int sent = __mul24((int)scp[p ^ 7], D[8 * (p ^ 7) + cc]);
                        L[8 * p + cc] = __mul24((int)scp[p], D[8 * p + cc]) + dpp_i<kDppHalfMirror>(sent);
                    }
                xor_stage<kDppQuadRev, 3, 4>(L);
                xor_stage<kDppXor1, 1, 2>(L);
                xor_stage1<kDppHalfMirror, 7, 8>(bm);
                xor_stage1<kDppQuadRev, 3, 4>(bm);
                xor_stage1<kDppXor1, 1, 2>(bm);
                const float cs = __fmul_rn(ws, qscale), mcs = __fmul_rn(ms, qscale);
#pragma unroll
                for (int cc = 0; cc < 8; ++cc) my[lane][cc] = __fmul_rn(cs, (float)L[cc]);
                my[lane][8] = __fmul_rn(mcs, (float)bm[0]);
                wave_sync();
#pragma unroll
                for (int q = 0; q < NCH; ++q) {
                    const int ch = g + q * SB;
                    if (ch < 9) {
#pragma unroll
                        for (int gg = 0; gg < SB; ++gg) {
                            if (c * SB + gg < nb) {
                                const float v = my[gbase + 8 * gg + k][ch];
                                acc[t][q] = ch < 8 ? __fadd_rn(acc[t][q], v) : __fsub_rn(acc[t][q], v);
                            }
                        }
                    }
                }
                wave_sync();
            }
        }
#pragma unroll
        for (int t = 0; t < TG; ++t) {
#pragma unroll
            for (int q = 0; q < NCH; ++q) my[lane][q] = acc[t][q];
            wave_sync();
            if (g == 0 && rl + k < d.rows && t0 + t < m) {
                float total = -0.0f;  // Iterator::sum::<f32>() starts from -0.0
#pragma unroll
                for (int ch = 0; ch < 8; ++ch) total = __fadd_rn(total, my[gbase + 8 * (ch % SB) + k][ch / SB]);
                const float minimum = my[gbase + 8 * (8 % SB) + k][8 / SB];
                float *dst = &y[((size_t)mat * m + t0 + t) * d.rows + rl + k];
                if (SRC == kSrcSlotDownSwiglu && fold.out) store_coherent(dst, __fadd_rn(minimum, total));
                else *dst = __fadd_rn(minimum, total);
            }
            wave_sync();
        }
    }
    if constexpr (SRC == kSrcSlotDownSwiglu) {
        if (!fold.out) return;
        __shared__ int s_last;
        const uint32_t tile = blockIdx.x, tiles = gridDim.x;
        const int token = plan->slots[mat].token;  // >= 0: slots without work left above
        wait_own_stores();
        __syncthreads();
        if (threadIdx.x == 0)
            s_last = counter_arrive(&fold.counters[(uint32_t)token * tiles + tile]) == (uint32_t)kTopK ? 1 : 0;
        __syncthreads();
        if (!s_last) return;
        const uint32_t H = d.rows, rows_per_tile = H / tiles;
        const float coef = plan->slots[token].coef;
        for (uint32_t r = threadIdx.x; r < rows_per_tile; r += blockDim.x) {
            const uint32_t c = tile * rows_per_tile + r;
            float o = __fmul_rn(load_coherent(&y[(size_t)token * H + c]), coef);
#pragma unroll
            for (int kk = 0; kk < kTopK; ++kk) {
                const int slot = plan->pair_slot[token * kTopK + kk];
                o = __fadd_rn(o, __fmul_rn(load_coherent(&y[(size_t)slot * H + c]), plan->weights[token][kk]));
            }
            const size_t i = (size_t)token * H + c;
            if (fold.resid) o = __fadd_rn(fold.resid[i], o);
            fold.out[i] = o;
        }
        if (threadIdx.x == 0) counter_reset(&fold.counters[(uint32_t)token * tiles + tile]);
    }
}

template <int LPR>
hipError_t launch_q4k_q8k_lpr(hipStream_t s, const uint8_t *const *tables, uint32_t count,
                              const MatrixDims &d, const uint32_t *q8, uint32_t m, float *y) {
    constexpr uint32_t rows_per_group = kQ4KWaves * 8 * (kWave / LPR);
    const dim3 grid((d.rows_padded + rows_per_group - 1) / rows_per_group, count);
    const dim3 block(kQ4KWaves * kWave);
    const Plan *none = nullptr;
    const float *nogu = nullptr;
    if (m <= 1)
        hipLaunchKernelGGL((q4k_q8k_gemv_kernel<LPR, 1, kSrcTables>), grid, block, 0, s, tables, none, d, q8, m, y, nogu, Fold{});
    else if (m <= 2)
        hipLaunchKernelGGL((q4k_q8k_gemv_kernel<LPR, 2, kSrcTables>), grid, block, 0, s, tables, none, d, q8, m, y, nogu, Fold{});
    else
        hipLaunchKernelGGL((q4k_q8k_gemv_kernel<LPR, 4, kSrcTables>), grid, block, 0, s, tables, none, d, q8, m, y, nogu, Fold{});
    return hipGetLastError();
}

template <int LPR>
hipError_t launch_q4k_q8k_slots_lpr(hipStream_t s, const Plan *plan, uint32_t n_slots, bool down,
                                    const MatrixDims &d, const uint32_t *q8, float *y, const float *gu,
                                    const Fold &fold) {
    constexpr uint32_t rows_per_group = kQ4KWaves * 8 * (kWave / LPR);
    const dim3 grid((d.rows_padded + rows_per_group - 1) / rows_per_group, down ? n_slots : 2 * n_slots);
    const dim3 block(kQ4KWaves * kWave);
    const uint8_t *const *none = nullptr;
    // the fold needs every wavefront of every workgroup to own rows
    if (fold.out && (!down || !gu || d.rows % rows_per_group || d.rows_padded != d.rows)) return hipErrorInvalidValue;
    if (down && gu)
        hipLaunchKernelGGL((q4k_q8k_gemv_kernel<LPR, 1, kSrcSlotDownSwiglu>), grid, block, 0, s, none, plan, d,
                           q8, 1u, y, gu, fold);
    else if (down)
        hipLaunchKernelGGL((q4k_q8k_gemv_kernel<LPR, 1, kSrcSlotDown>), grid, block, 0, s, none, plan, d, q8, 1u, y,
                           gu, Fold{});
    else
        hipLaunchKernelGGL((q4k_q8k_gemv_kernel<LPR, 1, kSrcSlotGateUp>), grid, block, 0, s, none, plan, d, q8, 1u,
                           y, gu, Fold{});
    return hipGetLastError();
}

hipError_t launch_q4k_q8k_gemv(hipStream_t s, const uint8_t *const *tables, uint32_t count,
                               const MatrixDims &d, const uint32_t *q8, uint32_t m, float *y) {
    if (d.lpr == 16) return launch_q4k_q8k_lpr<16>(s, tables, count, d, q8, m, y);
    if (d.lpr == 32) return launch_q4k_q8k_lpr<32>(s, tables, count, d, q8, m, y);
    return launch_q4k_q8k_lpr<64>(s, tables, count, d, q8, m, y);
}

hipError_t launch_q4k_q8k_slots(hipStream_t s, const Plan *plan, uint32_t n_slots, bool down,
                                const MatrixDims &d, const uint32_t *q8, float *y, const float *gu,
                                float *out, const float *resid, uint32_t *counters) {
    if (n_slots == 0 || n_slots > (uint32_t)kMaxSlots) return hipErrorInvalidValue;
    if (gu && (!down || d.blocks_padded > (uint32_t)kMaxRecBp || d.cols % 256)) return hipErrorInvalidValue;
    if (out && (!counters || n_slots % (kTopK + 1))) return hipErrorInvalidValue;
    const Fold fold{out, resid, counters};
    if (d.lpr == 16) return launch_q4k_q8k_slots_lpr<16>(s, plan, n_slots, down, d, q8, y, gu, fold);
    if (d.lpr == 32) return launch_q4k_q8k_slots_lpr<32>(s, plan, n_slots, down, d, q8, y, gu, fold);
    return launch_q4k_q8k_slots_lpr<64>(s, plan, n_slots, down, d, q8, y, gu, fold);
}

uint32_t q4k_fold_tiles(const MatrixDims &d) {
    const uint32_t rows_per_group = kQ4KWaves * 8 * (kWave / d.lpr);
    return (d.rows_padded + rows_per_group - 1) / rows_per_group;
}

bool q4k_fold_ok(const MatrixDims &d) {
    const uint32_t rows_per_group = kQ4KWaves * 8 * (kWave / d.lpr);
    return d.rows % rows_per_group == 0 && d.rows_padded == d.rows && d.blocks_padded <= (uint32_t)kMaxRecBp &&
           d.cols % 256 == 0 && q4k_fold_tiles(d) <= d.rows / 64;
}

// ---------------------------------------------------------------------------
// The MoE layer's combine (experts/mod.rs:1556-1568 per row, the arithmetic
// of :1610-1632): output = shared down x sigmoid(shared gate logit)
// (scale_in_place), then output += routed down x weight for each route in
// route order (add_scaled_in_place, weights.rs:267-281), each step one f32
// multiply and one f32 add; the stack's residual is added last
// (runtime.rs:777-802: h + moe(norm(h))).  One thread per (token, column).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void q4k_moe_combine_kernel(const Plan *__restrict__ plan,
                                                              const float *__restrict__ dn,
                                                              uint32_t m, uint32_t H,
                                                              const float *resid, float *y) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m * H || plan->status != 0) return;
    const uint32_t t = i / H, c = i % H;
    float o = __fmul_rn(dn[(size_t)t * H + c], plan->slots[t].coef);
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
        const int slot = plan->pair_slot[t * kTopK + k];
        o = __fadd_rn(o, __fmul_rn(dn[(size_t)slot * H + c], plan->weights[t][k]));
    }
    if (resid) o = __fadd_rn(resid[i], o);
    y[i] = o;
}

hipError_t launch_q4k_moe_combine(hipStream_t s, const Plan *plan, const float *dn, uint32_t m,
                                  uint32_t hidden, const float *resid, float *y) {
    const uint32_t n = m * hidden;
    hipLaunchKernelGGL(q4k_moe_combine_kernel, dim3((n + 255) / 256), dim3(256), 0, s, plan, dn, m,
                       hidden, resid, y);
    return hipGetLastError();
}

}  // namespace tqf
