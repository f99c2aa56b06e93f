// tqf_q6k.hip -- canonical Q6_K matrices (GGML super-blocks of 256 elements,
// 210 bytes: ql[128] low nibbles, qh[64] two high bits, 16 signed group
// scales, f16 d; format/quant/dequant.rs:190-218) on gfx950: the LM head of
// the canonical checkpoint (model/qwen36/runtime.rs:435, weights.rs:
// 1744).
//
//   * the lossless repack into the Q6_K row-lane layout (tqf_internal.h);
//   * the Q8_K integer matvec of matvec_payload for GgmlType::Q6K
//     (weights.rs:680-735, q6_k_dot_pre :1023-1101), bit-identical to the
//     scalar loop: exact integer lane sums, then the f32 combine in the
//     reference's order (per row, super-block after super-block, no fused
//     multiply-adds, the final iterator sum from -0.0);
//   * an optional fused top-4 epilogue with top_logit_candidates' semantics
//     (runtime/decode.rs:48-64: strict >, NaN and -inf never selected, ties
//     to the lower token), merged over workgroups by q6k_top4_merge_kernel.
#include <hip/hip_runtime.h>

#include "tqf_device.h"
#include "tqf_internal.h"

namespace tqf {

// ---------------------------------------------------------------------------
// Repack: GGML Q6_K -> Q6_K row-lane layout, one thread per (row, sub-block).
// Sub-block j (elements 32j..32j+31) of a super-block is, in ggml's order,
// group j mod 4 of half j / 4: element i takes the low nibble of ql[64 h +
// i] (j mod 4 = 0), ql[64 h + 32 + i] (1), the high nibble of ql[64 h + i]
// (2) or of ql[64 h + 32 + i] (3), and bits 2 (j mod 4) of qh[32 h + i];
// its scales are groups 2j and 2j + 1.  Stored per (octet, sub-block), in
// the XOR-permuted row positions of the Q4_K layout:
//   nibble slot   16 bytes, class order (byte 4i + t: element 2i + 8t low,
//                 2i + 1 + 8t high)
//   high-bit slot 8 bytes: dword c / 4, byte t, bits 2 (c mod 4) hold the
//                 high bits of element c + 8t with the upper bit flipped,
//                 so that (low | high << 4) is the 6-bit two's complement
//                 of q - 32
//   scale slot    2 bytes (int8 scales of groups 2j, 2j + 1)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void q6k_repack_kernel(const uint8_t *__restrict__ aos,
                                                         MatrixDims d, uint8_t *__restrict__ dst) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)d.rows * d.blocks) return;
    const uint32_t r = (uint32_t)(idx / d.blocks), b = (uint32_t)(idx % d.blocks);
    const uint32_t s = b >> 3;
    const int j = (int)(b & 7), h = j >> 2, grp = j & 3;
    const uint8_t *src = aos + ((size_t)r * (d.blocks >> 3) + s) * kQ6KBlock;
    const uint8_t *ql = src + 64 * h + ((grp & 1) ? 32 : 0);
    const uint8_t *qh = src + 128 + 32 * h;
    uint8_t lo[32], hi[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        lo[i] = (grp < 2) ? (ql[i] & 15) : (ql[i] >> 4);
        hi[i] = ((qh[i] >> (2 * grp)) & 3) ^ 2;
    }
    const size_t pr = q6k_slot_row(r, b);
    uint8_t *nib = dst + q6k_nibble_offset(d, pr, b);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int t = 0; t < 4; ++t) nib[4 * i + t] = (uint8_t)(lo[2 * i + 8 * t] | (lo[2 * i + 1 + 8 * t] << 4));
    uint8_t *hb = dst + q6k_high_offset(d, pr, b);
#pragma unroll
    for (int w = 0; w < 2; ++w)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t v = 0;
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) v |= (uint32_t)hi[4 * w + cc + 8 * t] << (2 * cc);
            hb[4 * w + t] = (uint8_t)v;
        }
    uint8_t *sc = dst + q6k_scale_offset(d, pr, b);
    sc[0] = src[192 + 2 * j];
    sc[1] = src[192 + 2 * j + 1];
    if (j == 0) {
        uint8_t *dd = dst + q6k_d_offset(d, r, s);
        dd[0] = src[208];
        dd[1] = src[209];
    }
}

hipError_t launch_q6k_repack(hipStream_t s, const uint8_t *d_aos, const MatrixDims &d,
                             uint8_t *dst) {
    const uint64_t n = (uint64_t)d.rows * d.blocks;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(q6k_repack_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s,
                       d_aos, d, dst);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Q8_K integer matvec (q6_k_dot_pre per row) over the Q8_K records of
// q8k_quantize_kernel (tqf_q4k.hip).  Geometry of the Q4_K matvec: lane b of
// a lane group owns sub-block b of the chunk for the octet's eight rows,
// register slot p holding row p ^ k (k = b mod 8).
//
// Per (slot, class c): the class's four values 4 (q - 32) (the stored 6-bit
// two's complement shifted left by two) times their group's int8 scale, as
// two int16 pairs (group 2j, group 2j + 1) formed once per chunk for all
// tokens, dotted with the class's Q8_K bytes as int16 pairs by two
// v_dot2_i32_i16: 4 x the reference's lane-sum term, exactly (|4 L| < 2^27).
// The butterfly of the Q4_K kernel sums a super-block's eight lanes; the combine
// sums[c] += (d * q8scale) * lane_sum runs super-block after super-block
// through LDS, and the row's first lane forms -0.0 + sums[0] + ... + sums[7].
//
// TOPK: the workgroup's rows also yield per-token top-4 candidates
// (top_logit_candidates' order) at cand[(blockIdx.x * m + t) * 4 ..].
// ---------------------------------------------------------------------------
constexpr int kQ6KWaves = 8;

struct Top4Cand {
    uint32_t token;
    float value;
};

// Top-4 of one value per lane over the wavefront (value, token), NaN and
// -inf excluded; results in every lane, empty slots (0, -inf).
__device__ __forceinline__ void wave_top4(float v, uint32_t tok, float (&bv)[4], uint32_t (&bt)[4]) {
    bool live = v > -INFINITY;  // false for NaN and -inf
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const float mv = group_reduce<64>(live ? v : -INFINITY, MaxOp());
        const int mt = group_reduce<64>((live && v == mv) ? (int)tok : 0x7FFFFFFF, MinOp());
        const bool found = mv > -INFINITY;
        bv[s] = found ? mv : -INFINITY;
        bt[s] = found ? (uint32_t)mt : 0u;
        if (found && live && v == mv && (int)tok == mt) live = false;
    }
}

template <typename T>
__device__ __forceinline__ T pick4(const T (&a)[4], int s) {
    return s == 0 ? a[0] : s == 1 ? a[1] : s == 2 ? a[2] : a[3];
}

// Folds one candidate per lane (lanes >= kTop4Lanes: ignored) into the
// running top-4 `best` (uniform): the running entries ride in the last four
// lanes of the same ranking.
constexpr int kTop4Lanes = kWave - 4;
__device__ __forceinline__ void fold_top4(float v, uint32_t tok, float (&best)[4], uint32_t (&btok)[4]) {
    const int lane = threadIdx.x % kWave;
    const int s = lane - kTop4Lanes;
    const float fv = s >= 0 ? pick4(best, s) : v;
    const uint32_t ft = s >= 0 ? pick4(btok, s) : tok;
    wave_top4(fv, ft, best, btok);
}

// int16 pairs for the int16 dot products: SDWA byte selects with sign
// extension, two instructions a pair.  scaled_pair<A, S>: bytes A and A + 1 of
// v, each times byte S of s (all signed; |product| <= 2^14, exact in int16).
// sext_pair<A>: bytes A and A + 1 of v.
template <int A, int S>
__device__ __forceinline__ uint32_t scaled_pair(uint32_t v, uint32_t s);
#define TQF_SCALED_PAIR(A0, A1, S)                                                                         \
    template <>                                                                                           \
    __device__ __forceinline__ uint32_t scaled_pair<A0, S>(uint32_t v, uint32_t s) {                    \
        uint32_t r;                                                                                       \
        asm("v_mul_lo_u16_sdwa %0, sext(%1), sext(%2) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_" #A0 \
            " src1_sel:BYTE_" #S                                                                          \
            : "=v"(r)                                                                                     \
            : "v"(v), "v"(s));                                                                            \
        asm("v_mul_lo_u16_sdwa %0, sext(%1), sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_" #A1 \
            " src1_sel:BYTE_" #S                                                                          \
            : "+v"(r)                                                                                     \
            : "v"(v), "v"(s));                                                                            \
        return r;                                                                                         \
    }
TQF_SCALED_PAIR(0, 1, 0)
TQF_SCALED_PAIR(0, 1, 2)
TQF_SCALED_PAIR(2, 3, 1)
TQF_SCALED_PAIR(2, 3, 3)
#undef TQF_SCALED_PAIR
template <int A>
__device__ __forceinline__ uint32_t sext_pair(uint32_t v);
#define TQF_SEXT_PAIR(A0, A1)                                                                             \
    template <>                                                                                           \
    __device__ __forceinline__ uint32_t sext_pair<A0>(uint32_t v) {                                      \
        uint32_t r;                                                                                       \
        asm("v_mov_b32_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_" #A0         \
            : "=v"(r)                                                                                     \
            : "v"(v));                                                                                    \
        asm("v_mov_b32_sdwa %0, sext(%1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_" #A1    \
            : "+v"(r)                                                                                     \
            : "v"(v));                                                                                    \
        return r;                                                                                         \
    }
TQF_SEXT_PAIR(0, 1)
TQF_SEXT_PAIR(2, 3)
#undef TQF_SEXT_PAIR
// A lane-permuting move whose every source lane is in range (mirrors and
// quad permutations): no old value to keep, so no register set up for one.
template <int CTRL>
__device__ __forceinline__ int dppz_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
// A token's eight Q8_K class dwords (record planes 0, 1 of one block) as
// int16 pairs: qa[c] = bytes 0, 1 (group 2j), qb[c] = bytes 2, 3 (group 2j + 1).
__device__ __forceinline__ void q8_class_pairs(const uint4 &xa, const uint4 &xb, uint32_t (&qa)[8],
                                               uint32_t (&qb)[8]) {
    const uint32_t qd[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
        qa[cc] = sext_pair<0>(qd[cc]);
        qb[cc] = sext_pair<2>(qd[cc]);
    }
}
// lo(a) lo(b) + hi(a) hi(b) (+ c) over signed int16 halves, exact in int32;
// the first form starts from an inline zero (no accumulator register).
__device__ __forceinline__ int dot2_i16_0(uint32_t a, uint32_t b) {
    int r;
    asm("v_dot2_i32_i16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ int dot2_i16(uint32_t a, uint32_t b, int c) {
    typedef short short2_t __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, a), __builtin_bit_cast(short2_t, b), c, false);
}

// One lane's share of a row octet's chunk for TG tokens: its sub-block's
// 6-bit values (nibbles nib, high bits hiv) and int8 group scales scv against
// each token's Q8_K class bytes as int16 pairs (xrec(t, qa, qb): qa[c] the
// class's group-2j bytes, qb[c] its group-2j+1 bytes), reduced over the
// super-block's eight lanes; sink(t, L) receives token t's L[cc] = 4 x the
// reference's lane sum of class cc for row (lane mod 8) of the octet in this
// super-block.
template <int TG, class XRec, class Sink>
__device__ __forceinline__ void q6k_octet_sums(const uint4 (&nib)[8], const uint4 (&hiv)[4], const uint4 &scv,
                                               XRec xrec, Sink sink) {
    // signed class values 4 (q - 32), slot-major
    int sv[64];
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const uint32_t wv[4] = {nib[p].x, nib[p].y, nib[p].z, nib[p].w};
        const uint4 hq = hiv[p >> 1];
        const uint32_t hw[2] = {(p & 1) ? hq.z : hq.x, (p & 1) ? hq.w : hq.y};
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) {
            const uint32_t w = wv[cc >> 1];
            const uint32_t lo = (cc & 1) ? ((w >> 2) & 0x3C3C3C3Cu) : ((w << 2) & 0x3C3C3C3Cu);
            const uint32_t hi = (hw[cc >> 2] << (6 - 2 * (cc & 3))) & 0xC0C0C0C0u;
            sv[8 * p + cc] = (int)(lo | hi);
        }
    }
    const uint32_t scw[4] = {scv.x, scv.y, scv.z, scv.w};
    // every value times its group's scale, once for all tokens, as int16
    // pairs (class bytes 0, 1: group 2j; bytes 2, 3: group 2j + 1;
    // |4 (q - 32) s| <= 2^14), so that a token's class term is two int16 dot2s
    uint32_t wa[64], wb[64];
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        // slot p's scales: bytes 2 (p mod 2) (group 2j) and 2 (p mod 2) + 1
        // (group 2j + 1) of scale dword p / 2
        const uint32_t sw = scw[p >> 1];
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) {
            const uint32_t v = (uint32_t)sv[8 * p + cc];
            wa[8 * p + cc] = (p & 1) ? scaled_pair<0, 2>(v, sw) : scaled_pair<0, 0>(v, sw);
            wb[8 * p + cc] = (p & 1) ? scaled_pair<2, 3>(v, sw) : scaled_pair<2, 1>(v, sw);
        }
    }
#pragma unroll
    for (int t = 0; t < TG; ++t) {
        uint32_t qa[8], qb[8];
        xrec(t, qa, qb);
        // slots p ^ 7 first: their terms move to the mirror lane (the same
        // row) and start slot p's dot2 chain
        int m7[32], L[32];
#pragma unroll
        for (int p = 0; p < 4; ++p)
#pragma unroll
            for (int cc = 0; cc < 8; ++cc)
                m7[8 * p + cc] = dot2_i16(wb[8 * (p ^ 7) + cc], qb[cc], dot2_i16_0(wa[8 * (p ^ 7) + cc], qa[cc]));
#pragma unroll
        for (int p = 0; p < 4; ++p)
#pragma unroll
            for (int cc = 0; cc < 8; ++cc)
                L[8 * p + cc] = dot2_i16(wb[8 * p + cc], qb[cc],
                                         dot2_i16(wa[8 * p + cc], qa[cc], dppz_i<kDppHalfMirror>(m7[8 * p + cc])));
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int cc = 0; cc < 8; ++cc) L[8 * p + cc] += dppz_i<kDppQuadRev>(L[8 * (p ^ 3) + cc]);
        int Lc[8];
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) Lc[cc] = L[cc] + dppz_i<kDppXor1>(L[8 + cc]);
        sink(t, Lc);
    }
}

template <int LPR, int TG, bool TOPK>
__global__ __launch_bounds__(kQ6KWaves * kWave) void q6k_q8k_gemv_kernel(
    const uint8_t *const *__restrict__ tables, MatrixDims d, const uint32_t *__restrict__ q8,
    uint32_t m, float *__restrict__ y, Top4Cand *__restrict__ cand) {
    constexpr int G = kWave / LPR;
    constexpr int SB = LPR / 8;
    constexpr int NCH = (8 + SB - 1) / SB;
    __shared__ float lds[kQ6KWaves][kWave][8];
    __shared__ float s_res[TOPK ? TG : 1][kQ6KWaves * 8 * G];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int jg = lane / LPR, b = lane % LPR, k = b & 7, g = b >> 3;
    const uint32_t mat = blockIdx.y;
    const uint32_t r0 = (blockIdx.x * kQ6KWaves + wave) * 8 * G;
    const bool active = r0 < d.rows_padded;
    if (!TOPK && !active) return;  // no workgroup barrier without TOPK
    const uint8_t *base = tables[mat];
    const uint32_t rl = active ? r0 + jg * 8 : 0;
    const uint32_t nb = d.blocks >> 3;
    const uint32_t chunks = d.blocks_padded / LPR;
    const size_t rstride = (size_t)d.blocks_padded * kQ8KRecDwords;
    const uint32_t bp = d.blocks_padded;
    const uint8_t *oct = base + q6k_nibble_offset(d, rl, 0);  // the octet chunk
    const uint8_t *d_row = base + q6k_d_offset(d, rl + k, 0);
    float(*my)[8] = lds[wave];
    const int gbase = jg * LPR;
    for (uint32_t t0 = 0; t0 < m; t0 += TG) {
        float acc[TG][NCH];
#pragma unroll
        for (int t = 0; t < TG; ++t)
#pragma unroll
            for (int q = 0; q < NCH; ++q) acc[t][q] = 0.0f;
        for (uint32_t c = 0; active && c < chunks; ++c) {
            const uint32_t blk = c * LPR + b;
            uint4 nib[8], hiv[4];
#pragma unroll
            for (int p = 0; p < 8; ++p) nib[p] = load_global_u4(oct + ((size_t)p * bp + blk) * 16);
#pragma unroll
            for (int q = 0; q < 4; ++q) hiv[q] = load_global_u4(oct + ((size_t)(8 + q) * bp + blk) * 16);
            const uint4 scv = load_global_u4(oct + ((size_t)12 * bp + blk) * 16);
            const uint32_t dw = *(const __attribute__((address_space(1))) uint16_t *)(d_row + (size_t)(blk >> 3) * 16);
            uint4 xa[TG], xb[TG], xc[TG];
#pragma unroll
            for (int t = 0; t < TG; ++t) {
                const uint32_t tt = t0 + t < m ? t0 + t : 0;
                const uint32_t *xr = q8 + tt * rstride + 4 * blk;
                xa[t] = load_global_u4(xr);
                xb[t] = load_global_u4(xr + 4 * bp);
                xc[t] = load_global_u4(xr + 8 * bp);
            }
            __builtin_amdgcn_sched_barrier(0);
            const float ws = f16_to_f32(dw);
            q6k_octet_sums<TG>(
                nib, hiv, scv, [&](int t, uint32_t (&qa)[8], uint32_t (&qb)[8]) { q8_class_pairs(xa[t], xb[t], qa, qb); },
                [&](int t, const int (&L)[8]) {
                    const float cs = __fmul_rn(ws, __uint_as_float(xc[t].y));
#pragma unroll
                    for (int cc = 0; cc < 8; ++cc) my[lane][cc] = __fmul_rn(cs, (float)(L[cc] >> 2));
                    wave_sync();
#pragma unroll
                    for (int q = 0; q < NCH; ++q) {
                        const int ch = g + q * SB;
                        if (ch < 8) {
#pragma unroll
                            for (int gg = 0; gg < SB; ++gg)
                                if (c * SB + gg < nb) acc[t][q] = __fadd_rn(acc[t][q], my[gbase + 8 * gg + k][ch]);
                        }
                    }
                    wave_sync();
                });
        }
#pragma unroll
        for (int t = 0; t < TG; ++t) {
            float res = 0.0f;
            if (active) {
#pragma unroll
                for (int q = 0; q < NCH; ++q) my[lane][q] = acc[t][q];
                wave_sync();
                float total = -0.0f;  // Iterator::sum::<f32>() starts from -0.0
#pragma unroll
                for (int ch = 0; ch < 8; ++ch) total = __fadd_rn(total, my[gbase + 8 * (ch % SB) + k][ch / SB]);
                res = total;
                if (g == 0 && rl + k < d.rows && t0 + t < m)
                    y[((size_t)mat * m + t0 + t) * d.rows + rl + k] = res;
                wave_sync();
            }
            if constexpr (TOPK) {
                if (g == 0) s_res[t][(wave * G + jg) * 8 + k] = (active && rl + k < d.rows) ? res : -INFINITY;
            }
        }
        if constexpr (TOPK) {
            __syncthreads();
            // wavefront t ranks token t0 + t over the workgroup's rows
            if (wave < TG && t0 + wave < m) {
                constexpr int NR = kQ6KWaves * 8 * G;
                float best[4];
                uint32_t btok[4];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    best[s] = -INFINITY;
                    btok[s] = 0;
                }
                const uint32_t row0 = blockIdx.x * kQ6KWaves * 8 * G;
                for (int i0 = 0; i0 < NR; i0 += kTop4Lanes) {
                    const int i = i0 + lane;
                    const bool in = lane < kTop4Lanes && i < NR;
                    fold_top4(in ? s_res[wave][in ? i : 0] : -INFINITY, row0 + (uint32_t)i, best, btok);
                }
                if (lane < 4) cand[((size_t)blockIdx.x * m + t0 + wave) * 4 + lane] = Top4Cand{pick4(btok, lane), pick4(best, lane)};
            }
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------------------
// The same matvec at the LM head's geometry (Bp = 64: one 64-lane chunk per
// row octet): a fixed grid of four-wavefront workgroups, each wavefront
// walking row octets o = first, first + W, ... (W wavefronts in the grid).
// The next octet's 13 KiB (nibbles, high bits, scales) is copied into the
// wavefront's LDS buffer (global_load_lds) while the current one computes
// from registers, so the weight stream runs on through the integer work; the
// tokens' Q8_K records are the same for every octet and stay in registers.
// Results as q6k_q8k_gemv_kernel; the top-4 candidates are per workgroup over
// all its octets.
// ---------------------------------------------------------------------------
constexpr int kQ6SWaves = 4;
constexpr uint32_t kQ6SGroups = 512;  // two workgroups per CU on a 256-CU part

__device__ __forceinline__ void q6k_copy_to_lds_16(const void *gaddr, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(gaddr) : "memory", "m0");
}

__host__ __device__ inline bool q6k_streams(const MatrixDims &d) { return d.blocks_padded == 64; }

__host__ __device__ inline uint32_t q6k_stream_groups(const MatrixDims &d) {
    const uint32_t octets = d.rows_padded >> 3;
    const uint32_t need = (octets + kQ6SWaves - 1) / kQ6SWaves;
    return need < kQ6SGroups ? need : kQ6SGroups;
}

// Per token: the top-4 of the workgroups' candidate lists (one workgroup of
// 1024 threads per token; every list is sorted, so the union's top-4 in
// top_logit_candidates' order is the answer).  Every thread loads its share
// first (one round trip), keeps a local top-4 by insertion, then the lists
// are merged per wavefront (four rounds of "largest head, lowest token") and
// across the 16 wavefronts in LDS.
__device__ __forceinline__ bool cand_before(float va, uint32_t ta, float vb, uint32_t tb) {
    return va > vb || (va == vb && ta < tb);
}

// Top-4 over the wavefront of per-lane sorted lists of four (value, token),
// empty entries (0, -inf); results uniform.
__device__ __forceinline__ void wave_merge4(float (&lv)[4], uint32_t (&lt)[4], float (&bv)[4],
                                            uint32_t (&bt)[4]) {
    int head = 0;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const float hv = head < 4 ? pick4(lv, head) : -INFINITY;
        const uint32_t ht = head < 4 ? pick4(lt, head) : 0u;
        const bool live = hv > -INFINITY;
        const float mv = group_reduce<64>(live ? hv : -INFINITY, MaxOp());
        const int mt = group_reduce<64>((live && hv == mv) ? (int)ht : 0x7FFFFFFF, MinOp());
        const bool found = mv > -INFINITY;
        bv[s] = found ? mv : -INFINITY;
        bt[s] = found ? (uint32_t)mt : 0u;
        if (found && live && hv == mv && (int)ht == mt) ++head;
    }
}

// Exchanges lane bits 3..5 with the register index: afterwards lane (g, k)
// (g = lane / 8) holds in v[e] what lane (e, k) held in v[g].  Three
// butterfly stages: lane bit 5 by v_permlane32_swap, bit 4 by
// v_permlane16_swap, bit 3 by row_ror:8 moves written to one half-row each.
__device__ __forceinline__ void transpose8_lanes(float (&v)[8]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[c]), __float_as_uint(v[c + 4]), false, false);
        v[c] = __uint_as_float(r[0]);
        v[c + 4] = __uint_as_float(r[1]);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        if (c & 2) continue;
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[c]), __float_as_uint(v[c + 2]), false, false);
        v[c] = __uint_as_float(r[0]);
        v[c + 2] = __uint_as_float(r[1]);
    }
#pragma unroll
    for (int c = 0; c < 8; c += 2) {
        const int lo = __float_as_int(v[c]), hi = __float_as_int(v[c + 1]);
        // lanes 8..15 of a row (banks 2, 3) take the partner's v[c + 1] into
        // v[c]; lanes 0..7 (banks 0, 1) the partner's v[c] into v[c + 1]
        v[c] = __int_as_float(__builtin_amdgcn_update_dpp(lo, hi, 0x128, 0xF, 0xC, false));
        v[c + 1] = __int_as_float(__builtin_amdgcn_update_dpp(hi, lo, 0x128, 0xF, 0x3, false));
    }
}

template <int TG, bool TOPK>
__global__ __launch_bounds__(kQ6SWaves * kWave, 2) void q6k_q8k_stream_kernel(
    const uint8_t *const *__restrict__ tables, MatrixDims d, const uint32_t *__restrict__ q8,
    uint32_t m, float *__restrict__ y, Top4Cand *__restrict__ cand) {
    __shared__ uint4 s_buf[kQ6SWaves][13][kWave];
    __shared__ uint4 s_x[TG][4][kWave];  // the tokens' Q8_K class bytes as int16 pairs
    __shared__ float s_acc[kQ6SWaves][TG][kWave];
    __shared__ Top4Cand s_cand[TOPK ? TG : 1][kQ6SWaves * 8][4];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int k = lane & 7, g = lane >> 3;
    const uint8_t *base = tables[blockIdx.y];
    const uint32_t n_oct = d.rows_padded >> 3;
    const uint32_t W = gridDim.x * kQ6SWaves;
    const uint32_t rounds = (n_oct + W - 1) / W;  // the same in every wavefront
    const uint32_t first = blockIdx.x * kQ6SWaves + wave;
    const size_t rstride = (size_t)64 * kQ8KRecDwords;
    const uint32_t nb = d.blocks >> 3;
    const uint8_t *d_base = base + q6k_d_base(d);
    const uint32_t buf = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)(
        reinterpret_cast<uint8_t *>(&s_buf[wave][0][0]));
    // octet o: its 13 KiB chunk into the buffer, and its lanes' f16 scales d
    // (row 8 o + k, super-block g)
    auto issue = [&](uint32_t o, uint32_t &dw) {
        const uint8_t *oct = base + (size_t)o * 13 * 1024 + (size_t)lane * 16;
#pragma unroll
        for (int i = 0; i < 13; ++i) q6k_copy_to_lds_16(oct + i * 1024, buf + i * 1024);
        dw = *(const __attribute__((address_space(1))) uint16_t *)(d_base + (size_t)o * 128 + lane * 2);
    };
    for (uint32_t t0 = 0; t0 < m; t0 += TG) {
        // token t0 + t's records: class dwords into LDS (wavefront t % 4), the
        // scale of the lane's super-block in a register
        float qscale[TG];
#pragma unroll
        for (int t = 0; t < TG; ++t) {
            const uint32_t tt = t0 + t < m ? t0 + t : 0;
            const uint32_t *xr = q8 + tt * rstride + 4 * lane;
            if (t % kQ6SWaves == wave) {
                uint32_t qa[8], qb[8];
                q8_class_pairs(load_global_u4(xr), load_global_u4(xr + 4 * 64), qa, qb);
                s_x[t][0][lane] = make_uint4(qa[0], qa[1], qa[2], qa[3]);
                s_x[t][1][lane] = make_uint4(qa[4], qa[5], qa[6], qa[7]);
                s_x[t][2][lane] = make_uint4(qb[0], qb[1], qb[2], qb[3]);
                s_x[t][3][lane] = make_uint4(qb[4], qb[5], qb[6], qb[7]);
            }
            qscale[t] = __uint_as_float(xr[8 * 64 + 1]);
        }
        __syncthreads();
        // lane (g, k), g < TG: the top-4 of token t0 + g over the rows 8 o + k
        // of this wavefront's octets, sorted as top_logit_candidates
        float lv[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        uint32_t lt[4] = {0, 0, 0, 0};
        uint32_t dw_next = 0;
        if (first < n_oct) issue(first, dw_next);
        uint32_t o = first;
        for (uint32_t r = 0; r < rounds; ++r, o += W) {
            const bool act = o < n_oct;
            // this octet's copies (and every earlier load) are in
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            uint4 nib[8], hiv[4];
#pragma unroll
            for (int p = 0; p < 8; ++p) nib[p] = s_buf[wave][p][lane];
#pragma unroll
            for (int q = 0; q < 4; ++q) hiv[q] = s_buf[wave][8 + q][lane];
            const uint4 scv = s_buf[wave][12][lane];
            const uint32_t dw = dw_next;
            // the reads are complete before the next octet's copies reuse the buffer
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (o + W < n_oct) issue(o + W, dw_next);
            if (act) {
                const float ws = f16_to_f32(dw);
                // per token: lane (g, k) scales its super-block g's eight class
                // sums of row k, the lanes exchange them so that lane (c, k)
                // holds class c of every super-block, and sums those in
                // super-block order
                float accs[TG];
                q6k_octet_sums<TG>(
                    nib, hiv, scv,
                    [&](int t, uint32_t (&qa)[8], uint32_t (&qb)[8]) {
                        const uint4 a0 = s_x[t][0][lane], a1 = s_x[t][1][lane], b0 = s_x[t][2][lane], b1 = s_x[t][3][lane];
                        qa[0] = a0.x; qa[1] = a0.y; qa[2] = a0.z; qa[3] = a0.w;
                        qa[4] = a1.x; qa[5] = a1.y; qa[6] = a1.z; qa[7] = a1.w;
                        qb[0] = b0.x; qb[1] = b0.y; qb[2] = b0.z; qb[3] = b0.w;
                        qb[4] = b1.x; qb[5] = b1.y; qb[6] = b1.z; qb[7] = b1.w;
                    },
                    [&](int t, const int (&L)[8]) {
                        const float cs = __fmul_rn(ws, qscale[t]);
                        float v[8];
#pragma unroll
                        for (int cc = 0; cc < 8; ++cc) v[cc] = __fmul_rn(cs, (float)(L[cc] >> 2));
                        transpose8_lanes(v);
                        float acc = 0.0f;
#pragma unroll
                        for (int gg = 0; gg < 8; ++gg)
                            if (gg < (int)nb) acc = __fadd_rn(acc, v[gg]);
                        accs[t] = acc;
                    });
#pragma unroll
                for (int t = 0; t < TG; ++t) s_acc[wave][t][lane] = accs[t];
                wave_sync();
                const uint32_t row = 8 * o + k;
#pragma unroll
                for (int t = 0; t < TG; ++t) {
                    float total = -0.0f;  // Iterator::sum::<f32>() starts from -0.0
#pragma unroll
                    for (int ch = 0; ch < 8; ++ch) total = __fadd_rn(total, s_acc[wave][t][8 * ch + k]);
                    if (g == 0 && row < d.rows && t0 + t < m)
                        y[((size_t)blockIdx.y * m + t0 + t) * d.rows + row] = total;
                    if constexpr (TOPK) {
                        // rows only grow along a lane, so a tie keeps the
                        // earlier (lower) token; NaN and -inf never enter
                        if (g == t && row < d.rows && total > -INFINITY) {
                            bool placed = false;
#pragma unroll
                            for (int s2 = 0; s2 < 4; ++s2) {
                                const bool here = !placed && cand_before(total, row, lv[s2], lt[s2]);
                                if (here) {
#pragma unroll
                                    for (int u = 3; u > s2; --u) {
                                        lv[u] = lv[u - 1];
                                        lt[u] = lt[u - 1];
                                    }
                                    lv[s2] = total;
                                    lt[s2] = row;
                                    placed = true;
                                }
                            }
                        }
                    }
                }
                wave_sync();
            }
        }
        if constexpr (TOPK) {
            // the workgroup's 32 lists per token, merged by wavefront t
            if (g < TG) {
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) s_cand[g][wave * 8 + k][s2] = Top4Cand{lt[s2], lv[s2]};
            }
            __syncthreads();
            if (wave < TG && t0 + wave < m) {
                float wv[4], bv[4];
                uint32_t wt[4], bt[4];
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) {
                    const Top4Cand c = lane < kQ6SWaves * 8 ? s_cand[wave][lane][s2] : Top4Cand{0u, -INFINITY};
                    wv[s2] = c.value;
                    wt[s2] = c.token;
                }
                wave_merge4(wv, wt, bv, bt);
                if (lane < 4)
                    cand[((size_t)blockIdx.x * m + t0 + wave) * 4 + lane] = Top4Cand{pick4(bt, lane), pick4(bv, lane)};
            }
        }
        __syncthreads();  // every wavefront is done with s_x and s_cand
    }
}

constexpr int kMergeThreads = 1024;
constexpr int kMergePer = 16;  // candidates per thread and pass

__global__ __launch_bounds__(kMergeThreads) void q6k_top4_merge_kernel(const Top4Cand *__restrict__ cand,
                                                                       uint32_t n_groups, uint32_t m,
                                                                       uint32_t *__restrict__ tokens4,
                                                                       float *__restrict__ logits4) {
    __shared__ Top4Cand s_best[kMergeThreads / kWave][4];
    const uint32_t t = blockIdx.x;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    float lv[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    uint32_t lt[4] = {0, 0, 0, 0};
    const uint32_t n = n_groups * 4;
    for (uint32_t base = 0; base < n; base += kMergeThreads * kMergePer) {
        Top4Cand c[kMergePer];
#pragma unroll
        for (int q = 0; q < kMergePer; ++q) {
            const uint32_t i = base + threadIdx.x + (uint32_t)q * kMergeThreads;
            c[q] = i < n ? cand[((size_t)(i / 4) * m + t) * 4 + (i % 4)] : Top4Cand{0u, -INFINITY};
        }
#pragma unroll
        for (int q = 0; q < kMergePer; ++q) {
            const float v = c[q].value;
            const uint32_t tk = c[q].token;
            if (!(v > -INFINITY)) continue;  // NaN / -inf / empty
            // insertion into the sorted local list
            bool placed = false;
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) {
                const bool here = !placed && cand_before(v, tk, lv[s2], lt[s2]);
                if (here) {
#pragma unroll
                    for (int u = 3; u > s2; --u) {
                        lv[u] = lv[u - 1];
                        lt[u] = lt[u - 1];
                    }
                    lv[s2] = v;
                    lt[s2] = tk;
                    placed = true;
                }
            }
        }
    }
    float bv[4];
    uint32_t bt[4];
    wave_merge4(lv, lt, bv, bt);
    if (lane == 0)
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) s_best[wave][s2] = Top4Cand{bt[s2], bv[s2]};
    __syncthreads();
    if (wave == 0) {
        // lanes 0..15 hold the wavefronts' lists
        float wv[4];
        uint32_t wt[4];
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
            const Top4Cand c = lane < kMergeThreads / kWave ? s_best[lane][s2] : Top4Cand{0u, -INFINITY};
            wv[s2] = c.value;
            wt[s2] = c.token;
        }
        wave_merge4(wv, wt, bv, bt);
        if (lane < 4) {
            tokens4[t * 4 + lane] = pick4(bt, lane);
            logits4[t * 4 + lane] = pick4(bv, lane);
        }
    }
}

template <int LPR, bool TOPK>
hipError_t launch_q6k_lpr(hipStream_t s, const uint8_t *const *tables, uint32_t count,
                          const MatrixDims &d, const uint32_t *q8, uint32_t m, float *y,
                          Top4Cand *cand) {
    constexpr uint32_t rows_per_group = kQ6KWaves * 8 * (kWave / LPR);
    const dim3 grid((d.rows_padded + rows_per_group - 1) / rows_per_group, count);
    const dim3 block(kQ6KWaves * kWave);
    if (m <= 1) hipLaunchKernelGGL((q6k_q8k_gemv_kernel<LPR, 1, TOPK>), grid, block, 0, s, tables, d, q8, m, y, cand);
    else if (m <= 2) hipLaunchKernelGGL((q6k_q8k_gemv_kernel<LPR, 2, TOPK>), grid, block, 0, s, tables, d, q8, m, y, cand);
    else hipLaunchKernelGGL((q6k_q8k_gemv_kernel<LPR, 4, TOPK>), grid, block, 0, s, tables, d, q8, m, y, cand);
    return hipGetLastError();
}

template <bool TOPK>
hipError_t launch_q6k_stream(hipStream_t s, const uint8_t *const *tables, uint32_t count,
                             const MatrixDims &d, const uint32_t *q8, uint32_t m, float *y,
                             Top4Cand *cand) {
    const dim3 grid(q6k_stream_groups(d), count);
    const dim3 block(kQ6SWaves * kWave);
    if (m <= 1) hipLaunchKernelGGL((q6k_q8k_stream_kernel<1, TOPK>), grid, block, 0, s, tables, d, q8, m, y, cand);
    else if (m <= 2) hipLaunchKernelGGL((q6k_q8k_stream_kernel<2, TOPK>), grid, block, 0, s, tables, d, q8, m, y, cand);
    else hipLaunchKernelGGL((q6k_q8k_stream_kernel<4, TOPK>), grid, block, 0, s, tables, d, q8, m, y, cand);
    return hipGetLastError();
}

uint32_t q6k_top4_groups(const MatrixDims &d) {
    if (q6k_streams(d)) return q6k_stream_groups(d);
    const uint32_t rows_per_group = kQ6KWaves * 8 * (kWave / d.lpr);
    return (d.rows_padded + rows_per_group - 1) / rows_per_group;
}

size_t q6k_top4_scratch_bytes(const MatrixDims &d, uint32_t m) {
    return (size_t)q6k_top4_groups(d) * m * 4 * sizeof(Top4Cand);
}

hipError_t launch_q6k_q8k_gemv(hipStream_t s, const uint8_t *const *tables, uint32_t count,
                               const MatrixDims &d, const uint32_t *q8, uint32_t m, float *y,
                               void *top4_scratch, uint32_t *tokens4, float *logits4) {
    Top4Cand *cand = static_cast<Top4Cand *>(top4_scratch);
    hipError_t e;
    if (cand) {
        if (q6k_streams(d)) e = launch_q6k_stream<true>(s, tables, count, d, q8, m, y, cand);
        else if (d.lpr == 16) e = launch_q6k_lpr<16, true>(s, tables, count, d, q8, m, y, cand);
        else if (d.lpr == 32) e = launch_q6k_lpr<32, true>(s, tables, count, d, q8, m, y, cand);
        else e = launch_q6k_lpr<64, true>(s, tables, count, d, q8, m, y, cand);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(q6k_top4_merge_kernel, dim3(m), dim3(kMergeThreads), 0, s, cand, q6k_top4_groups(d), m,
                           tokens4, logits4);
        return hipGetLastError();
    }
    if (q6k_streams(d)) return launch_q6k_stream<false>(s, tables, count, d, q8, m, y, nullptr);
    if (d.lpr == 16) return launch_q6k_lpr<16, false>(s, tables, count, d, q8, m, y, nullptr);
    if (d.lpr == 32) return launch_q6k_lpr<32, false>(s, tables, count, d, q8, m, y, nullptr);
    return launch_q6k_lpr<64, false>(s, tables, count, d, q8, m, y, nullptr);
}

}  // namespace tqf
