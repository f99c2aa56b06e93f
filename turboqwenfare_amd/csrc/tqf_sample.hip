// tqf_sample.hip -- Sampler::select's stochastic draw, bit-identical to the
// reference (sampling/mod.rs:68-106, 166-190, 227-266) for the filters the
// verify configuration uses (no repetition penalties, top_k, top_p or min_p:
// the early returns of apply_penalties, apply_top_k, apply_top_p and
// apply_min_p at their defaults).  Per row of logits l and uniform u (the
// draw's rng.next_f32()):
//
//   max   = fold(-inf, f32::max) over l           (NaN never wins)
//   e_x   = f32::exp((l_x - max) / T)             (ref_expf: the host expf)
//   total = -0 + e_0 + e_1 + ...                  (token order, f32, left to right)
//   p_x   = e_x / total if total > 0, else e_x
//   sort by p descending, NaN last, ties to the lower token (compare_desc
//        then token order: sort_unstable_by with a total order)
//   total2 = -0 + p_(0) + p_(1) + ...             (sorted order)
//   if total2 is not finite or <= 0: the first sorted token
//   target = u * total2; the first sorted token whose running sum
//        (from +0, sorted order) reaches target; else the last one.
//
// Every operation is the reference's, in its order: the sums are the
// sequential f32 folds themselves (one wavefront per row adds the terms one
// after another), the divisions are IEEE (correctly rounded), the sort is a
// stable descending radix sort of order-preserving keys over the token-
// ordered input.  Two shortcuts change no bit:
//   * in sorted order the terms do not increase while the running sum does
//     not decrease, so once a term is below half an ulp of the sum, that
//     term and every later one leave the sum unchanged (a tie at exactly
//     half an ulp can round up, so the test is strict): the folds stop
//     there.  A NaN (sorted last) would make total2 NaN, so a row with a NaN
//     probability takes the first sorted token without folding;
//   * the walk's running sum equals total2's fold at every position (both
//     add the same terms in the same order; -0 + p = +0 + p for p >= 0), so
//     a block whose last running sum is below target holds no hit.
//
// Kernels (rows <= 8 run side by side):
//   sel_max      chunk maxima of each row (1024 logits per workgroup)
//   sel_exp      the row maximum from the chunk maxima; e_x
//   sel_total    the token-order fold (one wavefront per row)
//   sel_keys     p_x and its sort key (NaN -> 0, else bits(p) + 1); token ids
//   (rocPRIM's stable descending radix sort of (key, token) per row)
//   sel_pick     total2, target, the walk (one wavefront per row)
// Temperature 0 is Sampler::Greedy: the caller's argmax (top_logit_candidates).
#include <hip/hip_runtime.h>

#include <rocprim/device/device_radix_sort.hpp>

#include "tqf_device.h"
#include "tqf_expf.h"
#include "tqf_internal.h"

namespace tqf {

namespace {

constexpr int kSelThreads = 256;
constexpr uint32_t kSelPer = 4;
constexpr uint32_t kSelChunk = kSelThreads * kSelPer;  // logits per workgroup
constexpr uint32_t kFold = 64;                         // terms per fold block
constexpr uint32_t kTile = 4096;                       // terms per LDS tile of a fold
// Rows of the e, key and token planes are padded to whole fold tiles, so a
// tile load never leaves the row's allocation (the padding is never folded).
constexpr uint32_t row_stride(uint32_t vocab) { return (vocab + kTile - 1) / kTile * kTile; }

struct SelRow {
    float total;       // the token-order fold
    uint32_t has_nan;  // some p_x is NaN
};

struct SelLayout {
    uint32_t nch, stride;
    size_t off_e, off_kin, off_kout, off_vin, off_vout, off_cmax, off_row, off_sort, total;
};

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

size_t sort_temp_bytes(uint32_t vocab) {
    size_t bytes = 0;
    (void)rocprim::radix_sort_pairs_desc(nullptr, bytes, (const uint32_t *)nullptr, (uint32_t *)nullptr,
                                         (const uint32_t *)nullptr, (uint32_t *)nullptr, vocab, 0u, 32u);
    return bytes;
}

SelLayout sel_layout(uint32_t rows, uint32_t vocab) {
    SelLayout L;
    L.nch = (vocab + kSelChunk - 1) / kSelChunk;
    L.stride = row_stride(vocab);
    const size_t plane = align256((size_t)rows * L.stride * 4);
    size_t o = 0;
    L.off_e = o, o += plane;
    L.off_kin = o, o += plane;
    L.off_kout = o, o += plane;
    L.off_vin = o, o += plane;
    L.off_vout = o, o += plane;
    L.off_cmax = o, o += align256((size_t)rows * L.nch * 4);
    L.off_row = o, o += align256((size_t)rows * sizeof(SelRow));
    L.off_sort = o, o += align256(sort_temp_bytes(vocab));
    L.total = o;
    return L;
}

struct SelArgs {
    const float *logits;
    uint32_t rows, vocab, nch, stride;
    float T;
    const float *u;
    int32_t *tokens;
    float *e;
    uint32_t *kin, *kout, *vin, *vout;
    float *cmax;
    SelRow *row;
};

// f32::max's fold: a NaN operand never wins (the other is kept).
__device__ __forceinline__ float nan_max(float m, float v) { return (v > m || m != m) ? v : m; }

__device__ __forceinline__ float block_max(float v, float *red) {
    for (int off = 32; off >= 1; off >>= 1) v = nan_max(v, __shfl_xor(v, off));
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
    for (int w = 1; w < kSelThreads / kWave; ++w) m = nan_max(m, red[w]);
    return m;
}

__global__ __launch_bounds__(kSelThreads) void sel_max_kernel(SelArgs a) {
    const uint32_t r = blockIdx.y, c = blockIdx.x;
    const float *l = a.logits + (size_t)r * a.vocab;
    float m = -__builtin_inff();
    for (uint32_t i = 0; i < kSelPer; ++i) {
        const uint32_t x = c * kSelChunk + i * kSelThreads + threadIdx.x;
        if (x < a.vocab) m = nan_max(m, l[x]);
    }
    __shared__ float red[kSelThreads / kWave];
    m = block_max(m, red);
    if (threadIdx.x == 0) a.cmax[(size_t)r * a.nch + c] = m;
}

__global__ __launch_bounds__(kSelThreads) void sel_exp_kernel(SelArgs a) {
    const uint32_t r = blockIdx.y, c = blockIdx.x;
    float m = -__builtin_inff();
    for (uint32_t i = threadIdx.x; i < a.nch; i += kSelThreads) m = nan_max(m, a.cmax[(size_t)r * a.nch + i]);
    __shared__ float red[kSelThreads / kWave];
    const float mx = block_max(m, red);  // every chunk's maximum, whatever their order
    const float *l = a.logits + (size_t)r * a.vocab;
    float *e = a.e + (size_t)r * a.stride;
    for (uint32_t i = 0; i < kSelPer; ++i) {
        const uint32_t x = c * kSelChunk + i * kSelThreads + threadIdx.x;
        if (x < a.vocab) e[x] = ref_expf((l[x] - mx) / a.T);
    }
    if (c == 0 && threadIdx.x == 0) a.row[r].has_nan = 0u;
}

// ---- sequential folds ---------------------------------------------------------
// One wavefront streams n words of a row through LDS, tile by tile (the next
// tile's loads in flight while the current one is folded), and hands each
// block of kFold words to blk(block, first index, count) in order; blk reads
// the block with broadcast LDS loads (every lane folds the same terms) and
// returns false to stop.
struct FoldLds {
    uint4 buf[2][kTile / 4];
};

template <class Blk>
__device__ void stream_blocks(const uint32_t *src, uint32_t n, FoldLds &lds, Blk blk) {
    const uint32_t lane = threadIdx.x;
    constexpr int kLoads = (int)(kTile / 4 / kWave);  // uint4 per lane per tile
    const uint32_t tiles = (n + kTile - 1) / kTile;
    uint4 reg[kLoads];
    if (tiles == 0) return;
#pragma unroll
    for (int k = 0; k < kLoads; ++k) reg[k] = reinterpret_cast<const uint4 *>(src)[k * kWave + lane];
    for (uint32_t t = 0; t < tiles; ++t) {
        uint4 *cur = lds.buf[t & 1];
#pragma unroll
        for (int k = 0; k < kLoads; ++k) cur[k * kWave + lane] = reg[k];
        __builtin_amdgcn_wave_barrier();
        if (t + 1 < tiles) {
#pragma unroll
            for (int k = 0; k < kLoads; ++k)
                reg[k] = reinterpret_cast<const uint4 *>(src + (size_t)(t + 1) * kTile)[k * kWave + lane];
        }
        const uint32_t base = t * kTile;
        const uint32_t cnt = n - base < kTile ? n - base : kTile;
        for (uint32_t b = 0; b < cnt; b += kFold)
            if (!blk(reinterpret_cast<const uint32_t *>(cur) + b, base + b, cnt - b < kFold ? cnt - b : kFold))
                return;
        __builtin_amdgcn_wave_barrier();
    }
}

// Folds `count` (<= kFold) terms of an LDS block into s, in order.
template <class Term>
__device__ __forceinline__ float fold_block(const uint32_t *blk, uint32_t count, float s, Term term) {
    if (count == kFold) {
        const uint4 *q = reinterpret_cast<const uint4 *>(blk);
#pragma unroll
        for (int k = 0; k < (int)(kFold / 4); ++k) {
            const uint4 v = q[k];
            s += term(v.x);
            s += term(v.y);
            s += term(v.z);
            s += term(v.w);
        }
    } else {
        for (uint32_t i = 0; i < count; ++i) s += term(blk[i]);
    }
    return s;
}

struct AsFloat {
    __device__ float operator()(uint32_t w) const { return __uint_as_float(w); }
};
// p of a sort key (keys of folded terms are never 0: NaN rows are not folded)
struct KeyValue {
    __device__ float operator()(uint32_t key) const { return __uint_as_float(key - 1u); }
};

// The token-order fold of e.
__global__ __launch_bounds__(kWave) void sel_total_kernel(SelArgs a) {
    __shared__ FoldLds lds;
    const uint32_t r = blockIdx.x;
    float s = -0.0f;
    stream_blocks(reinterpret_cast<const uint32_t *>(a.e + (size_t)r * a.stride), a.vocab, lds,
                  [&](const uint32_t *blk, uint32_t, uint32_t count) {
                      s = fold_block(blk, count, s, AsFloat());
                      return true;
                  });
    if (threadIdx.x == 0) a.row[r].total = s;
}

__global__ __launch_bounds__(kSelThreads) void sel_keys_kernel(SelArgs a) {
    const uint32_t r = blockIdx.y, c = blockIdx.x;
    const float total = a.row[r].total;
    const float *e = a.e + (size_t)r * a.stride;
    uint32_t *kin = a.kin + (size_t)r * a.stride, *vin = a.vin + (size_t)r * a.stride;
    bool nan = false;
    for (uint32_t i = 0; i < kSelPer; ++i) {
        const uint32_t x = c * kSelChunk + i * kSelThreads + threadIdx.x;
        if (x < a.vocab) {
            const float p = total > 0.0f ? e[x] / total : e[x];
            nan |= p != p;
            // order-preserving key of p >= +0 (exp and its quotient are never
            // negative); NaN below every number, so it sorts last
            kin[x] = p != p ? 0u : __float_as_uint(p) + 1u;
            vin[x] = x;
        }
    }
    if (__syncthreads_or(nan) && threadIdx.x == 0) atomicOr(&a.row[r].has_nan, 1u);
}

// Half an ulp of s > 0 (0 where it is below the smallest subnormal, so no
// term is ever taken as vanishing there).
__device__ __forceinline__ float half_ulp(float s) {
    const int ex = (int)((__float_as_uint(s) >> 23) & 0xffu);
    if (ex >= 25) return __uint_as_float((uint32_t)(ex - 24) << 23);
    if (ex >= 2) return __uint_as_float(1u << (ex - 2));
    return 0.0f;
}

__global__ __launch_bounds__(kWave) void sel_pick_kernel(SelArgs a) {
    __shared__ FoldLds lds;
    const uint32_t r = blockIdx.x, V = a.vocab;
    const uint32_t *keys = a.kout + (size_t)r * a.stride, *toks = a.vout + (size_t)r * a.stride;
    int32_t token = (int32_t)toks[0];
    if (!a.row[r].has_nan) {
        // total2, stopping at the first block whose last term vanishes: every
        // later term is no larger and the sum no smaller; `end` = terms folded
        float s = -0.0f;
        uint32_t end = V;
        stream_blocks(keys, V, lds, [&](const uint32_t *blk, uint32_t first, uint32_t count) {
            s = fold_block(blk, count, s, KeyValue());
            if (s > 0.0f && KeyValue()(blk[count - 1]) < half_ulp(s)) {
                end = first + count;
                return false;
            }
            return true;
        });
        const float total2 = s;
        if (__builtin_isfinite(total2) && total2 > 0.0f) {
            const float target = a.u[r] * total2;
            // the walk: whole blocks while their last running sum is below
            // target, then term by term inside the block that reaches it
            token = (int32_t)toks[V - 1];  // the reference's fallback: target past the last sum
            float cum = 0.0f;
            stream_blocks(keys, end, lds, [&](const uint32_t *blk, uint32_t first, uint32_t count) {
                const float next = fold_block(blk, count, cum, KeyValue());
                if (next < target) {
                    cum = next;
                    return true;
                }
                for (uint32_t i = 0; i < count; ++i) {
                    cum += KeyValue()(blk[i]);
                    if (cum >= target) {
                        token = (int32_t)toks[first + i];
                        break;
                    }
                }
                return false;
            });
        }
    }
    if (threadIdx.x == 0) a.tokens[r] = token;
}

__global__ void sel_greedy_kernel(const uint32_t *tokens4, uint32_t rows, int32_t *tokens) {
    if (threadIdx.x < rows) tokens[threadIdx.x] = (int32_t)tokens4[threadIdx.x * 4];
}

}  // namespace

size_t sample_scratch_bytes(uint32_t rows, uint32_t vocab) { return sel_layout(rows, vocab).total; }

hipError_t launch_sample_select(hipStream_t s, const float *logits, uint32_t rows, uint32_t vocab,
                                float temperature, const float *u, int32_t *tokens, void *scratch) {
    const SelLayout L = sel_layout(rows, vocab);
    uint8_t *base = static_cast<uint8_t *>(scratch);
    if (temperature == 0.0f) {
        // Sampler::Greedy: the argmax of top_logit_candidates
        uint32_t *t4 = reinterpret_cast<uint32_t *>(base + L.off_kin);
        float *l4 = reinterpret_cast<float *>(base + L.off_kout);
        hipError_t e = launch_top4(s, logits, rows, vocab, t4, l4);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(sel_greedy_kernel, dim3(1), dim3(kWave), 0, s, t4, rows, tokens);
        return hipGetLastError();
    }
    SelArgs a;
    a.logits = logits;
    a.rows = rows;
    a.vocab = vocab;
    a.nch = L.nch;
    a.stride = L.stride;
    a.T = temperature;
    a.u = u;
    a.tokens = tokens;
    a.e = reinterpret_cast<float *>(base + L.off_e);
    a.kin = reinterpret_cast<uint32_t *>(base + L.off_kin);
    a.kout = reinterpret_cast<uint32_t *>(base + L.off_kout);
    a.vin = reinterpret_cast<uint32_t *>(base + L.off_vin);
    a.vout = reinterpret_cast<uint32_t *>(base + L.off_vout);
    a.cmax = reinterpret_cast<float *>(base + L.off_cmax);
    a.row = reinterpret_cast<SelRow *>(base + L.off_row);
    const dim3 grid(L.nch, rows);
    hipLaunchKernelGGL(sel_max_kernel, grid, dim3(kSelThreads), 0, s, a);
    hipLaunchKernelGGL(sel_exp_kernel, grid, dim3(kSelThreads), 0, s, a);
    hipLaunchKernelGGL(sel_total_kernel, dim3(rows), dim3(kWave), 0, s, a);
    hipLaunchKernelGGL(sel_keys_kernel, grid, dim3(kSelThreads), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    size_t tmp_bytes = L.total - L.off_sort;
    for (uint32_t r = 0; r < rows; ++r) {
        const size_t o = (size_t)r * L.stride;
        e = rocprim::radix_sort_pairs_desc(base + L.off_sort, tmp_bytes, a.kin + o, a.kout + o, a.vin + o, a.vout + o,
                                           vocab, 0u, 32u, s);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(sel_pick_kernel, dim3(rows), dim3(kWave), 0, s, a);
    return hipGetLastError();
}

}  // namespace tqf
