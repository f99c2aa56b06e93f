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
// Every operation is the reference's, in its order: the divisions are IEEE
// (correctly rounded), the sort is a stable descending radix sort of
// order-preserving keys over the token-ordered input, and the two sums are
// the sequential f32 folds themselves -- computed exactly, but not one term
// at a time.
//
// The exact parallel fold.  Every term is >= +0, so the running sum s never
// decreases.  While s stays in one binade [2^k, 2^(k+1)) (or below 2^-125,
// where the spacing is the subnormals'), the values it can take are the
// multiples of g = ulp(s), and for a term t with s + t below the binade's top
//   fl(s + t) = s + g * rne(t / g),
// unless t / g lies exactly halfway between two integers (a tie: the rounding
// then depends on the parity of s / g).  A run of terms without a tie that
// keeps s below the top is therefore an integer sum on a fixed grid, which
// any order and any parallelism computes exactly; only the terms that cross a
// binade's top (at most one per binade the sum passes through) and the ties
// need the f32 add itself (tqf_fold.h).  The terms are cut into units of 256.
// Per row and sum:
//   fold_prefix  the float64 sum of the units before each unit (an estimate
//                of the running sum at the unit's start);
//   fold_units   every unit, one wavefront each, in parallel: two candidate
//                grids for the unit's start (the estimate's binade and its
//                neighbour on the side the estimate leans to), the unit's sum
//                in units of each grid (saturating), and whether a term is a
//                tie on it;
//   fold_row     one wavefront walks the units in order, 64 at a time (a wave
//                scan): a unit with a candidate grid that is the running
//                sum's, without a tie there, that keeps the sum below its
//                binade's top, adds its count; the first unit that does not
//                is folded term by term (each lane's four counts and a wave
//                scan up to the first crossing or tie, that term as one f32
//                add, then on from the next term), and the walk resumes after
//                it.  Units the prediction marks as likely to need that are
//                loaded ahead.
// A missed prediction costs time, never a bit: each unit's grid is checked
// against the exact running sum before its count is used.  Terms that are NaN
// (the sum is NaN) or +inf (it is +inf) short-cut the fold; a negative term,
// which the sampler never produces, takes the plain sequential fold.  The
// walk of the inverse CDF adds the same terms in the same order as the sorted
// fold (-0 + p = +0 + p for p >= 0), so it reads the fold's running sum at
// the end of every fourth unit, finds the first of those that reaches the
// target, and walks the four units before it.
//
// Kernels (rows <= 8 run side by side):
//   sel_max      chunk maxima of each row (1024 logits per workgroup)
//   sel_exp      the row maximum from the chunk maxima; e_x; unit sums
//   fold_prefix, fold_units (e, token order)
//   sel_total    fold_row of e
//   sel_keys     p_x and its sort key (NaN -> 0, else bits(p) + 1); token ids
//   (rocPRIM's stable descending radix sort of (key, token) per row)
//   sel_psum     unit sums of the sorted p
//   fold_prefix, fold_units (p, sorted order)
//   sel_pick     fold_row of the sorted p (total2), target, the walk
// Temperature 0 is Sampler::Greedy: the caller's argmax (top_logit_candidates).
#include <hip/hip_runtime.h>

#include <rocprim/device/device_radix_sort.hpp>

#include "tqf_device.h"
#include "tqf_expf.h"
#include "tqf_fold.h"
#include "tqf_internal.h"

namespace tqf {

namespace {

constexpr int kSelThreads = 256;
constexpr uint32_t kSelPer = 4;
constexpr uint32_t kSelChunk = kSelThreads * kSelPer;  // logits per workgroup
constexpr uint32_t kUnit = 4 * kWave;                  // terms per fold unit (4 per lane)
constexpr uint32_t kUnitsPerChunk = kSelChunk / kUnit;
constexpr uint32_t kMaxGroups = (1u << 22) / (4 * kUnit);  // vocab <= 2^22: walk checkpoints
// Rows of the e, key and token planes are padded to whole chunks, so a unit
// load never leaves the row's allocation (the padding is never folded).
constexpr uint32_t row_stride(uint32_t vocab) { return (vocab + kSelChunk - 1) / kSelChunk * kSelChunk; }


struct SelRow {
    float total;       // the token-order fold
    uint32_t has_nan;  // some p_x is NaN
};

// A fold unit's summary, for two candidate grids a and b of its start:
// meta = the grid exponent (bits 0-7), kTie, and (in meta_a) the unit's term
// flags kNan, kInf, kNeg and kLikely; q = the unit's count on that grid,
// saturated at kSat.
struct FoldUnit {
    uint32_t meta_a, q_a, meta_b, q_b;
};
constexpr uint32_t kLikely = 1u << 12;  // probably folded term by term

struct SelLayout {
    uint32_t nch, nu, stride;
    size_t off_e, off_kin, off_kout, off_vin, off_vout, off_cmax, off_dsum, off_dpre, off_info, off_flags, off_row,
        off_sort, total;
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
    L.nu = L.nch * kUnitsPerChunk;  // units of whole chunks (those past the row hold +0 terms)
    L.stride = row_stride(vocab);
    const size_t plane = align256((size_t)rows * L.stride * 4);
    size_t o = 0;
    L.off_e = o, o += plane;
    L.off_kin = o, o += plane;
    L.off_kout = o, o += plane;
    L.off_vin = o, o += plane;
    L.off_vout = o, o += plane;
    L.off_cmax = o, o += align256((size_t)rows * L.nch * 4);
    L.off_dsum = o, o += align256((size_t)rows * L.nu * sizeof(double));
    L.off_dpre = o, o += align256((size_t)rows * L.nu * sizeof(double));
    L.off_info = o, o += align256((size_t)rows * L.nu * sizeof(FoldUnit));
    L.off_flags = o, o += align256((size_t)rows * 4);
    L.off_row = o, o += align256((size_t)rows * sizeof(SelRow));
    L.off_sort = o, o += align256(sort_temp_bytes(vocab));
    L.total = o;
    return L;
}

struct SelArgs {
    const float *logits;
    uint32_t rows, vocab, nch, nu, stride;
    float T;
    const float *u;
    int32_t *tokens;
    float *sums;  // optional [rows x 2]: total, total2
    float *e;
    uint32_t *kin, *kout, *vin, *vout;
    float *cmax;
    double *dsum;    // per unit: the float64 sum of its terms
    double *dpre;    // per unit: the float64 sum of the units before it
    FoldUnit *info;  // per unit: fold_units' summary
    uint32_t *flags;  // per row: the current fold's term flags (kNan, kInf, kNeg)
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

// The float64 sums of the chunk's four units (unit i = elements i * 256 +
// thread of the chunk), from each thread's four values; a prediction only,
// so the order of the additions is immaterial.
__device__ __forceinline__ void unit_sums(const double (&v)[kSelPer], double *out) {
    __shared__ double red[kSelPer][kSelThreads / kWave];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
#pragma unroll
    for (uint32_t i = 0; i < kSelPer; ++i) {
        double x = v[i];
        for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
        if (lane == 0) red[i][wave] = x;
    }
    __syncthreads();
    if (threadIdx.x < kSelPer) {
        double t = 0.0;
        for (int w = 0; w < kSelThreads / kWave; ++w) t += red[threadIdx.x][w];
        out[threadIdx.x] = t;
    }
}

__global__ __launch_bounds__(kSelThreads) void sel_exp_kernel(SelArgs a) {
    const uint32_t r = blockIdx.y, c = blockIdx.x;
    float m = -__builtin_inff();
    for (uint32_t i = threadIdx.x; i < a.nch; i += kSelThreads) m = nan_max(m, a.cmax[(size_t)r * a.nch + i]);
    __shared__ float red[kSelThreads / kWave];
    const float mx = block_max(m, red);  // every chunk's maximum, whatever their order
    const float *l = a.logits + (size_t)r * a.vocab;
    float *e = a.e + (size_t)r * a.stride;
    double part[kSelPer];
    for (uint32_t i = 0; i < kSelPer; ++i) {
        const uint32_t x = c * kSelChunk + i * kSelThreads + threadIdx.x;
        part[i] = 0.0;
        if (x < a.vocab) {
            const float v = ref_expf((l[x] - mx) / a.T);
            e[x] = v;
            part[i] = (double)v;
        }
    }
    unit_sums(part, a.dsum + (size_t)r * a.nu + (size_t)c * kUnitsPerChunk);
    if (c == 0 && threadIdx.x == 0) a.row[r].has_nan = 0u;
}

// ---- the exact parallel fold (the grid rule: tqf_fold.h) ---------------------------
// Inclusive sum over the wavefront (row shifts within 16 lanes, then the
// row broadcasts of lanes 15 and 31); the caller keeps the total below 2^32.
__device__ __forceinline__ uint32_t wave_scan_add(uint32_t v) {
    const uint32_t lane = threadIdx.x % kWave, rl = lane % 16;
    uint32_t t = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x111, 0xf, 0xf, false);  // row_shr:1
    if (rl >= 1) v += t;
    t = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x112, 0xf, 0xf, false);  // row_shr:2
    if (rl >= 2) v += t;
    t = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x114, 0xf, 0xf, false);  // row_shr:4
    if (rl >= 4) v += t;
    t = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x118, 0xf, 0xf, false);  // row_shr:8
    if (rl >= 8) v += t;
    t = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x142, 0xf, 0xf, false);  // row_bcast:15
    if (lane % 32 >= 16) v += t;
    t = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x143, 0xf, 0xf, false);  // row_bcast:31
    if (lane >= 32) v += t;
    return v;
}

__device__ __forceinline__ uint32_t lane_value(uint32_t v, uint32_t l) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)l);
}

// Exclusive float64 prefix of each row's unit sums (one workgroup per row);
// also clears the row's term flags for fold_units.
__global__ __launch_bounds__(kSelThreads) void fold_prefix_kernel(const double *dsum, double *dpre, uint32_t nu,
                                                                  uint32_t *flags) {
    const uint32_t r = blockIdx.x, lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    if (threadIdx.x == 0) flags[r] = 0u;
    const double *in = dsum + (size_t)r * nu;
    double *out = dpre + (size_t)r * nu;
    __shared__ double wsum[kSelThreads / kWave];
    double carry = 0.0;
    for (uint32_t base = 0; base < nu; base += kSelThreads) {
        const uint32_t i = base + threadIdx.x;
        const double own = i < nu ? in[i] : 0.0;
        double v = own;
        for (int d = 1; d < kWave; d <<= 1) {
            const double o = __shfl_up(v, d);
            if ((int)lane >= d) v += o;
        }
        if (lane == kWave - 1) wsum[wave] = v;
        __syncthreads();
        double before = carry, all = carry;
        for (uint32_t w = 0; w < kSelThreads / kWave; ++w) {
            if (w < wave) before += wsum[w];
            all += wsum[w];
        }
        if (i < nu) out[i] = before + (v - own);
        carry = all;
        __syncthreads();
    }
}

// A unit's terms: lane l holds terms 4 l .. 4 l + 3 as f32 bits; terms past
// the row's n are +0.  kKeys: the words are sort keys, the term is the key
// minus 1.
__device__ __forceinline__ uint4 load_unit(const uint32_t *row, uint32_t u) {
    return reinterpret_cast<const uint4 *>(row + (size_t)u * kUnit)[threadIdx.x % kWave];
}

template <bool kKeys>
__device__ __forceinline__ void unit_terms(uint32_t u, uint32_t n, uint4 raw, float (&t)[4]) {
    const uint32_t first = u * kUnit + 4 * (threadIdx.x % kWave);
    const uint32_t v[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) t[j] = first + j < n ? __uint_as_float(kKeys ? v[j] - 1u : v[j]) : 0.0f;
}

struct FoldPass {
    const uint32_t *terms;  // row r at terms + r * stride
    uint32_t stride, n, nu;
    const double *dsum, *dpre;
    FoldUnit *info;
    uint32_t *flags;
};

// One wavefront per unit: two candidate grids for the unit's start (the
// binade of the float64 estimate, and its neighbour on the side the estimate
// leans to), the unit's count and tie flag on each, its term flags, and
// kLikely when fold_row will probably fold it term by term (unit 0, a tie on
// grid a, or an estimated end in another binade than the start).
template <bool kKeys>
__global__ __launch_bounds__(kWave) void fold_units_kernel(FoldPass f) {
    const uint32_t r = blockIdx.y, u = blockIdx.x, lane = threadIdx.x;
    const double acc = f.dpre[(size_t)r * f.nu + u];
    const uint32_t eb = __float_as_uint((float)acc);  // acc >= 0 (NaN or +inf: no grid)
    const uint32_t ee = eb >> 23, ee_end = __float_as_uint((float)(acc + f.dsum[(size_t)r * f.nu + u])) >> 23;
    uint32_t ga = ee > 1u ? ee : 1u, gb = (eb >> 22) & 1u ? ga + 1u : (ga > 1u ? ga - 1u : 2u);
    if (ee >= 254u) ga = gb = 255u;  // never a running sum's grid
    float t[4];
    unit_terms<kKeys>(u, f.n, load_unit(f.terms + (size_t)r * f.stride, u), t);
    uint32_t qa = 0, qb = 0, flags = 0, ta = 0, tb = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t fl = term_flags(__float_as_uint(t[j]));
        flags |= fl;
        bool tie_a, tie_b;
        const uint32_t ua = grid_units(t[j], ga < 255u ? ga : 254u, tie_a);
        const uint32_t ub = grid_units(t[j], gb < 255u ? gb : 254u, tie_b);
        if (!fl) qa = sat_add(qa, ua), qb = sat_add(qb, ub), ta |= tie_a, tb |= tie_b;
    }
    for (int off = 32; off >= 1; off >>= 1) {
        qa = sat_add(qa, __shfl_xor(qa, off));
        qb = sat_add(qb, __shfl_xor(qb, off));
        flags |= __shfl_xor(flags, off);
        ta |= __shfl_xor(ta, off);
        tb |= __shfl_xor(tb, off);
    }
    const uint32_t likely = u == 0 || ta || (ee_end > 1u ? ee_end : 1u) != ga ? kLikely : 0u;
    if (lane == 0) {
        f.info[(size_t)r * f.nu + u] = FoldUnit{ga | (ta ? kTie : 0u) | flags | likely, qa, gb | (tb ? kTie : 0u), qb};
        if (flags) atomicOr(f.flags + r, flags);
    }
}

constexpr uint32_t kNoHit = 0xffffffffu;

// Folds one unit's terms (t from unit_terms; cnt of them are the row's) into
// G by the grid rule: each lane's four counts and their running sum, a wave
// scan of the lanes' sums, the first crossing or tie, the counts before it
// added, that term as one f32 add, and on from the next term.  With walk,
// stops at the first term after which the running sum's bits reach target
// and returns its index in the unit; else (or without a hit) returns kNoHit.
// Each round either ends the unit or moves past at least one term, so the
// loop ends.
__device__ uint32_t fold_unit_terms(Grid &G, const float (&t)[4], uint32_t cnt, bool walk, uint32_t target) {
    const uint32_t lane = threadIdx.x % kWave;
    uint32_t pos = 0;  // first term still to fold
    while (pos < cnt) {
        uint32_t pl[4], run = 0, ties = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t idx = 4 * lane + (uint32_t)j;
            const bool live = idx >= pos && idx < cnt;
            bool tie;
            const uint32_t q = grid_units(t[j], G.eg, tie);  // <= 2^24
            run += live ? q : 0u;
            pl[j] = run;
            ties |= (live && tie ? 1u : 0u) << j;
        }
        const uint32_t rc = run < kSat ? run : kSat;  // a lane past kSat holds a crossing
        const uint32_t incl = wave_scan_add(rc);     // <= 64 * 2^25
        const uint32_t excl = incl - rc;
        bool found = false;
        uint32_t rv = 0, before = excl, tv = 0, hj = 4, prev = excl;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t idx = 4 * lane + (uint32_t)j;
            const bool live = idx >= pos && idx < cnt;
            const uint32_t P = excl + pl[j];
            const bool vio = live && (((ties >> j) & 1u) || G.n + P >= kTop);
            if (!found && vio) found = true, rv = (uint32_t)j, before = prev, tv = __float_as_uint(t[j]);
            if (walk && !found && live && hj == 4 && grid_bits(G.eg, G.n + P) >= target) hj = (uint32_t)j;
            prev = P;
        }
        const uint64_t vb = __ballot(found);
        const uint32_t fl = vb ? (uint32_t)__builtin_ctzll(vb) : kWave;
        if (walk) {
            const uint64_t hb = __ballot(hj < 4);
            const uint32_t hl = hb ? (uint32_t)__builtin_ctzll(hb) : kWave;
            if (hl < kWave && hl <= fl) return 4 * hl + lane_value(hj, hl);
        }
        if (!vb) {
            G.n += lane_value(incl, kWave - 1);
            break;
        }
        const uint32_t v = 4 * fl + lane_value(rv, fl);
        const float s = __uint_as_float(grid_bits(G.eg, G.n + lane_value(before, fl))) +
                        __uint_as_float(lane_value(tv, fl));
        G = grid_of(__float_as_uint(s));
        if (walk && __float_as_uint(s) >= target) return v;
        pos = v + 1;
    }
    return kNoHit;
}

// The unit's count if one of its candidate grids is G's and carries no tie
// (clean), else false.
__device__ __forceinline__ bool unit_count(const FoldUnit &fu, const Grid &G, uint32_t &q) {
    const bool ok_a = (fu.meta_a & (0xffu | kTie)) == G.eg, ok_b = (fu.meta_b & (0xffu | kTie)) == G.eg;
    q = ok_a ? fu.q_a : (ok_b ? fu.q_b : 0u);
    return ok_a || ok_b;
}

// fold_row's LDS: a block of unit summaries, and the terms of the block's
// units marked kLikely (the first kStageTerms of them), loaded together so
// that the walk over the units meets one memory latency per block.
constexpr uint32_t kStageUnits = 1024;
constexpr uint32_t kStageTerms = 24;
struct FoldLds {
    FoldUnit info[kStageUnits];
    uint4 terms[kStageTerms][kWave];
    uint32_t tidx[kStageTerms];  // their unit indices, ascending
};

// The sequential f32 fold from -0 of a row's n terms, from fold_units'
// summaries and the row's term flags; ckpt (LDS, may be null) receives the
// running sum's bits at the end of every fourth unit (entry g: after units
// 4g .. 4g + 3), except when the row has a NaN, +inf or negative term.
template <bool kKeys>
__device__ float fold_row(const uint32_t *row, uint32_t n, uint32_t nu, const FoldUnit *info, uint32_t flags,
                         uint32_t *ckpt, FoldLds &L) {
    const uint32_t lane = threadIdx.x % kWave;
    if (flags & kNeg) {
        // not a sampler term: the plain fold, one term after another
        float s = -0.0f;
        for (uint32_t i = 0; i < n; ++i) s += __uint_as_float(kKeys ? row[i] - 1u : row[i]);
        return s;
    }
    if (flags & kNan) return __uint_as_float(0x7fc00000u);  // NaN absorbs every term
    if (flags & kInf) return __builtin_inff();              // so does +inf every finite one
    Grid G = {1u, 0u};  // +0: after the first term, the same sum as from -0
    for (uint32_t blk = 0; blk < nu; blk += kStageUnits) {
        const uint32_t nb = nu - blk < kStageUnits ? nu - blk : kStageUnits;
        // stage the block's summaries, then its likely units' terms
        const uint4 *src = reinterpret_cast<const uint4 *>(info + blk);
        uint4 *dst = reinterpret_cast<uint4 *>(L.info);
        uint4 fu[kStageUnits / kWave];
#pragma unroll
        for (uint32_t i = 0; i < kStageUnits / kWave; ++i)
            fu[i] = lane + i * kWave < nb ? src[lane + i * kWave] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (uint32_t i = 0; i < kStageUnits / kWave; ++i) dst[lane + i * kWave] = fu[i];
        uint32_t nl = 0;
#pragma unroll
        for (uint32_t i = 0; i < kStageUnits / kWave; ++i) {
            const bool lk = lane + i * kWave < nb && (fu[i].x & kLikely);  // meta_a
            const uint64_t b = __ballot(lk);
            const uint32_t slot = nl + (uint32_t)__builtin_popcountll(b & ((1ull << lane) - 1ull));
            if (lk && slot < kStageTerms) L.tidx[slot] = blk + lane + i * kWave;
            nl += (uint32_t)__builtin_popcountll(b);
        }
        nl = nl < kStageTerms ? nl : kStageTerms;
        __syncthreads();
        uint4 tr[kStageTerms];
#pragma unroll
        for (uint32_t k = 0; k < kStageTerms; ++k)
            if (k < nl) tr[k] = load_unit(row, L.tidx[k]);
#pragma unroll
        for (uint32_t k = 0; k < kStageTerms; ++k)
            if (k < nl) L.terms[k][lane] = tr[k];
        __syncthreads();
        uint32_t li = 0;  // the next staged unit
        for (uint32_t c0 = 0; c0 < nb;) {
            const uint32_t c = c0 + lane, nvalid = nb - c0 < kWave ? nb - c0 : kWave;
            const bool valid = c < nb;
            uint32_t q;
            const bool clean = valid && unit_count(L.info[valid ? c : 0], G, q);
            const uint32_t incl = wave_scan_add(clean ? q : 0u);  // <= 64 * 2^25
            const uint64_t vb = __ballot(valid && (!clean || G.n + incl >= kTop));
            const uint32_t fv = vb ? (uint32_t)__builtin_ctzll(vb) : nvalid;
            if (ckpt && lane < fv && ((blk + c) & 3u) == 3u) ckpt[(blk + c) >> 2] = grid_bits(G.eg, G.n + incl);
            if (fv) G.n += lane_value(incl, fv - 1);
            if (!vb) {
                c0 += nvalid;
                continue;
            }
            const uint32_t u = blk + c0 + fv;
            while (li < nl && L.tidx[li] < u) ++li;
            const uint4 raw = li < nl && L.tidx[li] == u ? L.terms[li][lane] : load_unit(row, u);
            float t[4];
            unit_terms<kKeys>(u, n, raw, t);
            const uint32_t rest = n > u * kUnit ? n - u * kUnit : 0u;
            fold_unit_terms(G, t, rest < kUnit ? rest : kUnit, false, 0u);
            if (ckpt && lane == 0 && (u & 3u) == 3u) ckpt[u >> 2] = grid_bits(G.eg, G.n);
            c0 += fv + 1;
        }
        __syncthreads();
    }
    return __uint_as_float(grid_bits(G.eg, G.n));
}

// The token-order fold of e.
__global__ __launch_bounds__(kWave) void sel_total_kernel(SelArgs a) {
    __shared__ FoldLds lds;
    const uint32_t r = blockIdx.x;
    const float s = fold_row<false>(reinterpret_cast<const uint32_t *>(a.e + (size_t)r * a.stride), a.vocab, a.nu,
                                    a.info + (size_t)r * a.nu, a.flags[r], nullptr, lds);
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

// Unit sums of the sorted probabilities (the sorted fold's grid prediction).
__global__ __launch_bounds__(kSelThreads) void sel_psum_kernel(SelArgs a) {
    const uint32_t r = blockIdx.y, c = blockIdx.x;
    const uint32_t *keys = a.kout + (size_t)r * a.stride;
    double part[kSelPer];
    for (uint32_t i = 0; i < kSelPer; ++i) {
        const uint32_t x = c * kSelChunk + i * kSelThreads + threadIdx.x;
        part[i] = x < a.vocab ? (double)__uint_as_float(keys[x] - 1u) : 0.0;
    }
    unit_sums(part, a.dsum + (size_t)r * a.nu + (size_t)c * kUnitsPerChunk);
}

__global__ __launch_bounds__(kWave) void sel_pick_kernel(SelArgs a) {
    __shared__ uint32_t ckpt[kMaxGroups];
    __shared__ FoldLds lds;
    const uint32_t r = blockIdx.x, V = a.vocab, lane = threadIdx.x;
    const uint32_t *keys = a.kout + (size_t)r * a.stride, *toks = a.vout + (size_t)r * a.stride;
    const FoldUnit *info = a.info + (size_t)r * a.nu;
    int32_t token = (int32_t)toks[0];
    float total2 = __uint_as_float(0x7fc00000u);  // a NaN probability makes the sorted sum NaN
    if (!a.row[r].has_nan) {
        const uint32_t flags = a.flags[r];
        total2 = fold_row<true>(keys, V, a.nu, info, flags, ckpt, lds);
        if (__builtin_isfinite(total2) && total2 > 0.0f && flags) {
            // a negative probability (never produced from exponentials): the
            // walk one term after another
            const float target = a.u[r] * total2;
            token = (int32_t)toks[V - 1];
            float cum = 0.0f;
            for (uint32_t i = 0; i < V; ++i) {
                cum += __uint_as_float(keys[i] - 1u);
                if (cum >= target) {
                    token = (int32_t)toks[i];
                    break;
                }
            }
        } else if (__builtin_isfinite(total2) && total2 > 0.0f) {
            const uint32_t target = __float_as_uint(a.u[r] * total2);  // >= +0
            token = (int32_t)toks[V - 1];  // the reference's fallback: target past the last sum
            // the first group of four units whose end reaches target (the last
            // group, whole or not, ends at total2 >= target)
            const uint32_t ng = (a.nu + 3) / 4;
            uint32_t g = kNoHit;
            for (uint32_t g0 = 0; g0 < ng && g == kNoHit; g0 += kWave) {
                const uint32_t gi = g0 + lane;
                const bool reach = gi < ng && (gi == ng - 1 || ckpt[gi] >= target);
                const uint64_t b = __ballot(reach);
                if (b) g = g0 + (uint32_t)__builtin_ctzll(b);
            }
            // walk its units: a clean unit that ends below target is added
            // whole, the first other one term by term
            Grid G = grid_of(g ? ckpt[g - 1] : 0u);
            for (uint32_t u = 4 * g; u < 4 * g + 4 && u < a.nu; ++u) {
                const FoldUnit fu = info[u];
                uint32_t q;
                if (unit_count(fu, G, q) && G.n + q < kTop && grid_bits(G.eg, G.n + q) < target) {
                    G.n += q;
                    continue;
                }
                float t[4];
                unit_terms<true>(u, V, load_unit(keys, u), t);
                const uint32_t rest = V > u * kUnit ? V - u * kUnit : 0u;
                const uint32_t i = fold_unit_terms(G, t, rest < kUnit ? rest : kUnit, true, target);
                if (i != kNoHit) {
                    token = (int32_t)toks[u * kUnit + i];
                    break;
                }
            }
        }
    }
    if (lane == 0) {
        a.tokens[r] = token;
        if (a.sums) {
            a.sums[2 * r] = a.row[r].total;
            a.sums[2 * r + 1] = total2;
        }
    }
}

__global__ void sel_greedy_kernel(const uint32_t *tokens4, uint32_t rows, int32_t *tokens) {
    if (threadIdx.x < rows) tokens[threadIdx.x] = (int32_t)tokens4[threadIdx.x * 4];
}

}  // namespace

size_t sample_scratch_bytes(uint32_t rows, uint32_t vocab) { return sel_layout(rows, vocab).total; }

hipError_t launch_sample_select(hipStream_t s, const float *logits, uint32_t rows, uint32_t vocab,
                                float temperature, const float *u, int32_t *tokens, float *sums, void *scratch) {
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
    a.nu = L.nu;
    a.stride = L.stride;
    a.T = temperature;
    a.u = u;
    a.tokens = tokens;
    a.sums = sums;
    a.e = reinterpret_cast<float *>(base + L.off_e);
    a.kin = reinterpret_cast<uint32_t *>(base + L.off_kin);
    a.kout = reinterpret_cast<uint32_t *>(base + L.off_kout);
    a.vin = reinterpret_cast<uint32_t *>(base + L.off_vin);
    a.vout = reinterpret_cast<uint32_t *>(base + L.off_vout);
    a.cmax = reinterpret_cast<float *>(base + L.off_cmax);
    a.dsum = reinterpret_cast<double *>(base + L.off_dsum);
    a.dpre = reinterpret_cast<double *>(base + L.off_dpre);
    a.info = reinterpret_cast<FoldUnit *>(base + L.off_info);
    a.flags = reinterpret_cast<uint32_t *>(base + L.off_flags);
    a.row = reinterpret_cast<SelRow *>(base + L.off_row);
    const dim3 grid(L.nch, rows), ugrid(L.nu, rows);
    FoldPass f{reinterpret_cast<const uint32_t *>(a.e), L.stride, vocab, L.nu, a.dsum, a.dpre, a.info, a.flags};
    hipLaunchKernelGGL(sel_max_kernel, grid, dim3(kSelThreads), 0, s, a);
    hipLaunchKernelGGL(sel_exp_kernel, grid, dim3(kSelThreads), 0, s, a);
    hipLaunchKernelGGL(fold_prefix_kernel, dim3(rows), dim3(kSelThreads), 0, s, a.dsum, a.dpre, L.nu, a.flags);
    hipLaunchKernelGGL(fold_units_kernel<false>, ugrid, dim3(kWave), 0, s, f);
    hipLaunchKernelGGL(sel_total_kernel, dim3(rows), dim3(kWave), 0, s, a);
    hipLaunchKernelGGL(sel_keys_kernel, grid, dim3(kSelThreads), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    size_t tmp_bytes = L.total - L.off_sort;
    for (uint32_t r = 0; r < rows; ++r) {
        const size_t o = (size_t)r * L.stride;
        e = rocprim::radix_sort_pairs_desc(base + L.off_sort, tmp_bytes, a.kin + o, a.kout + o,
                                                       a.vin + o, a.vout + o, vocab, 0u, 32u, s);
        if (e != hipSuccess) return e;
    }
    f.terms = a.kout;
    hipLaunchKernelGGL(sel_psum_kernel, grid, dim3(kSelThreads), 0, s, a);
    hipLaunchKernelGGL(fold_prefix_kernel, dim3(rows), dim3(kSelThreads), 0, s, a.dsum, a.dpre, L.nu, a.flags);
    hipLaunchKernelGGL(fold_units_kernel<true>, ugrid, dim3(kWave), 0, s, f);
    hipLaunchKernelGGL(sel_pick_kernel, dim3(rows), dim3(kWave), 0, s, a);
    return hipGetLastError();
}

}  // namespace tqf
