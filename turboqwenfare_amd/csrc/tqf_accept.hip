// tqf_accept.hip -- k-token speculative acceptance over vocab logits (gfx950).
//
// Definition (identical, operation for operation, to the CPU statement the
// tests check it against; every sum is an exact unsigned-integer sum, so the
// result does not depend on the order in which the GPU adds):
//   texp(z)  = 0 if !(z >= -87); else Cody & Waite range reduction
//              n = rint(z log2e), r = fma(-n, ln2_hi, z), r = fma(-n, ln2_lo, r)
//              and a degree-7 Taylor polynomial of e^r by Horner with fma,
//              scaled by 2^n.
//   per row: M = max of the non-NaN logits; e_x = 0 for NaN, 1 if l_x == M,
//            else texp((l_x - M) / T); E_x = floor(e_x 2^40);
//            S_fix = sum E_x; S = rn_f32(S_fix) 2^-40.
//   p = ftz(e_p[d] / S_p), q = ftz(e_q[d] / S_q)   (ftz: |v| < FLT_MIN -> 0)
//   accept draft i  iff  (q > 0 ? u_i < p / q : p > 0)
//   i* = first rejection (or k); emitted tokens = drafts 0..i*-1, then
//   greedy:  argmax(target_{i*})   (strict '>', lowest index, NaN never wins)
//   i* < k:  inverse CDF of w_x = floor(ftz(max(0, p_x - q_x)) 2^62) with
//            u_resample[i*] (falling back to E_x of target i* if sum w == 0)
//   i* = k:  inverse CDF of E_x of target k with u_resample[k]
//   inverse CDF: t = floor(W u) exactly; first x with prefix_sum(w)_x > t.
//
// Kernels (chunks of 4096 logits per workgroup, coalesced 128-bit loads):
//   stats    per (row, chunk): max over non-NaN and the greedy arg-max; in
//            greedy mode the last workgroup emits the tokens.
//   sums     per (row, chunk): S_fix partials; the last workgroup forms the
//            row statistics and the decisions, and when every draft was
//            accepted it samples the bonus token itself.
//   residual per chunk, only after a rejection: residual mass; the last
//            workgroup samples the replacement token.
// Hand-offs inside a kernel use device-coherent stores and a counter; the
// counters return to zero in the workgroup that finishes the kernel.
#include <hip/hip_runtime.h>

#include <cstdlib>

#include "tqf_device.h"
#include "tqf_internal.h"

#pragma clang fp contract(off)

namespace tqf {

constexpr int kAccThreads = 256;
constexpr int kAccPerThread = 16;
constexpr int kAccChunk = kAccThreads * kAccPerThread;  // 4096
constexpr uint32_t kNone = 0xFFFFFFFFu;

// Control block at the start of the scratch, the same for every k, vocab and
// path: misc dwords (64 bytes) [0] i*, [1] counter (sums), [2] counter
// (residual), [3] counter (stats) of the three-kernel path; [4] exit counter
// and [5] sequence word of the one-launch path.
constexpr size_t kCtlBytes = 64;
constexpr int kFuseExitWord = 4, kFuseSeqWord = 5;

// One-launch path (acc_fused_kernel): chunks of kFuseThreads * ept logits
// (ept = 1..4 consecutive elements per thread, the fewest that keep the chunk
// count within the device's compute units), one per workgroup, every
// workgroup resident at once.  Workgroups exchange partials
// as tagged 64-bit words: the high half holds the launch's tag, the low half
// 32 bits of payload (a 64-bit payload takes two words).  A reader polls the
// words it needs until every tag is current, so one round trip to memory both
// waits for the data and delivers it, with no arrival counter.  The tag is
// one more than the sequence word, which the last workgroup out advances.
// The tagged words have a region of their own that nothing else writes, so a
// slot holds zero, a word of an earlier launch (an older tag) or this
// launch's word.
constexpr int kFuseThreads = 256;
constexpr uint32_t kFuseMaxGrid = 1024;  // vocab <= 1,048,576
constexpr int kFuseMaxRows = 2 * (kMaxTokens - 1) + 1;
struct FuseLayout {
    uint32_t rows, nch;
    // u64 arrays: max [rows][nch]; arg-max value and index [k+1][nch];
    // sums (low, high halves) [rows][nch]; residual weights (halves) [nch]
    size_t off_max, off_av, off_ai, off_slo, off_shi, off_wlo, off_whi, total;
};
__host__ __device__ inline FuseLayout fuse_layout(uint32_t k, uint32_t vocab, uint32_t ept) {
    FuseLayout L;
    L.rows = 2 * k + 1;
    L.nch = (vocab + kFuseThreads * ept - 1) / (kFuseThreads * ept);
    const size_t n = (size_t)L.rows * L.nch, nt = (size_t)(k + 1) * L.nch;
    L.off_max = kCtlBytes;
    L.off_av = L.off_max + n * 8;
    L.off_ai = L.off_av + nt * 8;
    L.off_slo = L.off_ai + nt * 8;
    L.off_shi = L.off_slo + n * 8;
    L.off_wlo = L.off_shi + n * 8;
    L.off_whi = L.off_wlo + (size_t)L.nch * 8;
    L.total = L.off_whi + (size_t)L.nch * 8;
    return L;
}
// End of the tagged region at its largest (k = kMaxTokens - 1, kFuseMaxGrid chunks).
constexpr size_t kFuseRegionEnd =
    kCtlBytes + 8 * (3 * (size_t)kFuseMaxRows * kFuseMaxGrid + 2 * (size_t)kMaxTokens * kFuseMaxGrid +
                     2 * (size_t)kFuseMaxGrid);

// Three-kernel path (vocab beyond the one-launch grid): partials after the
// tagged region.
struct AccLayout {
    uint32_t rows, nch;
    size_t off_max, off_av, off_ai, off_sum, off_w, off_misc, total;
};
__host__ __device__ inline AccLayout acc_layout(uint32_t k, uint32_t vocab) {
    AccLayout L;
    L.rows = 2 * k + 1;
    L.nch = (vocab + kAccChunk - 1) / kAccChunk;
    const size_t n = (size_t)L.rows * L.nch;
    L.off_misc = 0;
    L.off_max = kFuseRegionEnd;
    L.off_av = L.off_max + n * 4;
    L.off_ai = L.off_av + n * 4;
    L.off_sum = (L.off_ai + n * 4 + 7) & ~(size_t)7;
    L.off_w = L.off_sum + n * 8;
    L.total = L.off_w + (size_t)L.nch * 8;
    return L;
}

// ---- exact scalar building blocks ----------------------------------------
// exp of z: Cody-Waite reduction by ln 2 and a degree-7 Taylor polynomial;
// 0 below -87 (and for NaN), +inf above 88.  Straight-line (selects, no
// branches) so that independent elements interleave.
__device__ __forceinline__ float acc_exp(float z) {
    const float zc = fminf(fmaxf(z, -87.0f), 88.0f);  // z itself whenever the result is used
    const float n = __builtin_rintf(zc * 0x1.715476p+0f);
    float r = __builtin_fmaf(-n, 0x1.62e4p-1f, zc);
    r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float v = p * __uint_as_float((uint32_t)((int)n + 127) << 23);
    return !(z >= -87.0f) ? 0.0f : (z > 88.0f ? __builtin_inff() : v);
}

// floor(v * 2^shift) for v in [0, 1] and 32 < shift <= 62 (every caller's
// weights: E_x and residual probabilities), subnormal v giving 0.  Float
// arithmetic only, all of it exact: x = v * 2^(shift-32) is a scaling, x -
// floor(x) is exact, and the fraction times 2^32 is below 2^32, converted
// with truncation.
__device__ __forceinline__ uint64_t fix_shift(float v, int shift) {
    const float x = v * __builtin_ldexpf(1.0f, shift - 32);
    const float hi = __builtin_floorf(x);
    const uint32_t lo = (uint32_t)((x - hi) * 0x1p32f);
    return ((uint64_t)(uint32_t)hi << 32) | lo;
}

__device__ __forceinline__ float u64_to_f32_rn(uint64_t v) {
    if (v == 0) return 0.0f;
    const int lz = __builtin_clzll(v);
    const uint64_t norm = v << lz;
    uint32_t mant = (uint32_t)(norm >> 40);
    const uint64_t rest = norm & ((1ull << 40) - 1);
    const uint64_t half = 1ull << 39;
    int ex = 63 - lz;
    if (rest > half || (rest == half && (mant & 1u))) {
        mant += 1;
        if (mant == (1u << 24)) {
            mant >>= 1;
            ex += 1;
        }
    }
    return __uint_as_float(((uint32_t)(ex + 127) << 23) | (mant & 0x7FFFFFu));
}

// floor(total * u) for u in [0, 1), exact (88-bit product).
__device__ __forceinline__ uint64_t scale_floor(uint64_t total, float u) {
    const uint32_t b = __float_as_uint(u);
    const uint32_t ex = (b >> 23) & 0xFFu;
    if ((b & 0x80000000u) || ex == 0) return 0;
    const uint64_t m = (uint64_t)((b & 0x7FFFFFu) | 0x800000u);
    const int s = (int)ex - 127 - 23;
    if (s >= 0) return total;
    const uint64_t plo = (total & 0xFFFFFFFFull) * m;
    const uint64_t phi = (total >> 32) * m;
    const uint64_t p0 = plo + (phi << 32);
    const uint64_t p1 = (phi >> 32) + (p0 < plo ? 1 : 0);
    const int sh = -s;
    if (sh >= 128) return 0;
    if (sh >= 64) return p1 >> (sh - 64);
    return (p0 >> sh) | (p1 << (64 - sh));
}

__device__ __forceinline__ float ftz(float v) { return fabsf(v) < 1.17549435e-38f ? 0.0f : v; }

__device__ __forceinline__ float row_e(float l, float M, float T) {
    const float e = acc_exp((l - M) / T);
    return (l != l) ? 0.0f : (l == M ? 1.0f : e);
}

// a / T as the device's division sequence computes it (v_div_scale, v_rcp,
// one Newton step on the reciprocal, two corrected quotients, v_div_fmas,
// v_div_fixup), with the reciprocal step y1 taken once for the launch.  For
// T in [2^-30, 2^30] the scaling and fixup steps act only on quotients that
// are zero, subnormal, beyond 2^95 in magnitude or not finite, and exp of
// every such quotient is 0 or 1 either way, so row_e_y equals row_e there.
struct RecipT {
    float T, y1;
};
__device__ __forceinline__ RecipT recip_t(float T) {
    const float y0 = __builtin_amdgcn_rcpf(T);
    return RecipT{T, __builtin_fmaf(__builtin_fmaf(-T, y0, 1.0f), y0, y0)};
}
__device__ __forceinline__ float div_t(float a, const RecipT &d) {
    const float q0 = a * d.y1;
    const float q1 = __builtin_fmaf(__builtin_fmaf(-d.T, q0, a), d.y1, q0);
    return __builtin_fmaf(__builtin_fmaf(-d.T, q1, a), d.y1, q1);
}
__device__ __forceinline__ float row_e_y(float l, float M, const RecipT &d) {
    const float e = acc_exp(div_t(l - M, d));
    return (l != l) ? 0.0f : (l == M ? 1.0f : e);
}
// True when T is in the range where row_e_y equals row_e.
inline bool recip_t_exact(float T) { return T >= 0x1p-30f && T <= 0x1p30f; }

__device__ __forceinline__ float prob(float e, float s) { return s == 0.0f ? 0.0f : ftz(e / s); }

// Greedy candidate order: higher value, then lower index; kNone is empty.
__device__ __forceinline__ bool arg_better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i != kNone && bi != kNone && i < bi);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int off) {
    const uint32_t lo = __shfl_xor((uint32_t)v, off);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), off);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_up_u64(uint64_t v, int off) {
    const uint32_t lo = __shfl_up((uint32_t)v, off);
    const uint32_t hi = __shfl_up((uint32_t)(v >> 32), off);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
    const uint32_t lo = __shfl((uint32_t)v, src);
    const uint32_t hi = __shfl((uint32_t)(v >> 32), src);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
    for (int off = 32; off >= 1; off >>= 1) v += shfl_xor_u64(v, off);
    return v;
}
// Inclusive prefix sum over the wavefront (exact integers).
__device__ __forceinline__ uint64_t wave_scan_u64(uint64_t v, int lane) {
    for (int off = 1; off < 64; off <<= 1) {
        const uint64_t o = shfl_up_u64(v, off);
        if (lane >= off) v += o;
    }
    return v;
}

__device__ uint64_t block_sum_u64(uint64_t v, uint64_t *lds /*[4]*/) {
    v = wave_sum_u64(v);
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    __syncthreads();
    if (lane == 0) lds[wave] = v;
    __syncthreads();
    return (lds[0] + lds[1]) + (lds[2] + lds[3]);
}

__device__ __forceinline__ void store_coherent_u64(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent_u32(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_coherent_u32(const uint32_t *p) {
    return __hip_atomic_load(const_cast<uint32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent_f32(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent_f32(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Thread 0 arrives on `ctr` after every thread's coherent stores completed;
// returns (in every thread) whether this workgroup arrived last, and then
// resets the counter for the next launch.
__device__ bool arrive_last(uint32_t *ctr, uint32_t expected, int *s_flag) {
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = prev == expected - 1;
        if (last) store_coherent_u32(ctr, 0u);
        *s_flag = last ? 1 : 0;
    }
    __syncthreads();
    return *s_flag != 0;
}

struct AccArgs {
    const float *target;
    const float *draft;
    const int32_t *dtok;
    uint32_t k, vocab;
    float T;
    int32_t greedy;
    const float *u;
    const float *ures;
    int32_t *accepted;
    int32_t *tokens;
    uint8_t *scratch;
    uint32_t ept;  // one-launch path: elements per thread
    uint32_t fail_poll;  // one-launch path: workgroup 0 takes its first exchange (greedy: its
                         // arg-max gather) as timed out
    int32_t *host_flag;  // one-launch path: pinned host word set to 1 by a timed-out wait
};

struct Acc {
    AccLayout L;
    float *pmax, *pav;
    uint32_t *pai;
    uint64_t *psum, *pw;
    int32_t *misc;
    __device__ explicit Acc(const AccArgs &a) : L(acc_layout(a.k, a.vocab)) {
        pmax = reinterpret_cast<float *>(a.scratch + L.off_max);
        pav = reinterpret_cast<float *>(a.scratch + L.off_av);
        pai = reinterpret_cast<uint32_t *>(a.scratch + L.off_ai);
        psum = reinterpret_cast<uint64_t *>(a.scratch + L.off_sum);
        pw = reinterpret_cast<uint64_t *>(a.scratch + L.off_w);
        misc = reinterpret_cast<int32_t *>(a.scratch + L.off_misc);
    }
};

__device__ __forceinline__ const float *acc_row(const AccArgs &a, uint32_t r) {
    return r <= a.k ? a.target + (size_t)r * a.vocab : a.draft + (size_t)(r - a.k - 1) * a.vocab;
}

// The 16 logits of thread `tid` in chunk c: element i of the thread is
// x = c*4096 + (i/4)*1024 + tid*4 + i%4, read as four float4 loads when the
// row allows it (coalesced 1 KiB per wavefront).
__device__ __forceinline__ void load_chunk(const float *row, uint32_t vocab, uint32_t c, int tid,
                                           float (&v)[kAccPerThread], uint32_t (&x)[kAccPerThread]) {
    const uint32_t base = c * kAccChunk;
    const bool vec = (vocab % 4 == 0) && ((reinterpret_cast<uintptr_t>(row) & 15) == 0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t x0 = base + q * 1024 + tid * 4;
        if (vec && x0 + 3 < vocab) {
            const float4 f = *reinterpret_cast<const float4 *>(row + x0);
            v[q * 4 + 0] = f.x;
            v[q * 4 + 1] = f.y;
            v[q * 4 + 2] = f.z;
            v[q * 4 + 3] = f.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[q * 4 + j] = (x0 + j < vocab) ? row[x0 + j] : __int_as_float(0x7FC00000);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) x[q * 4 + j] = x0 + j;
    }
}

// ---- row statistics from the per-chunk partials (one wavefront per row) ---
struct RowStat {
    float M, S;
    uint64_t sfix;
};

__device__ RowStat wave_row_stat(const Acc &A, uint32_t r, bool coherent_sum, int lane) {
    float M = -__builtin_inff();
    uint64_t s = 0;
    for (uint32_t c = lane; c < A.L.nch; c += 64) {
        const size_t o = (size_t)r * A.L.nch + c;
        M = fmaxf(M, A.pmax[o]);
        s += coherent_sum ? load_coherent_u64(&A.psum[o]) : A.psum[o];
    }
    RowStat st;
    st.M = group_reduce<64>(M, MaxOp());
    st.sfix = wave_sum_u64(s);
    st.S = u64_to_f32_rn(st.sfix) * 0x1p-40f;
    return st;
}

__device__ uint32_t wave_row_argmax(const Acc &A, uint32_t r, bool coherent, int lane) {
    float bv = -__builtin_inff();
    uint32_t bi = kNone;
    for (uint32_t c = lane; c < A.L.nch; c += 64) {
        const size_t o = (size_t)r * A.L.nch + c;
        const float v = coherent ? load_coherent_f32(&A.pav[o]) : A.pav[o];
        const uint32_t i = coherent ? load_coherent_u32(&A.pai[o]) : A.pai[o];
        if (arg_better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
    // among lanes with the best value, the lowest index (kNone is largest)
    const float best = group_reduce<64>(bv, MaxOp());
    const int cand = (bv == best && bi != kNone) ? (int)bi : 0x7FFFFFFF;
    const int win = group_reduce<64>(cand, MinOp());
    return win == 0x7FFFFFFF ? 0u : (uint32_t)win;
}

// ---- weights of the sampled distribution -----------------------------------
struct SampleRows {
    const float *tr;  // target row i*
    const float *dr;  // draft row i* (residual mode)
    RowStat sp, sq;
    bool resid;
};

__device__ __forceinline__ uint64_t sample_w(const SampleRows &s, float l_t, float l_d, float T) {
    if (s.resid) {
        const float p = prob(row_e(l_t, s.sp.M, T), s.sp.S);
        const float q = prob(row_e(l_d, s.sq.M, T), s.sq.S);
        return fix_shift(ftz(fmaxf(0.0f, p - q)), 62);
    }
    return fix_shift(row_e(l_t, s.sp.M, T), 40);
}

// Inverse CDF over `parts` (per-chunk masses, total W > 0) with uniform u:
// the whole workgroup finds the first x with prefix(w)_x > floor(W u).
__device__ int32_t sample_token(const AccArgs &a, const Acc &A, const SampleRows &s,
                                const uint64_t *parts, bool coherent, uint64_t W, float u) {
    __shared__ uint64_t s_scan[4];
    __shared__ uint32_t s_chunk;
    __shared__ uint64_t s_base;
    __shared__ int32_t s_token;
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const uint64_t t = scale_floor(W, u);
    if (wave == 0) {
        uint64_t carry = 0;
        uint32_t found = kNone;
        uint64_t before = 0;
        for (uint32_t c0 = 0; c0 < A.L.nch && found == kNone; c0 += 64) {
            const uint32_t c = c0 + lane;
            const uint64_t v = c < A.L.nch ? (coherent ? load_coherent_u64(&parts[c]) : parts[c]) : 0;
            const uint64_t incl = carry + wave_scan_u64(v, lane);
            const uint64_t mask = __ballot(c < A.L.nch && incl > t);
            if (mask) {
                const int l = __builtin_ctzll(mask);
                found = c0 + l;
                before = shfl_u64(incl - v, l);
            }
            carry = shfl_u64(incl, 63);
        }
        if (lane == 0) {
            s_chunk = found;
            s_base = before;
            s_token = -1;
        }
    }
    __syncthreads();
    const uint32_t c = s_chunk;
    if (c != kNone) {
        // exact scan of the chunk in element order: thread tid owns elements
        // [c*4096 + tid*16, +16)
        const uint32_t base = c * kAccChunk + tid * kAccPerThread;
        uint64_t w[kAccPerThread];
        uint64_t mine = 0;
#pragma unroll
        for (int i = 0; i < kAccPerThread; ++i) {
            const uint32_t x = base + i;
            uint64_t v = 0;
            if (x < a.vocab) v = sample_w(s, s.tr[x], s.resid ? s.dr[x] : 0.0f, a.T);
            w[i] = v;
            mine += v;
        }
        const uint64_t incl = wave_scan_u64(mine, lane);
        if (lane == 63) s_scan[wave] = incl;
        __syncthreads();
        uint64_t before = 0;
        for (int wv = 0; wv < wave; ++wv) before += s_scan[wv];
        const uint64_t excl = s_base + before + (incl - mine);
        if (excl <= t && t < excl + mine) {
            uint64_t cum = excl;
            for (int i = 0; i < kAccPerThread; ++i) {
                cum += w[i];
                if (cum > t) {
                    s_token = (int32_t)(base + i);
                    break;
                }
            }
        }
    }
    __syncthreads();
    return s_token;
}

__device__ void emit(const AccArgs &a, uint32_t istar, int32_t token) {
    for (uint32_t j = threadIdx.x; j <= a.k; j += blockDim.x)
        a.tokens[j] = j < istar ? a.dtok[j] : (j == istar ? token : -1);
    if (threadIdx.x == 0) *a.accepted = (int32_t)istar;
}

// ---- kernel 1: per-chunk max and greedy arg-max ---------------------------
__global__ __launch_bounds__(kAccThreads) void acc_stats_kernel(AccArgs a) {
    const Acc A(a);
    __shared__ float s_mx[4], s_bv[4];
    __shared__ uint32_t s_bi[4];
    __shared__ int s_last;
    const uint32_t c = blockIdx.x, r = blockIdx.y;
    if (a.greedy && r > a.k) return;
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    float v[kAccPerThread];
    uint32_t xs[kAccPerThread];
    load_chunk(acc_row(a, r), a.vocab, c, tid, v, xs);
    float mx = -__builtin_inff();
    float bv = -__builtin_inff();
    uint32_t bi = kNone;
#pragma unroll
    for (int i = 0; i < kAccPerThread; ++i) {
        if (v[i] > mx) mx = v[i];
        if (arg_better(v[i], xs[i], bv, bi)) {
            bv = v[i];
            bi = xs[i];
        }
    }
    mx = group_reduce<64>(mx, MaxOp());
    {
        const float best = group_reduce<64>(bv, MaxOp());
        const int cand = (bv == best && bi != kNone) ? (int)bi : 0x7FFFFFFF;
        const int win = group_reduce<64>(cand, MinOp());
        bv = best;
        bi = win == 0x7FFFFFFF ? kNone : (uint32_t)win;
    }
    if (lane == 0) {
        s_mx[wave] = mx;
        s_bv[wave] = bv;
        s_bi[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; ++w) {
            mx = fmaxf(mx, s_mx[w]);
            if (arg_better(s_bv[w], s_bi[w], bv, bi)) {
                bv = s_bv[w];
                bi = s_bi[w];
            }
        }
        const size_t o = (size_t)r * A.L.nch + c;
        store_coherent_f32(&A.pmax[o], mx);
        store_coherent_f32(&A.pav[o], bv);
        store_coherent_u32(&A.pai[o], bi);
    }
    if (!a.greedy) return;
    // greedy: the last workgroup decides (runtime/decode.rs:48-64 argmax per
    // target row; accept while it equals the draft).
    if (!arrive_last(reinterpret_cast<uint32_t *>(&A.misc[3]), (a.k + 1) * A.L.nch, &s_last)) return;
    __shared__ uint32_t s_arg[kMaxTokens];
    for (uint32_t rr = wave; rr <= a.k; rr += 4) {
        const uint32_t am = wave_row_argmax(A, rr, true, lane);
        if (lane == 0) s_arg[rr] = am;
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t i = 0;
        while (i < a.k && (int32_t)s_arg[i] == a.dtok[i]) ++i;
        A.misc[0] = (int32_t)i;
        s_last = (int)s_arg[i];
    }
    __syncthreads();
    emit(a, (uint32_t)A.misc[0], s_last);
}

// ---- kernel 2: S_fix partials; the last workgroup decides -----------------
__global__ __launch_bounds__(kAccThreads) void acc_sums_kernel(AccArgs a) {
    if (a.greedy) return;
    const Acc A(a);
    const uint32_t c = blockIdx.x, r = blockIdx.y;
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    __shared__ float s_M;
    __shared__ uint64_t s_red[4];
    __shared__ int s_last;
    __shared__ RowStat s_st[2 * kMaxTokens];
    __shared__ float s_lt[kMaxTokens], s_ld[kMaxTokens];
    __shared__ uint32_t s_istar;
    __shared__ int32_t s_tok;
    // the chunk's loads first: their round trip overlaps wavefront 0's reads
    // of the row maxima
    float v[kAccPerThread];
    uint32_t xs[kAccPerThread];
    load_chunk(acc_row(a, r), a.vocab, c, tid, v, xs);
    if (wave == 0) {
        float M = -__builtin_inff();
        for (uint32_t cc = lane; cc < A.L.nch; cc += 64) M = fmaxf(M, A.pmax[(size_t)r * A.L.nch + cc]);
        M = group_reduce<64>(M, MaxOp());
        if (lane == 0) s_M = M;
    }
    __syncthreads();
    const float M = s_M;
    uint64_t s = 0;
#pragma unroll
    for (int i = 0; i < kAccPerThread; ++i)
        if (xs[i] < a.vocab) s += fix_shift(row_e(v[i], M, a.T), 40);
    s = block_sum_u64(s, s_red);
    if (tid == 0) store_coherent_u64(&A.psum[(size_t)r * A.L.nch + c], s);
    if (!arrive_last(reinterpret_cast<uint32_t *>(&A.misc[1]), A.L.rows * A.L.nch, &s_last)) return;

    // ---- last workgroup: row statistics and the decisions ------------------
    for (uint32_t rr = wave; rr < A.L.rows; rr += 4) {
        const RowStat st = wave_row_stat(A, rr, true, lane);
        if (lane == 0) s_st[rr] = st;
    }
    if (tid < (int)a.k) {
        const int32_t dt = a.dtok[tid];
        const bool ok = dt >= 0 && (uint32_t)dt < a.vocab;
        s_lt[tid] = ok ? a.target[(size_t)tid * a.vocab + dt] : 0.0f;
        s_ld[tid] = ok ? a.draft[(size_t)tid * a.vocab + dt] : 0.0f;
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t i = 0;
        for (; i < a.k; ++i) {
            const int32_t dt = a.dtok[i];
            if (dt < 0 || (uint32_t)dt >= a.vocab) break;  // out of vocabulary: rejected
            const RowStat sp = s_st[i], sq = s_st[a.k + 1 + i];
            const float p = prob(row_e(s_lt[i], sp.M, a.T), sp.S);
            const float q = prob(row_e(s_ld[i], sq.M, a.T), sq.S);
            const bool acc = (q > 0.0f) ? (a.u[i] < p / q) : (p > 0.0f);
            if (!acc) break;
        }
        s_istar = i;
        A.misc[0] = (int32_t)i;
    }
    __syncthreads();
    const uint32_t istar = s_istar;
    if (istar < a.k) return;  // the residual kernel samples the replacement
    // every draft accepted: the bonus token from target row k
    SampleRows srow{a.target + (size_t)a.k * a.vocab, nullptr, s_st[a.k], s_st[a.k], false};
    int32_t token;
    if (srow.sp.sfix == 0) {
        token = (int32_t)wave_row_argmax(A, a.k, false, lane);
        if (tid == 0) s_tok = token;
        __syncthreads();
        token = s_tok;
    } else {
        token = sample_token(a, A, srow, A.psum + (size_t)a.k * A.L.nch, true, srow.sp.sfix,
                             a.ures[a.k]);
    }
    emit(a, istar, token);
}

// ---- kernel 3: residual mass after a rejection; the last workgroup samples -
__global__ __launch_bounds__(kAccThreads) void acc_residual_kernel(AccArgs a) {
    if (a.greedy) return;
    const Acc A(a);
    const uint32_t istar = (uint32_t)A.misc[0];
    if (istar >= a.k) return;
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    __shared__ RowStat s_sp, s_sq;
    __shared__ uint64_t s_red[4];
    __shared__ int s_last;
    __shared__ int32_t s_tok;
    // the chunk's loads first: their round trip overlaps the row statistics
    const float *tr = a.target + (size_t)istar * a.vocab, *dr = a.draft + (size_t)istar * a.vocab;
    float vt[kAccPerThread], vd[kAccPerThread];
    uint32_t xs[kAccPerThread];
    load_chunk(tr, a.vocab, blockIdx.x, tid, vt, xs);
    load_chunk(dr, a.vocab, blockIdx.x, tid, vd, xs);
    if (wave < 2) {
        const RowStat st = wave_row_stat(A, wave == 0 ? istar : a.k + 1 + istar, false, lane);
        if (lane == 0) {
            if (wave == 0) s_sp = st;
            else s_sq = st;
        }
    }
    __syncthreads();
    const SampleRows srow{tr, dr, s_sp, s_sq, true};
    uint64_t s = 0;
#pragma unroll
    for (int i = 0; i < kAccPerThread; ++i)
        if (xs[i] < a.vocab) s += sample_w(srow, vt[i], vd[i], a.T);
    s = block_sum_u64(s, s_red);
    if (tid == 0) store_coherent_u64(&A.pw[blockIdx.x], s);
    if (!arrive_last(reinterpret_cast<uint32_t *>(&A.misc[2]), A.L.nch, &s_last)) return;

    // ---- last workgroup: W, fallbacks, the replacement token ----------------
    __shared__ uint64_t s_W;
    if (wave == 0) {
        uint64_t w = 0;
        for (uint32_t c = lane; c < A.L.nch; c += 64) w += load_coherent_u64(&A.pw[c]);
        w = wave_sum_u64(w);
        if (lane == 0) s_W = w;
    }
    __syncthreads();
    int32_t token;
    if (s_W > 0) {
        token = sample_token(a, A, srow, A.pw, true, s_W, a.ures[istar]);
    } else if (srow.sp.sfix > 0) {
        SampleRows e{srow.tr, nullptr, srow.sp, srow.sp, false};
        token = sample_token(a, A, e, A.psum + (size_t)istar * A.L.nch, false, srow.sp.sfix,
                             a.ures[istar]);
    } else {
        token = (int32_t)wave_row_argmax(A, istar, false, lane);
        if (tid == 0) s_tok = token;
        __syncthreads();
        token = s_tok;
    }
    emit(a, istar, token);
}

// ---- the acceptance as one launch --------------------------------------------
// Workgroup c holds logits [c * 1024, +1024) of every row in registers (4
// consecutive per thread) for the whole launch; grid barriers separate:
//   1  per-row chunk maxima (and arg-maxima of the target rows);
//   2  (stochastic) exact per-row chunk sums of E_x;
//   3  (stochastic, after a rejection) chunk sums of the residual weights.
// After each barrier every workgroup derives the same row statistics and
// decisions from the partials; the workgroup whose chunk holds the sampled
// prefix position scans it in element order and emits the tokens (greedy,
// and the arg-max fallbacks: workgroup 0).  Same definitions, hence the same
// bits, as the three-kernel path above: every sum is an exact integer sum.
// Barrier waits are bounded; a timed-out launch writes *accepted = -1.
// Order-preserving key of a float (never NaN here): larger floats have larger
// keys, and every value's key is above 0.
__device__ __forceinline__ uint32_t fkey(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float fkey_value(uint32_t key) {
    return __uint_as_float((key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key);
}
// Signed-integer key of a float (never NaN here) with the float's order, for
// integer max reductions.
__device__ __forceinline__ int skey(float v) {
    const int b = __float_as_int(v);
    return b >= 0 ? b : b ^ 0x7FFFFFFF;
}
__device__ __forceinline__ float skey_value(int key) { return __int_as_float(key >= 0 ? key : key ^ 0x7FFFFFFF); }
// Arg-max candidate as one key: higher value first, then lower index; an
// empty candidate (index kNone) sorts below every valid one of its value.
__device__ __forceinline__ unsigned long long argkey(float v, uint32_t i) {
    return ((unsigned long long)fkey(v) << 32) | (i == kNone ? 0u : ~i);
}
__device__ __forceinline__ uint32_t argkey_index(unsigned long long key) {
    const uint32_t lo = (uint32_t)key;
    return lo == 0 ? 0u : ~lo;  // no candidate at all: token 0
}
__device__ __forceinline__ uint64_t tagged(uint32_t tag, uint32_t payload) {
    return ((uint64_t)tag << 32) | payload;
}

// Polls items [0, n) of tagged words, spread over the workgroup (item i is
// lo[i], with hi[i] holding the payload's high half when hi is given), and
// calls fn(i, payload) once per item when its tags are current.  False in the
// calling thread after 20 ms without them.
template <typename Fn>
__device__ bool fuse_poll(const uint64_t *lo, const uint64_t *hi, uint32_t n, uint32_t tag, Fn fn) {
    constexpr int kB = 8;
    for (uint32_t base = 0; base < n; base += kB * kFuseThreads) {
        uint32_t pending = 0;
#pragma unroll
        for (int j = 0; j < kB; ++j)
            if (base + threadIdx.x + (uint32_t)j * kFuseThreads < n) pending |= 1u << j;
        int64_t t0 = 0;
        for (uint32_t spin = 1; pending != 0; ++spin) {
            uint64_t w0[kB], w1[kB];
#pragma unroll
            for (int j = 0; j < kB; ++j) {  // every load first: one round trip
                w0[j] = 0;
                w1[j] = 0;
                if (pending & (1u << j)) {
                    const uint32_t i = base + threadIdx.x + (uint32_t)j * kFuseThreads;
                    w0[j] = load_coherent_u64(&lo[i]);
                    if (hi) w1[j] = load_coherent_u64(&hi[i]);
                }
            }
#pragma unroll
            for (int j = 0; j < kB; ++j) {
                if ((pending & (1u << j)) && (uint32_t)(w0[j] >> 32) == tag &&
                    (!hi || (uint32_t)(w1[j] >> 32) == tag)) {
                    fn(base + threadIdx.x + (uint32_t)j * kFuseThreads, (w0[j] & 0xFFFFFFFFull) | (w1[j] << 32));
                    pending &= ~(1u << j);
                }
            }
            if (pending != 0) {
                if ((spin & 15) == 0) {
                    const int64_t now = wall_clock64();
                    if (t0 == 0) {
                        t0 = now;
                    } else if (now - t0 > 2000000) {  // 20 ms at 100 MHz
                        return false;
                    }
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
    }
    return true;
}

// The last workgroup out resets the exit counter and advances the sequence
// word to this launch's tag (every workgroup read the sequence before it
// counted itself out).
__device__ void fuse_exit(uint32_t *ctl, uint32_t tag) {
    __syncthreads();
    if (threadIdx.x == 0 &&
        __hip_atomic_fetch_add(&ctl[kFuseExitWord], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            gridDim.x - 1) {
        store_coherent_u32(&ctl[kFuseExitWord], 0u);
        store_coherent_u32(&ctl[kFuseSeqWord], tag);
    }
}

// Exact u64 sum over a wavefront: three 24-bit limbs, each an int32 DPP
// reduction (64 lanes x 2^24 < 2^31), recombined; exact whenever the true
// sum fits in 64 bits.
__device__ __forceinline__ uint64_t wave_sum_u64_dpp(uint64_t v) {
    const int lo = (int)(v & 0xFFFFFFu), mid = (int)((v >> 24) & 0xFFFFFFu), hi = (int)(v >> 48);
    const uint64_t slo = (uint32_t)group_reduce<64>(lo, AddOp());
    const uint64_t smid = (uint32_t)group_reduce<64>(mid, AddOp());
    const uint64_t shi = (uint32_t)group_reduce<64>(hi, AddOp());
    return slo + (smid << 24) + (shi << 48);
}

// The same for v < 2^48 in every lane: two 24-bit limbs.
__device__ __forceinline__ uint64_t wave_sum_u48_dpp(uint64_t v) {
    const int lo = (int)(v & 0xFFFFFFu), hi = (int)(v >> 24);
    const uint64_t slo = (uint32_t)group_reduce<64>(lo, AddOp());
    const uint64_t shi = (uint32_t)group_reduce<64>(hi, AddOp());
    return slo + (shi << 24);
}

// Block sum over 256 threads (4 wavefronts), result in every thread.
__device__ uint64_t fuse_sum_u64(uint64_t v, uint64_t *lds /*[4]*/) {
    v = wave_sum_u64_dpp(v);
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    __syncthreads();
    if (lane == 0) lds[wave] = v;
    __syncthreads();
    return (lds[0] + lds[1]) + (lds[2] + lds[3]);
}

// The owner of prefix position t (base = the weight before this chunk, w[]
// this thread's four weights in element order, x0 its first element) finds
// the first element whose inclusive prefix exceeds t, in every thread (-1:
// none); its exclusive prefix goes to *s_excl when given.
__device__ int32_t fuse_scan(const uint64_t (&w)[4], uint32_t x0, uint64_t base, uint64_t t, uint64_t *lds,
                             int32_t *s_tok, uint64_t *s_excl = nullptr) {
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint64_t mine = (w[0] + w[1]) + (w[2] + w[3]);
    const uint64_t incl = wave_scan_u64(mine, lane);
    __syncthreads();
    if (lane == 63) lds[wave] = incl;
    if (threadIdx.x == 0) *s_tok = -1;
    __syncthreads();
    uint64_t before = 0;
    for (int wv = 0; wv < wave; ++wv) before += lds[wv];
    const uint64_t excl = base + before + (incl - mine);
    if (excl <= t && t < excl + mine) {
        uint64_t cum = excl;
        for (int j = 0; j < 4; ++j) {
            if (cum + w[j] > t) {
                *s_tok = (int32_t)(x0 + (uint32_t)j);
                if (s_excl) *s_excl = cum;
                break;
            }
            cum += w[j];
        }
    }
    __syncthreads();
    return *s_tok;
}

// A thread's ept (<= 4) logits of a row from element x0 on; NaN in the
// unused slots and past the vocabulary.
__device__ __forceinline__ float4 load_ept(const float *row, uint32_t x0, uint32_t vocab, uint32_t ept) {
    const float nan = __int_as_float(0x7FC00000);
    float4 v = make_float4(nan, nan, nan, nan);
    if (ept == 4 && (vocab % 4 == 0) && x0 + 3 < vocab && ((reinterpret_cast<uintptr_t>(row) & 15) == 0)) {
        v = *reinterpret_cast<const float4 *>(row + x0);
    } else {
        if (0 < ept && x0 + 0 < vocab) v.x = row[x0 + 0];
        if (1 < ept && x0 + 1 < vocab) v.y = row[x0 + 1];
        if (2 < ept && x0 + 2 < vocab) v.z = row[x0 + 2];
        if (3 < ept && x0 + 3 < vocab) v.w = row[x0 + 3];
    }
    return v;
}

// The whole acceptance in one launch for up to R rows (2k + 1 <= R): each
// workgroup keeps its chunk of every row in LDS and exchanges the chunk
// maxima, the exact chunk sums of E_x and (on a rejection) the residual
// weights as tagged words.
template <int R, bool kRecip>
__global__ __launch_bounds__(kFuseThreads) void acc_fused_kernel(AccArgs a) {
    const FuseLayout L = fuse_layout(a.k, a.vocab, a.ept);
    uint32_t *ctl = reinterpret_cast<uint32_t *>(a.scratch);
    uint32_t tag = load_coherent_u32(&ctl[kFuseSeqWord]) + 1u;
    if (tag == 0) tag = 1;  // 0 is the tag of a zeroed slot
    __shared__ float4 s_v[R][kFuseThreads];
    __shared__ uint32_t s_key[R];
    __shared__ unsigned long long s_best[R], s_tot[R], s_bef[R];
    __shared__ float s_fm[R][4];
    __shared__ uint32_t s_fi[R][4];
    __shared__ uint64_t s_red[R][4], s_mine[R], s_scan[4], s_cw[kFuseMaxGrid], s_base;
    __shared__ float s_lt[kMaxTokens], s_ld[kMaxTokens], s_u[kMaxTokens], s_ur[kMaxTokens];
    __shared__ int32_t s_dt[kMaxTokens];
    __shared__ uint32_t s_istar;
    __shared__ int32_t s_tok;
    uint64_t *xmax = reinterpret_cast<uint64_t *>(a.scratch + L.off_max);
    uint64_t *xav = reinterpret_cast<uint64_t *>(a.scratch + L.off_av);
    uint64_t *xai = reinterpret_cast<uint64_t *>(a.scratch + L.off_ai);
    uint64_t *slo = reinterpret_cast<uint64_t *>(a.scratch + L.off_slo);
    uint64_t *shi = reinterpret_cast<uint64_t *>(a.scratch + L.off_shi);
    uint64_t *wlo = reinterpret_cast<uint64_t *>(a.scratch + L.off_wlo);
    uint64_t *whi = reinterpret_cast<uint64_t *>(a.scratch + L.off_whi);
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const uint32_t c = blockIdx.x, k = a.k, nch = L.nch;
    const uint32_t rows = a.greedy ? k + 1 : 2 * k + 1;
    const uint32_t ept = a.ept, chunk = kFuseThreads * ept;
    const RecipT rT = recip_t(a.T);
    // E_x of one logit against row maximum M
    auto rowe = [&](float l, float M) { return kRecip ? row_e_y(l, M, rT) : row_e(l, M, a.T); };
    const uint32_t x0 = c * chunk + (uint32_t)tid * ept;
    // the draft tokens and uniforms first (they arrive with the logits)
    int32_t my_dt = 0;
    float my_u = 0.0f, my_ur = 0.0f;
    if (tid < (int)k) my_dt = a.dtok[tid];
    if (!a.greedy && tid < (int)k) my_u = a.u[tid];
    if (!a.greedy && tid <= (int)k) my_ur = a.ures[tid];
    {
        // every row's four logits of this thread (NaN pads the tail), to LDS
        float4 v[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            if ((uint32_t)r < rows) v[r] = load_ept(acc_row(a, (uint32_t)r), x0, a.vocab, ept);
#pragma unroll
        for (int r = 0; r < R; ++r)
            if ((uint32_t)r < rows) s_v[r][tid] = v[r];
    }
    if (tid <= (int)k) {
        s_dt[tid] = my_dt;
        s_u[tid] = my_u;
        s_ur[tid] = my_ur;
    }
    if (tid < R) {
        s_key[tid] = 0;
        s_best[tid] = 0;
        s_tot[tid] = 0;
        s_bef[tid] = 0;
    }
    // ---- 1: chunk maxima; the target rows' arg-max candidates -----------------
    // (rows unrolled so that their wavefront reductions interleave).  A lane's
    // best candidate is its largest value above -inf at its lowest index, so
    // the wavefront's best value is the wavefront maximum (-inf: none), held
    // by the lowest such lane at the lowest index.
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if ((uint32_t)r < rows) {
            const float4 f = s_v[r][tid];
            // the lane's maximum (NaN ignored: the padding is NaN) and the
            // first element holding it, none when it is -inf
            const float lm = fmaxf(fmaxf(fmaxf(-__builtin_inff(), f.x), f.y), fmaxf(f.z, f.w));
            uint32_t bi = f.w == lm ? x0 + 3 : kNone;
            bi = f.z == lm ? x0 + 2 : bi;
            bi = f.y == lm ? x0 + 1 : bi;
            bi = f.x == lm ? x0 : bi;
            bi = lm > -__builtin_inff() ? bi : kNone;
            const float mx = skey_value(group_reduce<64>(skey(lm), MaxOp()));
            if ((uint32_t)r <= k) {
                const uint64_t held = __ballot(bi != kNone && lm == mx);
                const uint32_t win = held ? (uint32_t)readlane_i((int)bi, __ffsll((unsigned long long)held) - 1) : kNone;
                if (lane == 0) s_fi[r][wave] = win;
            }
            if (lane == 0) s_fm[r][wave] = mx;
        }
    }
    __syncthreads();
    if (tid < (int)rows) {
        const uint32_t r = (uint32_t)tid;
        const float mx = fmaxf(fmaxf(s_fm[r][0], s_fm[r][1]), fmaxf(s_fm[r][2], s_fm[r][3]));
        if (!a.greedy) store_coherent_u64(&xmax[(size_t)r * nch + c], tagged(tag, fkey(mx)));
        if (r <= k) {
            uint32_t bi = kNone;  // the first wavefront holding the maximum
            for (int w = 3; w >= 0; --w)
                if (s_fi[r][w] != kNone && s_fm[r][w] == mx) bi = s_fi[r][w];
            store_coherent_u64(&xav[(size_t)r * nch + c], tagged(tag, __float_as_uint(mx)));
            store_coherent_u64(&xai[(size_t)r * nch + c], tagged(tag, bi));
        }
    }
    // the draft tokens' logits, for the decisions: in flight during the first
    // exchange, to LDS after it
    float lt = 0.0f, ld = 0.0f;
    if (!a.greedy && tid < (int)k && my_dt >= 0 && (uint32_t)my_dt < a.vocab) {
        lt = a.target[(size_t)tid * a.vocab + my_dt];
        ld = a.draft[(size_t)tid * a.vocab + my_dt];
    }
    // arg-max of target rows r0..r1 over every chunk, into s_best
    auto argmax_rows = [&](uint32_t r0, uint32_t r1) {
        return fuse_poll(xav + (size_t)r0 * nch, xai + (size_t)r0 * nch, (r1 - r0 + 1) * nch, tag,
                         [&](uint32_t i, uint64_t p) {
                             atomicMax(&s_best[r0 + i / nch],
                                       argkey(__uint_as_float((uint32_t)p), (uint32_t)(p >> 32)));
                         });
    };
    // the outputs: accepted drafts, then the sampled token, then -1
    auto emit_fused = [&](uint32_t istar, int32_t token) {
        if (tid <= (int)k) a.tokens[tid] = (uint32_t)tid < istar ? s_dt[tid] : ((uint32_t)tid == istar ? token : -1);
        if (tid == 0) *a.accepted = (int32_t)istar;
    };
    auto fail = [&]() {
        if (tid == 0) {
            __hip_atomic_store(a.accepted, -1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (a.host_flag) __hip_atomic_store(a.host_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        fuse_exit(ctl, tag);
    };
    // ---- greedy: workgroup 0 decides -------------------------------------------
    if (a.greedy) {
        if (c == 0) {
            // (a forced timeout, TQF_HIP_ACCEPT_FAIL_POLL, takes this gather as
            // timed out once its words are in)
            if (__syncthreads_or(!argmax_rows(0, k) || a.fail_poll)) {
                fail();
                return;
            }
            if (tid == 0) {
                uint32_t i = 0;
                while (i < k && (int32_t)argkey_index(s_best[i]) == s_dt[i]) ++i;
                s_istar = i;
                s_tok = (int32_t)argkey_index(s_best[i]);
            }
            __syncthreads();
            emit_fused(s_istar, s_tok);
        }
        fuse_exit(ctl, tag);
        return;
    }
    // ---- 2: row maxima, then the chunk's exact sums of E_x ---------------------
    if (__syncthreads_or(!fuse_poll(xmax, nullptr, rows * nch, tag,
                                    [&](uint32_t i, uint64_t p) { atomicMax(&s_key[i / nch], (uint32_t)p); }) ||
                         (a.fail_poll && c == 0))) {
        fail();
        return;
    }
    if (tid < (int)k) {
        s_lt[tid] = lt;
        s_ld[tid] = ld;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if ((uint32_t)r < rows) {
            const float M = fkey_value(s_key[r]);
            const float4 f = s_v[r][tid];
            const float e[4] = {f.x, f.y, f.z, f.w};
            uint64_t sum = 0;  // the NaN padding adds 0; four terms <= 2^40 each
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if ((uint32_t)j < ept) sum += fix_shift(rowe(e[j], M), 40);
            sum = wave_sum_u48_dpp(sum);
            if (lane == 0) s_red[r][wave] = sum;
        }
    }
    __syncthreads();
    if (tid < (int)rows) {
        const uint32_t r = (uint32_t)tid;
        const uint64_t sum = (s_red[r][0] + s_red[r][1]) + (s_red[r][2] + s_red[r][3]);
        s_mine[r] = sum;
        store_coherent_u64(&slo[(size_t)r * nch + c], tagged(tag, (uint32_t)sum));
        store_coherent_u64(&shi[(size_t)r * nch + c], tagged(tag, (uint32_t)(sum >> 32)));
    }
    // ---- row totals and the sums before this chunk; the decisions -------------
    if (__syncthreads_or(!fuse_poll(slo, shi, rows * nch, tag, [&](uint32_t i, uint64_t p) {
            const uint32_t r = i / nch;
            atomicAdd(&s_tot[r], (unsigned long long)p);
            if (i - r * nch < c) atomicAdd(&s_bef[r], (unsigned long long)p);
        }))) {
        fail();
        return;
    }
    auto stat = [&](uint32_t r) {
        RowStat st;
        st.M = fkey_value(s_key[r]);
        st.sfix = s_tot[r];
        st.S = u64_to_f32_rn(st.sfix) * 0x1p-40f;
        return st;
    };
    if (wave == 0) {
        // lane i decides draft i; i* is the first rejection (k if none)
        bool stop = true;
        if ((uint32_t)lane < k) {
            const int32_t dt = s_dt[lane];
            if (dt >= 0 && (uint32_t)dt < a.vocab) {  // out of vocabulary: rejected
                const RowStat sp = stat(lane), sq = stat(k + 1 + lane);
                const float p = prob(rowe(s_lt[lane], sp.M), sp.S);
                const float q = prob(rowe(s_ld[lane], sq.M), sq.S);
                stop = !((q > 0.0f) ? (s_u[lane] < p / q) : (p > 0.0f));
            }
        }
        const uint64_t stops = __ballot(stop);
        if (lane == 0) s_istar = (uint32_t)__ffsll((unsigned long long)stops) - 1;
    }
    __syncthreads();
    const uint32_t istar = s_istar;
    const RowStat sp = stat(istar);
    const float4 ft = s_v[istar][tid];
    const float vt[4] = {ft.x, ft.y, ft.z, ft.w};
    int32_t token = -1;
    bool emitter = false;
    // weights of four elements: E_x of a target row, or the residual of pair i*
    auto e_weights = [&](const float (&x)[4], uint64_t (&w)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = (uint32_t)j < ept ? fix_shift(rowe(x[j], sp.M), 40) : 0;
    };
    const RowStat sq = stat(istar < k ? k + 1 + istar : istar);
    auto resid_weights = [&](const float (&xt)[4], const float (&xd)[4], uint64_t (&w)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            w[j] = 0;
            if ((uint32_t)j < ept) {  // the NaN padding past the vocabulary weighs 0
                const float p = prob(rowe(xt[j], sp.M), sp.S);
                const float q = prob(rowe(xd[j], sq.M), sq.S);
                w[j] = fix_shift(ftz(fmaxf(0.0f, p - q)), 62);
            }
        }
    };
    // a draw from E_x of target row r (sfix > 0) by the workgroup owning it,
    // from the chunk prefixes of the sums exchange
    auto draw_e = [&](uint32_t r) {
        const uint64_t t = scale_floor(sp.sfix, s_ur[r]);
        if (s_bef[r] <= t && t < s_bef[r] + s_mine[r]) {  // uniform per workgroup
            uint64_t w[4];
            e_weights(vt, w);
            token = fuse_scan(w, x0, s_bef[r], t, s_scan, &s_tok);
            emitter = true;
        }
    };
    // workgroup 0: the chunk that holds prefix position t = floor(total * u)
    // of the chunk weights in s_cw (s_base: the weight before that chunk); -1
    // for a zero total.  Every thread holds four consecutive chunks.
    auto locate = [&](float uu, uint64_t &t) -> int32_t {
        uint64_t cw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) cw[j] = (uint32_t)tid * 4 + j < nch ? s_cw[tid * 4 + j] : 0;
        const uint64_t mine = (cw[0] + cw[1]) + (cw[2] + cw[3]);
        const uint64_t incl = wave_scan_u64(mine, lane);
        __syncthreads();
        if (lane == 63) s_scan[wave] = incl;
        if (tid == 0) s_tok = -1;
        __syncthreads();
        uint64_t before = 0, total = 0;
        for (int wv = 0; wv < 4; ++wv) {
            if (wv < wave) before += s_scan[wv];
            total += s_scan[wv];
        }
        if (total == 0) return -1;  // uniform
        t = scale_floor(total, uu);
        const uint64_t excl = before + (incl - mine);
        if (excl <= t && t < excl + mine) {
            uint64_t cum = excl;
            for (int j = 0; j < 4; ++j) {
                if (cum + cw[j] > t) {
                    s_tok = tid * 4 + j;
                    s_base = cum;
                    break;
                }
                cum += cw[j];
            }
        }
        __syncthreads();
        return s_tok;
    };
    // workgroup 0: chunk cs's four logits of this thread in row r
    auto chunk_row = [&](int32_t cs, uint32_t r, float (&x)[4]) {
        const float4 g = load_ept(acc_row(a, r), (uint32_t)cs * chunk + (uint32_t)tid * ept, a.vocab, ept);
        x[0] = g.x;
        x[1] = g.y;
        x[2] = g.z;
        x[3] = g.w;
    };
    // the arg-max fallback of target row r, in workgroup 0
    auto draw_argmax = [&](uint32_t r) -> bool {
        if (__syncthreads_or(!argmax_rows(r, r))) return false;
        token = (int32_t)argkey_index(s_best[r]);
        emitter = true;
        return true;
    };
    bool ok = true;
    if (istar == k) {
        // ---- every draft accepted: the bonus token from E_x of target row k -------
        if (sp.sfix > 0)
            draw_e(k);
        else if (c == 0)
            ok = draw_argmax(k);
    } else {
        // ---- 3: the residual mass of pair i*: each workgroup hands its chunk's
        // weight to workgroup 0, which draws the chunk and scans it again ------
        const float4 fd = s_v[k + 1 + istar][tid];
        const float vd[4] = {fd.x, fd.y, fd.z, fd.w};
        uint64_t w[4];
        resid_weights(vt, vd, w);
        const uint64_t chunk_w = fuse_sum_u64((w[0] + w[1]) + (w[2] + w[3]), s_scan);
        if (tid == 0) {
            store_coherent_u64(&wlo[c], tagged(tag, (uint32_t)chunk_w));
            store_coherent_u64(&whi[c], tagged(tag, (uint32_t)(chunk_w >> 32)));
        }
        if (c != 0) {
            fuse_exit(ctl, tag);
            return;
        }
        if (__syncthreads_or(!fuse_poll(wlo, whi, nch, tag, [&](uint32_t i, uint64_t p) { s_cw[i] = p; }))) {
            fail();
            return;
        }
        uint64_t t = 0;
        int32_t cs = locate(s_ur[istar], t);
        if (cs >= 0) {
            float xt[4], xd[4];
            chunk_row(cs, istar, xt);
            chunk_row(cs, k + 1 + istar, xd);
            uint64_t wc[4];
            resid_weights(xt, xd, wc);
            token = fuse_scan(wc, (uint32_t)cs * chunk + (uint32_t)tid * ept, s_base, t, s_scan, &s_tok);
            emitter = true;
        } else if (sp.sfix > 0) {
            // no residual mass: E_x of target row i*, from its chunk sums
            if (__syncthreads_or(!fuse_poll(slo + (size_t)istar * nch, shi + (size_t)istar * nch, nch, tag,
                                            [&](uint32_t i, uint64_t p) { s_cw[i] = p; }))) {
                fail();
                return;
            }
            cs = locate(s_ur[istar], t);
            if (cs >= 0) {
                float xt[4];
                chunk_row(cs, istar, xt);
                uint64_t wc[4];
                e_weights(xt, wc);
                token = fuse_scan(wc, (uint32_t)cs * chunk + (uint32_t)tid * ept, s_base, t, s_scan, &s_tok);
                emitter = true;
            }
        } else {
            ok = draw_argmax(istar);
        }
    }
    if (!ok) {
        fail();
        return;
    }
    if (emitter) {
        __syncthreads();
        if (tid == 0) s_tok = token;
        __syncthreads();
        emit_fused(istar, s_tok);
    }
    fuse_exit(ctl, tag);
}

// Largest grid acc_fused_kernel<R> runs with: co-resident on this device (so
// the exchanges complete when the device runs nothing else; their waits are
// bounded either way) and at most kFuseMaxGrid.  0: none.
template <int R>
uint32_t fuse_max_grid() {
    static const uint32_t g = [] {
        int dev = 0, cus = 0, p0 = 0, p1 = 0;
        if (hipGetDevice(&dev) != hipSuccess) return 0u;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0u;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&p0, (const void *)acc_fused_kernel<R, false>, kFuseThreads,
                                                         0) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&p1, (const void *)acc_fused_kernel<R, true>, kFuseThreads,
                                                         0) != hipSuccess)
            return 0u;
        const uint32_t n = (uint32_t)(cus * (p0 < p1 ? p0 : p1));
        return n < kFuseMaxGrid ? n : kFuseMaxGrid;
    }();
    return g;
}

// Row capacity of the one-launch kernel for k: 3, 7 or 15 rows.
inline int fuse_cap(uint32_t k) { return 2 * k + 1 <= 3 ? 3 : (2 * k + 1 <= 7 ? 7 : 15); }

// Elements per thread: the fewest (1..4) whose chunks number no more than the
// device's compute units (4 beyond that).
uint32_t fuse_ept(uint32_t vocab) {
    static const uint32_t cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess) return 0u;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0u;
        return (uint32_t)n;
    }();
    for (uint32_t e = 1; e < 4; ++e)
        if (((uint64_t)vocab + kFuseThreads * e - 1) / (kFuseThreads * e) <= cus) return e;
    return 4;
}

bool fuse_fits(uint32_t k, uint32_t vocab) {
    const uint32_t nch = fuse_layout(k, vocab, fuse_ept(vocab)).nch;
    switch (fuse_cap(k)) {
    case 3: return nch <= fuse_max_grid<3>();
    case 7: return nch <= fuse_max_grid<7>();
    default: return nch <= fuse_max_grid<15>();
    }
}

// The device queries behind the launch choice, made once per process outside
// any stream capture (at context creation).
void accept_warm() {
    (void)fuse_ept(0);
    (void)fuse_max_grid<3>();
    (void)fuse_max_grid<7>();
    (void)fuse_max_grid<15>();
}

size_t accept_scratch_bytes(uint32_t k, uint32_t vocab) {
    return fuse_fits(k, vocab) ? fuse_layout(k, vocab, fuse_ept(vocab)).total : acc_layout(k, vocab).total;
}
size_t accept_multi_scratch_bytes(uint32_t k, uint32_t vocab) { return acc_layout(k, vocab).total; }
bool accept_one_launch(uint32_t k, uint32_t vocab) { return fuse_fits(k, vocab); }

hipError_t launch_accept(hipStream_t s, const float *target, const float *draft,
                         const int32_t *dtok, uint32_t k, uint32_t vocab, float temperature,
                         int32_t greedy, const float *u, const float *ures, int32_t *accepted,
                         int32_t *tokens, void *scratch, hipEvent_t ev_start, hipEvent_t ev_stop,
                         bool multi, int32_t *host_flag) {
    // a poll timeout forced from the host, for the tests of the failure path
    // (TQF_HIP_ACCEPT_FAIL_POLL = 1); read at every launch
    const char *fail_poll = std::getenv("TQF_HIP_ACCEPT_FAIL_POLL");
    AccArgs a{target, draft, dtok, k, vocab, temperature, greedy, u, ures, accepted, tokens,
              reinterpret_cast<uint8_t *>(scratch), fuse_ept(vocab),
              fail_poll && fail_poll[0] && fail_poll[0] != '0' ? 1u : 0u, host_flag};
    if (ev_start) (void)hipEventRecord(ev_start, s);
    if (!multi && fuse_fits(k, vocab)) {
        // one plain launch: a cooperative launch measured about 15 us of
        // extra dispatch time, and the grid fits co-resident anyway
        const dim3 grid(fuse_layout(k, vocab, a.ept).nch);
        const bool recip = !greedy && recip_t_exact(temperature);
        const dim3 block(kFuseThreads);
        switch (fuse_cap(k) * 2 + (recip ? 1 : 0)) {
        case 6: hipLaunchKernelGGL((acc_fused_kernel<3, false>), grid, block, 0, s, a); break;
        case 7: hipLaunchKernelGGL((acc_fused_kernel<3, true>), grid, block, 0, s, a); break;
        case 14: hipLaunchKernelGGL((acc_fused_kernel<7, false>), grid, block, 0, s, a); break;
        case 15: hipLaunchKernelGGL((acc_fused_kernel<7, true>), grid, block, 0, s, a); break;
        case 30: hipLaunchKernelGGL((acc_fused_kernel<15, false>), grid, block, 0, s, a); break;
        default: hipLaunchKernelGGL((acc_fused_kernel<15, true>), grid, block, 0, s, a); break;
        }
    } else {
        const AccLayout L = acc_layout(k, vocab);
        hipLaunchKernelGGL(acc_stats_kernel, dim3(L.nch, L.rows), dim3(kAccThreads), 0, s, a);
        hipLaunchKernelGGL(acc_sums_kernel, dim3(L.nch, L.rows), dim3(kAccThreads), 0, s, a);
        hipLaunchKernelGGL(acc_residual_kernel, dim3(L.nch), dim3(kAccThreads), 0, s, a);
    }
    if (ev_stop) (void)hipEventRecord(ev_stop, s);
    return hipGetLastError();
}

// ---- top_logit_candidates (runtime/decode.rs:48-64) ------------------------
// Order: higher logit first, lower index on ties; values that are not > -inf
// (and NaN) never enter; empty slots are (0, -inf).
struct Top4 {
    float v[4];
    uint32_t i[4];
};

__device__ __forceinline__ bool cand_before(float v, uint32_t i, float w, uint32_t j) {
    return v > w || (v == w && i < j);
}

__device__ __forceinline__ void top4_insert(Top4 &t, float v, uint32_t i) {
    if (!(v > -__builtin_inff())) return;
    int pos = 4;
    for (int s = 3; s >= 0; --s)
        if (cand_before(v, i, t.v[s], t.i[s])) pos = s;
    if (pos == 4) return;
    for (int s = 3; s > pos; --s) {
        t.v[s] = t.v[s - 1];
        t.i[s] = t.i[s - 1];
    }
    t.v[pos] = v;
    t.i[pos] = i;
}

__global__ __launch_bounds__(256) void top4_kernel(const float *__restrict__ logits,
                                                   uint32_t vocab, uint32_t *tokens4,
                                                   float *logits4) {
    const uint32_t r = blockIdx.x;
    const float *row = logits + (size_t)r * vocab;
    Top4 t;
    for (int s = 0; s < 4; ++s) {
        t.v[s] = -__builtin_inff();
        t.i[s] = kNone;
    }
    for (uint32_t x = threadIdx.x; x < vocab; x += 256) top4_insert(t, row[x], x);
    __shared__ Top4 s_t[256];
    s_t[threadIdx.x] = t;
    __syncthreads();
    for (int stride = 128; stride >= 1; stride >>= 1) {
        if ((int)threadIdx.x < stride) {
            Top4 m = s_t[threadIdx.x];
            const Top4 o = s_t[threadIdx.x + stride];
            for (int s = 0; s < 4; ++s)
                if (o.i[s] != kNone) top4_insert(m, o.v[s], o.i[s]);
            s_t[threadIdx.x] = m;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        for (int s = 0; s < 4; ++s) {
            const bool empty = s_t[0].i[s] == kNone;
            tokens4[(size_t)r * 4 + s] = empty ? 0u : s_t[0].i[s];
            logits4[(size_t)r * 4 + s] = empty ? -__builtin_inff() : s_t[0].v[s];
        }
    }
}

hipError_t launch_top4(hipStream_t s, const float *logits, uint32_t rows, uint32_t vocab,
                       uint32_t *tokens4, float *logits4) {
    hipLaunchKernelGGL(top4_kernel, dim3(rows), dim3(256), 0, s, logits, vocab, tokens4, logits4);
    return hipGetLastError();
}

}  // namespace tqf
