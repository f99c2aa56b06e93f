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

#include "tqf_device.h"
#include "tqf_internal.h"

#pragma clang fp contract(off)

namespace tqf {

constexpr int kAccThreads = 256;
constexpr int kAccPerThread = 16;
constexpr int kAccChunk = kAccThreads * kAccPerThread;  // 4096
constexpr uint32_t kNone = 0xFFFFFFFFu;

struct AccLayout {
    uint32_t rows, nch;
    size_t off_max, off_av, off_ai, off_sum, off_w, off_misc, total;
};

// misc (first 64 bytes, the same for every k and vocab so that the counters
// are never overlaid by another call's partials): [0] i*, [1] counter (sums),
// [2] counter (residual), [3] counter (stats).  Partials follow.
__host__ __device__ inline AccLayout acc_layout(uint32_t k, uint32_t vocab) {
    AccLayout L;
    L.rows = 2 * k + 1;
    L.nch = (vocab + kAccChunk - 1) / kAccChunk;
    const size_t n = (size_t)L.rows * L.nch;
    L.off_misc = 0;
    L.off_max = 64;
    L.off_av = L.off_max + n * 4;
    L.off_ai = L.off_av + n * 4;
    L.off_sum = (L.off_ai + n * 4 + 7) & ~(size_t)7;
    L.off_w = L.off_sum + n * 8;
    L.total = L.off_w + (size_t)L.nch * 8;
    return L;
}

size_t accept_scratch_bytes(uint32_t k, uint32_t vocab) { return acc_layout(k, vocab).total; }

// ---- exact scalar building blocks ----------------------------------------
__device__ __forceinline__ float acc_exp(float z) {
    if (!(z >= -87.0f)) return 0.0f;
    if (z > 88.0f) return __builtin_inff();
    const float n = __builtin_rintf(z * 0x1.715476p+0f);
    float r = __builtin_fmaf(-n, 0x1.62e4p-1f, z);
    r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int ni = (int)n;
    return p * __uint_as_float((uint32_t)(ni + 127) << 23);
}

__device__ __forceinline__ uint64_t fix_shift(float v, int shift) {
    const uint32_t b = __float_as_uint(v);
    if (b & 0x80000000u) return 0;
    const uint32_t ex = (b >> 23) & 0xFFu;
    if (ex == 0 || ex == 0xFF) return 0;
    const uint64_t m = (uint64_t)((b & 0x7FFFFFu) | 0x800000u);
    const int s = (int)ex - 127 - 23 + shift;
    if (s >= 0) return m << s;
    if (s <= -24) return 0;
    return m >> (-s);
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
    if (l != l) return 0.0f;
    if (l == M) return 1.0f;
    return acc_exp((l - M) / T);
}

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

hipError_t launch_accept(hipStream_t s, const float *target, const float *draft,
                         const int32_t *dtok, uint32_t k, uint32_t vocab, float temperature,
                         int32_t greedy, const float *u, const float *ures, int32_t *accepted,
                         int32_t *tokens, void *scratch, hipEvent_t ev_start, hipEvent_t ev_stop) {
    AccArgs a{target, draft, dtok, k, vocab, temperature, greedy, u, ures, accepted, tokens,
              reinterpret_cast<uint8_t *>(scratch)};
    const AccLayout L = acc_layout(k, vocab);
    if (ev_start) (void)hipEventRecord(ev_start, s);
    hipLaunchKernelGGL(acc_stats_kernel, dim3(L.nch, L.rows), dim3(kAccThreads), 0, s, a);
    hipLaunchKernelGGL(acc_sums_kernel, dim3(L.nch, L.rows), dim3(kAccThreads), 0, s, a);
    hipLaunchKernelGGL(acc_residual_kernel, dim3(L.nch), dim3(kAccThreads), 0, s, a);
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
