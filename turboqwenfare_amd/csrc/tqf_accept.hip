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
// Kernels (one pass over the logits each, chunks of 4096 per workgroup):
//   stats    per (row, chunk): max over non-NaN and the greedy arg-max
//   sums     per (row, chunk): S_fix partial (stochastic only)
//   residual per chunk: decisions (recomputed redundantly per workgroup from
//            the partials) and, if a draft was rejected, the residual mass
//   final    one workgroup: emitted tokens, locating the sampled token with
//            an exact prefix scan inside the selected chunk.
#include <hip/hip_runtime.h>

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

__host__ __device__ inline AccLayout acc_layout(uint32_t k, uint32_t vocab) {
    AccLayout L;
    L.rows = 2 * k + 1;
    L.nch = (vocab + kAccChunk - 1) / kAccChunk;
    const size_t n = (size_t)L.rows * L.nch;
    L.off_max = 0;
    L.off_av = L.off_max + n * 4;
    L.off_ai = L.off_av + n * 4;
    L.off_sum = (L.off_ai + n * 4 + 7) & ~(size_t)7;
    L.off_w = L.off_sum + n * 8;
    L.off_misc = L.off_w + (size_t)L.nch * 8;
    L.total = L.off_misc + 64;
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

__device__ uint64_t block_sum_u64(uint64_t v, uint64_t *lds /*[4]*/) {
    for (int off = 32; off >= 1; off >>= 1) v += shfl_xor_u64(v, off);
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    __syncthreads();
    if (lane == 0) lds[wave] = v;
    __syncthreads();
    return (lds[0] + lds[1]) + (lds[2] + lds[3]);
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

__device__ __forceinline__ const float *acc_row(const AccArgs &a, uint32_t r) {
    return r <= a.k ? a.target + (size_t)r * a.vocab : a.draft + (size_t)(r - a.k - 1) * a.vocab;
}

// ---- kernel 1: per-chunk max and greedy arg-max ---------------------------
__global__ __launch_bounds__(kAccThreads) void acc_stats_kernel(AccArgs a) {
    const AccLayout L = acc_layout(a.k, a.vocab);
    const uint32_t c = blockIdx.x, r = blockIdx.y;
    if (a.greedy && r > a.k) return;
    const float *row = acc_row(a, r);
    float mx = -__builtin_inff();
    float bv = -__builtin_inff();
    uint32_t bi = kNone;
    const uint32_t base = c * kAccChunk + threadIdx.x * kAccPerThread;
    for (int i = 0; i < kAccPerThread; ++i) {
        const uint32_t x = base + i;
        if (x >= a.vocab) break;
        const float l = row[x];
        if (l > mx) mx = l;
        if (l > bv) {
            bv = l;
            bi = x;
        }
    }
    __shared__ float s_mx[4], s_bv[4];
    __shared__ uint32_t s_bi[4];
    for (int off = 32; off >= 1; off >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, off));
        const float ov = __shfl_xor(bv, off);
        const uint32_t oi = __shfl_xor(bi, off);
        if (arg_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    if (lane == 0) {
        s_mx[wave] = mx;
        s_bv[wave] = bv;
        s_bi[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) {
            mx = fmaxf(mx, s_mx[w]);
            if (arg_better(s_bv[w], s_bi[w], bv, bi)) {
                bv = s_bv[w];
                bi = s_bi[w];
            }
        }
        const size_t o = (size_t)r * L.nch + c;
        reinterpret_cast<float *>(a.scratch + L.off_max)[o] = mx;
        reinterpret_cast<float *>(a.scratch + L.off_av)[o] = bv;
        reinterpret_cast<uint32_t *>(a.scratch + L.off_ai)[o] = bi;
    }
}

__device__ __forceinline__ float row_max(const AccArgs &a, const AccLayout &L, uint32_t r) {
    const float *pm = reinterpret_cast<const float *>(a.scratch + L.off_max) + (size_t)r * L.nch;
    float M = -__builtin_inff();
    for (uint32_t c = 0; c < L.nch; ++c) M = fmaxf(M, pm[c]);
    return M;
}

__device__ __forceinline__ uint64_t row_sfix(const AccArgs &a, const AccLayout &L, uint32_t r) {
    const uint64_t *ps =
        reinterpret_cast<const uint64_t *>(a.scratch + L.off_sum) + (size_t)r * L.nch;
    uint64_t s = 0;
    for (uint32_t c = 0; c < L.nch; ++c) s += ps[c];
    return s;
}

__device__ __forceinline__ uint32_t row_argmax(const AccArgs &a, const AccLayout &L, uint32_t r) {
    const float *pv = reinterpret_cast<const float *>(a.scratch + L.off_av) + (size_t)r * L.nch;
    const uint32_t *pi =
        reinterpret_cast<const uint32_t *>(a.scratch + L.off_ai) + (size_t)r * L.nch;
    float bv = -__builtin_inff();
    uint32_t bi = kNone;
    for (uint32_t c = 0; c < L.nch; ++c)
        if (arg_better(pv[c], pi[c], bv, bi)) {
            bv = pv[c];
            bi = pi[c];
        }
    return bi == kNone ? 0u : bi;
}

// ---- kernel 2: per-chunk S_fix partials -----------------------------------
__global__ __launch_bounds__(kAccThreads) void acc_sums_kernel(AccArgs a) {
    if (a.greedy) return;
    const AccLayout L = acc_layout(a.k, a.vocab);
    const uint32_t c = blockIdx.x, r = blockIdx.y;
    __shared__ float s_M;
    __shared__ uint64_t s_red[4];
    if (threadIdx.x == 0) s_M = row_max(a, L, r);
    __syncthreads();
    const float M = s_M;
    const float *row = acc_row(a, r);
    uint64_t s = 0;
    const uint32_t base = c * kAccChunk + threadIdx.x * kAccPerThread;
    for (int i = 0; i < kAccPerThread; ++i) {
        const uint32_t x = base + i;
        if (x >= a.vocab) break;
        s += fix_shift(row_e(row[x], M, a.T), 40);
    }
    s = block_sum_u64(s, s_red);
    if (threadIdx.x == 0)
        reinterpret_cast<uint64_t *>(a.scratch + L.off_sum)[(size_t)r * L.nch + c] = s;
}

struct RowStat {
    float M, S;
    uint64_t sfix;
};

__device__ RowStat row_stat(const AccArgs &a, const AccLayout &L, uint32_t r) {
    RowStat st;
    st.M = row_max(a, L, r);
    st.sfix = row_sfix(a, L, r);
    st.S = u64_to_f32_rn(st.sfix) * 0x1p-40f;
    return st;
}

// Decision sequence; returns i*.  Called by one thread.
__device__ uint32_t decide(const AccArgs &a, const AccLayout &L, RowStat &sp_star,
                           RowStat &sq_star) {
    for (uint32_t i = 0; i < a.k; ++i) {
        const RowStat sp = row_stat(a, L, i);
        const RowStat sq = row_stat(a, L, a.k + 1 + i);
        const int32_t dt = a.dtok[i];
        if (dt < 0 || (uint32_t)dt >= a.vocab) {  // out of vocabulary: rejected
            sp_star = sp;
            sq_star = sq;
            return i;
        }
        const uint32_t d = (uint32_t)dt;
        const float p = prob(row_e(a.target[(size_t)i * a.vocab + d], sp.M, a.T), sp.S);
        const float q = prob(row_e(a.draft[(size_t)i * a.vocab + d], sq.M, a.T), sq.S);
        const bool acc = (q > 0.0f) ? (a.u[i] < p / q) : (p > 0.0f);
        if (!acc) {
            sp_star = sp;
            sq_star = sq;
            return i;
        }
    }
    return a.k;
}

__device__ __forceinline__ uint64_t residual_w(const AccArgs &a, uint32_t istar, uint32_t x,
                                               const RowStat &sp, const RowStat &sq) {
    const float p = prob(row_e(a.target[(size_t)istar * a.vocab + x], sp.M, a.T), sp.S);
    const float q = prob(row_e(a.draft[(size_t)istar * a.vocab + x], sq.M, a.T), sq.S);
    return fix_shift(ftz(fmaxf(0.0f, p - q)), 62);
}

// ---- kernel 3: decisions + residual mass per chunk ------------------------
__global__ __launch_bounds__(kAccThreads) void acc_residual_kernel(AccArgs a) {
    if (a.greedy) return;
    const AccLayout L = acc_layout(a.k, a.vocab);
    __shared__ uint32_t s_istar;
    __shared__ RowStat s_sp, s_sq;
    __shared__ uint64_t s_red[4];
    if (threadIdx.x == 0) {
        RowStat sp{}, sq{};
        s_istar = decide(a, L, sp, sq);
        s_sp = sp;
        s_sq = sq;
        if (blockIdx.x == 0) reinterpret_cast<int32_t *>(a.scratch + L.off_misc)[0] = (int32_t)s_istar;
    }
    __syncthreads();
    const uint32_t istar = s_istar;
    if (istar >= a.k) return;
    const RowStat sp = s_sp, sq = s_sq;
    uint64_t s = 0;
    const uint32_t base = blockIdx.x * kAccChunk + threadIdx.x * kAccPerThread;
    for (int i = 0; i < kAccPerThread; ++i) {
        const uint32_t x = base + i;
        if (x >= a.vocab) break;
        s += residual_w(a, istar, x, sp, sq);
    }
    s = block_sum_u64(s, s_red);
    if (threadIdx.x == 0) reinterpret_cast<uint64_t *>(a.scratch + L.off_w)[blockIdx.x] = s;
}

// ---- kernel 4: emitted tokens ----------------------------------------------
__global__ __launch_bounds__(kAccThreads) void acc_final_kernel(AccArgs a) {
    const AccLayout L = acc_layout(a.k, a.vocab);
    __shared__ int32_t s_token;
    __shared__ uint32_t s_istar, s_chunk, s_mode;
    __shared__ uint64_t s_t, s_base;
    __shared__ RowStat s_sp, s_sq;
    __shared__ uint64_t s_scan[4];
    const int tid = threadIdx.x;
    if (a.greedy) {
        if (tid == 0) {
            uint32_t i = 0;
            for (; i < a.k; ++i) {
                const uint32_t am = row_argmax(a, L, i);
                if ((int32_t)am != a.dtok[i]) break;
                a.tokens[i] = a.dtok[i];
            }
            a.tokens[i] = (int32_t)row_argmax(a, L, i);
            for (uint32_t j = i + 1; j <= a.k; ++j) a.tokens[j] = -1;
            *a.accepted = (int32_t)i;
        }
        return;
    }
    // mode 0: residual weights of row pair i*; 1: E of target i*; 2: arg-max
    if (tid == 0) {
        const uint32_t istar = (uint32_t)reinterpret_cast<const int32_t *>(a.scratch + L.off_misc)[0];
        uint32_t mode = 1;
        uint64_t W = 0;
        const uint64_t *parts;
        if (istar < a.k) {
            parts = reinterpret_cast<const uint64_t *>(a.scratch + L.off_w);
            for (uint32_t c = 0; c < L.nch; ++c) W += parts[c];
            if (W > 0) mode = 0;
        }
        if (mode == 1) {
            parts = reinterpret_cast<const uint64_t *>(a.scratch + L.off_sum) + (size_t)istar * L.nch;
            W = 0;
            for (uint32_t c = 0; c < L.nch; ++c) W += parts[c];
            if (W == 0) mode = 2;
        }
        s_istar = istar;
        s_mode = mode;
        if (mode == 2) {
            s_token = (int32_t)row_argmax(a, L, istar);
        } else {
            const uint64_t t = scale_floor(W, a.ures[istar]);
            uint64_t cum = 0;
            uint32_t c = 0;
            for (; c < L.nch; ++c) {
                if (cum + parts[c] > t) break;
                cum += parts[c];
            }
            s_chunk = c;
            s_base = cum;
            s_t = t;
            s_sp = row_stat(a, L, istar);
            s_sq = (mode == 0) ? row_stat(a, L, a.k + 1 + istar) : s_sp;
            s_token = -1;
        }
    }
    __syncthreads();
    const uint32_t istar = s_istar;
    if (s_mode != 2) {
        const uint32_t c = s_chunk;
        const RowStat sp = s_sp, sq = s_sq;
        const bool resid = (s_mode == 0);
        uint64_t w[kAccPerThread];
        uint64_t mine = 0;
        const uint32_t base = c * kAccChunk + tid * kAccPerThread;
        for (int i = 0; i < kAccPerThread; ++i) {
            const uint32_t x = base + i;
            uint64_t v = 0;
            if (x < a.vocab) {
                v = resid ? residual_w(a, istar, x, sp, sq)
                          : fix_shift(row_e(a.target[(size_t)istar * a.vocab + x], sp.M, a.T), 40);
            }
            w[i] = v;
            mine += v;
        }
        // exclusive scan of `mine` across the workgroup (exact integers)
        const int wave = tid / 64, lane = tid % 64;
        uint64_t incl = mine;
        for (int off = 1; off < 64; off <<= 1) {
            const uint64_t o = shfl_up_u64(incl, off);
            if (lane >= off) incl += o;
        }
        if (lane == 63) s_scan[wave] = incl;
        __syncthreads();
        uint64_t before = 0;
        for (int wv = 0; wv < wave; ++wv) before += s_scan[wv];
        const uint64_t excl = s_base + before + (incl - mine);
        const uint64_t t = s_t;
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
        __syncthreads();
    }
    if (tid == 0) {
        for (uint32_t j = 0; j < istar; ++j) a.tokens[j] = a.dtok[j];
        a.tokens[istar] = s_token;
        for (uint32_t j = istar + 1; j <= a.k; ++j) a.tokens[j] = -1;
        *a.accepted = (int32_t)istar;
    }
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
    hipLaunchKernelGGL(acc_final_kernel, dim3(1), dim3(kAccThreads), 0, s, a);
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
