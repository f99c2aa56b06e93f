// tqf_device.h -- device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tqf_internal.h"

namespace tqf {

__device__ __forceinline__ float f16_to_f32(uint32_t h16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h16 & 0xFFFFu));
}

// Lanes of this wavefront holding the same 9-bit key (a match-any from nine
// ballots; every lane of the wavefront must take part).
__device__ __forceinline__ uint64_t match_peers(uint32_t key) {
    uint64_t peers = ~0ull;
#pragma unroll
    for (int bit = 0; bit < 9; ++bit) {
        const uint64_t m = __ballot((key >> bit) & 1u);
        peers &= ((key >> bit) & 1u) ? m : ~m;
    }
    return peers;
}

// ---- wavefront reductions with DPP (no LDS round trip) ---------------------
// gfx9 DPP controls: quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1]
// (lane ^ 2), row_half_mirror (lane i <- 7 - i within 8), row_mirror
// (lane i <- 15 - i within 16).  After the four steps every lane of a 16-lane
// row holds the row's result; rows are combined through v_readlane.
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}

struct AddOp {
    __device__ float operator()(float a, float b) const { return a + b; }
    __device__ int operator()(int a, int b) const { return a + b; }
};
struct MaxOp {
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
    __device__ int operator()(int a, int b) const { return a > b ? a : b; }
};
struct MinOp {
    __device__ int operator()(int a, int b) const { return a < b ? a : b; }
};

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ int readlane_i(int v, int lane) {
    return __builtin_amdgcn_readlane(v, lane);
}

// The wavefront's maximum of an unsigned key, broadcast through scalar
// registers: each DPP step is one fused v_max_u32_dpp (a float maximum needs
// a move, a canonicalise and the maximum per step), then the four rows'
// maxima are combined in scalar registers.  Every lane must be active.
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppXor1, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppXor2, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppHalfMirror, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppMirror, 0xF, 0xF, false));
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
    const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
    const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return max(max(a, b), max(c, d));
}
// Order-preserving map of a float (not NaN) to an unsigned key, and back.
__device__ __forceinline__ uint32_t f2key(float x) {
    const uint32_t b = __float_as_uint(x);
    return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
    return __uint_as_float(k ^ ((uint32_t)((int32_t)~k >> 31) | 0x80000000u));
}
// The wavefront's maximum of four floats per lane (none NaN), to every lane.
__device__ __forceinline__ float wave_max4(const float (&v)[4]) {
    return key2f(wave_umax(max(max(f2key(v[0]), f2key(v[1])), max(f2key(v[2]), f2key(v[3])))));
}

// The router's top-8 (experts/mod.rs:134-197: the stable descending sort of
// the probabilities, so equal probabilities in ascending id order) of the
// E <= 256 probabilities p[i] of ids lane + 64 i, in the order taken.  Keys
// (bits(p) + 1) << 2 | (3 - i) order entries by probability (0 <= p <= 1, so
// the bits order as the values and the key fits 32 bits), then by the smaller
// i, i.e. the smaller id (lane < 64); equal keys are broken by the lowest
// lane, the smallest id again; 0 marks no expert.  Each lane first orders its
// four keys, then 8 rounds take the largest lane head.  Every lane of the
// wavefront must be active; psel / idsel are uniform.
__device__ __forceinline__ void top8_by_probability(const float (&p)[4], int lane, uint32_t E, float (&psel)[8],
                                                    int (&idsel)[8]) {
    uint32_t q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        q[i] = ((uint32_t)lane + 64u * i < E) ? ((__float_as_uint(p[i]) + 1u) << 2) | (3u - (uint32_t)i) : 0u;
    auto order = [&](int x, int y) {
        const uint32_t hi = max(q[x], q[y]), lo = min(q[x], q[y]);
        q[x] = hi;
        q[y] = lo;
    };
    order(0, 1);
    order(2, 3);
    order(0, 2);
    order(1, 3);
    order(1, 2);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t best = wave_umax(q[0]);
        const int l_win = (int)__builtin_ctzll(__ballot(q[0] == best));
        psel[k] = __uint_as_float((best >> 2) - 1u);
        idsel[k] = l_win + 64 * (int)(3u - (best & 3u));
        const bool won = lane == l_win;
        q[0] = won ? q[1] : q[0];
        q[1] = won ? q[2] : q[1];
        q[2] = won ? q[3] : q[2];
        q[3] = won ? 0u : q[3];
    }
}

// All-reduce over aligned groups of LANES lanes (2..64); every lane of a
// group receives the group's result.  All lanes of a group must be active.
template <int LANES, typename Op>
__device__ __forceinline__ float group_reduce(float v, Op op) {
    if constexpr (LANES >= 2) v = op(v, dpp_f<kDppXor1>(v));
    if constexpr (LANES >= 4) v = op(v, dpp_f<kDppXor2>(v));
    if constexpr (LANES >= 8) v = op(v, dpp_f<kDppHalfMirror>(v));
    if constexpr (LANES >= 16) v = op(v, dpp_f<kDppMirror>(v));
    if constexpr (LANES >= 32) {
        const float a = readlane_f(v, 0), b = readlane_f(v, 16);
        const float c = readlane_f(v, 32), d = readlane_f(v, 48);
        if constexpr (LANES == 32)
            v = (threadIdx.x & 32) ? op(c, d) : op(a, b);
        else
            v = op(op(a, b), op(c, d));
    }
    return v;
}
template <int LANES, typename Op>
__device__ __forceinline__ int group_reduce(int v, Op op) {
    if constexpr (LANES >= 2) v = op(v, dpp_i<kDppXor1>(v));
    if constexpr (LANES >= 4) v = op(v, dpp_i<kDppXor2>(v));
    if constexpr (LANES >= 8) v = op(v, dpp_i<kDppHalfMirror>(v));
    if constexpr (LANES >= 16) v = op(v, dpp_i<kDppMirror>(v));
    if constexpr (LANES >= 32) {
        const int a = readlane_i(v, 0), b = readlane_i(v, 16);
        const int c = readlane_i(v, 32), d = readlane_i(v, 48);
        if constexpr (LANES == 32)
            v = (threadIdx.x & 32) ? op(c, d) : op(a, b);
        else
            v = op(op(a, b), op(c, d));
    }
    return v;
}

// Scale of a 32-element activation block: x = X * 2^e with |X| <= 2^22.
// Returns 2^e; 0 for a block whose max |x| is below 2^-100 (its products are
// below fp32 resolution of any finite output); NaN if the block holds a
// non-finite value, so the non-finite input propagates to the outputs.
__device__ __forceinline__ float block_scale(float amax, bool bad, int &e) {
    e = 0;
    if (bad) return __int_as_float(0x7FC00000);
    if (!(amax >= 0x1p-100f)) return 0.0f;
    e = (int)((__float_as_uint(amax) >> 23) & 0xFFu) - 127 - 21;
    return __uint_as_float((uint32_t)(e + 127) << 23);
}

// X = rint(x * 2^-e) as six balanced base-16 digits d_k in [-8, 7]:
// X = sum_k d_k 16^k (|X| <= 2^22 < 7 (16^6 - 1) / 15, so six digits suffice).
__device__ __forceinline__ void split_digits16(float x, int e, float scale, int (&d)[6]) {
    int X = 0;
    if (scale > 0.0f) X = (int)__builtin_rintf(__builtin_ldexpf(x, -e));
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        d[k] = ((X + 8) & 15) - 8;
        X = (X - d[k]) >> 4;
    }
}
// Nibble position of block element j (0..31) in the record's digit dwords:
// it mirrors the Q4_0 byte order (element j < 16 is the low nibble of qs[j],
// element j + 16 the high nibble), so dword i of a digit plane pairs with
// bytes 4i..4i+3 of qs nibble for nibble.
__device__ __forceinline__ int rec_dword_of(int j) { return (j & 15) >> 2; }
__device__ __forceinline__ int rec_shift_of(int j) { return 4 * (2 * (j & 3) + (j >> 4)); }

// Address of dword `dw` (0..27) of the record of block b in one activation
// row's record planes (layout in tqf_internal.h: plane dw/4, block b, word
// dw%4).
__device__ __forceinline__ uint32_t *rec_dw(uint32_t *row, uint32_t bp, uint32_t b, int dw) {
    return row + (size_t)(dw >> 2) * 4 * bp + 4 * b + (dw & 3);
}

// Writes one xprep record for a 32-element block held by a group of
// 32/EPL lanes (EPL consecutive elements per lane, group-aligned lanes).
struct OrOp {
    __device__ int operator()(int a, int b) const { return a | b; }
};
template <int EPL>
__device__ __forceinline__ void prep_block(const float (&v)[EPL], int lane_in_group,
                                           uint32_t *__restrict__ row, uint32_t bp,
                                           uint32_t block) {
    constexpr int LPB = 32 / EPL;
    float amax = 0.0f;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        float a = fabsf(v[i]);
        bool b = !(a <= 3.402823466e38f);
        bad |= b;
        amax = fmaxf(amax, b ? 0.0f : a);
    }
    int badi = bad ? 1 : 0;
    if constexpr (LPB > 1) {
        amax = group_reduce<LPB>(amax, MaxOp());
        badi = group_reduce<LPB>(badi, MaxOp());
    }
    int e;
    const float scale = block_scale(amax, badi != 0, e);
    int part[24];
#pragma unroll
    for (int q = 0; q < 24; ++q) part[q] = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int j = lane_in_group * EPL + i;
        int d[6];
        split_digits16(v[i], e, scale, d);
        const int dw = rec_dword_of(j), sh = rec_shift_of(j);
#pragma unroll
        for (int k = 0; k < 6; ++k)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                part[4 * k + q] |= (q == dw) ? (int)(((uint32_t)d[k] & 15u) << sh) : 0;
    }
    if constexpr (LPB > 1) {
#pragma unroll
        for (int q = 0; q < 24; ++q) part[q] = group_reduce<LPB>(part[q], OrOp());
    }
    if (lane_in_group == 0) {
#pragma unroll
        for (int q = 0; q < 24; ++q) *rec_dw(row, bp, block, q) = (uint32_t)part[q];
        *rec_dw(row, bp, block, 24) = __float_as_uint(scale);
    }
}

// Store policies for prep_block32: plain stores (the writer's own later
// kernels read the record) or device-coherent stores (another workgroup of
// the same persistent kernel reads it after a grid barrier).
struct PlainStore {
    __device__ void operator()(uint32_t *p, uint32_t v) const { *p = v; }
};
struct CoherentStore {
    __device__ void operator()(uint32_t *p, uint32_t v) const {
        __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
};

// prep_block for one element per lane over an aligned half-wavefront (j =
// lane & 31); the digit nibbles of the eight elements that share a record
// dword (a quad and the quad 16 lanes away) are OR-combined across lanes so
// that the record is written with dword stores only.  `active` (uniform per
// half) suppresses the stores of a half that carries no block.
template <typename Store>
__device__ __forceinline__ void prep_block32(float v, int j, bool active, uint32_t *row,
                                             uint32_t bp, uint32_t block, Store st) {
    const float a = fabsf(v);
    const bool bad = !(a <= 3.402823466e38f);
    const float amax = group_reduce<32>(bad ? 0.0f : a, MaxOp());
    const int badi = group_reduce<32>(bad ? 1 : 0, MaxOp());
    int e;
    const float scale = block_scale(amax, badi != 0, e);
    int d[6];
    split_digits16(v, e, scale, d);
    const int sh = rec_shift_of(j);
    int p[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        p[k] = (int)(((uint32_t)d[k] & 15u) << sh);
        p[k] |= dpp_i<kDppXor1>(p[k]);
        p[k] |= dpp_i<kDppXor2>(p[k]);
        p[k] |= __shfl_xor(p[k], 16);
    }
    if (active && (j & 19) == 0) {  // j in {0, 4, 8, 12}: dword j / 4 of every digit
#pragma unroll
        for (int k = 0; k < 6; ++k) st(rec_dw(row, bp, block, 4 * k + (j >> 2)), (uint32_t)p[k]);
    }
    if (active && j == 0) st(rec_dw(row, bp, block, 24), __float_as_uint(scale));
}

// Device-coherent 32/64-bit accesses for data exchanged between workgroups
// of one launch (agent scope: not left in, or served from, one XCD's L2).
__device__ __forceinline__ void store_coherent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_coherent_u64(const uint64_t *p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_own_stores() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ uint32_t counter_arrive(uint32_t *c) {
    return __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void counter_reset(uint32_t *c) {
    __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The 16 nibble bytes of a Q4_0 block as signed int4 (q - 8): q ^ 8 is the
// 4-bit two's complement of q - 8 for q in 0..15.
__device__ __forceinline__ uint4 q4_signed(const uint4 w) {
    return make_uint4(w.x ^ 0x88888888u, w.y ^ 0x88888888u, w.z ^ 0x88888888u, w.w ^ 0x88888888u);
}

// sum_j (q_j - 8) * x_j of one Q4_0 block against one xprep record, in fp32.
// `ws` is the block's nibbles after q4_signed: six independent chains of
// four v_dot8_i32_i4 (one per activation digit), recombined exactly in int32
// (|sum| <= 32 * 8 * 2^22 = 2^30), then scaled by the record's 2^e.
__device__ __forceinline__ float q4_block_dot(const uint4 ws, const uint32_t *__restrict__ xp) {
    const int w4[4] = {(int)ws.x, (int)ws.y, (int)ws.z, (int)ws.w};
    int acc[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        int s = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) s = __builtin_amdgcn_sdot8(w4[i], (int)xp[4 * k + i], s, false);
        acc[k] = s;
    }
    int v = acc[5];
#pragma unroll
    for (int k = 4; k >= 0; --k) v = v * 16 + acc[k];
    return (float)v * __uint_as_float(xp[24]);
}

// ---- transpose-reduce: per-lane partial sums of NL rows -> one row per lane
// Lanes are grouped LPR to a matrix row (LPR in {16, 32, 64}); every lane
// holds NL partials.  Each halving stage pairs value i with value i + K/2;
// lanes whose stage bit is set keep the second member and add their
// partner's copy of it, so K halves per stage and no work is wasted.  The
// cross-row stages use gfx950's v_permlane32_swap / v_permlane16_swap, the
// in-row stages DPP mirrors.  Result: the sum over the group's LPR lanes of
// value index (lane % LPR) >> log2(LPR / NL), replicated LPR / NL times.
constexpr int kDppQuadRev = 0x1B;  // quad_perm [3,2,1,0]

template <int CTRL, int K>
__device__ __forceinline__ void dpp_stage(float *v, bool hi) {
    if constexpr (K >= 2) {
#pragma unroll
        for (int i = 0; i < K / 2; ++i) {
            const float a = v[i], b = v[i + K / 2];
            v[i] = (hi ? b : a) + dpp_f<CTRL>(hi ? a : b);
        }
    } else {
        v[0] = v[0] + dpp_f<CTRL>(v[0]);
    }
}

template <int K>
__device__ __forceinline__ void permlane32_stage(float *v) {
    if constexpr (K >= 2) {
#pragma unroll
        for (int i = 0; i < K / 2; ++i) {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]),
                                                            __float_as_uint(v[i + K / 2]), false, false);
            v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[0]), __float_as_uint(v[0]),
                                                        false, false);
        v[0] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}

template <int K>
__device__ __forceinline__ void permlane16_stage(float *v) {
    if constexpr (K >= 2) {
#pragma unroll
        for (int i = 0; i < K / 2; ++i) {
            const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]),
                                                            __float_as_uint(v[i + K / 2]), false, false);
            v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
    } else {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[0]), __float_as_uint(v[0]),
                                                        false, false);
        v[0] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}

constexpr int half_or_one(int k) { return k > 1 ? k / 2 : 1; }
constexpr int ilog2(int v) { return v <= 1 ? 0 : 1 + ilog2(v / 2); }

template <int LPR, int NL>
__device__ __forceinline__ float transpose_reduce(float (&v)[NL]) {
    static_assert(LPR == 16 || LPR == 32 || LPR == 64, "lanes per row");
    static_assert(NL >= 1 && NL <= LPR && (NL & (NL - 1)) == 0, "values per lane");
    const int lane = threadIdx.x & 63;
    constexpr int K0 = NL;
    if constexpr (LPR == 64) permlane32_stage<K0>(v);
    constexpr int K1 = LPR == 64 ? half_or_one(K0) : K0;
    if constexpr (LPR >= 32) permlane16_stage<K1>(v);
    constexpr int K2 = LPR >= 32 ? half_or_one(K1) : K1;
    dpp_stage<kDppMirror, K2>(v, lane & 8);
    constexpr int K3 = half_or_one(K2);
    dpp_stage<kDppHalfMirror, K3>(v, lane & 4);
    constexpr int K4 = half_or_one(K3);
    dpp_stage<kDppQuadRev, K4>(v, lane & 2);
    constexpr int K5 = half_or_one(K4);
    dpp_stage<kDppXor1, K5>(v, lane & 1);
    return v[0];
}
// Value index a lane holds after transpose_reduce, and whether it is the
// first of the replicated copies.
template <int LPR, int NL>
__device__ __forceinline__ int reduced_index(int lane) {
    return (lane % LPR) >> (ilog2(LPR) - ilog2(NL));
}
template <int LPR, int NL>
__device__ __forceinline__ bool reduced_first_copy(int lane) {
    return ((lane % LPR) & ((LPR / NL) - 1)) == 0;
}

// ---- row-lane matrix access ------------------------------------------------
// Octet-chunk layout (tqf_internal.h): rows 8o..8o+7 are one contiguous chunk
// of 9 * Bp * 16 bytes: their nibble rows, then one 16-byte scale vector per
// block.
struct RowLane {
    const uint8_t *base;
    uint32_t bp;  // padded blocks per row
};
__device__ __forceinline__ RowLane row_lane(const uint8_t *base, uint32_t bp) {
    RowLane r;
    r.base = base;
    r.bp = bp;
    return r;
}
// Loads from device memory through global (not flat) instructions: the
// matrix pointers come from tables in memory, which the compiler cannot
// prove are global.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_global_u4(const void *p) {
    const u32x4 v = *(const __attribute__((address_space(1))) u32x4 *)(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 load_global_f4(const float *p) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 v = *(const __attribute__((address_space(1))) f32x4 *)(p);
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float load_global_f(const float *p) {
    return *(const __attribute__((address_space(1))) float *)(p);
}
template <typename T>
__device__ __forceinline__ T load_global_ptr(T const *p) {
    return *(T const __attribute__((address_space(1))) *)(p);
}
__device__ __forceinline__ uint4 load_nibbles(const RowLane &m, uint32_t row, uint32_t block) {
    return load_global_u4(m.base + (((size_t)(row >> 3) * 9 + (row & 7)) * m.bp + block) * 16);
}
// Scales of rows 8*octet .. 8*octet+7 of one block.
__device__ __forceinline__ uint4 load_scales(const RowLane &m, uint32_t octet, uint32_t block) {
    return load_global_u4(m.base + (((size_t)octet * 9 + 8) * m.bp + block) * 16);
}
// The record of block b of one activation row into registers: seven 16-byte
// loads, each part of a contiguous 1 KiB wavefront access when lane = block.
__device__ __forceinline__ void load_xrec(const uint32_t *row, uint32_t bp, uint32_t b,
                                          uint32_t (&x)[28]) {
#pragma unroll
    for (int i = 0; i < 7; ++i) {
        const uint4 q = load_global_u4(row + (size_t)i * 4 * bp + 4 * b);
        x[4 * i + 0] = q.x;
        x[4 * i + 1] = q.y;
        x[4 * i + 2] = q.z;
        x[4 * i + 3] = q.w;
    }
}

// Scale j (0..7) of a per-lane vector of eight f16 scales.
__device__ __forceinline__ float octet_scale(const uint4 s, int j) {
    const uint32_t sv[4] = {s.x, s.y, s.z, s.w};
    const uint32_t word = sv[j >> 1];
    return f16_to_f32((j & 1) ? (word >> 16) : word);
}


// ---- integer butterflies of the K-quant matvecs (tqf_q4k.hip, tqf_q6k.hip) ----
// Wavefront-local LDS hand-off: this wavefront's LDS stores complete before
// any of its lanes reads them.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int CTRL, int MASK, int K>
__device__ __forceinline__ void xor_stage(int *v) {
    // slots p < K/2 (in units of 8 values) keep p and add the partner's p ^ MASK
#pragma unroll
    for (int p = 0; p < K / 2; ++p)
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) v[8 * p + cc] += dpp_i<CTRL>(v[8 * (p ^ MASK) + cc]);
}
template <int CTRL, int MASK, int K>
__device__ __forceinline__ void xor_stage1(int *v) {
#pragma unroll
    for (int p = 0; p < K / 2; ++p) v[p] += dpp_i<CTRL>(v[p ^ MASK]);
}

// ---------------------------------------------------------------------------
// Block-wide reduction of N floats per thread (256 threads); result valid in
// every thread.
// ---------------------------------------------------------------------------
template <int N>
__device__ __forceinline__ void block_sum_256(float (&v)[N], float (*lds)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = group_reduce<64>(v[i], AddOp());
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    __syncthreads();
    if (lane == 0)
#pragma unroll
        for (int i = 0; i < N; ++i) lds[wave][i] = v[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = (lds[0][i] + lds[1][i]) + (lds[2][i] + lds[3][i]);
}

// quantize_q8_k (model/qwen36/weights.rs:898-931) of one 256-element chunk
// by one wavefront, from lane 8k + c's four values v[i] = element 32k + c +
// 8i of the chunk, into the Q8_K record row `row` (12 dwords per sub-block,
// row stride 12 bp) at sub-blocks 8 chunk .. 8 chunk + 7.
__device__ __forceinline__ void q8k_quantize_values(const float (&v)[4], uint32_t *row, uint32_t bp,
                                                    uint32_t chunk) {
    const int lane = threadIdx.x & 63, k = lane >> 3, c = lane & 7;
    float am = -1.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = fabsf(v[i]);
        am = (a == a && a > am) ? a : am;
    }
    const float amax = group_reduce<64>(am, MaxOp());
    const uint32_t blk = chunk * 8 + (uint32_t)k;
    uint32_t word = 0;
    int sum = 0;
    float scale = 0.0f;
    if (amax > 0.0f) {
        int idx = 256;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (fabsf(v[i]) == amax) idx = min(idx, 32 * k + c + 8 * i);
        idx = group_reduce<64>(idx, MinOp());
        const int slot = (idx >> 3) & 3;
        const float vs = slot == 0 ? v[0] : slot == 1 ? v[1] : slot == 2 ? v[2] : v[3];
        const float smax = readlane_f(vs, 8 * (idx >> 5) + (idx & 7));
        const float inv = __fdiv_rn(-127.0f, smax);
        scale = __frcp_rn(inv);
        int s = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float q = __builtin_rintf(__fmul_rn(v[i], inv));
            if (!(q <= 127.0f)) q = 127.0f;
            if (q < -128.0f) q = -128.0f;
            const int qi = (int)q;
            s += qi;
            word |= ((uint32_t)qi & 0xFFu) << (8 * i);
        }
        sum = group_reduce<8>(s, AddOp());
    }
    row[(size_t)(c >> 2) * 4 * bp + 4 * blk + (c & 3)] = word;
    if (c == 0) {
        row[(size_t)8 * bp + 4 * blk] = (uint32_t)sum;
        row[(size_t)8 * bp + 4 * blk + 1] = __float_as_uint(scale);
    }
}

}  // namespace tqf
