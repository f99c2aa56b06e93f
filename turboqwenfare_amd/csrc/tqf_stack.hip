// tqf_stack.hip -- the persistent MoE-stack kernel for gfx950.
//
// One cooperative launch runs every layer of a stack over M <= 4 verify rows:
//   h <- h + MoE_l(rmsnorm_l(h))        (model/qwen36/runtime.rs:777-802)
// with MoE_l = shared expert * sigmoid(gate . x) + sum_k w_k expert_k(x) over
// the router's top-8 (experts/mod.rs:1540-1634).  Per layer three phases are
// separated by grid barriers (every workgroup is resident, one per CU):
//
//   A  the first ~33 workgroups: RMSNorm of the M rows (the sum of squares
//      comes from per-team partials written by the previous phase C), one
//      router row (or the shared-expert input gate) per wavefront, and the
//      activation records of the M x 64 blocks of x.
//   B  every workgroup: the routes (softmax, stable top-8, renormalise;
//      experts/mod.rs:134-197) from the logits -- computed identically in
//      every workgroup, so the plan needs no further exchange -- then
//      gate/up units of (expert, 32 rows) for ALL tokens routed to that
//      expert: its weights are read once, its activation records staged
//      through LDS; h = silu(g) * u is written as records per (expert, token)
//      pair.
//   C  teams of workgroups own 64 output rows each; a team member takes a
//      contiguous share of the expert-sorted pair list (8 rows per
//      wavefront, every weight load issued up front), and the last member to
//      finish sums the members' partials in member order, adds the residual
//      and writes h plus the team's sum of squares for the next layer.
//
// Everything exchanged between workgroups is written with agent-scope
// atomic stores and read with agent-scope atomic loads, and every thread
// drains its stores (s_waitcnt) before the barrier arrival, so no L2
// write-back / invalidate is needed.  Barrier waits are bounded in time: a
// wait that exceeds kSpinLimit sets `abort`, after which every workgroup
// leaves at its next barrier and the launch reports TQF_HIP_ERR_DEVICE; the
// last workgroup to exit resets the barrier state for the next launch.
#include <hip/hip_runtime.h>

#include "tqf_device.h"
#include "tqf_internal.h"

namespace tqf {

namespace {

constexpr int kThreads = 512;  // 8 wavefronts
constexpr int kWaves = kThreads / kWave;
constexpr int MT = kStackMT;
constexpr int H = kStackHidden;
constexpr int kBpGate = H / 32;        // 64 blocks per gate/up row: one per lane
constexpr int64_t kSpinLimit = 2000000;  // wall-clock ticks (100 MHz): 20 ms

// Routes and the pair plan of the current layer (identical in every
// workgroup).  Group 0 is the shared expert (all M tokens); groups 1..U the
// distinct routed experts in first-demand order.  Pairs: [0, M) shared,
// then each routed group's tokens in ascending token order.
struct RoutePlan {
    int32_t ids[MT][kTopK];
    float w[MT][kTopK];
    float gate_logit[MT];
    int32_t bad;
    int32_t n_groups, n_pairs;
    int32_t grp_expert[1 + MT * kTopK];
    int32_t grp_cnt[1 + MT * kTopK];
    int32_t grp_base[1 + MT * kTopK];   // first pair index of the group
    int32_t grp_tok[1 + MT * kTopK][MT];
    int32_t pair_expert[MT * (kTopK + 1)];
    int32_t pair_tok[64 + 64];  // [0, 9 MT): pairs; [64, 128): plan scratch
    float pair_coef[MT * (kTopK + 1)];
    float inv_rms[MT];
    int32_t last;
    int32_t ok;
};

// Workgroup-shared state (file scope, so that every access is a ds_* access).
__shared__ RoutePlan P;
__shared__ float s_h[MT][32];
__shared__ const uint8_t *s_mats[(256 + 1) * 3];  // the layer's expert matrix table
extern __shared__ uint4 s_dyn[];

// Phase C's down weights are prefetched into LDS during phase B with direct
// global -> LDS loads, where they fit: a wavefront's share of one pair is the
// contiguous octet chunk of its 8 rows (nibbles of 8 rows x LPRD blocks, then
// their scales: 9 LPRD 16 B), copied byte for byte.  The images sit above
// every phase's own LDS region.
template <int LPRD, int MAXP>
struct DownPrefetch {
    static constexpr uint32_t kWaveBytes = 9 * LPRD * 16;
    static constexpr bool kOn = LPRD == 16 && MAXP <= 5;
    static constexpr uint32_t kBytes = kOn ? MAXP * kWaves * kWaveBytes : 0;
};
constexpr uint32_t kPrefOffset = MT * H * 4;  // phase A's h rows, the largest region
static_assert(MT * 7 * kBpGate * 16 <= kPrefOffset, "phase B region");
static_assert(5 * 7 * 16 * 16 <= kPrefOffset, "phase C region of the prefetching variant");

// Workgroup barrier for LDS data only: this wavefront's LDS accesses
// complete (lgkmcnt(0)), then s_barrier.  __syncthreads() would also wait for
// every outstanding vector-memory operation, including direct global -> LDS
// loads still in flight, which the gate/up units must not wait for.
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt / expcnt at their maxima, lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Direct global -> LDS copies: lane l's `size` bytes at gaddr land at LDS
// byte address lds + l * size (m0 holds the wavefront's LDS base).  Issued as
// inline assembly so that the compiler adds no LDS-alias waits for them:
// every reader of the destination runs after a full s_waitcnt and a barrier
// (the grid barrier before phase C).  An operation the compiler does not
// count can only make its own vmcnt waits stricter, since loads retire in
// order.
__device__ __forceinline__ uint32_t lds_addr(uint32_t byte_off) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)(
               reinterpret_cast<uint8_t *>(s_dyn)) + byte_off;
}
__device__ __forceinline__ void copy_to_lds_16(const void *gaddr, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(gaddr) : "memory", "m0");
}
__device__ __forceinline__ void copy_to_lds_4(const void *gaddr, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(gaddr) : "memory", "m0");
}

// Copies n 64-bit words written by other workgroups into LDS: every load of
// a thread is issued before the first LDS store (one round trip).
template <int PER_THREAD>
__device__ __forceinline__ void stage_coherent(uint64_t *dst, const uint64_t *src, uint32_t n) {
    uint64_t v[PER_THREAD];
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const uint32_t k = threadIdx.x + (uint32_t)i * kThreads;
        v[i] = k < n ? load_coherent_u64(src + k) : 0;
    }
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const uint32_t k = threadIdx.x + (uint32_t)i * kThreads;
        if (k < n) dst[k] = v[i];
    }
}

// ---- grid barrier ------------------------------------------------------------
__device__ bool grid_sync(StackSync *sync, uint32_t &epoch, int32_t *status) {
    wait_own_stores();
    __syncthreads();
    ++epoch;
    if (threadIdx.x == 0) {
        const uint32_t target = epoch * gridDim.x;
        int ok = 1;
        if (counter_arrive(&sync->barrier) + 1 == target) {
            // last arrival: release everyone (the poll line sees no atomics)
            __hip_atomic_store(&sync->release, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            uint64_t *word = reinterpret_cast<uint64_t *>(&sync->release);
            int64_t t0 = 0;
            for (uint32_t spin = 1;; ++spin) {
                const uint64_t v = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if ((uint32_t)v >= epoch) break;
                if (v >> 32) {  // another workgroup timed out
                    ok = 0;
                    break;
                }
                if ((spin & 63) == 0) {
                    const int64_t now = wall_clock64();
                    if (t0 == 0) {
                        t0 = now;
                    } else if (now - t0 > kSpinLimit) {
                        __hip_atomic_store(&sync->abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        if (status)
                            __hip_atomic_store(status, (int32_t)TQF_HIP_ERR_DEVICE, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                        ok = 0;
                        break;
                    }
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
        P.ok = ok;
    }
    __syncthreads();
    return P.ok != 0;
}

// Last workgroup out resets the barrier state (every workgroup reaches this,
// including after an abort).
__device__ void stack_exit(StackSync *sync) {
    wait_own_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        if (counter_arrive(&sync->exit) == gridDim.x - 1) {
            counter_reset(&sync->barrier);
            counter_reset(&sync->release);
            counter_reset(&sync->abort);
            counter_reset(&sync->exit);
        }
    }
}

// ---- phase A -------------------------------------------------------------------
// Every workgroup: router row(s) blockIdx.x + k * gridDim.x (row E is the
// shared-expert input gate), the 2048 columns split over the 8 wavefronts
// (lane l of wavefront w: columns 256 w + 4 l ..); wavefront 1 of the first
// m * 32 workgroups also writes two activation records.  h rows [m x H] are
// staged in LDS.
__device__ void phase_a(const StackArgs &a, const StackLayer &L, const float *hin) {
    float *s_hx = reinterpret_cast<float *>(s_dyn);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const uint32_t m = a.m, E = a.E;
    const uint32_t col = 256 * wave + 4 * lane;
    const float4 nw = load_global_f4(L.norm + col);
    // this workgroup's first router row (gridDim.x <= E + 1), issued ahead of
    // the h staging so that the two round trips overlap
    const uint32_t e0 = blockIdx.x;
    const float4 r_first = load_global_f4((e0 < E ? L.router + (size_t)e0 * H : L.gate_vec) + col);
    float sq[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
        sq[t] = load_coherent(&a.ssq[(lane % kStackTeams) * MT + ((uint32_t)t < m ? t : 0)]);
    stage_coherent<MT * H / 2 / kThreads>(reinterpret_cast<uint64_t *>(s_hx),
                                          reinterpret_cast<const uint64_t *>(hin), m * H / 2);
    if (wave == 0) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const float v = group_reduce<64>(lane < kStackTeams ? sq[t] : 0.0f, AddOp());
            if (lane == 0) P.inv_rms[t] = 1.0f / sqrtf(v / (float)H + 1e-6f);
        }
    }
    __syncthreads();
    float4 xn[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const float4 hv = *reinterpret_cast<const float4 *>(s_hx + (size_t)(t < (int)m ? t : 0) * H + col);
        const float inv = P.inv_rms[t < (int)m ? t : 0];
        xn[t] = make_float4(hv.x * inv * nw.x, hv.y * inv * nw.y, hv.z * inv * nw.z, hv.w * inv * nw.w);
    }
    for (uint32_t e = blockIdx.x; e <= E; e += gridDim.x) {
        const float4 r = e == e0 ? r_first : load_global_f4((e < E ? L.router + (size_t)e * H : L.gate_vec) + col);
        float dot[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            float s0 = xn[t].x * r.x;
            s0 = fmaf(xn[t].y, r.y, s0);
            s0 = fmaf(xn[t].z, r.z, s0);
            s0 = fmaf(xn[t].w, r.w, s0);
            dot[t] = group_reduce<64>(s0, AddOp());
        }
        if (lane == 0)
#pragma unroll
            for (int t = 0; t < MT; ++t) s_h[t][wave] = dot[t];
        __syncthreads();
        if (wave == 0 && lane < (int)m) {
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) v += s_h[lane][w];
            store_coherent(&a.logits[lane * (E + 1) + e], v);
        }
        __syncthreads();
    }
    // activation records q = 2 blockIdx.x + half, q < m * 64
    if (wave == 1 && 2 * blockIdx.x < m * kBpGate) {
        const uint32_t q = 2 * blockIdx.x + (uint32_t)(lane >> 5);
        const bool active = q < m * kBpGate;
        const uint32_t t = active ? q / kBpGate : 0, kb = q % kBpGate;
        const uint32_t c = kb * 32 + (lane & 31);
        const float x = s_hx[(size_t)t * H + c] * P.inv_rms[t] * load_global_f(L.norm + c);
        prep_block32(x, lane & 31, active, a.xprep + (size_t)t * kBpGate * kXprepDwords, kBpGate, kb,
                     CoherentStore());
    }
}

// ---- phase B: the loads of one gate/up unit ----------------------------------------
// Wavefront w's rows 4w..4w+3 of the unit in gate and up (one block per lane,
// raw nibbles) and their scales, held in registers between issue and use.
constexpr int kRecRow = 7 * kBpGate * 2;  // 64-bit words of one token's records
constexpr int kRecPer = (MT * kRecRow + kThreads - 1) / kThreads;
struct UnitLoads {
    uint4 ng[4], nu[4], sg, su;
};

__device__ __forceinline__ void unit_loads(const StackArgs &a, int expert, int blk32, UnitLoads &U) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const RowLane Wg = row_lane(s_mats[expert * 3 + 0], kBpGate), Wu = row_lane(s_mats[expert * 3 + 1], kBpGate);
    const uint32_t r = (uint32_t)blk32 * 32 + 4 * wave;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
        U.ng[n] = load_nibbles(Wg, r + n, lane);
        U.nu[n] = load_nibbles(Wu, r + n, lane);
    }
    U.sg = load_scales(Wg, r / 8, lane);
    U.su = load_scales(Wu, r / 8, lane);
}

// This workgroup's first unit (blockIdx.x) from the routes alone, before the
// pair plan exists: its group is the shared expert or the g-th distinct routed
// expert in first-demand order (the plan's group order).  Every wavefront
// issues its weight loads, which then fly while wavefront 0 builds the plan.
// False: the workgroup has no unit.
__device__ __forceinline__ bool early_unit_loads(const StackArgs &a, UnitLoads &U) {
    const int lane = threadIdx.x % kWave;
    const int nb32 = (int)a.F / 32;
    const int g = (int)blockIdx.x / nb32, blk32 = (int)blockIdx.x % nb32;
    const int m = (int)a.m, n = m * kTopK;
    int expert;
    if (g == 0) {
        expert = (int)a.E;
    } else {
        // route entry i = (t, k) on lane i; other lanes carry distinct dummy keys
        const int e_i = lane < n ? P.ids[lane / kTopK][lane % kTopK] : 256 + lane;
        const uint64_t peers = match_peers((uint32_t)e_i);
        const uint64_t below = (1ull << lane) - 1ull;
        const uint64_t firsts = __ballot(lane < n && (peers & below) == 0);
        if (g > __builtin_popcountll(firsts)) return false;
        uint64_t mk = firsts;
        for (int r = 1; r < g; ++r) mk &= mk - 1ull;
        expert = __builtin_amdgcn_readlane(e_i, (int)__builtin_ctzll(mk));
    }
    unit_loads(a, expert, blk32, U);
    return true;
}

// ---- phase B: routes ------------------------------------------------------------
// `pre`: whether this workgroup's first unit's loads were issued (in `U`).
__device__ void compute_routes(const StackArgs &a, UnitLoads &U, bool &pre) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const uint32_t m = a.m, E = a.E;
    if (threadIdx.x == 0) P.bad = 0;
    __syncthreads();
    if (wave < (int)m) {
        const int t = wave;
        const float *lt = a.logits + (size_t)t * (E + 1);
        float lv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // unconditional loads: one round trip
            const uint32_t e = (uint32_t)lane + 64u * i;
            lv[i] = load_coherent(lt + (e < E ? e : E - 1));
        }
        const float glog = load_coherent(lt + E);
        bool fin = true;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t e = (uint32_t)lane + 64u * i;
            if (e >= E) lv[i] = -INFINITY;
            else if (!(fabsf(lv[i]) <= 3.402823466e38f)) fin = false;
        }
        if (lane == 0) P.gate_logit[t] = glog;
        if (__any(!fin)) {
            if (lane == 0) P.bad = 1;
        } else {
            const float mx = group_reduce<64>(fmaxf(fmaxf(lv[0], lv[1]), fmaxf(lv[2], lv[3])), MaxOp());
            float p[4], ssum = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t e = (uint32_t)lane + 64u * i;
                p[i] = e < E ? expf(lv[i] - mx) : 0.0f;
                ssum += p[i];
            }
            ssum = group_reduce<64>(ssum, AddOp());
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = ((uint32_t)lane + 64u * i < E) ? p[i] / ssum : -1.0f;
            // 8 rounds of: the wave's largest probability, then the lowest id
            // holding it (ids ascend with i, then with the lane), via ballots
            float psel[kTopK];
            int idsel[kTopK];
#pragma unroll
            for (int k = 0; k < kTopK; ++k) {
                const float best =
                    group_reduce<64>(fmaxf(fmaxf(p[0], p[1]), fmaxf(p[2], p[3])), MaxOp());
                const uint64_t m0 = __ballot(p[0] == best), m1 = __ballot(p[1] == best);
                const uint64_t m2 = __ballot(p[2] == best), m3 = __ballot(p[3] == best);
                const int i_win = m0 ? 0 : m1 ? 1 : m2 ? 2 : 3;
                const uint64_t mw = m0 ? m0 : m1 ? m1 : m2 ? m2 : m3;
                const int l_win = __builtin_ctzll(mw);
                psel[k] = best;
                idsel[k] = l_win + 64 * i_win;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (lane == l_win && i == i_win) p[i] = -1.0f;
            }
            // renormalise (experts/mod.rs:159-166): the total is the route-order
            // sum; each lane k < 8 divides its own weight
            float total = -0.0f;
#pragma unroll
            for (int k = 0; k < kTopK; ++k) total += psel[k];
            float mine = psel[0];
            int mid = idsel[0];
#pragma unroll
            for (int k = 1; k < kTopK; ++k)
                if (lane == k) {
                    mine = psel[k];
                    mid = idsel[k];
                }
            const float wk = mine / total;
            float wsum = 0.0f;
#pragma unroll
            for (int k = 0; k < kTopK; ++k) wsum += readlane_f(wk, k);
            if (lane < kTopK) {
                P.ids[t][lane] = mid;
                P.w[t][lane] = wk;
            }
            if (lane == 0 && !(fabsf(wsum - 1.0f) <= 1e-4f)) P.bad = 1;
        }
    }
    __syncthreads();
    pre = false;
    if (P.bad) {
        if (threadIdx.x == 0) {
            P.n_groups = 0;
            P.n_pairs = 0;
        }
        __syncthreads();
        return;
    }
    pre = early_unit_loads(a, U);
    // the pair plan, one route entry i = (t, k) per lane of wavefront 0: the
    // entries of the same expert as bits of one mask (broadcast LDS reads)
    if (wave == 0) {
        const int n = (int)m * kTopK;
        const int *flat = &P.ids[0][0];
        const int e_i = lane < n ? flat[lane] : -1 - lane;
        uint32_t eq = 0;
#pragma unroll
        for (int j = 0; j < MT * kTopK; ++j) eq |= (j < n && flat[j] == e_i) ? (1u << j) : 0u;
        const int cnt = __builtin_popcount(eq);
        const int rank = __builtin_popcount(eq & ((1u << (lane & 31)) - 1u));
        const int first = lane < n ? __builtin_ctz(eq) : lane;
        const bool flag = lane < n && first == lane;
        const uint64_t fmask = __ballot(flag);
        P.pair_tok[64 + lane] = first;  // scratch row: every entry's group start
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        int before = 0;  // route entries whose group starts before this entry's group
#pragma unroll
        for (int j = 0; j < MT * kTopK; ++j)
            before += (j < n && P.pair_tok[64 + j] < first) ? 1 : 0;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        const int g = 1 + __builtin_popcountll(fmask & ((1ull << first) - 1ull));
        if (lane < n) {
            const int t = lane / kTopK;
            const int pair = (int)m + before + rank;
            P.pair_expert[pair] = e_i;
            P.pair_tok[pair] = t;
            P.pair_coef[pair] = P.w[t][lane % kTopK];
            P.grp_tok[g][rank] = t;
            if (flag) {
                P.grp_expert[g] = e_i;
                P.grp_cnt[g] = cnt;
                P.grp_base[g] = (int)m + before;
            }
        }
        if (lane < (int)m) {
            P.pair_expert[lane] = (int)E;
            P.pair_tok[lane] = lane;
            P.pair_coef[lane] = 1.0f / (1.0f + expf(-P.gate_logit[lane]));
            P.grp_tok[0][lane] = lane;
        }
        if (lane == 0) {
            P.grp_expert[0] = (int)E;
            P.grp_cnt[0] = (int)m;
            P.grp_base[0] = 0;
            P.n_groups = 1 + __builtin_popcountll(fmask);
            P.n_pairs = (int)m * (kTopK + 1);
        }
    }
    __syncthreads();
}

// ---- phase B: prefetch of phase C's down weights ------------------------------------
// This workgroup's phase C share (the same member / pair split as phase_c):
// per pair, wavefront w's octet chunk of the pair's down matrix into its LDS
// image.  Issued inside the workgroup's first gate/up unit once its own loads
// are consumed, so the copies overlap the unit's compute (whose barriers are
// LDS-only); the grid barrier before phase C drains them.
template <int LPRD, int MAXP>
__device__ void prefetch_down(const StackArgs &a) {
    using PF = DownPrefetch<LPRD, MAXP>;
    if constexpr (PF::kOn) {
        const uint32_t K = a.members;
        const uint32_t tau = blockIdx.x % kStackTeams, k = blockIdx.x / kStackTeams;
        if (k >= K) return;
        const int n_pairs = P.n_pairs;
        const int p0 = (int)(k * n_pairs / K), p1 = (int)((k + 1) * n_pairs / K);
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
        const int lane = threadIdx.x % kWave;
        const uint32_t octet = tau * 8 + (uint32_t)wave;  // rows tau * 64 + 8 wave ..
        const uint32_t img = kPrefOffset + (uint32_t)wave * MAXP * PF::kWaveBytes;
#pragma unroll
        for (int q = 0; q < MAXP; ++q) {
            if (p0 + q < p1) {
                const uint8_t *chunk = s_mats[P.pair_expert[p0 + q] * 3 + 2] + (size_t)octet * PF::kWaveBytes;
                const uint32_t dst = img + (uint32_t)q * PF::kWaveBytes;
#pragma unroll
                for (int i = 0; i < LPRD / 8; ++i)  // nibbles: 1 KiB per instruction
                    copy_to_lds_16(chunk + i * 1024 + lane * 16, lds_addr(dst + i * 1024));
#pragma unroll
                for (int i = 0; i < LPRD / 16; ++i)  // scales: 256 B per instruction
                    copy_to_lds_4(chunk + 8 * LPRD * 16 + i * 256 + lane * 4, lds_addr(dst + 8 * LPRD * 16 + i * 256));
            }
        }
    }
}

// ---- phase B: gate/up units ---------------------------------------------------
// Unit = (group g, rows [32 blk32, +32)) for all of g's tokens.  Wavefront w
// owns rows 4w..4w+3 of the unit in both matrices.
// `preloaded`: U already holds this unit's loads (early_unit_loads).
template <int LPRD, int MAXP>
__device__ void gate_up_unit(const StackArgs &a, const StackLayer &L, int unit, bool prefetch,
                             UnitLoads &U, bool preloaded) {
    uint4 *s_x = s_dyn;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int nb32 = (int)a.F / 32;
    const int g = unit / nb32, blk32 = unit % nb32;
    const int cnt = P.grp_cnt[g];
    // weights (HBM) and the activation records of the group's tokens: one
    // round trip for both, issued here unless they are already in flight
    if (!preloaded) unit_loads(a, P.grp_expert[g], blk32, U);
    const uint32_t r = (uint32_t)blk32 * 32 + 4 * wave;
    const int pos = (int)(r & 7);  // 0 or 4
    {
        uint64_t v[kRecPer];
#pragma unroll
        for (int i = 0; i < kRecPer; ++i) {
            const int k = (int)threadIdx.x + i * kThreads;
            const int ti = k / kRecRow, off = k % kRecRow;
            const uint64_t *src = reinterpret_cast<const uint64_t *>(
                a.xprep + (size_t)P.grp_tok[g][ti < cnt ? ti : 0] * kBpGate * kXprepDwords);
            v[i] = ti < cnt ? load_coherent_u64(src + off) : 0;
        }
        uint64_t *dst = reinterpret_cast<uint64_t *>(s_x);  // 7 planes x 64 blocks per token
#pragma unroll
        for (int i = 0; i < kRecPer; ++i) {
            const int k = (int)threadIdx.x + i * kThreads;
            if (k < cnt * kRecRow) dst[k] = v[i];
        }
    }
    lds_barrier();
    // every load of this unit is consumed here (waited for explicitly, on
    // every path), so no later wait of the unit covers the prefetch's copies
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt / lgkmcnt at their maxima
    if (prefetch) prefetch_down<LPRD, MAXP>(a);
    uint4 ng[4], nu[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
        ng[n] = q4_signed(U.ng[n]);
        nu[n] = q4_signed(U.nu[n]);
    }
    const uint4 sg = U.sg, su = U.su;
    for (int i = 0; i < cnt; ++i) {
        uint32_t x[28];
#pragma unroll
        for (int qd = 0; qd < 7; ++qd) {
            const uint4 v = s_x[((size_t)i * 7 + qd) * kBpGate + lane];
            x[4 * qd] = v.x;
            x[4 * qd + 1] = v.y;
            x[4 * qd + 2] = v.z;
            x[4 * qd + 3] = v.w;
        }
        float v[8];
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            v[2 * n] = octet_scale(sg, pos + n) * q4_block_dot(ng[n], x);
            v[2 * n + 1] = octet_scale(su, pos + n) * q4_block_dot(nu[n], x);
        }
        const float gate = transpose_reduce<64, 8>(v);  // lanes 16n..: gate n, 16n+8..: up n
        const float up = dpp_f<0x108>(gate);            // row_shl:8
        if ((lane & 15) == 0) s_h[i][4 * wave + (lane >> 4)] = (gate / (1.0f + expf(-gate))) * up;
    }
    lds_barrier();
    // h records: two tokens per wavefront
    if (2 * wave < cnt) {
        const int i = 2 * wave + (lane >> 5);
        const bool active = i < cnt;
        const int ii = active ? i : 2 * wave;
        const int pair = P.grp_base[g] + ii;
        prep_block32(s_h[ii][lane & 31], lane & 31, active,
                     a.hprep + (size_t)pair * LPRD * kXprepDwords, LPRD, (uint32_t)blk32,
                     CoherentStore());
    }
    lds_barrier();
}

// ---- phase C -------------------------------------------------------------------
template <int LPRD, int MAXP>
__device__ void phase_c(const StackArgs &a, const StackLayer &L, const float *hin) {
    uint4 *s_x = s_dyn;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    constexpr int G = kWave / LPRD;   // lane groups per wavefront
    constexpr int RG = 8 / G;         // rows per lane group (a wavefront owns one octet)
    constexpr int NL = MT * RG;       // values per lane before the transpose
    static_assert(NL <= LPRD, "transpose width");
    const uint32_t K = a.members;
    const uint32_t tau = blockIdx.x % kStackTeams, k = blockIdx.x / kStackTeams;
    if (k >= K) return;
    const int n_pairs = P.n_pairs;
    const int p0 = (int)(k * n_pairs / K), p1 = (int)((k + 1) * n_pairs / K);
    const int cnt = p1 - p0;
    const uint32_t j = (uint32_t)lane / LPRD, b = (uint32_t)lane % LPRD;
    const uint32_t r0 = tau * 64 + 8 * wave;  // this wavefront's octet
    // every weight load of the member up front (pair index clamped into the
    // member's range), then the h records of its pairs into LDS (7 planes x
    // LPRD blocks each)
    using PF = DownPrefetch<LPRD, MAXP>;
    uint4 nib[MAXP][RG], sc[MAXP];
    if (!PF::kOn && cnt > 0) {
#pragma unroll
        for (int q = 0; q < MAXP; ++q) {
            const int pq = p0 + (q < cnt ? q : cnt - 1);
            const RowLane W = row_lane(s_mats[P.pair_expert[pq] * 3 + 2], LPRD);
#pragma unroll
            for (int rr = 0; rr < RG; ++rr) nib[q][rr] = q4_signed(load_nibbles(W, r0 + j * RG + rr, b));
            sc[q] = load_scales(W, r0 / 8, b);
        }
    }
    stage_coherent<(MAXP * 7 * LPRD * 2 + kThreads - 1) / kThreads>(
        reinterpret_cast<uint64_t *>(s_x),
        reinterpret_cast<const uint64_t *>(a.hprep + (size_t)p0 * LPRD * kXprepDwords),
        (uint32_t)cnt * 7 * LPRD * 2);
    __syncthreads();
    float acc[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) acc[i] = 0.0f;
    const bool pad = b >= a.F / 32;
#pragma unroll
    for (int q = 0; q < MAXP; ++q) {
        if (q < cnt) {
            const int pq = p0 + q;
            const int tok = P.pair_tok[pq];
            const float coef = P.pair_coef[pq];
            uint32_t x[28];
#pragma unroll
            for (int qd = 0; qd < 7; ++qd) {
                const uint4 v = s_x[((size_t)q * 7 + qd) * LPRD + b];
                x[4 * qd] = v.x;
                x[4 * qd + 1] = v.y;
                x[4 * qd + 2] = v.z;
                x[4 * qd + 3] = v.w;
            }
            if (pad) x[24] = 0;
            if constexpr (PF::kOn) {  // this wavefront's image of the pair (prefetch_down)
                const uint8_t *img = reinterpret_cast<const uint8_t *>(s_dyn) + kPrefOffset +
                                     ((size_t)wave * MAXP + q) * PF::kWaveBytes;
#pragma unroll
                for (int rr = 0; rr < RG; ++rr)
                    nib[q][rr] = q4_signed(*reinterpret_cast<const uint4 *>(img + ((j * RG + rr) * LPRD + b) * 16));
                sc[q] = *reinterpret_cast<const uint4 *>(img + 8 * LPRD * 16 + b * 16);
            }
#pragma unroll
            for (int rr = 0; rr < RG; ++rr) {
                const float v = coef * (octet_scale(sc[q], (int)(j * RG) + rr) * q4_block_dot(nib[q][rr], x));
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    if (t == tok) acc[t * RG + rr] += v;
            }
        }
    }
    const float s = transpose_reduce<LPRD, NL>(acc);
    const int idx = reduced_index<LPRD, NL>(lane);
    const int t = idx / RG, rr = idx % RG;
    if (reduced_first_copy<LPRD, NL>(lane) && t < (int)a.m)
        store_coherent(&a.partial[(((size_t)tau * K + k) * MT + t) * 64 + 8 * wave + j * RG + rr], s);
    // team combine: the last member sums the members' partials in order
    wait_own_stores();
    __syncthreads();
    if (threadIdx.x == 0) P.last = counter_arrive(&a.sync->team[tau]) == K - 1 ? 1 : 0;
    __syncthreads();
    if (!P.last) return;
    float *s_red = reinterpret_cast<float *>(s_x);  // [MT][64] squares
    const uint32_t m = a.m;
    for (uint32_t i = threadIdx.x; i < MT * 64; i += kThreads) {
        const uint32_t tt = i / 64, row = i % 64;
        float sq = 0.0f;
        if (tt < m) {
            constexpr int kMaxMembers = 16;
            float pv[kMaxMembers];
#pragma unroll
            for (int kk = 0; kk < kMaxMembers; ++kk)
                pv[kk] = kk < (int)K ? load_coherent(&a.partial[(((size_t)tau * K + kk) * MT + tt) * 64 + row])
                                     : 0.0f;
            const size_t o = (size_t)tt * H + tau * 64 + row;
            const float res = load_coherent(hin + o);
            float sum = 0.0f;
#pragma unroll
            for (int kk = 0; kk < kMaxMembers; ++kk)
                if (kk < (int)K) sum += pv[kk];
            const float out = res + sum;
            store_coherent(&a.h[o], out);
            sq = out * out;
        }
        s_red[i] = sq;
    }
    __syncthreads();
    if (wave < MT) {
        const float v = group_reduce<64>(s_red[wave * 64 + lane], AddOp());
        if (lane == 0 && wave < (int)m) store_coherent(&a.ssq[tau * MT + wave], v);
    }
    if (threadIdx.x == 0) counter_reset(&a.sync->team[tau]);
}

// sum of squares of h rows of the team (prologue for the first layer)
__device__ void team_ssq(const StackArgs &a) {
    float *s_red = reinterpret_cast<float *>(s_dyn);
    const uint32_t tau = blockIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    for (uint32_t i = threadIdx.x; i < MT * 64; i += kThreads) {
        const uint32_t tt = i / 64, row = i % 64;
        float v = 0.0f;
        if (tt < a.m) v = load_coherent(&a.h_in[(size_t)tt * H + tau * 64 + row]);
        s_red[i] = v * v;
    }
    __syncthreads();
    if (wave < MT) {
        const float v = group_reduce<64>(s_red[wave * 64 + lane], AddOp());
        if (lane == 0 && wave < (int)a.m) store_coherent(&a.ssq[tau * MT + wave], v);
    }
}

}  // namespace

template <int LPRD, int MAXP>
__global__ __launch_bounds__(kThreads) void stack_kernel(StackArgs a) {
    uint32_t epoch = 0;
    if (blockIdx.x < (uint32_t)kStackTeams) team_ssq(a);
    bool ok = grid_sync(a.sync, epoch, a.status);
    for (uint32_t l = 0; ok && l < a.n_layers; ++l) {
        const StackLayer L = a.layers[l];
        const float *hin = l == 0 ? a.h_in : a.h;
        // the layer's expert-matrix pointers: loads issued now, stored to LDS
        // after phase A (read by phases B and C)
        constexpr int kPtrPer = ((256 + 1) * 3 + kThreads - 1) / kThreads;
        const uint8_t *mp[kPtrPer];
#pragma unroll
        for (int i = 0; i < kPtrPer; ++i) {
            const uint32_t k = threadIdx.x + (uint32_t)i * kThreads;
            mp[i] = load_global_ptr(L.mats + (k < (a.E + 1) * 3 ? k : 0));
        }
        phase_a(a, L, hin);
#pragma unroll
        for (int i = 0; i < kPtrPer; ++i) {
            const uint32_t k = threadIdx.x + (uint32_t)i * kThreads;
            if (k < (a.E + 1) * 3) s_mats[k] = mp[i];
        }
        if (!(ok = grid_sync(a.sync, epoch, a.status))) break;
        UnitLoads U;
        bool pre;
        compute_routes(a, U, pre);
        if (blockIdx.x == 0 && threadIdx.x < a.m * kTopK) {
            const uint32_t t = threadIdx.x / kTopK, kk = threadIdx.x % kTopK;
            if (a.ids_out) a.ids_out[((size_t)l * a.m + t) * kTopK + kk] = P.bad ? 0 : (uint16_t)P.ids[t][kk];
            if (a.w_out) a.w_out[((size_t)l * a.m + t) * kTopK + kk] = P.bad ? 0.0f : P.w[t][kk];
        }
        if (blockIdx.x == 0 && threadIdx.x == 0 && P.bad && a.status)
            __hip_atomic_store(a.status, (int32_t)TQF_HIP_ERR_ROUTER, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        const int n_units = P.n_groups * (int)(a.F / 32);
        bool prefetch = true;  // with the first unit's loads, or alone
        for (int u = blockIdx.x; u < n_units; u += gridDim.x) {
            gate_up_unit<LPRD, MAXP>(a, L, u, prefetch, U, pre && u == (int)blockIdx.x);
            prefetch = false;
        }
        if (prefetch) prefetch_down<LPRD, MAXP>(a);
        if (!(ok = grid_sync(a.sync, epoch, a.status))) break;
        phase_c<LPRD, MAXP>(a, L, hin);
        if (l + 1 < a.n_layers && !(ok = grid_sync(a.sync, epoch, a.status))) break;
    }
    stack_exit(a.sync);
}

size_t stack_lds_bytes(uint32_t bp_down, uint32_t members) {
    const size_t a = (size_t)MT * H * 4;                        // phase A: h rows
    const size_t b = (size_t)MT * 7 * kBpGate * 16;             // phase B: x records
    const uint32_t maxp = (MT * (kTopK + 1) + members - 1) / members;
    const size_t c = (size_t)maxp * 7 * bp_down * 16;           // phase C: h records
    size_t m = a > b ? a : b;
    m = m > c ? m : c;
    // the prefetching variant (pick: bp_down 16, maxp <= 5) adds its images
    if (bp_down == 16 && maxp <= 5) m = (m > kPrefOffset ? m : kPrefOffset) + DownPrefetch<16, 5>::kBytes;
    return m;
}

namespace {
template <int LPRD>
const void *pick(uint32_t maxp, int &chosen) {
    if (maxp <= 5) { chosen = 5; return (const void *)stack_kernel<LPRD, 5>; }
    if (maxp <= 9) { chosen = 9; return (const void *)stack_kernel<LPRD, 9>; }
    chosen = 0;
    return nullptr;
}
const void *kernel_for(uint32_t bp_down, uint32_t members) {
    const uint32_t maxp = (MT * (kTopK + 1) + members - 1) / members;
    int chosen = 0;
    if (bp_down == 16) return pick<16>(maxp, chosen);
    if (bp_down == 32) return pick<32>(maxp, chosen);
    if (bp_down == 64) return pick<64>(maxp, chosen);
    return nullptr;
}
}  // namespace

uint32_t stack_grid(int device, uint32_t bp_down) {
    int coop = 0, cus = 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, device) != hipSuccess || !coop)
        return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
        return 0;
    uint32_t grid = (uint32_t)cus;
    uint32_t members = grid / kStackTeams;
    if (members == 0) return 0;
    if (members > 16) {  // the team combine reads at most 16 member partials
        members = 16;
        grid = members * kStackTeams;
    }
    // dynamic LDS beyond the default limit, set once per context for every
    // variant this grid can launch (bp_down 16 / 32 / 64)
    for (uint32_t bp : {16u, 32u, 64u}) {
        const void *kv = kernel_for(bp, members);
        if (kv && hipFuncSetAttribute(kv, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)stack_lds_bytes(bp, members)) != hipSuccess)
            return 0;
    }
    const void *k = kernel_for(bp_down, members);
    if (!k) return 0;
    int per_cu = 0;
    const size_t lds = stack_lds_bytes(bp_down, members);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kThreads, lds) != hipSuccess || per_cu < 1)
        return 0;
    return grid;
}

hipError_t launch_stack(hipStream_t s, const StackArgs &a, uint32_t grid, uint32_t bp_down) {
    const void *k = kernel_for(bp_down, a.members);
    if (!k) return hipErrorInvalidValue;
    StackArgs args = a;
    void *params[] = {&args};
    return hipLaunchCooperativeKernel(k, dim3(grid), dim3(kThreads), params,
                                      (unsigned int)stack_lds_bytes(bp_down, a.members), s);
}

}  // namespace tqf
