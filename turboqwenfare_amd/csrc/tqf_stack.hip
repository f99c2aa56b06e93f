// tqf_stack.hip -- the persistent MoE-stack kernel for gfx950.
//
// One persistent launch (one workgroup per CU, all co-resident) runs every
// layer of a stack over M <= 4 verify rows:
//   h <- h + MoE_l(rmsnorm_l(h))        (model/qwen36/runtime.rs:777-802)
// with MoE_l = shared expert * sigmoid(gate . x) + sum_k w_k expert_k(x) over
// the router's top-8 (experts/mod.rs:1540-1634).  Per layer two phases are
// separated by a grid barrier (every workgroup is resident, one per CU); the
// input side of a layer (RMSNorm, router logits, activation records) is
// produced by the previous layer's phase C (by a prologue for layer 0), and
// the layer's routing waits on those words themselves (the counted logit
// words and tagged sums of squares) instead of on a second barrier:
//
//   B  every workgroup: 1/rms of the M rows from the per-team sums of
//      squares; the router logits = 1/rms x the fixed-point sum of the
//      teams' partial logits; the routes (softmax, stable top-8,
//      renormalise; experts/mod.rs:134-197) on wavefronts 0..M-1 --
//      computed identically in every workgroup, so the plan needs no further
//      exchange -- then gate/up units of 64 rows (one row octet per
//      wavefront; 32 rows in the kernel instantiation for M <= 2) of one
//      routed (expert, token) pair, with the activation records of
//      y = h * w_norm of every row in LDS (1/rms scales the dot products:
//      rmsnorm(h) . W = (1/rms) (y . W)); h = silu(g) * u is written as
//      records per pair.  M = 4 tokens have 32 routed pairs: 256 units of
//      equal work, one per workgroup.  The shared expert (all M tokens) is
//      spread thinner: every workgroup takes two of its rows, one (row,
//      token) per wavefront, computed inside its unit while the unit's first
//      weights are in flight, and writes raw h values; the phase C member
//      that owns the shared pairs turns them into records.
//   C  teams of workgroups own 64 output rows each; a team member takes a
//      contiguous share of the expert-sorted pair list (8 rows per
//      wavefront, every weight load issued up front) and publishes its
//      partial rows as tagged words; every member polls all the team's
//      words, sums them in member order and adds the residual (kept in
//      registers across layers: each member holds the team's rows, the same
//      bits in all of them), and the members share the next layer's inputs
//      from the team's 64 rows: the sums of squares, the records of
//      y = h * w_norm, and the partial router logits sum_c R[e][c] y[c] of
//      every expert (member k: experts [k E / K, (k + 1) E / K)) and of the
//      shared-expert gate, added into a 2^-32 fixed-point accumulator with
//      counted integer atomics (exact, so the sum over teams does not depend
//      on their order), after the member's own record and sum-of-squares
//      stores have completed.  h itself is written once, after the last
//      layer.
//
// Everything exchanged between workgroups is written with agent-scope
// atomic stores and read with agent-scope atomic loads, and every thread
// drains its stores (s_waitcnt) before the barrier arrival or, in the tail,
// before its counted logit adds, so no L2 write-back / invalidate is needed.
// What the removed second barrier ordered still holds: the next layer's
// phase B writes (records of h, shared rows, tail inputs) can only start in a
// workgroup once every member of every team has counted into every logit
// word, i.e. has finished the layer (staging and exchange included), and the
// partial words and the accumulator parity a layer zeroes stay ordered by
// the layer's barrier.  (Workgroup-scope stores and loads do
// not suffice even between the members of a team: their partial words were
// not seen within the spin limit.)  Barrier waits are bounded in time: a
// wait that exceeds kSpinLimit sets `abort`, after which every workgroup
// leaves at its next barrier or wait and the launch reports TQF_HIP_ERR_DEVICE (in
// dev_status, and as 1 in the host flag); the last workgroup to exit resets
// the barrier state for the next launch.  The library then re-runs the stack
// through the per-layer kernels from the prologue's copy of h_in.
#include <hip/hip_runtime.h>

#include "tqf_device.h"
#include "tqf_internal.h"
#include "tqf_tags.h"

namespace tqf {

namespace {

// The thread index through an opaque register move, so that the compiler
// rederives each phase's lane arithmetic inside the layer loop instead of
// hoisting all of it out of the loop, where the hoisted values of every phase
// would stay live across every other phase (and spill).
__device__ __forceinline__ uint32_t tid() {
    uint32_t t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Marks loaded registers as used here: on a path that never uses the data,
// the loads then complete at this point, instead of leaving the compiler to
// wait for them (with every later load) wherever the paths join.
__device__ __forceinline__ void consume(uint32_t v) { asm volatile("" ::"v"(v)); }
__device__ __forceinline__ void consume(const uint4 &v) {
    asm volatile("" ::"v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
}

constexpr int kThreads = 512;  // 8 wavefronts
constexpr int kWaves = kThreads / kWave;
constexpr int MT = kStackMT;
constexpr int kMaxMembers = 16;  // phase C workgroups per team
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
    int32_t pair_tok[MT * (kTopK + 1)];
    float pair_coef[MT * (kTopK + 1)];
    float inv_rms[MT];
    int32_t last;
    int32_t ok;
    int32_t arrived_last;  // this workgroup released the current grid barrier
    int32_t xcd_local;     // the team exchange goes through the XCD's L2 (xcd_local_ok)
};

// Workgroup-shared state (file scope, so that every access is a ds_* access).
__shared__ RoutePlan P;
__shared__ float s_h[MT][64];
__shared__ float s_lv[MT][33];  // the tail's gathered partial logits (column 32: the shared gate)
__shared__ const uint8_t *s_mats[(256 + 1) * 3];  // the layer's expert matrix table
extern __shared__ uint4 s_dyn[];

// Phase C's down weights are prefetched into LDS during phase B with direct
// global -> LDS loads, where they fit: a wavefront's share of one pair is the
// contiguous octet chunk of its 8 rows (nibbles of 8 rows x LPRD blocks, then
// their scales: 9 LPRD 16 B), copied byte for byte.
template <int LPRD, int MAXP>
struct DownPrefetch {
    static constexpr uint32_t kWaveBytes = 9 * LPRD * 16;
    static constexpr bool kOn = LPRD == 16 && MAXP <= 5;
    static constexpr uint32_t kBytes = kOn ? MAXP * kWaves * kWaveBytes : 0;
};
// Dynamic LDS, in phase order:
//   [0, PF::kBytes)          from the arrival at the barrier before phase C
//                            on: the prefetched down weights;
//   [xr, xr + kXrBytes)      phase B: the activation records of the M rows
//                            (7 planes x 64 blocks x 16 B per row);
//   [xr, ...)                phase C: the h records of the member's pairs,
//                            then the team tail's rows (2 x MT x 64 floats).
constexpr uint32_t kXrBytes = MT * 7 * kBpGate * 16;
template <int LPRD, int MAXP>
struct LdsLayout {
    static constexpr uint32_t kXr = DownPrefetch<LPRD, MAXP>::kBytes;
    static constexpr uint32_t kCStage = MAXP * 7 * LPRD * 16;
    static constexpr uint32_t kTotal = kXr + (kXrBytes > kCStage ? kXrBytes : kCStage);
};

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
// The same at agent scope (sc1), for data other workgroups wrote.
__device__ __forceinline__ void copy_to_lds_16_coherent(const void *gaddr, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off sc1" ::"s"(lds), "v"(gaddr) : "memory", "m0");
}

// Copies n 64-bit words written by other workgroups into LDS: every load of
// a thread is issued before the first LDS store (one round trip).
template <int PER_THREAD>
__device__ __forceinline__ void stage_coherent(uint64_t *dst, const uint64_t *src, uint32_t n) {
    uint64_t v[PER_THREAD];
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const uint32_t k = tid() + (uint32_t)i * kThreads;
        v[i] = k < n ? load_coherent_u64(src + k) : 0;
    }
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const uint32_t k = tid() + (uint32_t)i * kThreads;
        if (k < n) dst[k] = v[i];
    }
}

// Zeroes this workgroup's share (workgroup `part` of `parts`) of one parity of
// the accumulator.
__device__ __forceinline__ void zero_lacc(uint64_t *acc, uint32_t part, uint32_t parts) {
    for (uint32_t k = part * kThreads + tid(); k < kLaccWords; k += parts * kThreads)
        __hip_atomic_store(acc + k, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Router logits travel between layers as 2^-32 fixed point in 64-bit words
// that also count their contributors: each of the 32 teams adds
// 2^58 + llrint(partial * 2^32) + 2^52 with an integer atomic, so the low 58
// bits hold the exact sum (independent of the teams' order) plus 32 * 2^52,
// and the top 6 bits count the teams that have added.  The next layer's
// routing polls the words until all 32 have counted: the words carry their
// own completion, and no grid barrier separates a layer's tail from the
// next layer's routing.  |partial| must stay below 2^20 (about 931,000); a
// partial that is larger or not finite sets a bit of the accumulator's flag
// word instead and never counts, and the routing polls the flag with the
// words.  A non-finite partial (kFlagNonFinite) is the router error of the
// reference's validation; a finite one beyond the range (kFlagRange: rows of
// h with |h| around 10^7, whose normalised logits are ordinary) is a limit of
// this accumulator only, so the routing aborts the launch, and with recovery
// on the library re-runs the stack through the per-layer kernels, which sum
// the logits in f32.
constexpr uint64_t kCountOne = 1ull << 58, kTermBias = 1ull << 52;
constexpr uint64_t kFlagNonFinite = 1, kFlagRange = 2;
__device__ __forceinline__ void add_counted(uint64_t *word, uint64_t *flag, float v) {
    const double d = (double)v * 4294967296.0;
    if (fabs(d) < 4.0e15) {
        __hip_atomic_fetch_add(word, kCountOne + (uint64_t)(__double2ll_rn(d) + (int64_t)kTermBias), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    } else {
        __hip_atomic_fetch_or(flag, fabsf(v) <= 3.402823466e38f ? kFlagRange : kFlagNonFinite, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
    }
}
__device__ __forceinline__ bool counted_done(uint64_t w) { return (w >> 58) == kStackTeams; }
__device__ __forceinline__ uint64_t counted_value(uint64_t w) {
    return (w & (kCountOne - 1)) - (uint64_t)kStackTeams * kTermBias;
}
__device__ __forceinline__ float logit_of(uint64_t fixed, float inv_rms) {
    return (float)((double)(int64_t)fixed * 0x1p-32 * (double)inv_rms);
}

// ---- grid barrier ------------------------------------------------------------
// Split phase: barrier_arrive counts this workgroup in once every thread's
// stores are complete (the caller waits for them) and the last arrival
// releases everyone; grid_wait polls for the release.  Work placed between
// the two overlaps the barrier, and grid_wait uses only an LDS barrier, so
// loads issued in between (the down weight prefetch) are not waited for.
// One thread arrives and polls: lane 0 of the last wavefront, which issues
// none of the prefetch's copies (its poll loads would wait for them).
constexpr int kPoller = (kWaves - 1) * kWave;
constexpr int kDmaWaves = 6;  // wavefronts 0..5 issue the down prefetch

__device__ void barrier_arrive(StackSync *sync, uint32_t &epoch) {
    lds_barrier();
    ++epoch;
    if (tid() == kPoller) {
        // first the workgroup's group line, then (last of its group) the grid's
        const uint32_t G = kStackBarrierGroups;
        const uint32_t grp = blockIdx.x % G, groups = gridDim.x < G ? gridDim.x : G;
        const uint32_t per = (gridDim.x - grp + G - 1) / G;  // workgroups in group grp
        bool last = false;
        if (counter_arrive(&sync->group[grp][0]) + 1 == epoch * per)
            last = counter_arrive(&sync->barrier) + 1 == epoch * groups;
        // last arrival: release everyone (the poll line sees no atomics)
        if (last) __hip_atomic_store(&sync->release, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        P.arrived_last = last ? 1 : 0;
    }
}

__device__ void grid_arrive(StackSync *sync, uint32_t &epoch) {
    wait_own_stores();
    barrier_arrive(sync, epoch);
}

__device__ __forceinline__ uint64_t poll_load(const uint64_t *word) {
    return __hip_atomic_load(const_cast<uint64_t *>(word), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The poller keeps three loads of the release word in flight, so a release
// is seen about one round trip after it lands rather than up to two.
// `fail` takes the wait as timed out without polling (a timeout forced from
// the host, so that the abort path can be tested with every wait bounded).
__device__ bool grid_wait(StackSync *sync, uint32_t epoch, int32_t *status, bool fail = false) {
    if (tid() == kPoller) {
        int ok = 1;
        if (fail) {
            __hip_atomic_store(&sync->abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (status)
                __hip_atomic_store(status, (int32_t)TQF_HIP_ERR_DEVICE, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            ok = 0;
        } else if (!P.arrived_last) {
            const uint64_t *word = reinterpret_cast<const uint64_t *>(&sync->release);
            uint64_t v0 = poll_load(word);
            __builtin_amdgcn_s_sleep(1);
            uint64_t v1 = poll_load(word);
            int64_t t0 = 0;
            for (uint32_t spin = 1;; ++spin) {
                __builtin_amdgcn_s_sleep(1);
                const uint64_t v2 = poll_load(word);
                if ((uint32_t)v0 >= epoch) break;
                if (v0 >> 32) {  // another workgroup timed out
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
                v0 = v1;
                v1 = v2;
            }
            // the loads still in flight complete here, in this wavefront,
            // rather than at a later reuse of their registers by every one
            asm volatile("s_waitcnt vmcnt(0)" ::"v"(v0), "v"(v1) : "memory");
        }
        P.ok = ok;
    }
    lds_barrier();
    return P.ok != 0;
}

__device__ bool grid_sync(StackSync *sync, uint32_t &epoch, int32_t *status) {
    grid_arrive(sync, epoch);
    return grid_wait(sync, epoch, status);
}

// Last workgroup out resets the barrier state (every workgroup reaches this,
// including after an abort), advances the layer-step base of the partial
// words' tags by this launch's depth (stack_next_base) and reports the
// outcome in the host flag; after an abort it also zeroes the logit
// accumulators, which a completed launch leaves at zero.
__device__ void stack_exit(StackSync *sync, uint64_t *lacc, uint32_t base, uint32_t n_layers,
                           int32_t *host_flag) {
    wait_own_stores();
    __syncthreads();
    if (tid() == 0) {
        P.last = 0;
        if (counter_arrive(&sync->exit) == gridDim.x - 1) {
            P.last = __hip_atomic_load(&sync->abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ? 2 : 1;
            // the launch's outcome for the host (read once the launch has ended)
            if (host_flag)
                __hip_atomic_store(host_flag, P.last == 2 ? 1 : 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            counter_reset(&sync->barrier);
            for (int g = 0; g < kStackBarrierGroups; ++g) counter_reset(&sync->group[g][0]);
            counter_reset(&sync->release);
            counter_reset(&sync->abort);
            counter_reset(&sync->xcd_bad);
            counter_reset(&sync->exit);
            __hip_atomic_store(&sync->step_base, stack_next_base(base, n_layers), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __syncthreads();
    if (P.last == 2) zero_lacc(lacc, 0, 1), zero_lacc(lacc + kLaccWords, 0, 1);
}

// ---- phase B: gate/up units ------------------------------------------------------
// A unit is R = 8 URW rows of one routed pair's gate and up, URW rows per
// wavefront: URW = 8 (64 rows, one octet per wavefront) in the kernel for
// M >= 3, URW = 4 (32 rows) in the one for M <= 2, where 64-row units would
// leave most compute units without gate/up loads (a quarter of them carry the
// weight stream at M = 1); with 32-row units the 8 M F / R units cover half
// the grid at M = 1 and all of it at M = 2.  Unit u < 8 M (F / R) is rows
// [R (u % (F / R)), +R) of routed pair M + u / (F / R) in the plan's pair
// order (wavefront w: rows URW w .. URW w + URW - 1 of the unit).
struct UnitDesc {
    int pair, row0, rw;  // pair, first row, rows per wavefront
};
template <int URW>
__device__ __forceinline__ UnitDesc unit_desc(int u, int F, int m) {
    UnitDesc d;
    d.rw = URW;
    d.pair = m + u / (F / (8 * URW));
    d.row0 = (u % (F / (8 * URW))) * 8 * URW;
    return d;
}

// Wavefront w's rows of the unit in gate and up (one block per lane, raw
// nibbles) and their scale octets, held in registers between issue and use.
constexpr int kRecBytes = 7 * kBpGate * 16;  // one token's activation records (7 KiB)
constexpr int kRecWaves = kWaves - MT;        // the wavefronts that route no token copy them
struct UnitLoads {
    uint4 ng[8], nu[8], sg, su;
};

// The records of the M rows (written by the previous layer's phase C) into
// LDS, copied directly by wavefronts MT.. (1 KiB per instruction); the
// caller waits for them (vmcnt) before the barrier that publishes them.
template <int LPRD, int MAXP>
__device__ __forceinline__ void record_copies(const StackArgs &a, int wave, int lane) {
    if (wave < MT) return;
    const uint32_t chunks = a.m * (kRecBytes / 1024);
    for (uint32_t c = (uint32_t)(wave - MT); c < chunks; c += kRecWaves)
        copy_to_lds_16_coherent(reinterpret_cast<const uint8_t *>(a.xprep) + (size_t)c * 1024 + lane * 16,
                                lds_addr(LdsLayout<LPRD, MAXP>::kXr + c * 1024));
}

// ---- phase B: the shared expert's rows ------------------------------------------
// Wavefront w of workgroup b: row 2 b + (w & 1) (then + 2 G, ...) of the
// shared expert's gate and up for token w >> 1; the raw value silu(g) * u goes
// to hshared[token][row].
struct SharedLoads {
    uint4 ng, nu;
    uint32_t sg, su;  // the lane's block scale of the row (binary16 bits)
};
__device__ __forceinline__ void consume_shared(const SharedLoads &S) {
    consume(S.ng);
    consume(S.nu);
    consume(S.sg);
    consume(S.su);
}
__device__ __forceinline__ uint32_t load_scale_row(const RowLane &m, uint32_t row, uint32_t block) {
    return *(const __attribute__((address_space(1))) uint16_t *)(m.base + (((size_t)(row >> 3) * 9 + 8) * m.bp + block) * 16 +
                                                                 (row & 7) * 2);
}
__device__ __forceinline__ void shared_row_loads(const StackArgs &a, uint32_t row, SharedLoads &S) {
    const int lane = tid() % kWave;
    const RowLane Wg = row_lane(s_mats[a.E * 3 + 0], kBpGate), Wu = row_lane(s_mats[a.E * 3 + 1], kBpGate);
    S.ng = load_nibbles(Wg, row, lane);
    S.nu = load_nibbles(Wu, row, lane);
    S.sg = load_scale_row(Wg, row, lane);
    S.su = load_scale_row(Wu, row, lane);
}
template <int LPRD, int MAXP>
__device__ void shared_rows(const StackArgs &a, const SharedLoads &S0) {
    const uint4 *xr = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint8_t *>(s_dyn) +
                                                      LdsLayout<LPRD, MAXP>::kXr);
    const int wave = __builtin_amdgcn_readfirstlane(tid() / kWave);
    const int lane = tid() % kWave;
    const uint32_t t = (uint32_t)wave >> 1;
    if (t >= a.m || 2 * blockIdx.x + (wave & 1) >= a.F) {
        consume_shared(S0);
        return;
    }
    SharedLoads S = S0;
    for (uint32_t row = 2 * blockIdx.x + (wave & 1), i = 0; row < a.F; row += 2 * gridDim.x, ++i) {
        if (i > 0) shared_row_loads(a, row, S);
        uint32_t x[28];
#pragma unroll
        for (int qd = 0; qd < 7; ++qd) {
            const uint4 v = xr[((size_t)t * 7 + qd) * kBpGate + lane];
            x[4 * qd] = v.x;
            x[4 * qd + 1] = v.y;
            x[4 * qd + 2] = v.z;
            x[4 * qd + 3] = v.w;
        }
        float v[2] = {f16_to_f32(S.sg) * q4_block_dot(q4_signed(S.ng), x),
                      f16_to_f32(S.su) * q4_block_dot(q4_signed(S.nu), x)};
        // lanes 0..31: gate, 32..63: up; the records hold y = h * w_norm, so
        // 1/rms scales the dot products
        const float gate = transpose_reduce<64, 2>(v) * P.inv_rms[t];
        const float up = __shfl_xor(gate, 32);
        if (lane == 0) store_coherent(&a.hshared[(size_t)t * a.F + row], (gate / (1.0f + expf(-gate))) * up);
    }
}

// A unit's rows are software-pipelined: the loads of its first kAhead rows
// (and the scale octets) are issued here, and gate_up_compute issues row
// n + kAhead's just before it computes row n.  Issuing all of a wavefront's
// rows at once stalls the wavefront until the shared weight stream has
// nearly drained (the memory pipeline takes the loads only as fast as HBM
// serves the whole chip), so its digit dots could only start after the
// stream; pipelined, the dots of the rows that have landed run while the
// later rows stream (measured per 40-layer launch: 1208 us issuing all
// eight rows up front, 1152 / 1142 / 1147 / 1162 us with 1 / 3 / 4 / 6
// rows ahead).
constexpr int kAhead = 3;
template <int RW>
__device__ __forceinline__ void unit_loads_rw(int expert, int row0, UnitLoads &U) {
    const int wave = __builtin_amdgcn_readfirstlane(tid() / kWave);
    const int lane = tid() % kWave;
    const RowLane Wg = row_lane(s_mats[expert * 3 + 0], kBpGate), Wu = row_lane(s_mats[expert * 3 + 1], kBpGate);
    const uint32_t r = (uint32_t)row0 + RW * wave;
    U.sg = load_scales(Wg, r / 8, lane);
    U.su = load_scales(Wu, r / 8, lane);
#pragma unroll
    for (int n = 0; n < (RW < kAhead ? RW : kAhead); ++n) {
        U.ng[n] = load_nibbles(Wg, r + n, lane);
        U.nu[n] = load_nibbles(Wu, r + n, lane);
    }
}
__device__ __forceinline__ void unit_loads(int expert, const UnitDesc &d, UnitLoads &U) {
    if (d.rw == 8) unit_loads_rw<8>(expert, d.row0, U);
    else unit_loads_rw<4>(expert, d.row0, U);
}

// The pair plan's order (experts/mod.rs forward_batch's union: groups in
// first-demand order, a group's tokens ascending) for route entry i = (t, k)
// on lane i of a wavefront, from the routes alone: the lanes of equal experts
// (match_peers), the group's first entry, this entry's rank in its group,
// and the entries of the groups that start before it (an exclusive prefix
// sum, in lane order, of each group's size at its first entry).  Lanes >= n
// carry distinct dummy keys.  The entry's pair is m + before + rank.
struct RouteEntry {
    int e, first, rank, cnt, before;
    uint64_t fmask;  // lanes that start a group
};
__device__ __forceinline__ RouteEntry route_entry(int lane, int n) {
    RouteEntry r;
    r.e = lane < n ? P.ids[lane / kTopK][lane % kTopK] : 256 + lane;
    const uint64_t peers = match_peers((uint32_t)r.e);
    r.first = (int)__builtin_ctzll(peers);
    r.rank = __builtin_popcountll(peers & ((1ull << lane) - 1ull));
    r.cnt = __builtin_popcountll(peers);
    const bool starts = lane < n && r.first == lane;
    r.fmask = __ballot(starts);
    const int size_at_first = starts ? r.cnt : 0;
    int incl = size_at_first;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const int o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
    }
    r.before = __shfl(incl - size_at_first, r.first);
    return r;
}

// This workgroup's first unit (blockIdx.x) from the route entries: every
// wavefront issues its first rows' weight loads (unit_loads_rw).  False: the
// workgroup has no unit.
template <int URW>
__device__ __forceinline__ bool early_unit_loads(const StackArgs &a, const RouteEntry &r, UnitLoads &U) {
    const int lane = tid() % kWave;
    const int m = (int)a.m, n = m * kTopK;
    const int u = (int)blockIdx.x;
    if (u >= n * ((int)a.F / (8 * URW))) return false;
    const UnitDesc d = unit_desc<URW>(u, (int)a.F, m);
    const uint64_t hit = __ballot(lane < n && m + r.before + r.rank == d.pair);
    const int expert = __builtin_amdgcn_readlane(r.e, (int)__builtin_ctzll(hit));
    unit_loads(expert, d, U);
    return true;
}


// ---- phase B: routes ------------------------------------------------------------
// `pre`: whether this workgroup's first unit's loads were issued (in `U`).
// After the loads are issued only LDS barriers are used: __syncthreads()
// would wait for them.
template <int LPRD, int MAXP, int URW>
__device__ void compute_routes(const StackArgs &a, uint32_t l, UnitLoads &U, SharedLoads &S, bool &pre, uint32_t base) {
    const int wave = __builtin_amdgcn_readfirstlane(tid() / kWave);
    const int lane = tid() % kWave;
    const uint32_t m = a.m, E = a.E;
    if (tid() == 0) P.bad = 0;
    lds_barrier();
    // the routing wavefronts' logit words and sums of squares first, then the
    // loads that need no routes (the M rows' records, this wavefront's
    // shared-expert row), so that the logits are not queued behind them
    const int t = wave;
    const uint64_t *acc = a.lacc + (size_t)(l & 1) * kLaccWords;
    const uint64_t *lt = acc + (size_t)(t < (int)m ? t : 0) * (E + 1);
    uint64_t fx[4], gfx = 0, flag = 0;
    float sq = 0.0f;
    if (wave < (int)m) {
        // the words carry their own completion: poll until every team has
        // counted into every logit word and stored its tagged sum of squares
        // (or a team flagged a bad partial, or the wait times out)
        const uint32_t qtag = stack_part_tag(base, l);
        bool aborted = false;
        const uint64_t *sq64 = reinterpret_cast<const uint64_t *>(a.ssq) + (lane % kStackTeams) * MT + t;
        int64_t t0 = 0;
        for (uint32_t spin = 1;; ++spin) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t e = (uint32_t)lane + 64u * i;
                fx[i] = load_coherent_u64(lt + (e < E ? e : E - 1));
            }
            gfx = load_coherent_u64(lt + E);
            flag = load_coherent_u64(acc + (size_t)MT * (E + 1));
            const uint64_t sw = load_coherent_u64(sq64);
            sq = __uint_as_float((uint32_t)sw);
            bool done = counted_done(gfx) && (uint32_t)(sw >> 32) == qtag;
#pragma unroll
            for (int i = 0; i < 4; ++i) done = done && counted_done(fx[i]);
            if (__all(done) || flag != 0) break;
            if ((spin & 15) == 0) {
                if (__hip_atomic_load(&a.sync->abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                    aborted = true;  // no routes; the launch reports the abort
                    break;
                }
                const int64_t now = wall_clock64();
                if (t0 == 0) {
                    t0 = now;
                } else if (now - t0 > kSpinLimit) {
                    __hip_atomic_store(&a.sync->abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (a.dev_status)
                        __hip_atomic_store(a.dev_status, (int32_t)TQF_HIP_ERR_DEVICE, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                    aborted = true;
                    break;
                }
            }
            __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) fx[i] = counted_value(fx[i]);
        gfx = counted_value(gfx);
        if (!aborted && (flag & kFlagRange) && !(flag & kFlagNonFinite)) {
            // a finite partial beyond the accumulator's range: abort (every
            // workgroup leaves at its next wait; without recovery the call
            // reports the router error, with it the library re-runs the stack)
            if (lane == 0) {
                __hip_atomic_store(&a.sync->abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (a.dev_status)
                    __hip_atomic_store(a.dev_status, (int32_t)TQF_HIP_ERR_ROUTER, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
            aborted = true;
        }
        if (aborted && lane == 0) P.bad = 2;
    }
    // the records only once the routing words are in (their 7 MB over all
    // workgroups would otherwise queue ahead of them), by the wavefronts
    // that do not route
    float v = 0.0f;
    if (wave < (int)m) v = group_reduce<64>(lane < kStackTeams ? sq : 0.0f, AddOp());
    lds_barrier();
    record_copies<LPRD, MAXP>(a, wave, lane);
    {
        const uint32_t row = 2 * blockIdx.x + (wave & 1);
        if (row < a.F && (uint32_t)(wave >> 1) < m) shared_row_loads(a, row, S);
    }
    // the other parity, summed into by this layer's phase C: back to zero
    if (blockIdx.x * kThreads < kLaccWords)
        zero_lacc(a.lacc + (size_t)((l + 1) & 1) * kLaccWords, blockIdx.x, gridDim.x);
    float lv[4], glog = 0.0f;
    if (wave < (int)m && P.bad != 2) {  // 2: the wait for the words ended in an abort
        // 1/rms (RMSNorm, weights.rs:216-239) of row t from the 32 teams' sums
        const float inv = 1.0f / sqrtf(v / (float)H + 1e-6f);
        if (lane == 0) P.inv_rms[t] = inv;
#pragma unroll
        for (int i = 0; i < 4; ++i) lv[i] = logit_of(fx[i], inv);
        glog = logit_of(gfx, inv);
        if ((flag & kFlagNonFinite) && lane == 0) P.bad = 1;  // a non-finite partial logit
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
            const float mx = wave_max4(lv);
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
            // top-8 by (probability descending, id ascending), as the stable
            // descending sort of from_logits
            float psel[kTopK];
            int idsel[kTopK];
            top8_by_probability(p, lane, E, psel, idsel);
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
    if (wave >= MT) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the record copies
    lds_barrier();
    pre = false;
    if (P.bad) {
        if (tid() == 0) {
            P.n_groups = 0;
            P.n_pairs = 0;
        }
        // no unit uses the shared-expert row: its loads complete here
        consume_shared(S);
        lds_barrier();
        return;
    }
    // the pair plan, one route entry i = (t, k) per lane (every wavefront
    // computes the entries for its own first unit; wavefront 0 also writes
    // the plan)
    const int n = (int)m * kTopK;
    const RouteEntry r = route_entry(lane, n);
    if (wave == 0) {
        const int g = 1 + __builtin_popcountll(r.fmask & ((1ull << r.first) - 1ull));
        if (lane < n) {
            const int t = lane / kTopK;
            const int pair = (int)m + r.before + r.rank;
            P.pair_expert[pair] = r.e;
            P.pair_tok[pair] = t;
            P.pair_coef[pair] = P.w[t][lane % kTopK];
            P.grp_tok[g][r.rank] = t;
            if (r.first == lane) {
                P.grp_expert[g] = r.e;
                P.grp_cnt[g] = r.cnt;
                P.grp_base[g] = (int)m + r.before;
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
            P.n_groups = 1 + __builtin_popcountll(r.fmask);
            P.n_pairs = (int)m * (kTopK + 1);
        }
    }
    pre = early_unit_loads<URW>(a, r, U);
    lds_barrier();
}

// ---- phase C's pair shares -----------------------------------------------------------
// Member k (of K) of a team: the shared pairs s = k, k + K, ... < M (at most
// one when K >= M, so that the shared records, which the member builds from
// raw rows, are spread over the members), then an equal contiguous share of
// the routed pairs [M, n_pairs).
struct MemberShare {
    int k, K, ns, r0, r1;
    __device__ int cnt() const { return ns + r1 - r0; }
    __device__ int pair(int q) const { return q < ns ? k + K * q : r0 + q - ns; }
};
// URW: the kernel's unit rows per wavefront.  In the kernel for M <= 2
// (URW = 4), at M = 1 the routed pairs are split with the shared pair counted
// as two routed ones (member 0, which builds the shared pair's records from
// raw rows, takes fewer routed pairs): 865 -> 830 us per 40-layer launch;
// the same weighting cost 31 us at M = 2 and 8 us at M = 4.
template <int URW>
__device__ __forceinline__ MemberShare member_share(int k, int K, int m, int n_pairs) {
    MemberShare s;
    s.k = k;
    s.K = K;
    if (n_pairs == 0) {  // routing failed: no pairs
        s.ns = s.r0 = s.r1 = 0;
        return s;
    }
    s.ns = k < m ? (m - 1 - k) / K + 1 : 0;
    const int R = n_pairs - m;
    if (URW == 4 && m == 1) {
        constexpr int W = 2;
        const int T = R + W;
        auto start = [&](int kk) {
            const int v = kk * T / K - (kk > 0 ? W : 0);
            return v < 0 ? 0 : v > R ? R : v;
        };
        s.r0 = m + start(k);
        s.r1 = m + start(k + 1);
    } else {
        s.r0 = m + k * R / K;
        s.r1 = m + (k + 1) * R / K;
    }
    return s;
}

// ---- phase B: prefetch of phase C's down weights ------------------------------------
// This workgroup's phase C share (the same member / pair split as phase_c):
// per pair, wavefront w's octet chunk of the pair's down matrix into its LDS
// image.  Issued after the workgroup has arrived at the barrier before phase
// C (its gate/up loads and h record stores are complete by then), so the
// copies stream while the barrier completes; phase C's first wait drains
// them before the images are read.
template <int LPRD, int MAXP>
struct PrefetchOps {
    static constexpr int kParts = LPRD / 8 + LPRD / 16;  // copies per image: nibble KiBs, scale rows
    static constexpr int kOps = MAXP * kWaves * kParts;
    static constexpr int kPerWave = kOps / kDmaWaves;
    static_assert(kOps % kDmaWaves == 0, "prefetch copies split evenly");
};

// Every image slot gets a copy (slots past the member's pairs repeat its last
// pair, or the shared expert's down matrix when it has none), so each of
// wavefronts 0..5 issues exactly PrefetchOps::kPerWave copies.  The poller's
// wavefront issues none.  Returns whether this wavefront issued copies.
template <int LPRD, int MAXP, int URW>
__device__ bool prefetch_down(const StackArgs &a) {
    using PF = DownPrefetch<LPRD, MAXP>;
    using OPS = PrefetchOps<LPRD, MAXP>;
    if constexpr (PF::kOn) {
        const uint32_t K = a.members;
        const uint32_t tau = blockIdx.x % kStackTeams, k = blockIdx.x / kStackTeams;
        const int wave = __builtin_amdgcn_readfirstlane(tid() / kWave);
        if (k >= K || wave >= kDmaWaves) return false;
        const MemberShare sh = member_share<URW>((int)k, (int)K, (int)a.m, P.n_pairs);
        const int cnt = sh.cnt();
        const int lane = tid() % kWave;
#pragma unroll
        for (int i = 0; i < OPS::kPerWave; ++i) {
            const int o = wave * OPS::kPerWave + i;
            const int img = o / OPS::kParts, part = o % OPS::kParts;
            const int q = img / kWaves, w = img % kWaves;  // pair slot, octet wavefront
            const int e = cnt > 0 ? P.pair_expert[sh.pair(q < cnt ? q : cnt - 1)] : (int)a.E;
            const uint8_t *chunk = s_mats[e * 3 + 2] + (size_t)(tau * 8 + w) * PF::kWaveBytes;
            const uint32_t dst = ((uint32_t)w * MAXP + q) * PF::kWaveBytes;
            if (part < LPRD / 8)  // nibbles: 1 KiB per instruction
                copy_to_lds_16(chunk + part * 1024 + lane * 16, lds_addr(dst + part * 1024));
            else  // scales: 256 B per instruction
                copy_to_lds_4(chunk + 8 * LPRD * 16 + (part - LPRD / 8) * 256 + lane * 4,
                              lds_addr(dst + 8 * LPRD * 16 + (part - LPRD / 8) * 256));
        }
        return true;
    }
    return false;
}

// ---- phase B: one gate/up unit -------------------------------------------------
// `preloaded`: U already holds this unit's loads (early_unit_loads).
template <int RW, int LPRD, int MAXP, class Hook>
__device__ void gate_up_compute(const StackArgs &a, const UnitDesc &d, UnitLoads &U, Hook &&hook) {
    // one token: the pair's
    const uint4 *xr = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint8_t *>(s_dyn) +
                                                      LdsLayout<LPRD, MAXP>::kXr);
    const int wave = __builtin_amdgcn_readfirstlane(tid() / kWave);
    const int lane = tid() % kWave;
    const int pos = (int)(((uint32_t)d.row0 + RW * wave) & 7);  // 0, or 4 in a 32-row unit
    const int expert = P.pair_expert[d.pair];
    const RowLane Wg = row_lane(s_mats[expert * 3 + 0], kBpGate), Wu = row_lane(s_mats[expert * 3 + 1], kBpGate);
    const uint32_t rbase = (uint32_t)d.row0 + RW * wave;
    const uint4 sg = U.sg, su = U.su;
    {
        const int i = 0, t = P.pair_tok[d.pair];
        uint32_t x[28];
#pragma unroll
        for (int qd = 0; qd < 7; ++qd) {
            const uint4 v = xr[((size_t)t * 7 + qd) * kBpGate + lane];
            x[4 * qd] = v.x;
            x[4 * qd + 1] = v.y;
            x[4 * qd + 2] = v.z;
            x[4 * qd + 3] = v.w;
        }
        float v[2 * RW];
#pragma unroll
        for (int n = 0; n < RW; ++n) {
            // row n + kAhead's loads, then row n's dots; the scheduling
            // barriers keep the compiler from hoisting every load to the top
            if (n + kAhead < RW) {
                U.ng[n + kAhead] = load_nibbles(Wg, rbase + n + kAhead, lane);
                U.nu[n + kAhead] = load_nibbles(Wu, rbase + n + kAhead, lane);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (n == 0) {  // the caller's work while the first rows' weights are in flight
                hook();
                __builtin_amdgcn_sched_barrier(0);
            }
            v[2 * n] = octet_scale(sg, pos + n) * q4_block_dot(q4_signed(U.ng[n]), x);
            v[2 * n + 1] = octet_scale(su, pos + n) * q4_block_dot(q4_signed(U.nu[n]), x);
            __builtin_amdgcn_sched_barrier(0);
        }
        // value 2n (gate row n) lands on lanes (64 / RW) n .., value 2n + 1 (up
        // row n) on the lanes 32 / RW above them
        // the records hold y = h * w_norm: 1/rms scales the dot products
        const float gate = transpose_reduce<64, 2 * RW>(v) * P.inv_rms[t];
        const float up = RW == 8 ? dpp_f<0x104>(gate) : dpp_f<0x108>(gate);  // row_shl:4 / :8
        if ((lane & (64 / RW - 1)) == 0)
            s_h[i][RW * wave + lane / (64 / RW)] = (gate / (1.0f + expf(-gate))) * up;
    }
}

template <int LPRD, int MAXP, int URW, class Hook>
__device__ void gate_up_unit(const StackArgs &a, const UnitDesc &d, UnitLoads &U, bool preloaded, Hook &&hook) {
    const int wave = __builtin_amdgcn_readfirstlane(tid() / kWave);
    const int lane = tid() % kWave;
    const int cnt = 1;
    // the weights (HBM), unless early_unit_loads already issued them; the
    // activation records are in LDS
    if (!preloaded) unit_loads(P.pair_expert[d.pair], d, U);
    gate_up_compute<URW, LPRD, MAXP>(a, d, U, hook);
    lds_barrier();
    // h records: one (token, 32-row block) per half-wavefront, from the last
    // wavefront down (the wavefronts that issue no prefetch copies)
    const int nblk = d.rw / 4;  // 32-row blocks in the unit
    const int rwave = kWaves - 1 - wave;
    if (2 * rwave < cnt * nblk) {
        const int q = 2 * rwave + (lane >> 5);
        const bool active = q < cnt * nblk;
        const int qq = active ? q : 2 * rwave;
        const int i = qq / nblk, kb = qq % nblk;
        const int pair = d.pair;
        prep_block32(s_h[i][32 * kb + (lane & 31)], lane & 31, active,
                     a.hprep + (size_t)pair * LPRD * kXprepDwords, LPRD,
                     (uint32_t)(d.row0 / 32 + kb), CoherentStore());
    }
    lds_barrier();
}

// ---- the team tail: the next layer's inputs from the team's 64 rows -------------
// Every member of team tau ends a layer holding the team's new rows of h (the
// same bits in each: the members' partials summed in member order), thread
// tid < MT * 64 row tid % 64 of token tid / 64, and shares out the next
// layer's inputs: member t % K writes the records of token t's two y blocks
// (y = h * w_norm), member 0 the sums of squares, member K - 1 the
// shared-expert gate, and member k the partial logits of experts
// [k E / K, (k + 1) E / K) (thread (el, cg) = (tid / 16, tid % 16): expert
// e0 + 32 i + el over columns 4 cg ..).  A member's loads go out while the
// barrier before phase C completes and land during phase C.
static_assert(MT * 64 <= kThreads, "one team row value per thread");
constexpr int kShareIt = 2;  // expert passes held in registers (E / K <= 64)
struct ShareLoads {
    float4 r[kShareIt];
    float g, wn;
};
__device__ __forceinline__ void share_loads(const StackArgs &a, uint32_t ln, ShareLoads &S) {
    const uint32_t K = a.members, tau = blockIdx.x % kStackTeams, k = blockIdx.x / kStackTeams;
    if (k >= K) return;
    const StackLayer Ln = a.layers[ln];
    const uint32_t epm = (a.E + K - 1) / K, e0 = k * epm;
    const uint32_t el = tid() >> 4, cg = tid() & 15;
#pragma unroll
    for (int i = 0; i < kShareIt; ++i) {
        const uint32_t e = e0 + 32 * i + el;
        S.r[i] = load_global_f4(Ln.router + (size_t)(e < a.E ? e : 0) * H + tau * 64 + 4 * cg);
    }
    S.g = load_global_f(Ln.gate_vec + tau * 64 + (tid() % 64));
    S.wn = load_global_f(Ln.norm + tau * 64 + (tid() % 64));
}

// hv: this thread's row of h (0 past the m tokens); acc: the parity of the
// logit accumulator layer ln reads; s_y: LDS for the team's [MT][64] y rows.
// The partial logits go to the accumulator as full-wavefront atomics: each
// pass's 32 x M values (and the shared-expert gate's M) are gathered in LDS
// and added one (token, expert) per lane by the first wavefronts.  The device
// pays per atomic instruction: 4-lane atomics straight from the reductions'
// lanes took 1131 us per 40-layer launch, the gathered form 1098 us.
__device__ void member_tail(const StackArgs &a, uint32_t tau, uint32_t k, const ShareLoads &S, float hv,
                            float *s_y, uint64_t *acc, uint32_t ln, uint32_t base) {
    const int wave = __builtin_amdgcn_readfirstlane(tid() / kWave);
    const int lane = tid() % kWave;
    const uint32_t m = a.m, E = a.E, K = a.members;
    uint64_t *flag = acc + (size_t)MT * (E + 1);
    const float y = hv * S.wn;  // tid % 64 is this thread's column, the weight it loaded
    if (tid() < MT * 64) s_y[tid()] = y;
    if (wave < (int)m) {  // wavefront t holds token t's 64 rows
        const uint32_t t = (uint32_t)wave;
        if (k == t % K) {  // records: half-wavefront = block 2 tau + half
            const uint32_t half = (uint32_t)lane >> 5;
            prep_block32(y, lane & 31, true, a.xprep + (size_t)t * kBpGate * kXprepDwords, kBpGate,
                         2 * tau + half, CoherentStore());
        }
        if (k == 0) {
            const float v = group_reduce<64>(hv * hv, AddOp());
            if (lane == 0)
                __hip_atomic_store(reinterpret_cast<uint64_t *>(a.ssq) + tau * MT + t,
                                   ((uint64_t)stack_part_tag(base, ln) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        if (k == K - 1) {  // the shared-expert gate, one column per lane
            const float g = group_reduce<64>(S.g * y, AddOp());
            if (lane == 0) s_lv[t][32] = g;
        }
    }
    __syncthreads();
    const uint32_t epm = (E + K - 1) / K, e0 = k * epm, e1 = e0 + epm < E ? e0 + epm : E;
    const uint32_t el = tid() >> 4, cg = tid() & 15;
    auto pass = [&](uint32_t i, const float4 &r) {
        const uint32_t e = e0 + 32 * i + el;
        const bool valid = e < e1;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (t < (int)m) {
                const float4 yv = *reinterpret_cast<const float4 *>(s_y + t * 64 + 4 * cg);
                float v = r.x * yv.x;
                v = fmaf(r.y, yv.y, v);
                v = fmaf(r.z, yv.z, v);
                v = fmaf(r.w, yv.w, v);
                v = group_reduce<16>(valid ? v : 0.0f, AddOp());
                if (cg == 0) s_lv[t][el] = v;
            }
        }
        lds_barrier();
        if (i == 0) wait_own_stores();  // records and sums of squares before any count
        const uint32_t t = tid() / 32, ee = e0 + 32 * i + tid() % 32;
        if (tid() < MT * 32 && t < m && ee < e1) add_counted(acc + (size_t)t * (E + 1) + ee, flag, s_lv[t][tid() % 32]);
        if (i == 0 && k == K - 1 && tid() >= MT * 32 && tid() < MT * 32 + m)
            add_counted(acc + (size_t)(tid() - MT * 32) * (E + 1) + E, flag, s_lv[tid() - MT * 32][32]);
        lds_barrier();  // s_lv is rewritten by the next pass
    };
#pragma unroll
    for (int i = 0; i < kShareIt; ++i)
        if (e0 + 32 * i < e1 || i == 0) pass(i, S.r[i]);  // pass 0 also adds the shared gate
    const StackLayer Ln = a.layers[ln];
    for (uint32_t i = kShareIt; e0 + 32 * i < e1; ++i) {
        const uint32_t e = e0 + 32 * i + el;
        pass(i, load_global_f4(Ln.router + (size_t)(e < e1 ? e : e0) * H + tau * 64 + 4 * cg));
    }
}

// Layer 0's inputs: every member takes its team's rows of h_in (kept as the
// first layer's residual in hres) and does its share of the tail.  Member 0
// also copies the rows to h_save, from which the library re-runs the stack
// after an aborted launch: every workgroup runs this prologue before any
// grid barrier, and h (which may be h_in) is written only after the last
// layer, which no workgroup reaches before all have passed the first barrier,
// so the copy is of the input even when the launch updates h in place.
__device__ void team_prologue(const StackArgs &a, float &hres, uint32_t base) {
    const uint32_t tau = blockIdx.x % kStackTeams, k = blockIdx.x / kStackTeams;
    if (k >= a.members) return;
    ShareLoads S;
    share_loads(a, 0, S);
    const uint32_t tt = tid() / 64, row = tid() % 64;
    hres = tid() < MT * 64 && tt < a.m ? load_coherent(&a.h_in[(size_t)tt * H + tau * 64 + row]) : 0.0f;
    if (k == 0 && a.h_save && tid() < MT * 64 && tt < a.m) a.h_save[(size_t)tt * H + tau * 64 + row] = hres;
    member_tail(a, tau, k, S, hres, reinterpret_cast<float *>(s_dyn), a.lacc, 0, base);
}

// Phase C's partials travel as tagged 64-bit words: tag << 32 | f32 bits, the
// tag counting layer steps over every launch on this scratch with the high
// bit set (stack_part_tag: strictly increasing whatever the depth of each
// launch), so a word left by an earlier layer or launch (or the zeroed
// allocation) never carries the current tag.  Readers poll the words
// themselves, bounded like grid_wait.

// ---- the team exchange within one XCD ------------------------------------------------
// Workgroup b runs on XCD b mod 8 under the dispatcher's round-robin placement
// (checked at every launch: a workgroup that reads another id from its
// XCC_ID register sets sync->xcd_bad before the first barrier), so the 8
// members of team tau (workgroups tau + 32 k) share one L2.  Their partial
// words then need not travel to the memory side: a plain store lands in the
// L2 (the vector L1 is write-through), and a non-temporal load misses the
// L1 and reads the L2 -- a round trip of about 0.8 us between two idle
// compute units against 1.0-1.2 us at agent scope (measured).  Without the
// placement, or with another team size, the exchange stays at agent scope.
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v;
}
constexpr uint32_t kLocalMembers = 8;
__device__ __forceinline__ void store_l2(uint64_t *p, uint64_t v) {
    asm volatile("global_store_dwordx2 %0, %1, off" ::"v"(p), "v"(v) : "memory");
}
// The eight members' words of one row (stride MT * 64 words), all loads in
// flight at once, then one wait.
__device__ __forceinline__ void load8_l2(const uint64_t *w0, uint64_t (&w)[8]) {
    constexpr size_t S = (size_t)MT * 64;
    asm volatile(
        "global_load_dwordx2 %0, %8, off nt\n\t"
        "global_load_dwordx2 %1, %9, off nt\n\t"
        "global_load_dwordx2 %2, %10, off nt\n\t"
        "global_load_dwordx2 %3, %11, off nt\n\t"
        "global_load_dwordx2 %4, %12, off nt\n\t"
        "global_load_dwordx2 %5, %13, off nt\n\t"
        "global_load_dwordx2 %6, %14, off nt\n\t"
        "global_load_dwordx2 %7, %15, off nt\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]), "=&v"(w[6]), "=&v"(w[7])
        : "v"(w0), "v"(w0 + S), "v"(w0 + 2 * S), "v"(w0 + 3 * S), "v"(w0 + 4 * S), "v"(w0 + 5 * S),
          "v"(w0 + 6 * S), "v"(w0 + 7 * S)
        : "memory");
}

// This thread's K partials (member order) of word `w0` (stride MT * 64 words
// per member), but for member `own`'s (the caller's own, which it already
// holds); false after a timeout (which sets abort) or another workgroup's
// abort.
__device__ bool poll_partials(const StackArgs &a, const uint64_t *w0, uint32_t K, uint32_t tag,
                              float (&pv)[kMaxMembers], bool local, uint32_t own) {
    uint32_t need = ((1u << K) - 1u) & ~(1u << own);
    int64_t t0 = 0;
    for (uint32_t spin = 1;; ++spin) {
        if (local) {  // K == kLocalMembers, through the L2
            uint64_t w[8];
            load8_l2(w0, w);
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                if (((need >> kk) & 1u) && (uint32_t)(w[kk] >> 32) == tag) {
                    pv[kk] = __uint_as_float((uint32_t)w[kk]);
                    need &= ~(1u << kk);
                }
            }
        } else {
#pragma unroll
            for (int kk = 0; kk < kMaxMembers; ++kk) {
                if ((need >> kk) & 1u) {
                    const uint64_t w = poll_load(w0 + (size_t)kk * MT * 64);
                    if ((uint32_t)(w >> 32) == tag) {
                        pv[kk] = __uint_as_float((uint32_t)w);
                        need &= ~(1u << kk);
                    }
                }
            }
        }
        if (!need) return true;
        if ((spin & 15) == 0) {
            if (__hip_atomic_load(&a.sync->abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
            const int64_t now = wall_clock64();
            if (t0 == 0) {
                t0 = now;
            } else if (now - t0 > kSpinLimit) {
                __hip_atomic_store(&a.sync->abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (a.dev_status)
                    __hip_atomic_store(a.dev_status, (int32_t)TQF_HIP_ERR_DEVICE, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                return false;
            }
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// ---- phase C -------------------------------------------------------------------
template <int LPRD, int MAXP, int URW>
__device__ void phase_c(const StackArgs &a, uint32_t l, uint32_t base, float &hres, const ShareLoads &SL) {
    uint4 *s_x = reinterpret_cast<uint4 *>(reinterpret_cast<uint8_t *>(s_dyn) + LdsLayout<LPRD, MAXP>::kXr);
    const int wave = __builtin_amdgcn_readfirstlane(tid() / kWave);
    const int lane = tid() % kWave;
    constexpr int G = kWave / LPRD;   // lane groups per wavefront
    constexpr int RG = 8 / G;         // rows per lane group (a wavefront owns one octet)
    constexpr int NL = MT * RG;       // values per lane before the transpose
    static_assert(NL <= LPRD, "transpose width");
    const uint32_t K = a.members;
    const uint32_t tau = blockIdx.x % kStackTeams, k = blockIdx.x / kStackTeams;
    if (k >= K) return;
    const MemberShare share = member_share<URW>((int)k, (int)K, (int)a.m, P.n_pairs);
    const int cnt = share.cnt();
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
            const int pq = share.pair(q < cnt ? q : cnt - 1);
            const RowLane W = row_lane(s_mats[P.pair_expert[pq] * 3 + 2], LPRD);
#pragma unroll
            for (int rr = 0; rr < RG; ++rr) nib[q][rr] = q4_signed(load_nibbles(W, r0 + j * RG + rr, b));
            sc[q] = load_scales(W, r0 / 8, b);
        }
    }
    // routed pairs (staging slots ns..): their records from phase B; shared
    // pairs (slots 0..ns-1): records of the raw rows, one (pair, block) per
    // half-wavefront and round
    stage_coherent<(MAXP * 7 * LPRD * 2 + kThreads - 1) / kThreads>(
        reinterpret_cast<uint64_t *>(s_x) + (size_t)share.ns * 7 * LPRD * 2,
        reinterpret_cast<const uint64_t *>(a.hprep + (size_t)share.r0 * LPRD * kXprepDwords),
        (uint32_t)(share.r1 - share.r0) * 7 * LPRD * 2);
    {
        // kIt rounds (the most a member can own: ceil(M / K) shared pairs of
        // LPRD blocks over 16 half-wavefronts); every round's loads go out
        // before the first build
        constexpr int kIt = MT * LPRD / (2 * kWaves);
        const int nb = (int)a.F / 32, n_sh = share.ns * nb;
        const int hw = (int)(tid() >> 5), jj = lane & 31;
        float vv[kIt];
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
            const int q = it * 2 * kWaves + hw;  // uniform per half-wavefront
            const int qq = q < n_sh ? q : 0;
            const int pair = share.pair(qq / nb), blk = qq % nb;
            vv[it] = q < n_sh ? load_coherent(&a.hshared[(size_t)P.pair_tok[pair] * a.F + blk * 32 + jj]) : 0.0f;
        }
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
            const int q = it * 2 * kWaves + hw;
            if (it * 2 * kWaves < n_sh) {  // uniform over the workgroup
                const bool active = q < n_sh;
                const int qq = active ? q : 0;
                prep_block32(vv[it], jj, active,
                             reinterpret_cast<uint32_t *>(s_x) + (size_t)(qq / nb) * 7 * LPRD * 4, LPRD,
                             (uint32_t)(qq % nb), PlainStore());
            }
        }
    }
    __syncthreads();
    float acc[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) acc[i] = 0.0f;
    const bool pad = b >= a.F / 32;
#pragma unroll
    for (int q = 0; q < MAXP; ++q) {
        if (q < cnt) {
            const int pq = share.pair(q);
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
                const uint8_t *img = reinterpret_cast<const uint8_t *>(s_dyn) +
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
    // every token slot, so each word this launch reads was last written by it
    // or by the previous launch
    const uint32_t tag = stack_part_tag(base, l);
    if (reduced_first_copy<LPRD, NL>(lane)) {
        uint64_t *word = &a.partial[(((size_t)tau * K + k) * MT + t) * 64 + 8 * wave + j * RG + rr];
        const uint64_t v = ((uint64_t)tag << 32) | __float_as_uint(s);
        if (P.xcd_local) store_l2(word, v);
        else __hip_atomic_store(word, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_h[t][8 * wave + j * RG + rr] = s;  // this member's own partial, for the combine
    }
    // team combine: every member takes its own partials from LDS and polls the
    // other K - 1 members' words, then sums them in member order (the same
    // bits in every member) and takes its share of the next layer's inputs.
    // Only an LDS barrier: the poll need not wait for this member's own
    // stores to complete (1141 -> 1131 us per 40-layer launch against
    // polling its own word too).
    if (tid() == 0) P.ok = 1;
    lds_barrier();
    const uint32_t m = a.m, tt = tid() / 64, row = tid() % 64;
    const bool next = l + 1 < a.n_layers;
    if (tid() < MT * 64 && tt < m) {
        float pv[kMaxMembers];
        pv[k < kMaxMembers ? k : 0] = s_h[tt][row];
        if (poll_partials(a, a.partial + ((size_t)tau * K * MT + tt) * 64 + row, K, tag, pv, P.xcd_local != 0, k)) {
            float sum = 0.0f;
#pragma unroll
            for (int kk = 0; kk < kMaxMembers; ++kk)
                if (kk < (int)K) sum += pv[kk];
            hres += sum;
            if (!next && k == 0) store_coherent(&a.h[(size_t)tt * H + tau * 64 + row], hres);
        } else {
            P.ok = 0;
        }
    }
    __syncthreads();
    if (!P.ok) return;
    if (!next) {
        // nothing reads this parity any more: leave it at zero
        zero_lacc(a.lacc + (size_t)(l & 1) * kLaccWords, k * kStackTeams + tau, K * kStackTeams);
        return;
    }
    member_tail(a, tau, k, SL, hres, reinterpret_cast<float *>(s_x), a.lacc + (size_t)((l + 1) & 1) * kLaccWords,
                l + 1, base);
}

}  // namespace

template <int LPRD, int MAXP, int URW>
__global__ __launch_bounds__(kThreads) void stack_kernel(StackArgs a) {
    uint32_t epoch = 0;
    // layer 0's expert-matrix table into LDS (later layers': during the
    // previous layer's phase C), and layer 0's inputs from h_in
    constexpr int kPtrPer = ((256 + 1) * 3 + kThreads - 1) / kThreads;
    {
        const StackLayer L0 = a.layers[0];
#pragma unroll
        for (int i = 0; i < kPtrPer; ++i) {
            const uint32_t k = tid() + (uint32_t)i * kThreads;
            if (k < (a.E + 1) * 3) s_mats[k] = load_global_ptr(L0.mats + k);
        }
    }
    // layer steps of every earlier launch on this scratch (the tags' base)
    const uint32_t base = __hip_atomic_load(&a.sync->step_base, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the team exchange's placement check (before the first barrier's drain)
    if (tid() == 0 && xcc_id() != blockIdx.x % kStackBarrierGroups)
        __hip_atomic_fetch_or(&a.sync->xcd_bad, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float hres = 0.0f;  // the residual: this thread's team row of h (phase C members)
    team_prologue(a, hres, base);
    bool ok = grid_sync(a.sync, epoch, a.dev_status);
    if (tid() == 0)
        P.xcd_local = a.members == kLocalMembers && gridDim.x == kLocalMembers * kStackTeams &&
                      kStackTeams % kStackBarrierGroups == 0 &&
                      __hip_atomic_load(&a.sync->xcd_bad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0;
    __syncthreads();
    for (uint32_t l = 0; ok && l < a.n_layers; ++l) {
        UnitLoads U;
        SharedLoads S;
        bool pre;
        compute_routes<LPRD, MAXP, URW>(a, l, U, S, pre, base);
        if (blockIdx.x == 0 && tid() < a.m * kTopK) {
            const uint32_t t = tid() / kTopK, kk = tid() % kTopK;
            if (a.ids_out) a.ids_out[((size_t)l * a.m + t) * kTopK + kk] = P.bad ? 0 : (uint16_t)P.ids[t][kk];
            if (a.w_out) a.w_out[((size_t)l * a.m + t) * kTopK + kk] = P.bad ? 0.0f : P.w[t][kk];
        }
        if (blockIdx.x == 0 && tid() == 0 && P.bad == 1 && a.status)
            __hip_atomic_store(a.status, (int32_t)TQF_HIP_ERR_ROUTER, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        const int n_units = P.n_groups > 0 ? (int)a.m * kTopK * (int)(a.F / (8 * URW)) : 0;
        // the preloaded first unit (pre holds exactly when blockIdx.x <
        // n_units); both branches use U, so no path leaves its loads pending
        // the shared expert's rows go inside the first unit, once its first
        // kAhead + 1 rows' loads are issued: they compute while those rows'
        // weights are in flight (measured per 40-layer launch: 1055 us before
        // the unit's loads are issued, 1038 us here, 1055 / 1071 / 1108 /
        // 1131 us after rows 0 / 1 / 2 / 3's dot products)
        if (pre) {
            gate_up_unit<LPRD, MAXP, URW>(a, unit_desc<URW>(blockIdx.x, (int)a.F, (int)a.m), U, true,
                                     [&] { shared_rows<LPRD, MAXP>(a, S); });
        } else {
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                consume(U.ng[n]);
                consume(U.nu[n]);
            }
            consume(U.sg);
            consume(U.su);
            if (P.n_groups > 0) shared_rows<LPRD, MAXP>(a, S);
        }
        for (int u = blockIdx.x + gridDim.x; u < n_units; u += gridDim.x)
            gate_up_unit<LPRD, MAXP, URW>(a, unit_desc<URW>(u, (int)a.F, (int)a.m), U, false, [] {});
        // arrive once every load of phase B is consumed and this thread's
        // record and row stores are complete (a compiler-visible wait, which
        // also settles the compiler's own bookkeeping of those loads); then
        // phase C's down weights stream while the barrier completes (issuing
        // them stalls until the memory pipeline takes them, so they go out
        // after the arrival)
        grid_arrive(a.sync, epoch);
        prefetch_down<LPRD, MAXP, URW>(a);
        // this member's share of the next layer's router rows, gate and norm
        ShareLoads SL;
        if (l + 1 < a.n_layers) share_loads(a, l + 1, SL);
        if (!(ok = grid_wait(a.sync, epoch, a.dev_status, l == a.fail_at && blockIdx.x == 0))) break;
        // the next layer's expert-matrix table: loads now, LDS after phase C
        // (whose down weights still come from this layer's table)
        const bool more = l + 1 < a.n_layers;
        const uint8_t *mp[kPtrPer];
        if (more) {
            const StackLayer Ln = a.layers[l + 1];
#pragma unroll
            for (int i = 0; i < kPtrPer; ++i) {
                const uint32_t k = tid() + (uint32_t)i * kThreads;
                mp[i] = load_global_ptr(Ln.mats + (k < (a.E + 1) * 3 ? k : 0));
            }
        }
        phase_c<LPRD, MAXP, URW>(a, l, base, hres, SL);
        if (!(ok = P.ok != 0)) break;
        if (more) {
            __syncthreads();  // every wavefront is past phase C's table reads
#pragma unroll
            for (int i = 0; i < kPtrPer; ++i) {
                const uint32_t k = tid() + (uint32_t)i * kThreads;
                if (k < (a.E + 1) * 3) s_mats[k] = mp[i];
            }
        }
    }
    stack_exit(a.sync, a.lacc, base, a.n_layers, a.host_flag);
}

namespace {
template <int LPRD>
size_t lds_bytes_for(uint32_t maxp) {
    return maxp <= 5 ? LdsLayout<LPRD, 5>::kTotal : LdsLayout<LPRD, 9>::kTotal;
}
}  // namespace

// The most pairs a phase C member owns (member_share).
uint32_t member_max_pairs(uint32_t members) {
    return (MT + members - 1) / members + (MT * kTopK + members - 1) / members;
}

size_t stack_lds_bytes(uint32_t bp_down, uint32_t members) {
    const uint32_t maxp = member_max_pairs(members);
    if (bp_down == 16) return lds_bytes_for<16>(maxp);
    if (bp_down == 32) return lds_bytes_for<32>(maxp);
    return lds_bytes_for<64>(maxp);
}

namespace {
template <int LPRD, int URW>
const void *pick(uint32_t maxp, int &chosen) {
    if (maxp <= 5) { chosen = 5; return (const void *)stack_kernel<LPRD, 5, URW>; }
    if (maxp <= 9) { chosen = 9; return (const void *)stack_kernel<LPRD, 9, URW>; }
    chosen = 0;
    return nullptr;
}
// small: the kernel for M <= 2 (32-row gate/up units)
const void *kernel_for(uint32_t bp_down, uint32_t members, bool small) {
    const uint32_t maxp = member_max_pairs(members);
    int chosen = 0;
    if (bp_down == 16) return small ? pick<16, 4>(maxp, chosen) : pick<16, 8>(maxp, chosen);
    if (bp_down == 32) return small ? pick<32, 4>(maxp, chosen) : pick<32, 8>(maxp, chosen);
    if (bp_down == 64) return small ? pick<64, 4>(maxp, chosen) : pick<64, 8>(maxp, chosen);
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
        for (bool small : {false, true}) {
            const void *kv = kernel_for(bp, members, small);
            if (kv && hipFuncSetAttribute(kv, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)stack_lds_bytes(bp, members)) != hipSuccess)
                return 0;
        }
    }
    const size_t lds = stack_lds_bytes(bp_down, members);
    for (bool small : {false, true}) {
        const void *k = kernel_for(bp_down, members, small);
        int per_cu = 0;
        if (!k || hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kThreads, lds) != hipSuccess ||
            per_cu < 1)
            return 0;
    }
    return grid;
}

// A plain launch: the grid (one workgroup per compute unit, checked against
// the occupancy limit by stack_grid) is co-resident whenever the device runs
// nothing else, and every grid-barrier wait is bounded (a timeout reports
// TQF_HIP_ERR_DEVICE), so the cooperative launch's guarantee is not needed;
// it cost about 15 us of dispatch per launch.
hipError_t launch_stack(hipStream_t s, const StackArgs &a, uint32_t grid, uint32_t bp_down) {
    const void *k = kernel_for(bp_down, a.members, a.m <= 2);
    if (!k) return hipErrorInvalidValue;
    StackArgs args = a;
    void *params[] = {&args};
    return hipLaunchKernel(k, dim3(grid), dim3(kThreads), params, (unsigned int)stack_lds_bytes(bp_down, a.members),
                           s);
}

}  // namespace tqf
