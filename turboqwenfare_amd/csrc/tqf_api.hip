// tqf_api.hip -- the C ABI (include/tqf_hip.h): context, weights arena,
// scratch, host/device entry points, HIP-graph replay and event profiling.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/tqf_hip.h"
#include "../../include/tqf_hip_synth.h"
#include "tqf_internal.h"

using namespace tqf;

namespace tqf {
struct GraphEntry {
    std::vector<uint64_t> key;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};
}  // namespace tqf

// ---- allocation-free acceptance scratch -----------------------------------
// tqf_hip_accept_device_noalloc runs the acceptance kernels on this array
// instead of a context-allocated buffer: one copy per GPU, held until the
// process ends, shared by every call on that GPU (calls that overlap on one
// GPU race).  The kernels' hand-off counters live in its first 64 bytes and
// start at zero (the array is zero-initialised when the code object loads);
// every launch returns them to zero before it ends.  The partials after them
// are rewritten by each launch before they are read.  In host code `scratch`
// names a host-side stand-in; kernels get the per-device address that
// hipGetSymbolAddress returns (tqf_hip_create resolves it once per device).
namespace {
constexpr size_t kNoAllocScratchBytes = size_t(256) << 10;
constexpr int kMaxDevices = 64;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device `device` (resolved
// once per device); nullptr on failure.
void *noalloc_scratch_for(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
        g_scratch_ptr[device] = ptr;
    }
    return g_scratch_ptr[device];
}
}  // namespace

namespace {

constexpr size_t kSlabBytes = size_t(256) << 20;
constexpr size_t kAlign = 256;
constexpr int kRingSize = 4096;
constexpr size_t kMaxGraphs = 16;
// the context's pinned abort flags (tqf_hip_ctx::h_flags)
constexpr int kFlagStack = 0;
constexpr int kFlagAccept = 1;

int32_t fail(tqf_hip_ctx *ctx, int32_t code, const std::string &msg) {
    if (ctx) ctx->last_error = msg;
    return code;
}

int32_t hip_fail(tqf_hip_ctx *ctx, const char *what, hipError_t e) {
    return fail(ctx, TQF_HIP_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

#define TQF_HIP(ctx, expr)                                  \
    do {                                                    \
        hipError_t _e = (expr);                             \
        if (_e != hipSuccess) return hip_fail(ctx, #expr, _e); \
    } while (0)

#define TQF_ENTER(ctx)                                                      \
    do {                                                                    \
        if (!(ctx)) return TQF_HIP_ERR_INVALID;                             \
        (ctx)->last_error.clear();                                          \
        hipError_t _e = hipSetDevice((ctx)->device);                        \
        if (_e != hipSuccess) return hip_fail(ctx, "hipSetDevice", _e);     \
    } while (0)

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ---- arena ----------------------------------------------------------------
hipError_t arena_alloc(tqf_hip_ctx *ctx, size_t bytes, void **out) {
    bytes = align_up(bytes ? bytes : 1, kAlign);
    if (bytes > kSlabBytes / 2) {
        uint8_t *p = nullptr;
        hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) return e;
        ctx->slabs.push_back(Slab{p, bytes, bytes, 1});
        *out = p;
        return hipSuccess;
    }
    for (auto it = ctx->slabs.rbegin(); it != ctx->slabs.rend(); ++it) {
        if (it->size == kSlabBytes && it->size - it->used >= bytes) {
            *out = it->base + it->used;
            it->used += bytes;
            it->live += 1;
            return hipSuccess;
        }
    }
    uint8_t *p = nullptr;
    hipError_t e = hipMalloc(&p, kSlabBytes);
    if (e != hipSuccess) return e;
    ctx->slabs.push_back(Slab{p, kSlabBytes, bytes, 1});
    *out = p;
    return hipSuccess;
}

void arena_free(tqf_hip_ctx *ctx, void *ptr) {
    if (!ptr) return;
    uint8_t *p = static_cast<uint8_t *>(ptr);
    for (size_t i = 0; i < ctx->slabs.size(); ++i) {
        Slab &s = ctx->slabs[i];
        if (p >= s.base && p < s.base + s.size) {
            if (--s.live == 0) {
                (void)hipFree(s.base);
                ctx->slabs.erase(ctx->slabs.begin() + (long)i);
            }
            return;
        }
    }
}

// ---- graphs ---------------------------------------------------------------
void drop_graphs(tqf_hip_ctx *ctx) {
    for (GraphEntry *g : ctx->graphs) {
        if (g->exec) (void)hipGraphExecDestroy(g->exec);
        if (g->graph) (void)hipGraphDestroy(g->graph);
        delete g;
    }
    ctx->graphs.clear();
}

GraphEntry *find_graph(tqf_hip_ctx *ctx, const std::vector<uint64_t> &key) {
    for (GraphEntry *g : ctx->graphs)
        if (g->key == key) return g;
    return nullptr;
}

// ---- scratch --------------------------------------------------------------
template <typename T>
hipError_t grow(T *&ptr, size_t &have, size_t need) {
    if (have >= need && ptr) return hipSuccess;
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    have = 0;
    hipError_t e = hipMalloc(&ptr, need);
    if (e == hipSuccess) have = need;
    return e;
}

int32_t ensure_moe_scratch(tqf_hip_ctx *ctx, uint32_t hidden, uint32_t width, uint32_t experts) {
    Scratch &sc = ctx->scratch;
    if (sc.xprep && hidden <= sc.hidden && width <= sc.width && experts <= sc.experts)
        return TQF_HIP_OK;
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    drop_graphs(ctx);
    hidden = std::max(hidden, sc.hidden);
    width = std::max(width, sc.width);
    experts = std::max(experts, sc.experts);
    (void)hipFree(sc.xprep);
    (void)hipFree(sc.hprep);
    (void)hipFree(sc.logits);
    (void)hipFree(sc.plan);
    (void)hipFree(sc.partial);
    (void)hipFree(sc.counters);
    sc.xprep = sc.hprep = sc.counters = nullptr;
    sc.logits = nullptr;
    sc.partial = nullptr;
    sc.plan = nullptr;
    sc.hidden = sc.width = sc.experts = 0;
    // padding records stay zero: kernels only write real blocks
    const size_t xprep = (size_t)kMaxTokens * padded_blocks(hidden / 32) * kXprepDwords * 4;
    const size_t hprep = (size_t)kMaxSlots * padded_blocks(width / 32) * kXprepDwords * 4;
    const size_t logits = (size_t)kMaxTokens * (experts + 1) * 8;
    const size_t partial = (size_t)kMaxSlots * kMaxTokens * hidden * 4;
    const size_t counters = counter_count(hidden) * 4;
    TQF_HIP(ctx, hipMalloc(&sc.xprep, xprep));
    TQF_HIP(ctx, hipMalloc(&sc.hprep, hprep));
    TQF_HIP(ctx, hipMalloc(&sc.logits, logits));
    TQF_HIP(ctx, hipMalloc(&sc.plan, sizeof(Plan)));
    TQF_HIP(ctx, hipMalloc(&sc.partial, partial));
    TQF_HIP(ctx, hipMalloc(&sc.counters, counters));
    TQF_HIP(ctx, hipMemset(sc.xprep, 0, xprep));
    TQF_HIP(ctx, hipMemset(sc.hprep, 0, hprep));
    TQF_HIP(ctx, hipMemset(sc.plan, 0, sizeof(Plan)));
    TQF_HIP(ctx, hipMemset(sc.counters, 0, counters));
    TQF_HIP(ctx, hipMemset(sc.logits, 0, logits));  // zero carries no launch's tag
    sc.hidden = hidden;
    sc.width = width;
    sc.experts = experts;
    return TQF_HIP_OK;
}

int32_t ensure_accept_scratch(tqf_hip_ctx *ctx, size_t bytes) {
    Scratch &sc = ctx->scratch;
    if (sc.accept && sc.accept_bytes >= bytes) return TQF_HIP_OK;
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    drop_graphs(ctx);
    TQF_HIP(ctx, grow(sc.accept, sc.accept_bytes, bytes));
    TQF_HIP(ctx, hipMemset(sc.accept, 0, sc.accept_bytes));  // counters start at zero
    return TQF_HIP_OK;
}

// Scratch of the persistent stack kernel (sized for kStackMT tokens).
int32_t ensure_stack_scratch(tqf_hip_ctx *ctx, uint32_t experts, uint32_t bp_down,
                             uint32_t members) {
    StackScratch &sc = ctx->stack;
    if (sc.sync && experts <= sc.experts && bp_down <= sc.bp_down && members <= sc.members)
        return TQF_HIP_OK;
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    drop_graphs(ctx);
    experts = std::max(experts, sc.experts);
    bp_down = std::max(bp_down, sc.bp_down);
    members = std::max(members, sc.members);
    (void)hipFree(sc.sync);
    (void)hipFree(sc.lacc);
    (void)hipFree(sc.xprep);
    (void)hipFree(sc.hprep);
    (void)hipFree(sc.hshared);
    (void)hipFree(sc.partial);
    (void)hipFree(sc.ssq);
    (void)hipFree(sc.h_save);
    sc = StackScratch();
    TQF_HIP(ctx, hipMalloc(&sc.sync, sizeof(StackSync)));
    TQF_HIP(ctx, hipMemset(sc.sync, 0, sizeof(StackSync)));
    // the accumulators start (and every launch leaves them) at zero
    TQF_HIP(ctx, hipMalloc(&sc.lacc, 2 * (size_t)kLaccWords * 8));
    TQF_HIP(ctx, hipMemset(sc.lacc, 0, 2 * (size_t)kLaccWords * 8));
    TQF_HIP(ctx, hipMalloc(&sc.xprep, (size_t)kStackMT * (kStackHidden / 32) * kXprepDwords * 4));
    TQF_HIP(ctx, hipMalloc(&sc.hprep, (size_t)kStackMT * (kTopK + 1) * bp_down * kXprepDwords * 4));
    TQF_HIP(ctx, hipMalloc(&sc.hshared, (size_t)kStackMT * bp_down * 32 * 4));
    // tagged words: zero holds no launch's tag
    TQF_HIP(ctx, hipMalloc(&sc.partial, (size_t)kStackTeams * members * kStackMT * 64 * 8));
    TQF_HIP(ctx, hipMemset(sc.partial, 0, (size_t)kStackTeams * members * kStackMT * 64 * 8));
    TQF_HIP(ctx, hipMalloc(&sc.ssq, (size_t)kStackTeams * kStackMT * 8));
    TQF_HIP(ctx, hipMemset(sc.ssq, 0, (size_t)kStackTeams * kStackMT * 8));
    TQF_HIP(ctx, hipMalloc(&sc.h_save, (size_t)kStackMT * kStackHidden * 4));
    sc.experts = experts;
    sc.bp_down = bp_down;
    sc.members = members;
    return TQF_HIP_OK;
}

int32_t ensure_stage(tqf_hip_ctx *ctx, size_t bytes) {
    if (ctx->d_stage && ctx->stage_bytes >= bytes) return TQF_HIP_OK;
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    TQF_HIP(ctx, grow(ctx->d_stage, ctx->stage_bytes, std::max(bytes, size_t(1) << 20)));
    return TQF_HIP_OK;
}

// ---- profiling ------------------------------------------------------------
hipEvent_t take_event(tqf_hip_ctx *ctx) {
    if (!ctx->event_pool.empty()) {
        hipEvent_t e = ctx->event_pool.back();
        ctx->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

void resolve_profile(tqf_hip_ctx *ctx) {
    if (ctx->prof_pending.empty()) return;
    (void)hipStreamSynchronize(ctx->stream);
    for (const ProfileSlot &p : ctx->prof_pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
            ctx->prof_launches[p.kind] += 1;
            ctx->prof_ms[p.kind] += ms;
            double bytes = p.fixed_bytes;
            if (p.ring_index >= 0) bytes += p.per_slot_bytes * (ctx->prof_ring[p.ring_index] + 1);
            ctx->prof_bytes[p.kind] += bytes;
        }
        ctx->event_pool.push_back(p.start);
        ctx->event_pool.push_back(p.stop);
    }
    ctx->prof_pending.clear();
    ctx->prof_ring_next = 0;
}

struct Prof {
    tqf_hip_ctx *ctx;
    hipEvent_t start = nullptr;
    explicit Prof(tqf_hip_ctx *c) : ctx(c) {
        if (ctx->profiling && !ctx->capturing) {
            if (ctx->prof_ring_next >= kRingSize) resolve_profile(ctx);
            start = take_event(ctx);
            if (start) (void)hipEventRecord(start, ctx->stream);
        }
    }
    // per_slot_bytes > 0 is charged once per distinct expert of the launch
    // just made: (plan->n_union + 1) including the shared expert.
    void end(int kind, double fixed_bytes, double per_slot_bytes, const Plan *plan) {
        if (!start) return;
        hipEvent_t stop = take_event(ctx);
        if (!stop) return;
        (void)hipEventRecord(stop, ctx->stream);
        int ring = -1;
        if (per_slot_bytes > 0 && plan) {
            ring = ctx->prof_ring_next++;
            (void)hipMemcpyAsync(&ctx->prof_ring[ring], &plan->n_union, sizeof(int32_t),
                                 hipMemcpyDeviceToHost, ctx->stream);
        }
        ctx->prof_pending.push_back(ProfileSlot{start, stop, kind, fixed_bytes, per_slot_bytes, ring});
        start = nullptr;
    }
};

double q4_bytes(uint32_t rows, uint32_t cols) { return (double)rows * (cols / 32) * kQ4Block; }

// ---- validation -----------------------------------------------------------
bool valid_weights(const tqf_hip_weights *w) {
    return w && w->tiles && w->format == TQF_HIP_FORMAT_Q4_0;
}
bool valid_q4k(const tqf_hip_weights *w) {
    return w && w->tiles && w->format == TQF_HIP_FORMAT_Q4_K;
}
bool valid_q6k(const tqf_hip_weights *w) {
    return w && w->tiles && w->format == TQF_HIP_FORMAT_Q6_K;
}

// ---- the layer sequence ---------------------------------------------------
// One MoE layer: route (optionally RMSNorm) -> gate/up -> down (+ residual).
int32_t enqueue_layer(tqf_hip_ctx *ctx, const LayerDev &L, const float *h, const float *norm,
                      uint32_t m, const float *resid, float *out, uint16_t *ids, float *w,
                      int32_t *status) {
    Scratch &sc = ctx->scratch;
    const double H = L.hidden, F = L.width;
    const double pairs = (double)m * (kTopK + 1);
    {
        Prof p(ctx);
        hipError_t e = launch_route(ctx->stream, L, h, norm, m, sc, ids, w, status);
        if (e != hipSuccess) return hip_fail(ctx, "route kernel launch", e);
        p.end(TQF_HIP_KERNEL_ROUTE, (L.n_experts + 1) * H * 4 + m * H * 4 + (norm ? H * 4 : 0), 0,
              nullptr);
    }
    {
        Prof p(ctx);
        hipError_t e = launch_gate_up(ctx->stream, L, m * (kTopK + 1), sc.plan, sc.xprep, sc.hprep);
        if (e != hipSuccess) return hip_fail(ctx, "gate/up kernel launch", e);
        p.end(TQF_HIP_KERNEL_GATE_UP, m * H * 4 + pairs * F * 4, 2 * q4_bytes(L.width, L.hidden),
              sc.plan);
    }
    {
        Prof p(ctx);
        hipError_t e = launch_down(ctx->stream, L, m, m * (kTopK + 1), sc, sc.plan, sc.hprep, resid, out);
        if (e != hipSuccess) return hip_fail(ctx, "down kernel launch", e);
        p.end(TQF_HIP_KERNEL_DOWN, pairs * F * 4 + m * H * 4 * (resid ? 2 : 1),
              q4_bytes(L.hidden, L.width), sc.plan);
    }
    return TQF_HIP_OK;
}

// Device views of the Q4_K layer's buffers in ctx->d_q4k, sized for m rows.
struct Q4KLayerBufs {
    float *gu, *dn;
    uint32_t *q8x, *q8h;
    size_t bytes;
};
Q4KLayerBufs q4k_layer_bufs(uint8_t *base, uint32_t H, uint32_t F, uint32_t m) {
    const uint32_t S = m * (kTopK + 1);
    const size_t qx = align_up((size_t)m * padded_blocks(H / 32) * kQ8KRecDwords * 4, kAlign);
    const size_t gu = align_up((size_t)2 * S * F * 4, kAlign);
    const size_t qh = align_up((size_t)S * padded_blocks(F / 32) * kQ8KRecDwords * 4, kAlign);
    const size_t dn = align_up((size_t)S * H * 4, kAlign);
    Q4KLayerBufs b;
    b.q8x = reinterpret_cast<uint32_t *>(base);
    b.gu = reinterpret_cast<float *>(base + qx);
    b.q8h = reinterpret_cast<uint32_t *>(base + qx + gu);
    b.dn = reinterpret_cast<float *>(base + qx + gu + qh);
    b.bytes = qx + gu + qh + dn;
    return b;
}

// Sized for kMaxTokens rows, so that a captured graph never needs to grow it.
int32_t ensure_q4k_layer_scratch(tqf_hip_ctx *ctx, uint32_t H, uint32_t F) {
    const size_t need = q4k_layer_bufs(nullptr, H, F, kMaxTokens).bytes;
    if (ctx->d_q4k && ctx->q4k_bytes >= need) return TQF_HIP_OK;
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    drop_graphs(ctx);
    TQF_HIP(ctx, grow(ctx->d_q4k, ctx->q4k_bytes, need));
    return TQF_HIP_OK;
}

// One MoE layer with Q4_K experts, every expert matvec on the Q8_K path of
// matvec_payload (weights.rs:680-735): route (with the RMSNorm and the Q8_K
// records of the rows) -> gate and up of all 9 M slots -> down of all slots
// (each workgroup first quantizes its slot's silu_mul(gate, up) in LDS) ->
// combine in route order (+ residual).  The caller has run
// ensure_moe_scratch and ensure_q4k_layer_scratch.
int32_t enqueue_layer_q4k(tqf_hip_ctx *ctx, const LayerDev &L, const float *h, const float *norm,
                          uint32_t m, const float *resid, float *out, uint16_t *ids, float *w,
                          int32_t *status) {
    Scratch &sc = ctx->scratch;
    const uint32_t H = L.hidden, F = L.width, S = m * (kTopK + 1);
    const MatrixDims dgu = matrix_dims(F, H), dd = matrix_dims(H, F);
    const Q4KLayerBufs b = q4k_layer_bufs(ctx->d_q4k, H, F, m);
    if (!ctx->d_q4k || ctx->q4k_bytes < b.bytes) return fail(ctx, TQF_HIP_ERR_INVALID, "Q4_K layer scratch missing");
    hipError_t e = hipSuccess;
    {
        Prof p(ctx);
        e = launch_route(ctx->stream, L, h, norm, m, sc, ids, w, status, false, b.q8x, dgu.blocks_padded);
        if (e != hipSuccess) return hip_fail(ctx, "route kernel launch", e);
        p.end(TQF_HIP_KERNEL_ROUTE, (L.n_experts + 1) * (double)H * 4 + m * (double)H * 4, 0, nullptr);
    }
    {
        Prof p(ctx);
        e = launch_q4k_q8k_slots(ctx->stream, sc.plan, S, false, dgu, b.q8x, b.gu);
        if (e != hipSuccess) return hip_fail(ctx, "Q4_K gate/up kernel launch", e);
        p.end(TQF_HIP_KERNEL_Q4K_MATVEC, 2.0 * S * ((double)F * H / 256 * kQ4KBlock + F * 4.0), 0, nullptr);
    }
    // the combine folded into the down launch; TQF_HIP_Q4K_FOLD=0 in the
    // environment keeps the separate combine launch (the same arithmetic)
    const bool fold = ctx->variant[TQF_HIP_VARIANT_Q4K_FOLD] != 0 && q4k_fold_ok(dd);
    {
        Prof p(ctx);
        e = fold ? launch_q4k_q8k_slots(ctx->stream, sc.plan, S, true, dd, nullptr, b.dn, b.gu, out, resid,
                                        sc.counters + counter_fold_offset(H))
                 : launch_q4k_q8k_slots(ctx->stream, sc.plan, S, true, dd, nullptr, b.dn, b.gu);
        if (e != hipSuccess) return hip_fail(ctx, "Q4_K down kernel launch", e);
        p.end(TQF_HIP_KERNEL_Q4K_MATVEC, S * ((double)F * H / 256 * kQ4KBlock + H * 4.0), 0, nullptr);
    }
    if (!fold) {
        e = launch_q4k_moe_combine(ctx->stream, sc.plan, b.dn, m, H, resid, out);
        if (e != hipSuccess) return hip_fail(ctx, "combine kernel launch", e);
    }
    return TQF_HIP_OK;
}

int32_t enqueue_moe(tqf_hip_ctx *ctx, const tqf_hip_layer *layer, const float *h, const float *norm,
                    uint32_t m, const float *resid, float *out, uint16_t *ids, float *w,
                    int32_t *status) {
    if (layer->format == TQF_HIP_FORMAT_Q4_K)
        return enqueue_layer_q4k(ctx, layer->dev, h, norm, m, resid, out, ids, w, status);
    return enqueue_layer(ctx, layer->dev, h, norm, m, resid, out, ids, w, status);
}

// Scratch of every kernel a layer's format runs (outside any graph capture).
int32_t ensure_layer_scratch(tqf_hip_ctx *ctx, const LayerDev &L, int32_t format) {
    if (int32_t rc = ensure_moe_scratch(ctx, L.hidden, L.width, L.n_experts)) return rc;
    if (format == TQF_HIP_FORMAT_Q4_K) return ensure_q4k_layer_scratch(ctx, L.hidden, L.width);
    return TQF_HIP_OK;
}

int32_t enqueue_stack(tqf_hip_ctx *ctx, const tqf_hip_stack *st, const float *d_h_in, float *d_h,
                      uint32_t m, uint16_t *d_ids, float *d_w, int32_t *d_status) {
    for (size_t l = 0; l < st->layers.size(); ++l) {
        uint16_t *ids = d_ids ? d_ids + l * (size_t)m * kTopK : nullptr;
        float *w = d_w ? d_w + l * (size_t)m * kTopK : nullptr;
        const float *in = (l == 0 && d_h_in) ? d_h_in : d_h;
        int32_t rc = enqueue_moe(ctx, st->layers[l], in, st->norms[l], m, in, d_h, ids, w, d_status);
        if (rc) return rc;
    }
    return TQF_HIP_OK;
}

// The persistent path: model geometry, m <= kStackMT, a device that can
// co-schedule one workgroup per CU.
bool stack_persistent_ok(tqf_hip_ctx *ctx, const tqf_hip_stack *st, uint32_t m) {
    if (!ctx->variant[TQF_HIP_VARIANT_PERSISTENT]) return false;
    if (st->format != TQF_HIP_FORMAT_Q4_0) return false;  // the persistent kernel reads Q4_0
    if (!st->d_layers || m > (uint32_t)kStackMT || st->hidden != (uint32_t)kStackHidden ||
        st->experts == 0 || st->experts > 256 || st->width % 256 || st->width > 2048)
        return false;
    const uint32_t bp_down = padded_blocks(st->width / 32);
    if (ctx->stack_grid == 0) ctx->stack_grid = stack_grid(ctx->device, bp_down);
    // phase A writes the activation records of block q from workgroup q / 2
    return ctx->stack_grid >= (uint32_t)kStackTeams && ctx->stack_grid >= (uint32_t)kStackMT * 32;
}

// recover: the launch reports an abort in the context's host flag (set to -1
// here, 0 or 1 by the launch's last workgroup) instead of TQF_HIP_ERR_DEVICE
// in d_status, and copies h_in to the stack scratch's h_save, from which
// rerun_stack restarts.
int32_t enqueue_stack_persistent(tqf_hip_ctx *ctx, const tqf_hip_stack *st, const float *d_h_in,
                                 float *d_h, uint32_t m, uint16_t *d_ids, float *d_w,
                                 int32_t *d_status, bool recover) {
    const uint32_t bp_down = padded_blocks(st->width / 32);
    const uint32_t grid = ctx->stack_grid;
    const uint32_t members = grid / kStackTeams;
    if (int32_t rc = ensure_stack_scratch(ctx, st->experts, bp_down, members)) return rc;
    const StackScratch &sc = ctx->stack;
    StackArgs a;
    a.layers = st->d_layers;
    a.n_layers = (uint32_t)st->layers.size();
    a.E = st->experts;
    a.F = st->width;
    a.m = m;
    a.h_in = d_h_in ? d_h_in : d_h;
    a.h = d_h;
    a.ids_out = d_ids;
    a.w_out = d_w;
    a.status = d_status;
    a.lacc = sc.lacc;
    a.xprep = sc.xprep;
    a.hprep = sc.hprep;
    a.hshared = sc.hshared;
    a.partial = sc.partial;
    a.ssq = sc.ssq;
    a.sync = sc.sync;
    a.members = members;
    a.dev_status = recover ? nullptr : d_status;
    a.h_save = sc.h_save;
    a.host_flag = recover ? ctx->d_flags + kFlagStack : nullptr;
    if (recover) ctx->h_flags[kFlagStack] = -1;  // no launch on this context is in flight
    // a barrier timeout forced from the host, for the tests of the abort path
    // (TQF_HIP_STACK_FAIL_AT_LAYER = l); read at every launch
    const char *fail_at = std::getenv("TQF_HIP_STACK_FAIL_AT_LAYER");
    a.fail_at = fail_at && *fail_at ? (uint32_t)std::strtoul(fail_at, nullptr, 10) : ~0u;
    Prof p(ctx);
    hipError_t e = launch_stack(ctx->stream, a, grid, bp_down);
    if (e != hipSuccess) return hip_fail(ctx, "persistent stack kernel launch", e);
    p.end(TQF_HIP_KERNEL_STACK, 0.0, 0.0, nullptr);
    return TQF_HIP_OK;
}

// recover: a timed-out one-launch acceptance reports in the context's host
// flag (zeroed here) as well as in *acc.  multi: the three-kernel path.
int32_t enqueue_accept(tqf_hip_ctx *ctx, const float *t, const float *d, const int32_t *dt,
                       uint32_t k, uint32_t vocab, float T, int32_t greedy, const float *u,
                       const float *ur, int32_t *acc, int32_t *tok, bool recover = false,
                       bool multi = false) {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    Prof p(ctx);
    if (recover) ctx->h_flags[kFlagAccept] = 0;
    hipError_t e = launch_accept(ctx->stream, t, d, dt, k, vocab, T, greedy, u, ur, acc, tok,
                                 ctx->scratch.accept, e0, e1, multi,
                                 recover ? ctx->d_flags + kFlagAccept : nullptr);
    if (e != hipSuccess) return hip_fail(ctx, "acceptance kernel launch", e);
    p.end(TQF_HIP_KERNEL_ACCEPT, (double)(greedy ? k + 1 : 2 * k + 1) * vocab * 4, 0, nullptr);
    return TQF_HIP_OK;
}

// Runs `enqueue` eagerly, or captures it once per key into a HIP graph and
// replays it.  Profiling forces eager execution so events bracket kernels;
// variant TQF_HIP_VARIANT_GRAPHS = 0 disables capture (eager launches of the
// same kernels), e.g. under tracing tools that do not follow graphs.
template <typename F>
int32_t run_graphed(tqf_hip_ctx *ctx, const std::vector<uint64_t> &key, F enqueue) {
    if (ctx->profiling || !ctx->variant[TQF_HIP_VARIANT_GRAPHS]) return enqueue();
    GraphEntry *g = find_graph(ctx, key);
    if (!g) {
        if (ctx->graphs.size() >= kMaxGraphs) {
            // the evicted graph may still be executing on the stream
            TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
            GraphEntry *old = ctx->graphs.front();
            (void)hipGraphExecDestroy(old->exec);
            (void)hipGraphDestroy(old->graph);
            delete old;
            ctx->graphs.erase(ctx->graphs.begin());
        }
        TQF_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
        ctx->capturing = true;
        int32_t rc = enqueue();
        ctx->capturing = false;
        hipGraph_t graph = nullptr;
        hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
        if (rc) {
            if (graph) (void)hipGraphDestroy(graph);
            return rc;
        }
        if (e != hipSuccess) return hip_fail(ctx, "hipStreamEndCapture", e);
        hipGraphExec_t exec = nullptr;
        e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            (void)hipGraphDestroy(graph);
            return hip_fail(ctx, "hipGraphInstantiate", e);
        }
        g = new GraphEntry{key, graph, exec};
        ctx->graphs.push_back(g);
    }
    TQF_HIP(ctx, hipGraphLaunch(g->exec, ctx->stream));
    return TQF_HIP_OK;
}

uint64_t k64(const void *p) { return (uint64_t)(uintptr_t)p; }

// ---- recovery from a timed-out persistent launch -----------------------------
// The persistent stack kernel and the one-launch acceptance need every
// workgroup resident at once.  When other work holds compute units, their
// waits time out after 20 ms and the launch aborts (TQF_HIP_ERR_DEVICE /
// accepted = -1).  With TQF_HIP_VARIANT_RECOVER (the default) the entry
// points that run one wait for it, read the flag the launch leaves in pinned
// host memory, and after an abort re-run the work through kernels that never
// wait on one another: the per-layer stack kernels from the copy of h_in the
// persistent prologue made, and the three-kernel acceptance.  The reruns are
// counted (tqf_hip_recovery_counts).  This is the GPU-side counterpart of the
// reference's fallback from a failed GPU path to a working one
// (experts/mod.rs:480-497).
bool recovering(const tqf_hip_ctx *ctx) {
    return ctx->variant[TQF_HIP_VARIANT_RECOVER] != 0 && ctx->d_flags != nullptr;
}

int32_t rerun_stack(tqf_hip_ctx *ctx, const tqf_hip_stack *st, float *d_h, uint32_t m, uint16_t *d_ids,
                    float *d_w, int32_t *d_status) {
    ++ctx->reruns[kFlagStack];
    if (int32_t rc = ensure_layer_scratch(ctx, st->layers[0]->dev, st->format)) return rc;
    const float *h_in = ctx->stack.h_save;
    std::vector<uint64_t> key = {3, k64(st), k64(h_in), k64(d_h), m, k64(d_ids), k64(d_w), k64(d_status)};
    return run_graphed(ctx, key, [&]() { return enqueue_stack(ctx, st, h_in, d_h, m, d_ids, d_w, d_status); });
}

int32_t rerun_accept(tqf_hip_ctx *ctx, const float *t, const float *d, const int32_t *dt, uint32_t k,
                     uint32_t vocab, float T, int32_t greedy, const float *u, const float *ur, int32_t *acc,
                     int32_t *tok) {
    ++ctx->reruns[kFlagAccept];
    if (int32_t rc = ensure_accept_scratch(ctx, accept_multi_scratch_bytes(k, vocab))) return rc;
    return enqueue_accept(ctx, t, d, dt, k, vocab, T, greedy, u, ur, acc, tok, false, true);
}

}  // namespace

// ===========================================================================
// context
// ===========================================================================
extern "C" int32_t tqf_hip_create(int32_t device, tqf_hip_ctx **out) {
    if (!out) return TQF_HIP_ERR_INVALID;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return TQF_HIP_ERR_DEVICE;
    if (device < 0 || device >= count) return TQF_HIP_ERR_INVALID;
    if (hipSetDevice(device) != hipSuccess) return TQF_HIP_ERR_DEVICE;
    tqf_hip_ctx *ctx = new tqf_hip_ctx();
    ctx->device = device;
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return TQF_HIP_ERR_DEVICE;
    }
    if (hipHostMalloc(reinterpret_cast<void **>(&ctx->prof_ring), kRingSize * sizeof(int32_t),
                      hipHostMallocDefault) != hipSuccess) {
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return TQF_HIP_ERR_NOMEM;
    }
    const size_t adhoc = align_up(3 * sizeof(void *), kAlign) + sizeof(Plan);
    uint8_t *p = nullptr;
    if (hipMalloc(&p, adhoc) != hipSuccess) {
        (void)hipHostFree(ctx->prof_ring);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return TQF_HIP_ERR_NOMEM;
    }
    ctx->d_adhoc_mats = reinterpret_cast<const uint8_t **>(p);
    ctx->d_adhoc_plan = reinterpret_cast<Plan *>(p + align_up(3 * sizeof(void *), kAlign));
    // set-up of the allocation-free entry point: this device's copy of
    // `scratch` (the device is current here)
    ctx->noalloc_scratch = noalloc_scratch_for(device);
    if (!ctx->noalloc_scratch) {
        (void)hipFree(p);
        (void)hipHostFree(ctx->prof_ring);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return TQF_HIP_ERR_DEVICE;
    }
    // the abort flags the persistent launches write for the host (recovery)
    if (hipHostMalloc(reinterpret_cast<void **>(&ctx->h_flags), 2 * sizeof(int32_t), hipHostMallocMapped) !=
            hipSuccess ||
        hipHostGetDevicePointer(reinterpret_cast<void **>(&ctx->d_flags), ctx->h_flags, 0) != hipSuccess) {
        (void)hipHostFree(ctx->h_flags);
        (void)hipFree(p);
        (void)hipHostFree(ctx->prof_ring);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return TQF_HIP_ERR_NOMEM;
    }
    ctx->h_flags[kFlagStack] = ctx->h_flags[kFlagAccept] = 0;
    tqf::accept_warm();  // device queries of the acceptance launch, outside any capture
    static const char *const kVariantEnv[TQF_HIP_VARIANTS] = {"TQF_HIP_PERSISTENT", "TQF_HIP_Q4K_FOLD",
                                                              "TQF_HIP_GRAPHS", "TQF_HIP_RECOVER"};
    for (int i = 0; i < TQF_HIP_VARIANTS; ++i) {
        const char *v = std::getenv(kVariantEnv[i]);
        ctx->variant[i] = (v && v[0] == '0') ? 0 : 1;
    }
    *out = ctx;
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_set_variant(tqf_hip_ctx *ctx, int32_t variant, int32_t value) {
    TQF_ENTER(ctx);
    if (variant < 0 || variant >= TQF_HIP_VARIANTS || (value != 0 && value != 1))
        return fail(ctx, TQF_HIP_ERR_INVALID, "unknown variant or value");
    if (ctx->variant[variant] == value) return TQF_HIP_OK;
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    drop_graphs(ctx);
    ctx->variant[variant] = value;
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_get_variant(tqf_hip_ctx *ctx, int32_t variant, int32_t *value) {
    TQF_ENTER(ctx);
    if (variant < 0 || variant >= TQF_HIP_VARIANTS || !value)
        return fail(ctx, TQF_HIP_ERR_INVALID, "unknown variant or null pointer");
    *value = ctx->variant[variant];
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_destroy(tqf_hip_ctx *ctx) {
    if (!ctx) return TQF_HIP_ERR_INVALID;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    drop_graphs(ctx);
    for (const ProfileSlot &p : ctx->prof_pending) {
        (void)hipEventDestroy(p.start);
        (void)hipEventDestroy(p.stop);
    }
    for (hipEvent_t e : ctx->event_pool) (void)hipEventDestroy(e);
    Scratch &sc = ctx->scratch;
    (void)hipFree(sc.xprep);
    (void)hipFree(sc.hprep);
    (void)hipFree(sc.logits);
    (void)hipFree(sc.plan);
    (void)hipFree(sc.partial);
    (void)hipFree(sc.counters);
    (void)hipFree(sc.accept);
    (void)hipFree(ctx->stack.sync);
    (void)hipFree(ctx->stack.lacc);
    (void)hipFree(ctx->stack.xprep);
    (void)hipFree(ctx->stack.hprep);
    (void)hipFree(ctx->stack.hshared);
    (void)hipFree(ctx->stack.partial);
    (void)hipFree(ctx->stack.ssq);
    (void)hipFree(ctx->stack.h_save);
    (void)hipFree(ctx->d_stage);
    (void)hipFree(ctx->d_table);
    (void)hipFree(ctx->d_gemv_xprep);
    (void)hipFree(ctx->d_q4k);
    (void)hipFree(ctx->d_lm);
    (void)hipFree(ctx->d_grouped);
    (void)hipFree(ctx->d_sample);
    (void)hipFree(const_cast<const uint8_t **>(ctx->d_adhoc_mats));
    for (Slab &s : ctx->slabs) (void)hipFree(s.base);
    (void)hipHostFree(ctx->prof_ring);
    (void)hipHostFree(ctx->h_flags);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return TQF_HIP_OK;
}

extern "C" const char *tqf_hip_last_error(const tqf_hip_ctx *ctx) {
    return ctx ? ctx->last_error.c_str() : "null context";
}

extern "C" int32_t tqf_hip_synchronize(tqf_hip_ctx *ctx) {
    TQF_ENTER(ctx);
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_device_info(tqf_hip_ctx *ctx, char *name, size_t name_len,
                                       int32_t *cu_count) {
    TQF_ENTER(ctx);
    hipDeviceProp_t prop;
    TQF_HIP(ctx, hipGetDeviceProperties(&prop, ctx->device));
    if (name && name_len) {
        std::snprintf(name, name_len, "%s (%s)", prop.name, prop.gcnArchName);
    }
    if (cu_count) *cu_count = prop.multiProcessorCount;
    return TQF_HIP_OK;
}

// ===========================================================================
// plain buffers
// ===========================================================================
extern "C" int32_t tqf_hip_buffer_alloc(tqf_hip_ctx *ctx, size_t bytes, void **dptr) {
    TQF_ENTER(ctx);
    if (!dptr) return fail(ctx, TQF_HIP_ERR_INVALID, "null output pointer");
    *dptr = nullptr;
    hipError_t e = hipMalloc(dptr, bytes ? bytes : 1);
    if (e != hipSuccess) {
        *dptr = nullptr;
        return fail(ctx, TQF_HIP_ERR_NOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
    }
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_buffer_free(tqf_hip_ctx *ctx, void *dptr) {
    TQF_ENTER(ctx);
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    TQF_HIP(ctx, hipFree(dptr));
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_memcpy_h2d(tqf_hip_ctx *ctx, void *dst, const void *src, size_t bytes) {
    TQF_ENTER(ctx);
    TQF_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_memcpy_d2h(tqf_hip_ctx *ctx, void *dst, const void *src, size_t bytes) {
    TQF_ENTER(ctx);
    TQF_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_memcpy_d2d(tqf_hip_ctx *ctx, void *dst, const void *src, size_t bytes) {
    TQF_ENTER(ctx);
    if (bytes == 0) return TQF_HIP_OK;
    if (!dst || !src) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    TQF_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return TQF_HIP_OK;
}

// ===========================================================================
// weights
// ===========================================================================
extern "C" uint64_t tqf_hip_weights_bytes_for(uint32_t rows, uint32_t cols) {
    if (rows == 0 || cols == 0 || cols % 32) return 0;
    return align_up(layout_bytes(matrix_dims(rows, cols)), kAlign) + kAlign;
}

namespace {
int32_t weights_alloc(tqf_hip_ctx *ctx, uint32_t rows, uint32_t cols, tqf_hip_weights **out,
                      int32_t format = TQF_HIP_FORMAT_Q4_0) {
    const MatrixDims d = matrix_dims(rows, cols);
    const size_t bytes = format == TQF_HIP_FORMAT_Q4_K   ? q4k_layout_bytes(d)
                         : format == TQF_HIP_FORMAT_Q6_K ? q6k_layout_bytes(d)
                                                         : layout_bytes(d);
    void *tiles = nullptr, *self = nullptr;
    hipError_t e = arena_alloc(ctx, bytes, &tiles);
    if (e != hipSuccess) return fail(ctx, TQF_HIP_ERR_NOMEM, "weights allocation failed");
    e = arena_alloc(ctx, sizeof(void *), &self);
    if (e != hipSuccess) {
        arena_free(ctx, tiles);
        return fail(ctx, TQF_HIP_ERR_NOMEM, "weights allocation failed");
    }
    const uint8_t *tp = static_cast<const uint8_t *>(tiles);
    e = hipMemsetAsync(tiles, 0, bytes, ctx->stream);
    if (e == hipSuccess) e = hipMemcpy(self, &tp, sizeof(void *), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        arena_free(ctx, self);
        arena_free(ctx, tiles);
        return hip_fail(ctx, "weights initialisation", e);
    }
    tqf_hip_weights *w = new tqf_hip_weights();
    w->dims = d;
    w->format = format;
    w->tiles = static_cast<uint8_t *>(tiles);
    w->bytes = bytes;
    w->d_self = static_cast<const uint8_t **>(self);
    *out = w;
    return TQF_HIP_OK;
}

void weights_release(tqf_hip_ctx *ctx, tqf_hip_weights *w) {
    arena_free(ctx, const_cast<const uint8_t **>(w->d_self));
    arena_free(ctx, w->tiles);
    delete w;
}

int32_t check_q4_shape(tqf_hip_ctx *ctx, size_t len, uint32_t rows, uint32_t cols) {
    if (rows == 0 || cols == 0 || cols % 32)
        return fail(ctx, TQF_HIP_ERR_INVALID, "Q4_0 matrix needs rows > 0 and cols a positive multiple of 32");
    if (len != (size_t)rows * (cols / 32) * kQ4Block)
        return fail(ctx, TQF_HIP_ERR_INVALID, "Q4_0 byte length does not match rows x cols");
    return TQF_HIP_OK;
}
}  // namespace

extern "C" int32_t tqf_hip_weights_upload(tqf_hip_ctx *ctx, const uint8_t *q4_0, size_t len,
                                          uint32_t rows, uint32_t cols, tqf_hip_weights **out) {
    TQF_ENTER(ctx);
    if (!q4_0 || !out) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    *out = nullptr;
    if (int32_t rc = check_q4_shape(ctx, len, rows, cols)) return rc;
    if (int32_t rc = ensure_stage(ctx, len)) return rc;
    tqf_hip_weights *w = nullptr;
    if (int32_t rc = weights_alloc(ctx, rows, cols, &w)) return rc;
    hipError_t e = hipMemcpyAsync(ctx->d_stage, q4_0, len, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess)
        e = launch_repack(ctx->stream, static_cast<const uint8_t *>(ctx->d_stage), w->dims, w->tiles);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        weights_release(ctx, w);
        return hip_fail(ctx, "weights upload", e);
    }
    *out = w;
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_weights_upload_device(tqf_hip_ctx *ctx, const void *d_q4_0, size_t len,
                                                 uint32_t rows, uint32_t cols,
                                                 tqf_hip_weights **out) {
    TQF_ENTER(ctx);
    if (!d_q4_0 || !out) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    *out = nullptr;
    if (int32_t rc = check_q4_shape(ctx, len, rows, cols)) return rc;
    tqf_hip_weights *w = nullptr;
    if (int32_t rc = weights_alloc(ctx, rows, cols, &w)) return rc;
    hipError_t e = launch_repack(ctx->stream, static_cast<const uint8_t *>(d_q4_0), w->dims, w->tiles);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        weights_release(ctx, w);
        return hip_fail(ctx, "weights upload", e);
    }
    *out = w;
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_weights_synth_recipe(tqf_hip_ctx *ctx, uint32_t rows, uint32_t cols,
                                                uint32_t tensor_id, uint32_t seed, uint32_t recipe,
                                                tqf_hip_weights **out) {
    TQF_ENTER(ctx);
    if (!out) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    *out = nullptr;
    if (rows == 0 || cols == 0 || cols % 32)
        return fail(ctx, TQF_HIP_ERR_INVALID, "Q4_0 matrix needs cols a positive multiple of 32");
    if (recipe != TQF_HIP_SYNTH_UNIFORM && recipe != TQF_HIP_SYNTH_ZERO_MEAN)
        return fail(ctx, TQF_HIP_ERR_INVALID, "unknown synthetic recipe");
    tqf_hip_weights *w = nullptr;
    if (int32_t rc = weights_alloc(ctx, rows, cols, &w)) return rc;
    hipError_t e = launch_synth_q4_0(ctx->stream, w->dims, tensor_id, seed, recipe, w->tiles);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        weights_release(ctx, w);
        return hip_fail(ctx, "synthetic weights", e);
    }
    *out = w;
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_weights_synth(tqf_hip_ctx *ctx, uint32_t rows, uint32_t cols,
                                         uint32_t tensor_id, uint32_t seed, tqf_hip_weights **out) {
    return tqf_hip_weights_synth_recipe(ctx, rows, cols, tensor_id, seed, TQF_HIP_SYNTH_UNIFORM, out);
}

extern "C" int32_t tqf_hip_weights_download(tqf_hip_ctx *ctx, const tqf_hip_weights *w,
                                            uint8_t *q4_0, size_t len) {
    TQF_ENTER(ctx);
    if (!valid_weights(w) || !q4_0) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    const MatrixDims &d = w->dims;
    const uint32_t blocks = d.cols / 32;
    if (len != (size_t)d.rows * blocks * kQ4Block)
        return fail(ctx, TQF_HIP_ERR_INVALID, "Q4_0 byte length does not match the matrix");
    std::vector<uint8_t> tiles(w->bytes);
    TQF_HIP(ctx, hipMemcpyAsync(tiles.data(), w->tiles, w->bytes, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (uint32_t r = 0; r < d.rows; ++r) {
        for (uint32_t b = 0; b < blocks; ++b) {
            uint8_t *dst = q4_0 + ((size_t)r * blocks + b) * kQ4Block;
            std::memcpy(dst, tiles.data() + scale_offset(d, r, b), 2);
            std::memcpy(dst + 2, tiles.data() + nibble_offset(d, r, b), 16);
        }
    }
    return TQF_HIP_OK;
}

extern "C" uint64_t tqf_hip_weights_bytes(const tqf_hip_weights *w) { return w ? w->bytes : 0; }

extern "C" int32_t tqf_hip_weights_free(tqf_hip_ctx *ctx, tqf_hip_weights *w) {
    TQF_ENTER(ctx);
    if (!w) return TQF_HIP_OK;
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    drop_graphs(ctx);
    weights_release(ctx, w);
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_tensor_upload(tqf_hip_ctx *ctx, const float *data, size_t count,
                                         tqf_hip_tensor **out) {
    TQF_ENTER(ctx);
    if (!data || !out || count == 0) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer or empty tensor");
    *out = nullptr;
    void *p = nullptr;
    if (arena_alloc(ctx, count * sizeof(float), &p) != hipSuccess)
        return fail(ctx, TQF_HIP_ERR_NOMEM, "tensor allocation failed");
    hipError_t e = hipMemcpyAsync(p, data, count * sizeof(float), hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        arena_free(ctx, p);
        return hip_fail(ctx, "tensor upload", e);
    }
    *out = new tqf_hip_tensor{static_cast<float *>(p), count};
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_tensor_free(tqf_hip_ctx *ctx, tqf_hip_tensor *t) {
    TQF_ENTER(ctx);
    if (!t) return TQF_HIP_OK;
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    drop_graphs(ctx);
    arena_free(ctx, t->data);
    delete t;
    return TQF_HIP_OK;
}

// ===========================================================================
// GEMV
// ===========================================================================
namespace {
// Device table of `count` matrices (same shape, one format) for batched
// launches; rewritten only when the list changes.
int32_t set_table(tqf_hip_ctx *ctx, const tqf_hip_weights *const *ws, uint32_t count,
                  bool (*valid)(const tqf_hip_weights *)) {
    if (count > 65535) return fail(ctx, TQF_HIP_ERR_INVALID, "count must be <= 65535");
    std::vector<const uint8_t *> table(count);
    for (uint32_t i = 0; i < count; ++i) {
        if (!valid(ws[i])) return fail(ctx, TQF_HIP_ERR_INVALID, "null or wrong-format weights in batch");
        if (ws[i]->dims.rows != ws[0]->dims.rows || ws[i]->dims.cols != ws[0]->dims.cols)
            return fail(ctx, TQF_HIP_ERR_INVALID, "batched matrices must share one shape");
        table[i] = ws[i]->tiles;
    }
    if (table != ctx->table_shadow) {
        TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
        drop_graphs(ctx);
        TQF_HIP(ctx, grow(ctx->d_table, ctx->table_cap, count * sizeof(void *)));
        TQF_HIP(ctx, hipMemcpy(ctx->d_table, table.data(), count * sizeof(void *), hipMemcpyHostToDevice));
        ctx->table_shadow = table;
    }
    return TQF_HIP_OK;
}

int32_t gemv_enqueue(tqf_hip_ctx *ctx, const uint8_t *const *table, uint32_t count,
                     const MatrixDims &d, const float *d_x, uint32_t m, float *d_y) {
    const uint32_t bp = d.blocks_padded;
    const size_t xb = (size_t)m * bp * kXprepDwords * 4;
    if (!ctx->d_gemv_xprep || ctx->gemv_xprep_bytes < xb) {
        TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
        drop_graphs(ctx);
        TQF_HIP(ctx, grow(ctx->d_gemv_xprep, ctx->gemv_xprep_bytes, xb));
    }
    hipError_t e = launch_prep(ctx->stream, d_x, m, d.cols, bp, ctx->d_gemv_xprep);
    if (e != hipSuccess) return hip_fail(ctx, "prep kernel launch", e);
    Prof p(ctx);
    e = launch_gemv(ctx->stream, table, count, d, ctx->d_gemv_xprep, m, d_y);
    if (e != hipSuccess) return hip_fail(ctx, "gemv kernel launch", e);
    p.end(TQF_HIP_KERNEL_GEMV,
          (double)count * (q4_bytes(d.rows, d.cols) + (double)m * d.rows * 4) + (double)m * d.cols * 4,
          0, nullptr);
    return TQF_HIP_OK;
}
}  // namespace

extern "C" int32_t tqf_hip_q4_gemv(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *x,
                                   uint32_t m, float *y) {
    TQF_ENTER(ctx);
    if (!valid_weights(w) || !x || !y) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (m == 0 || m > kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "m must be in 1..8");
    const MatrixDims &d = w->dims;
    const size_t xb = (size_t)m * d.cols * 4, yb = (size_t)m * d.rows * 4;
    if (int32_t rc = ensure_stage(ctx, align_up(xb, kAlign) + yb)) return rc;
    float *dx = static_cast<float *>(ctx->d_stage);
    float *dy = reinterpret_cast<float *>(static_cast<uint8_t *>(ctx->d_stage) + align_up(xb, kAlign));
    TQF_HIP(ctx, hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, ctx->stream));
    if (int32_t rc = gemv_enqueue(ctx, w->d_self, 1, d, dx, m, dy)) return rc;
    TQF_HIP(ctx, hipMemcpyAsync(y, dy, yb, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_q4_gemv_device(tqf_hip_ctx *ctx, const tqf_hip_weights *w,
                                          const float *d_x, uint32_t m, float *d_y) {
    TQF_ENTER(ctx);
    if (!valid_weights(w) || !d_x || !d_y) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (m == 0 || m > kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "m must be in 1..8");
    return gemv_enqueue(ctx, w->d_self, 1, w->dims, d_x, m, d_y);
}

extern "C" int32_t tqf_hip_q4_gemv_batched_device(tqf_hip_ctx *ctx,
                                                  const tqf_hip_weights *const *ws, uint32_t count,
                                                  const float *d_x, float *d_y) {
    TQF_ENTER(ctx);
    if (!ws || !d_x || !d_y || count == 0) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer or count 0");
    if (int32_t rc = set_table(ctx, ws, count, valid_weights)) return rc;
    return gemv_enqueue(ctx, ctx->d_table, count, ws[0]->dims, d_x, 1, d_y);
}

// ===========================================================================
// Q4_K
// ===========================================================================
namespace {
double q4k_bytes_of(uint32_t rows, uint32_t cols) { return (double)rows * (cols / 256) * kQ4KBlock; }

int32_t check_q4k_shape(tqf_hip_ctx *ctx, size_t len, uint32_t rows, uint32_t cols) {
    if (rows == 0 || cols == 0 || cols % 256)
        return fail(ctx, TQF_HIP_ERR_INVALID, "Q4_K matrix needs rows > 0 and cols a positive multiple of 256");
    if (len != (size_t)rows * (cols / 256) * kQ4KBlock)
        return fail(ctx, TQF_HIP_ERR_INVALID, "Q4_K byte length does not match rows x cols");
    return TQF_HIP_OK;
}

int32_t q4k_upload_from(tqf_hip_ctx *ctx, const uint8_t *d_src, uint32_t rows, uint32_t cols,
                        tqf_hip_weights **out) {
    tqf_hip_weights *w = nullptr;
    if (int32_t rc = weights_alloc(ctx, rows, cols, &w, TQF_HIP_FORMAT_Q4_K)) return rc;
    hipError_t e = launch_q4k_repack(ctx->stream, d_src, w->dims, w->tiles);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        weights_release(ctx, w);
        return hip_fail(ctx, "Q4_K weights upload", e);
    }
    *out = w;
    return TQF_HIP_OK;
}

// Grows the shared record buffer to `bytes` (synchronising first, as a
// resize may free memory an earlier launch still reads).
int32_t ensure_gemv_records(tqf_hip_ctx *ctx, size_t bytes) {
    if (ctx->d_gemv_xprep && ctx->gemv_xprep_bytes >= bytes) return TQF_HIP_OK;
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    drop_graphs(ctx);
    TQF_HIP(ctx, grow(ctx->d_gemv_xprep, ctx->gemv_xprep_bytes, bytes));
    return TQF_HIP_OK;
}

int32_t q4k_gemv_enqueue(tqf_hip_ctx *ctx, const uint8_t *const *table, uint32_t count,
                         const MatrixDims &d, const float *d_x, uint32_t m, float *d_y) {
    const uint32_t bp = d.blocks_padded;
    if (int32_t rc = ensure_gemv_records(ctx, (size_t)m * bp * kXprepDwords * 4)) return rc;
    hipError_t e = launch_q4k_prep(ctx->stream, d_x, m, d.cols, bp, ctx->d_gemv_xprep);
    if (e != hipSuccess) return hip_fail(ctx, "Q4_K prep kernel launch", e);
    Prof p(ctx);
    e = launch_q4k_gemv(ctx->stream, table, count, d, ctx->d_gemv_xprep, m, d_y);
    if (e != hipSuccess) return hip_fail(ctx, "Q4_K gemv kernel launch", e);
    p.end(TQF_HIP_KERNEL_Q4K_GEMV,
          (double)count * (q4k_bytes_of(d.rows, d.cols) + (double)m * d.rows * 4) + (double)m * d.cols * 4,
          0, nullptr);
    return TQF_HIP_OK;
}

int32_t q4k_matvec_enqueue(tqf_hip_ctx *ctx, const uint8_t *const *table, uint32_t count,
                           const MatrixDims &d, const float *d_x, uint32_t m, float *d_y) {
    const uint32_t bp = d.blocks_padded;
    if (int32_t rc = ensure_gemv_records(ctx, (size_t)m * bp * kQ8KRecDwords * 4)) return rc;
    hipError_t e = launch_q8k_quantize(ctx->stream, d_x, m, d.cols, bp, ctx->d_gemv_xprep);
    if (e != hipSuccess) return hip_fail(ctx, "Q8_K quantize kernel launch", e);
    Prof p(ctx);
    e = launch_q4k_q8k_gemv(ctx->stream, table, count, d, ctx->d_gemv_xprep, m, d_y);
    if (e != hipSuccess) return hip_fail(ctx, "Q4_K matvec kernel launch", e);
    p.end(TQF_HIP_KERNEL_Q4K_MATVEC,
          (double)count * (q4k_bytes_of(d.rows, d.cols) + (double)m * d.rows * 4) + (double)m * d.cols * 4,
          0, nullptr);
    return TQF_HIP_OK;
}

using Q4kEnqueue = int32_t (*)(tqf_hip_ctx *, const uint8_t *const *, uint32_t, const MatrixDims &,
                               const float *, uint32_t, float *);

// Host-pointer form: stage x, run, copy y back, wait.
int32_t q4k_host_call(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *x, uint32_t m,
                      float *y, Q4kEnqueue enqueue) {
    if (!valid_q4k(w) || !x || !y) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer or not Q4_K weights");
    if (m == 0 || m > kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "m must be in 1..8");
    const MatrixDims &d = w->dims;
    const size_t xb = (size_t)m * d.cols * 4, yb = (size_t)m * d.rows * 4;
    if (int32_t rc = ensure_stage(ctx, align_up(xb, kAlign) + yb)) return rc;
    float *dx = static_cast<float *>(ctx->d_stage);
    float *dy = reinterpret_cast<float *>(static_cast<uint8_t *>(ctx->d_stage) + align_up(xb, kAlign));
    TQF_HIP(ctx, hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, ctx->stream));
    if (int32_t rc = enqueue(ctx, w->d_self, 1, d, dx, m, dy)) return rc;
    TQF_HIP(ctx, hipMemcpyAsync(y, dy, yb, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TQF_HIP_OK;
}
}  // namespace

extern "C" uint64_t tqf_hip_q4k_weights_bytes_for(uint32_t rows, uint32_t cols) {
    if (rows == 0 || cols == 0 || cols % 256) return 0;
    return align_up(q4k_layout_bytes(matrix_dims(rows, cols)), kAlign) + kAlign;
}

extern "C" int32_t tqf_hip_q4k_weights_upload(tqf_hip_ctx *ctx, const uint8_t *q4_k, size_t len,
                                              uint32_t rows, uint32_t cols,
                                              tqf_hip_weights **out) {
    TQF_ENTER(ctx);
    if (!q4_k || !out) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    *out = nullptr;
    if (int32_t rc = check_q4k_shape(ctx, len, rows, cols)) return rc;
    if (int32_t rc = ensure_stage(ctx, len)) return rc;
    TQF_HIP(ctx, hipMemcpyAsync(ctx->d_stage, q4_k, len, hipMemcpyHostToDevice, ctx->stream));
    return q4k_upload_from(ctx, static_cast<const uint8_t *>(ctx->d_stage), rows, cols, out);
}

extern "C" int32_t tqf_hip_q4k_weights_upload_device(tqf_hip_ctx *ctx, const void *d_q4_k,
                                                     size_t len, uint32_t rows, uint32_t cols,
                                                     tqf_hip_weights **out) {
    TQF_ENTER(ctx);
    if (!d_q4_k || !out) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    *out = nullptr;
    if (int32_t rc = check_q4k_shape(ctx, len, rows, cols)) return rc;
    return q4k_upload_from(ctx, static_cast<const uint8_t *>(d_q4_k), rows, cols, out);
}

extern "C" int32_t tqf_hip_q4k_weights_download(tqf_hip_ctx *ctx, const tqf_hip_weights *w,
                                                uint8_t *q4_k, size_t len) {
    TQF_ENTER(ctx);
    if (!valid_q4k(w) || !q4_k) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer or not Q4_K weights");
    const MatrixDims &d = w->dims;
    const uint32_t nb = d.cols / 256;
    if (len != (size_t)d.rows * nb * kQ4KBlock)
        return fail(ctx, TQF_HIP_ERR_INVALID, "Q4_K byte length does not match the matrix");
    std::vector<uint8_t> tiles(w->bytes);
    TQF_HIP(ctx, hipMemcpyAsync(tiles.data(), w->tiles, w->bytes, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (uint32_t r = 0; r < d.rows; ++r) {
        for (uint32_t s = 0; s < nb; ++s) {
            uint8_t *dst = q4_k + ((size_t)r * nb + s) * kQ4KBlock;
            std::memcpy(dst, tiles.data() + q4k_dm_offset(d, r, s), 4);
            uint32_t sc[8], mn[8];
            for (int j = 0; j < 8; ++j) {
                const uint8_t *p = tiles.data() + scale_offset(d, q4k_slot_row(r, s * 8 + j), s * 8 + j);
                sc[j] = p[0];
                mn[j] = p[1];
            }
            // the 12-byte packing that q4_k_scale_min (weights.rs:933-942) unpacks
            for (int i = 0; i < 4; ++i) {
                dst[4 + i] = (uint8_t)(sc[i] | ((sc[i + 4] >> 4) << 6));
                dst[8 + i] = (uint8_t)(mn[i] | ((mn[i + 4] >> 4) << 6));
                dst[12 + i] = (uint8_t)((sc[i + 4] & 15) | ((mn[i + 4] & 15) << 4));
            }
            for (int j = 0; j < 8; ++j) {
                const uint8_t *nib = tiles.data() + nibble_offset(d, q4k_slot_row(r, s * 8 + j), s * 8 + j);
                uint8_t q[32];
                for (int i = 0; i < 4; ++i)
                    for (int t = 0; t < 4; ++t) {
                        q[2 * i + 8 * t] = nib[4 * i + t] & 15;
                        q[2 * i + 1 + 8 * t] = nib[4 * i + t] >> 4;
                    }
                uint8_t *qs = dst + 16 + 32 * (j >> 1);
                for (int e = 0; e < 32; ++e)
                    qs[e] = (j & 1) ? (uint8_t)((qs[e] & 15) | (q[e] << 4)) : q[e];
            }
        }
    }
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_q4k_gemv(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *x,
                                    uint32_t m, float *y) {
    TQF_ENTER(ctx);
    return q4k_host_call(ctx, w, x, m, y, q4k_gemv_enqueue);
}

extern "C" int32_t tqf_hip_q4k_gemv_device(tqf_hip_ctx *ctx, const tqf_hip_weights *w,
                                           const float *d_x, uint32_t m, float *d_y) {
    TQF_ENTER(ctx);
    if (!valid_q4k(w) || !d_x || !d_y) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer or not Q4_K weights");
    if (m == 0 || m > kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "m must be in 1..8");
    return q4k_gemv_enqueue(ctx, w->d_self, 1, w->dims, d_x, m, d_y);
}

extern "C" int32_t tqf_hip_q4k_gemv_batched_device(tqf_hip_ctx *ctx,
                                                   const tqf_hip_weights *const *ws,
                                                   uint32_t count, const float *d_x, float *d_y) {
    TQF_ENTER(ctx);
    if (!ws || !d_x || !d_y || count == 0) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer or count 0");
    if (int32_t rc = set_table(ctx, ws, count, valid_q4k)) return rc;
    return q4k_gemv_enqueue(ctx, ctx->d_table, count, ws[0]->dims, d_x, 1, d_y);
}

extern "C" int32_t tqf_hip_q4k_matvec(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *x,
                                      uint32_t m, float *y) {
    TQF_ENTER(ctx);
    return q4k_host_call(ctx, w, x, m, y, q4k_matvec_enqueue);
}

extern "C" int32_t tqf_hip_q4k_matvec_device(tqf_hip_ctx *ctx, const tqf_hip_weights *w,
                                             const float *d_x, uint32_t m, float *d_y) {
    TQF_ENTER(ctx);
    if (!valid_q4k(w) || !d_x || !d_y) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer or not Q4_K weights");
    if (m == 0 || m > kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "m must be in 1..8");
    return q4k_matvec_enqueue(ctx, w->d_self, 1, w->dims, d_x, m, d_y);
}

extern "C" int32_t tqf_hip_q4k_matvec_batched_device(tqf_hip_ctx *ctx,
                                                     const tqf_hip_weights *const *ws,
                                                     uint32_t count, const float *d_x,
                                                     float *d_y) {
    TQF_ENTER(ctx);
    if (!ws || !d_x || !d_y || count == 0) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer or count 0");
    if (int32_t rc = set_table(ctx, ws, count, valid_q4k)) return rc;
    return q4k_matvec_enqueue(ctx, ctx->d_table, count, ws[0]->dims, d_x, 1, d_y);
}

namespace {
// One Q4_K expert over m rows: Q8_K(x) -> gate, up -> silu_mul -> Q8_K(h)
// -> down, every matvec with q4_k_dot_pre's arithmetic.
int32_t q4k_expert_enqueue(tqf_hip_ctx *ctx, const tqf_hip_weights *gate,
                           const tqf_hip_weights *up, const tqf_hip_weights *down,
                           const float *d_x, uint32_t m, float *d_y) {
    const MatrixDims &dg = gate->dims, &dd = down->dims;
    const uint32_t F = dg.rows, H = dg.cols;
    const size_t qx = align_up((size_t)m * dg.blocks_padded * kQ8KRecDwords * 4, kAlign);
    const size_t qh = align_up((size_t)m * dd.blocks_padded * kQ8KRecDwords * 4, kAlign);
    const size_t gu = align_up((size_t)2 * m * F * 4, kAlign);
    const size_t need = qx + qh + gu;
    if (!ctx->d_q4k || ctx->q4k_bytes < need) {
        TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
        drop_graphs(ctx);
        TQF_HIP(ctx, grow(ctx->d_q4k, ctx->q4k_bytes, need));
    }
    uint32_t *q8x = reinterpret_cast<uint32_t *>(ctx->d_q4k);
    uint32_t *q8h = reinterpret_cast<uint32_t *>(ctx->d_q4k + qx);
    float *dgu = reinterpret_cast<float *>(ctx->d_q4k + qx + qh);
    hipError_t e = launch_q8k_quantize(ctx->stream, d_x, m, H, dg.blocks_padded, q8x);
    if (e == hipSuccess) e = launch_q4k_q8k_gemv(ctx->stream, gate->d_self, 1, dg, q8x, m, dgu);
    if (e == hipSuccess)
        e = launch_q4k_q8k_gemv(ctx->stream, up->d_self, 1, up->dims, q8x, m, dgu + (size_t)m * F);
    if (e == hipSuccess) e = launch_q8k_swiglu_quantize(ctx->stream, dgu, m, F, dd.blocks_padded, q8h);
    if (e == hipSuccess) e = launch_q4k_q8k_gemv(ctx->stream, down->d_self, 1, dd, q8h, m, d_y);
    if (e != hipSuccess) return hip_fail(ctx, "Q4_K expert kernels", e);
    (void)H;
    return TQF_HIP_OK;
}

int32_t check_q4k_expert(tqf_hip_ctx *ctx, const tqf_hip_weights *gate, const tqf_hip_weights *up,
                         const tqf_hip_weights *down, uint32_t m) {
    if (!valid_q4k(gate) || !valid_q4k(up) || !valid_q4k(down))
        return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer or not Q4_K weights");
    if (m == 0 || m > kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "m must be in 1..8");
    const uint32_t F = gate->dims.rows, H = gate->dims.cols;
    if (up->dims.rows != F || up->dims.cols != H || down->dims.rows != H || down->dims.cols != F)
        return fail(ctx, TQF_HIP_ERR_INVALID, "expert shapes: gate/up [width x hidden], down [hidden x width]");
    return TQF_HIP_OK;
}
}  // namespace

extern "C" int32_t tqf_hip_q4k_expert_forward(tqf_hip_ctx *ctx, const tqf_hip_weights *gate,
                                              const tqf_hip_weights *up,
                                              const tqf_hip_weights *down, const float *x,
                                              uint32_t m, float *y) {
    TQF_ENTER(ctx);
    if (!x || !y) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (int32_t rc = check_q4k_expert(ctx, gate, up, down, m)) return rc;
    const size_t xb = (size_t)m * gate->dims.cols * 4;
    if (int32_t rc = ensure_stage(ctx, 2 * align_up(xb, kAlign))) return rc;
    float *dx = static_cast<float *>(ctx->d_stage);
    float *dy = reinterpret_cast<float *>(static_cast<uint8_t *>(ctx->d_stage) + align_up(xb, kAlign));
    TQF_HIP(ctx, hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, ctx->stream));
    if (int32_t rc = q4k_expert_enqueue(ctx, gate, up, down, dx, m, dy)) return rc;
    TQF_HIP(ctx, hipMemcpyAsync(y, dy, xb, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_q4k_expert_forward_device(tqf_hip_ctx *ctx,
                                                     const tqf_hip_weights *gate,
                                                     const tqf_hip_weights *up,
                                                     const tqf_hip_weights *down,
                                                     const float *d_x, uint32_t m, float *d_y) {
    TQF_ENTER(ctx);
    if (!d_x || !d_y) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (int32_t rc = check_q4k_expert(ctx, gate, up, down, m)) return rc;
    return q4k_expert_enqueue(ctx, gate, up, down, d_x, m, d_y);
}

// ===========================================================================
// Q6_K and the LM head
// ===========================================================================
namespace {
double q6k_bytes_of(uint32_t rows, uint32_t cols) { return (double)rows * (cols / 256) * kQ6KBlock; }

int32_t check_q6k_shape(tqf_hip_ctx *ctx, size_t len, uint32_t rows, uint32_t cols) {
    if (rows == 0 || cols == 0 || cols % 256)
        return fail(ctx, TQF_HIP_ERR_INVALID, "Q6_K matrix needs rows > 0 and cols a positive multiple of 256");
    if (len != (size_t)rows * (cols / 256) * kQ6KBlock)
        return fail(ctx, TQF_HIP_ERR_INVALID, "Q6_K byte length does not match rows x cols");
    return TQF_HIP_OK;
}

int32_t q6k_upload_from(tqf_hip_ctx *ctx, const uint8_t *d_src, uint32_t rows, uint32_t cols,
                        tqf_hip_weights **out) {
    tqf_hip_weights *w = nullptr;
    if (int32_t rc = weights_alloc(ctx, rows, cols, &w, TQF_HIP_FORMAT_Q6_K)) return rc;
    hipError_t e = launch_q6k_repack(ctx->stream, d_src, w->dims, w->tiles);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        weights_release(ctx, w);
        return hip_fail(ctx, "Q6_K weights upload", e);
    }
    *out = w;
    return TQF_HIP_OK;
}

// Q8_K records of x, then the matvec (with the top-4 candidates when tokens4
// is given).  Scratch: [records | candidates] in ctx->d_lm.
int32_t q6k_enqueue(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *d_x, uint32_t m,
                    float *d_y, uint32_t *d_tokens4, float *d_logits4) {
    const MatrixDims &d = w->dims;
    const size_t rec = align_up((size_t)m * d.blocks_padded * kQ8KRecDwords * 4, kAlign);
    const size_t cand = d_tokens4 ? q6k_top4_scratch_bytes(d, m) : 0;
    if (!ctx->d_lm || ctx->lm_bytes < rec + cand) {
        TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
        drop_graphs(ctx);
        TQF_HIP(ctx, grow(ctx->d_lm, ctx->lm_bytes, rec + cand));
    }
    uint32_t *q8 = reinterpret_cast<uint32_t *>(ctx->d_lm);
    hipError_t e = launch_q8k_quantize(ctx->stream, d_x, m, d.cols, d.blocks_padded, q8);
    if (e != hipSuccess) return hip_fail(ctx, "Q8_K quantize kernel launch", e);
    Prof p(ctx);
    e = launch_q6k_q8k_gemv(ctx->stream, w->d_self, 1, d, q8, m, d_y,
                            d_tokens4 ? ctx->d_lm + rec : nullptr, d_tokens4, d_logits4);
    if (e != hipSuccess) return hip_fail(ctx, "Q6_K matvec kernel launch", e);
    p.end(TQF_HIP_KERNEL_Q6K_MATVEC,
          q6k_bytes_of(d.rows, d.cols) + (double)m * d.rows * 4 + (double)m * d.cols * 4, 0, nullptr);
    return TQF_HIP_OK;
}

int32_t check_q6k_call(tqf_hip_ctx *ctx, const tqf_hip_weights *w, uint32_t m) {
    if (!valid_q6k(w)) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer or not Q6_K weights");
    if (m == 0 || m > kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "m must be in 1..8");
    return TQF_HIP_OK;
}

int32_t q6k_host_call(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *x, uint32_t m,
                      float *y, uint32_t *tokens4, float *logits4) {
    if (!x || !y || (!tokens4) != (!logits4)) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (int32_t rc = check_q6k_call(ctx, w, m)) return rc;
    const MatrixDims &d = w->dims;
    const size_t xb = (size_t)m * d.cols * 4, yb = (size_t)m * d.rows * 4, cb = (size_t)m * 16;
    if (int32_t rc = ensure_stage(ctx, align_up(xb, kAlign) + align_up(yb, kAlign) + 2 * cb)) return rc;
    uint8_t *st = static_cast<uint8_t *>(ctx->d_stage);
    float *dx = reinterpret_cast<float *>(st);
    float *dy = reinterpret_cast<float *>(st + align_up(xb, kAlign));
    uint32_t *dt = reinterpret_cast<uint32_t *>(st + align_up(xb, kAlign) + align_up(yb, kAlign));
    float *dl = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(dt) + cb);
    TQF_HIP(ctx, hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, ctx->stream));
    if (int32_t rc = q6k_enqueue(ctx, w, dx, m, dy, tokens4 ? dt : nullptr, tokens4 ? dl : nullptr)) return rc;
    TQF_HIP(ctx, hipMemcpyAsync(y, dy, yb, hipMemcpyDeviceToHost, ctx->stream));
    if (tokens4) {
        TQF_HIP(ctx, hipMemcpyAsync(tokens4, dt, cb, hipMemcpyDeviceToHost, ctx->stream));
        TQF_HIP(ctx, hipMemcpyAsync(logits4, dl, cb, hipMemcpyDeviceToHost, ctx->stream));
    }
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TQF_HIP_OK;
}
}  // namespace

extern "C" uint64_t tqf_hip_q6k_weights_bytes_for(uint32_t rows, uint32_t cols) {
    if (rows == 0 || cols == 0 || cols % 256) return 0;
    return align_up(q6k_layout_bytes(matrix_dims(rows, cols)), kAlign) + kAlign;
}

extern "C" int32_t tqf_hip_q6k_weights_upload(tqf_hip_ctx *ctx, const uint8_t *q6_k, size_t len,
                                              uint32_t rows, uint32_t cols,
                                              tqf_hip_weights **out) {
    TQF_ENTER(ctx);
    if (!q6_k || !out) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    *out = nullptr;
    if (int32_t rc = check_q6k_shape(ctx, len, rows, cols)) return rc;
    if (int32_t rc = ensure_stage(ctx, len)) return rc;
    TQF_HIP(ctx, hipMemcpyAsync(ctx->d_stage, q6_k, len, hipMemcpyHostToDevice, ctx->stream));
    return q6k_upload_from(ctx, static_cast<const uint8_t *>(ctx->d_stage), rows, cols, out);
}

extern "C" int32_t tqf_hip_q6k_weights_upload_device(tqf_hip_ctx *ctx, const void *d_q6_k,
                                                     size_t len, uint32_t rows, uint32_t cols,
                                                     tqf_hip_weights **out) {
    TQF_ENTER(ctx);
    if (!d_q6_k || !out) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    *out = nullptr;
    if (int32_t rc = check_q6k_shape(ctx, len, rows, cols)) return rc;
    return q6k_upload_from(ctx, static_cast<const uint8_t *>(d_q6_k), rows, cols, out);
}

extern "C" int32_t tqf_hip_q6k_weights_download(tqf_hip_ctx *ctx, const tqf_hip_weights *w,
                                                uint8_t *q6_k, size_t len) {
    TQF_ENTER(ctx);
    if (!valid_q6k(w) || !q6_k) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer or not Q6_K weights");
    const MatrixDims &d = w->dims;
    const uint32_t nb = d.cols / 256;
    if (len != (size_t)d.rows * nb * kQ6KBlock)
        return fail(ctx, TQF_HIP_ERR_INVALID, "Q6_K byte length does not match the matrix");
    std::vector<uint8_t> tiles(w->bytes);
    TQF_HIP(ctx, hipMemcpyAsync(tiles.data(), w->tiles, w->bytes, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (uint32_t r = 0; r < d.rows; ++r) {
        for (uint32_t s = 0; s < nb; ++s) {
            uint8_t *dst = q6_k + ((size_t)r * nb + s) * kQ6KBlock;
            std::memset(dst, 0, kQ6KBlock);
            std::memcpy(dst + 208, tiles.data() + q6k_d_offset(d, r, s), 2);
            for (int j = 0; j < 8; ++j) {
                const uint32_t b = s * 8 + j;
                const size_t pr = q6k_slot_row(r, b);
                const uint8_t *nib = tiles.data() + q6k_nibble_offset(d, pr, b);
                const uint8_t *hb = tiles.data() + q6k_high_offset(d, pr, b);
                const uint8_t *sc = tiles.data() + q6k_scale_offset(d, pr, b);
                dst[192 + 2 * j] = sc[0];
                dst[192 + 2 * j + 1] = sc[1];
                const int h = j >> 2, grp = j & 3;
                for (int e = 0; e < 32; ++e) {
                    const int c = e & 7, t = e >> 3;
                    const uint8_t byte = nib[4 * (c >> 1) + t];
                    const int lo = (c & 1) ? (byte >> 4) : (byte & 15);
                    const int hi = ((hb[4 * (c >> 2) + t] >> (2 * (c & 3))) & 3) ^ 2;
                    uint8_t &q = dst[64 * h + ((grp & 1) ? 32 : 0) + e];
                    q = (uint8_t)(q | (grp < 2 ? lo : lo << 4));
                    dst[128 + 32 * h + e] = (uint8_t)(dst[128 + 32 * h + e] | (hi << (2 * grp)));
                }
            }
        }
    }
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_q6k_matvec(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *x,
                                      uint32_t m, float *y) {
    TQF_ENTER(ctx);
    return q6k_host_call(ctx, w, x, m, y, nullptr, nullptr);
}

extern "C" int32_t tqf_hip_q6k_matvec_device(tqf_hip_ctx *ctx, const tqf_hip_weights *w,
                                             const float *d_x, uint32_t m, float *d_y) {
    TQF_ENTER(ctx);
    if (!d_x || !d_y) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (int32_t rc = check_q6k_call(ctx, w, m)) return rc;
    return q6k_enqueue(ctx, w, d_x, m, d_y, nullptr, nullptr);
}

extern "C" int32_t tqf_hip_lm_head_logits(tqf_hip_ctx *ctx, const tqf_hip_weights *w,
                                          const float *x, uint32_t m, float *logits,
                                          uint32_t *tokens4, float *logits4) {
    TQF_ENTER(ctx);
    if (!tokens4 || !logits4) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    return q6k_host_call(ctx, w, x, m, logits, tokens4, logits4);
}

extern "C" int32_t tqf_hip_lm_head_logits_device(tqf_hip_ctx *ctx, const tqf_hip_weights *w,
                                                 const float *d_x, uint32_t m, float *d_logits,
                                                 uint32_t *d_tokens4, float *d_logits4) {
    TQF_ENTER(ctx);
    if (!d_x || !d_logits || !d_tokens4 || !d_logits4) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (int32_t rc = check_q6k_call(ctx, w, m)) return rc;
    return q6k_enqueue(ctx, w, d_x, m, d_logits, d_tokens4, d_logits4);
}

// ===========================================================================
// expert forward
// ===========================================================================
extern "C" int32_t tqf_hip_expert_forward(tqf_hip_ctx *ctx, const tqf_hip_weights *gate,
                                          const tqf_hip_weights *up, const tqf_hip_weights *down,
                                          const float *x, uint32_t m, float *y) {
    TQF_ENTER(ctx);
    if (!valid_weights(gate) || !valid_weights(up) || !valid_weights(down) || !x || !y)
        return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (m == 0 || m > kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "m must be in 1..8");
    const uint32_t F = gate->dims.rows, H = gate->dims.cols;
    if (up->dims.rows != F || up->dims.cols != H || down->dims.rows != H || down->dims.cols != F)
        return fail(ctx, TQF_HIP_ERR_INVALID, "expert shapes: gate/up [width x hidden], down [hidden x width]");
    if (H % 256 || F % 256 || H > 2048 || F > 2048)
        return fail(ctx, TQF_HIP_ERR_INVALID, "expert hidden and width must be multiples of 256, at most 2048");
    if (int32_t rc = ensure_moe_scratch(ctx, H, F, 0)) return rc;
    const size_t xb = (size_t)m * H * 4;
    if (int32_t rc = ensure_stage(ctx, 2 * align_up(xb, kAlign))) return rc;
    float *dx = static_cast<float *>(ctx->d_stage);
    float *dy = reinterpret_cast<float *>(static_cast<uint8_t *>(ctx->d_stage) + align_up(xb, kAlign));
    const uint8_t *mats[3] = {gate->tiles, up->tiles, down->tiles};
    Plan plan;
    std::memset(&plan, 0, sizeof plan);
    plan.n_slots = (int32_t)m;
    plan.n_union = 0;
    plan.m = (int32_t)m;
    for (uint32_t t = 0; t < m; ++t) {
        plan.slots[t] = SlotRec{{gate->tiles, up->tiles, down->tiles}, (int32_t)t, 1.0f};
        plan.slot_expert[t] = 0;
    }
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    drop_graphs(ctx);
    TQF_HIP(ctx, hipMemcpy(ctx->d_adhoc_mats, mats, sizeof mats, hipMemcpyHostToDevice));
    TQF_HIP(ctx, hipMemcpy(ctx->d_adhoc_plan, &plan, sizeof plan, hipMemcpyHostToDevice));
    TQF_HIP(ctx, hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, ctx->stream));
    LayerDev L{nullptr, nullptr, ctx->d_adhoc_mats, 0, H, F};
    Scratch &sc = ctx->scratch;
    hipError_t e = launch_prep(ctx->stream, dx, m, H, padded_blocks(H / 32), sc.xprep);
    if (e == hipSuccess)
        e = launch_gate_up(ctx->stream, L, m, ctx->d_adhoc_plan, sc.xprep, sc.hprep);
    if (e == hipSuccess)
        e = launch_down(ctx->stream, L, m, m, sc, ctx->d_adhoc_plan, sc.hprep, nullptr, dy);
    if (e != hipSuccess) return hip_fail(ctx, "expert kernels", e);
    TQF_HIP(ctx, hipMemcpyAsync(y, dy, xb, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TQF_HIP_OK;
}

// ===========================================================================
// MoE layer
// ===========================================================================
extern "C" int32_t tqf_hip_moe_layer_prepare(tqf_hip_ctx *ctx, const tqf_hip_moe_weights *mw,
                                             tqf_hip_layer **out) {
    TQF_ENTER(ctx);
    if (!mw || !out) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    *out = nullptr;
    const uint32_t E = mw->n_experts, H = mw->hidden, F = mw->width;
    if (E != 256) return fail(ctx, TQF_HIP_ERR_INVALID, "router requires n_experts == 256 (experts/mod.rs:135)");
    if (H == 0 || H % 256 || H > 2048) return fail(ctx, TQF_HIP_ERR_INVALID, "hidden must be a multiple of 256, at most 2048");
    if (F == 0 || F % 256 || F > 2048)
        return fail(ctx, TQF_HIP_ERR_INVALID, "width must be a multiple of 256, at most 2048");
    if (!mw->router || mw->router->count != (size_t)E * H)
        return fail(ctx, TQF_HIP_ERR_INVALID, "router must be f32 [n_experts x hidden]");
    if (!mw->shared_input_gate || mw->shared_input_gate->count != H)
        return fail(ctx, TQF_HIP_ERR_INVALID, "shared_input_gate must be f32 [hidden]");
    if (!mw->routed_gate || !mw->routed_up || !mw->routed_down)
        return fail(ctx, TQF_HIP_ERR_INVALID, "null routed expert table");
    // Every expert matrix of a layer has one format: Q4_0 (the configs'
    // group-32 format) or Q4_K (the canonical checkpoint's experts).
    const int32_t format = mw->shared_gate && mw->shared_gate->tiles ? mw->shared_gate->format : -1;
    if (format != TQF_HIP_FORMAT_Q4_0 && format != TQF_HIP_FORMAT_Q4_K)
        return fail(ctx, TQF_HIP_ERR_INVALID, "expert matrices must be Q4_0 or Q4_K weights");
    auto ok_fmt = [&](const tqf_hip_weights *w) { return w && w->tiles && w->format == format; };
    auto ok_gu = [&](const tqf_hip_weights *w) { return ok_fmt(w) && w->dims.rows == F && w->dims.cols == H; };
    auto ok_d = [&](const tqf_hip_weights *w) { return ok_fmt(w) && w->dims.rows == H && w->dims.cols == F; };
    std::vector<const uint8_t *> mats((size_t)(E + 1) * 3);
    for (uint32_t e = 0; e <= E; ++e) {
        const tqf_hip_weights *g = e < E ? mw->routed_gate[e] : mw->shared_gate;
        const tqf_hip_weights *u = e < E ? mw->routed_up[e] : mw->shared_up;
        const tqf_hip_weights *d = e < E ? mw->routed_down[e] : mw->shared_down;
        if (!ok_gu(g) || !ok_gu(u) || !ok_d(d))
            return fail(ctx, TQF_HIP_ERR_INVALID,
                        "expert " + std::to_string(e) +
                            ": gate/up must be [width x hidden] and down [hidden x width], all of one format");
        mats[(size_t)e * 3 + 0] = g->tiles;
        mats[(size_t)e * 3 + 1] = u->tiles;
        mats[(size_t)e * 3 + 2] = d->tiles;
    }
    if (int32_t rc = ensure_moe_scratch(ctx, H, F, E)) return rc;
    if (format == TQF_HIP_FORMAT_Q4_K)
        if (int32_t rc = ensure_q4k_layer_scratch(ctx, H, F)) return rc;
    void *dm = nullptr;
    if (arena_alloc(ctx, mats.size() * sizeof(void *), &dm) != hipSuccess)
        return fail(ctx, TQF_HIP_ERR_NOMEM, "layer table allocation failed");
    hipError_t e = hipMemcpy(dm, mats.data(), mats.size() * sizeof(void *), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        arena_free(ctx, dm);
        return hip_fail(ctx, "layer table upload", e);
    }
    tqf_hip_layer *layer = new tqf_hip_layer();
    layer->d_mats = static_cast<const uint8_t **>(dm);
    layer->dev = LayerDev{mw->router->data, mw->shared_input_gate->data, layer->d_mats, E, H, F};
    layer->format = format;
    *out = layer;
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_moe_layer_free(tqf_hip_ctx *ctx, tqf_hip_layer *layer) {
    TQF_ENTER(ctx);
    if (!layer) return TQF_HIP_OK;
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    drop_graphs(ctx);
    arena_free(ctx, const_cast<const uint8_t **>(layer->d_mats));
    delete layer;
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_moe_layer_device(tqf_hip_ctx *ctx, const tqf_hip_layer *layer,
                                            const float *d_x, uint32_t m, float *d_y,
                                            uint16_t *d_ids, float *d_w, int32_t *d_status) {
    TQF_ENTER(ctx);
    if (!layer || !d_x || !d_y) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (m == 0 || m > kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "m must be in 1..8");
    if (d_x == d_y) return fail(ctx, TQF_HIP_ERR_INVALID, "x and y must not alias");
    if (int32_t rc = ensure_layer_scratch(ctx, layer->dev, layer->format)) return rc;
    return enqueue_moe(ctx, layer, d_x, nullptr, m, nullptr, d_y, d_ids, d_w, d_status);
}

extern "C" int32_t tqf_hip_moe_layer(tqf_hip_ctx *ctx, const tqf_hip_layer *layer, const float *x,
                                     uint32_t m, float *y, uint16_t *ids, float *w) {
    TQF_ENTER(ctx);
    if (!layer || !x || !y) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (m == 0 || m > kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "m must be in 1..8");
    const LayerDev &L = layer->dev;
    if (int32_t rc = ensure_layer_scratch(ctx, L, layer->format)) return rc;
    const size_t xb = align_up((size_t)m * L.hidden * 4, kAlign);
    const size_t ib = align_up((size_t)m * kTopK * 2, kAlign), wb = align_up((size_t)m * kTopK * 4, kAlign);
    if (int32_t rc = ensure_stage(ctx, 2 * xb + ib + wb + kAlign)) return rc;
    uint8_t *base = static_cast<uint8_t *>(ctx->d_stage);
    float *dx = reinterpret_cast<float *>(base);
    float *dy = reinterpret_cast<float *>(base + xb);
    uint16_t *dids = reinterpret_cast<uint16_t *>(base + 2 * xb);
    float *dw = reinterpret_cast<float *>(base + 2 * xb + ib);
    int32_t *dstatus = reinterpret_cast<int32_t *>(base + 2 * xb + ib + wb);
    const int32_t zero = 0;
    TQF_HIP(ctx, hipMemcpyAsync(dstatus, &zero, 4, hipMemcpyHostToDevice, ctx->stream));
    TQF_HIP(ctx, hipMemcpyAsync(dx, x, (size_t)m * L.hidden * 4, hipMemcpyHostToDevice, ctx->stream));
    if (int32_t rc = enqueue_moe(ctx, layer, dx, nullptr, m, nullptr, dy, dids, dw, dstatus)) return rc;
    int32_t status = 0;
    TQF_HIP(ctx, hipMemcpyAsync(&status, dstatus, 4, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipMemcpyAsync(y, dy, (size_t)m * L.hidden * 4, hipMemcpyDeviceToHost, ctx->stream));
    if (ids) TQF_HIP(ctx, hipMemcpyAsync(ids, dids, (size_t)m * kTopK * 2, hipMemcpyDeviceToHost, ctx->stream));
    if (w) TQF_HIP(ctx, hipMemcpyAsync(w, dw, (size_t)m * kTopK * 4, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (status != 0)
        return fail(ctx, TQF_HIP_ERR_ROUTER, "exact router logits must all be finite (experts/mod.rs:136-141)");
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_moe_layer_bf16(tqf_hip_ctx *ctx, const tqf_hip_layer *layer,
                                          const uint16_t *x_bf16, uint32_t m, float *y,
                                          uint16_t *ids, float *w) {
    TQF_ENTER(ctx);
    if (!layer || !x_bf16 || !y) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (m == 0 || m > kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "m must be in 1..8");
    const size_t n = (size_t)m * layer->dev.hidden;
    std::vector<float> x(n);
    for (size_t i = 0; i < n; ++i) {
        const uint32_t bits = (uint32_t)x_bf16[i] << 16;
        std::memcpy(&x[i], &bits, 4);
    }
    return tqf_hip_moe_layer(ctx, layer, x.data(), m, y, ids, w);
}

// ===========================================================================
// stack
// ===========================================================================
extern "C" int32_t tqf_hip_stack_prepare(tqf_hip_ctx *ctx, const tqf_hip_layer *const *layers,
                                         const tqf_hip_tensor *const *ffn_norms, uint32_t n_layers,
                                         tqf_hip_stack **out) {
    TQF_ENTER(ctx);
    if (!layers || !ffn_norms || !out || n_layers == 0)
        return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer or no layers");
    *out = nullptr;
    tqf_hip_stack *st = new tqf_hip_stack();
    st->hidden = layers[0] ? layers[0]->dev.hidden : 0;
    st->width = layers[0] ? layers[0]->dev.width : 0;
    st->experts = layers[0] ? layers[0]->dev.n_experts : 0;
    st->format = layers[0] ? layers[0]->format : TQF_HIP_FORMAT_Q4_0;
    for (uint32_t l = 0; l < n_layers; ++l) {
        const tqf_hip_layer *L = layers[l];
        const tqf_hip_tensor *nw = ffn_norms[l];
        if (!L || !nw || L->dev.hidden != st->hidden || L->dev.width != st->width ||
            L->dev.n_experts != st->experts || nw->count != st->hidden ||
            L->format != layers[0]->format) {
            delete st;
            return fail(ctx, TQF_HIP_ERR_INVALID,
                        "layer " + std::to_string(l) +
                            ": layers must share one geometry and expert format, and norms be f32 [hidden]");
        }
        st->layers.push_back(L);
        st->norms.push_back(nw->data);
    }
    std::vector<StackLayer> table(n_layers);
    for (uint32_t l = 0; l < n_layers; ++l)
        table[l] = StackLayer{st->layers[l]->dev.router, st->layers[l]->dev.shared_input_gate,
                              st->norms[l], st->layers[l]->dev.mats};
    hipError_t e = hipMalloc(&st->d_layers, n_layers * sizeof(StackLayer));
    if (e == hipSuccess)
        e = hipMemcpy(st->d_layers, table.data(), n_layers * sizeof(StackLayer), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(st->d_layers);
        delete st;
        return hip_fail(ctx, "stack layer table", e);
    }
    *out = st;
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_stack_free(tqf_hip_ctx *ctx, tqf_hip_stack *stack) {
    TQF_ENTER(ctx);
    if (!stack) return TQF_HIP_OK;
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    drop_graphs(ctx);
    (void)hipFree(stack->d_layers);
    delete stack;
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_stack_forward_device(tqf_hip_ctx *ctx, const tqf_hip_stack *stack,
                                                const float *d_h_in, float *d_h, uint32_t m,
                                                uint16_t *d_ids, float *d_w, int32_t *d_status) {
    TQF_ENTER(ctx);
    if (!stack || !d_h) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (m == 0 || m > kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "m must be in 1..8");
    if (stack_persistent_ok(ctx, stack, m)) {
        const bool rec = recovering(ctx);
        if (int32_t rc = enqueue_stack_persistent(ctx, stack, d_h_in, d_h, m, d_ids, d_w, d_status, rec))
            return rc;
        if (!rec) return TQF_HIP_OK;
        TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->h_flags[kFlagStack] != 0) return rerun_stack(ctx, stack, d_h, m, d_ids, d_w, d_status);
        return TQF_HIP_OK;
    }
    if (int32_t rc = ensure_layer_scratch(ctx, stack->layers[0]->dev, stack->format)) return rc;
    std::vector<uint64_t> key = {1, k64(stack), k64(d_h_in), k64(d_h), m, k64(d_ids), k64(d_w),
                                 k64(d_status)};
    return run_graphed(ctx, key, [&]() {
        return enqueue_stack(ctx, stack, d_h_in, d_h, m, d_ids, d_w, d_status);
    });
}

// ===========================================================================
// acceptance
// ===========================================================================
namespace {
int32_t check_accept(tqf_hip_ctx *ctx, uint32_t k, uint32_t vocab, float T, int32_t greedy,
                     bool have_draft, bool have_u) {
    if (vocab == 0) return fail(ctx, TQF_HIP_ERR_INVALID, "vocab must be > 0");
    if (k > kMaxTokens - 1) return fail(ctx, TQF_HIP_ERR_INVALID, "k must be <= 7");
    if (!greedy) {
        if (!(T > 0.0f) || !(T <= 3.402823466e38f))
            return fail(ctx, TQF_HIP_ERR_INVALID, "temperature must be finite and > 0 when sampling");
        if (!have_draft || !have_u)
            return fail(ctx, TQF_HIP_ERR_INVALID, "stochastic acceptance needs draft logits and uniforms");
    }
    return TQF_HIP_OK;
}
}  // namespace

extern "C" int32_t tqf_hip_accept_device(tqf_hip_ctx *ctx, const float *d_target,
                                         const float *d_draft, const int32_t *d_draft_tokens,
                                         uint32_t k, uint32_t vocab, float temperature,
                                         int32_t greedy, const float *d_u, const float *d_ures,
                                         int32_t *d_accepted, int32_t *d_tokens) {
    TQF_ENTER(ctx);
    if (!d_target || !d_accepted || !d_tokens || (k > 0 && !d_draft_tokens))
        return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (int32_t rc = check_accept(ctx, k, vocab, temperature, greedy, d_draft != nullptr,
                                  d_u != nullptr && d_ures != nullptr))
        return rc;
    if (int32_t rc = ensure_accept_scratch(ctx, accept_scratch_bytes(k, vocab))) return rc;
    const bool rec = recovering(ctx) && accept_one_launch(k, vocab);
    if (int32_t rc = enqueue_accept(ctx, d_target, d_draft, d_draft_tokens, k, vocab, temperature, greedy,
                                    d_u, d_ures, d_accepted, d_tokens, rec))
        return rc;
    if (!rec) return TQF_HIP_OK;
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->h_flags[kFlagAccept] != 0)
        return rerun_accept(ctx, d_target, d_draft, d_draft_tokens, k, vocab, temperature, greedy, d_u, d_ures,
                            d_accepted, d_tokens);
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_embed_rows_device(tqf_hip_ctx *ctx, const tqf_hip_weights *emb,
                                             const int32_t *d_tokens, uint32_t n, const float *d_add,
                                             float *d_out, int32_t *d_status) {
    TQF_ENTER(ctx);
    if (!valid_weights(emb) || !d_tokens || !d_out) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (emb->format != TQF_HIP_FORMAT_Q4_0)
        return fail(ctx, TQF_HIP_ERR_INVALID, "the embedding rows need a Q4_0 matrix");
    if (n == 0) return TQF_HIP_OK;
    hipError_t e = tqf::launch_embed_rows(ctx->stream, emb->tiles, emb->dims, d_tokens, n, d_add, d_out, d_status);
    if (e != hipSuccess) return hip_fail(ctx, "embedding rows launch", e);
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_rmsnorm_rows_device(tqf_hip_ctx *ctx, const float *d_x, uint32_t n, uint32_t cols,
                                               const tqf_hip_tensor *w, float *d_out) {
    TQF_ENTER(ctx);
    if (!d_x || !w || !w->data || !d_out) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (w->count != cols || cols == 0) return fail(ctx, TQF_HIP_ERR_INVALID, "norm weight length != cols");
    if (n == 0) return TQF_HIP_OK;
    hipError_t e = tqf::launch_rmsnorm_rows(ctx->stream, d_x, n, cols, w->data, d_out);
    if (e != hipSuccess) return hip_fail(ctx, "rmsnorm rows launch", e);
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_accept_device_noalloc(tqf_hip_ctx *ctx, const float *d_target,
                                                 const float *d_draft, const int32_t *d_draft_tokens,
                                                 uint32_t k, uint32_t vocab, float temperature,
                                                 int32_t greedy, const float *d_u, const float *d_ures,
                                                 int32_t *d_accepted, int32_t *d_tokens) {
    TQF_ENTER(ctx);
    if (!d_target || !d_accepted || !d_tokens || (k > 0 && !d_draft_tokens))
        return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (int32_t rc = check_accept(ctx, k, vocab, temperature, greedy, d_draft != nullptr,
                                  d_u != nullptr && d_ures != nullptr))
        return rc;
    if (accept_scratch_bytes(k, vocab) > kNoAllocScratchBytes)
        return fail(ctx, TQF_HIP_ERR_INVALID,
                    "k and vocab need " + std::to_string(accept_scratch_bytes(k, vocab)) +
                        " scratch bytes; the allocation-free scratch holds " +
                        std::to_string(kNoAllocScratchBytes));
    if (!ctx->noalloc_scratch) return fail(ctx, TQF_HIP_ERR_DEVICE, "allocation-free scratch not resolved");
    // no profiling events here: an empty event pool would create events
    hipError_t e = launch_accept(ctx->stream, d_target, d_draft, d_draft_tokens, k, vocab, temperature,
                                 greedy, d_u, d_ures, d_accepted, d_tokens, ctx->noalloc_scratch,
                                 nullptr, nullptr);
    if (e != hipSuccess) return hip_fail(ctx, "acceptance kernel launch", e);
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_accept(tqf_hip_ctx *ctx, const float *target, const float *draft,
                                  const int32_t *draft_tokens, uint32_t k, uint32_t vocab,
                                  float temperature, int32_t greedy, const float *u,
                                  const float *u_resample, int32_t *accepted,
                                  int32_t *tokens_out) {
    TQF_ENTER(ctx);
    if (!target || !accepted || !tokens_out || (k > 0 && !draft_tokens))
        return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (int32_t rc = check_accept(ctx, k, vocab, temperature, greedy, draft != nullptr,
                                  u != nullptr && u_resample != nullptr))
        return rc;
    for (uint32_t i = 0; i < k; ++i)
        if (draft_tokens[i] < 0 || (uint32_t)draft_tokens[i] >= vocab)
            return fail(ctx, TQF_HIP_ERR_INVALID, "draft token out of vocabulary");
    if (!greedy) {
        for (uint32_t i = 0; i < k; ++i)
            if (!(u[i] >= 0.0f && u[i] < 1.0f)) return fail(ctx, TQF_HIP_ERR_INVALID, "uniforms must lie in [0, 1)");
        for (uint32_t i = 0; i <= k; ++i)
            if (!(u_resample[i] >= 0.0f && u_resample[i] < 1.0f))
                return fail(ctx, TQF_HIP_ERR_INVALID, "uniforms must lie in [0, 1)");
    }
    const size_t tb = align_up((size_t)(k + 1) * vocab * 4, kAlign);
    const size_t db = greedy ? 0 : align_up((size_t)k * vocab * 4, kAlign);
    const size_t small = 4 * kAlign;
    if (int32_t rc = ensure_stage(ctx, tb + db + small)) return rc;
    if (int32_t rc = ensure_accept_scratch(ctx, accept_scratch_bytes(k, vocab))) return rc;
    uint8_t *base = static_cast<uint8_t *>(ctx->d_stage);
    float *dt = reinterpret_cast<float *>(base);
    float *dd = greedy ? nullptr : reinterpret_cast<float *>(base + tb);
    uint8_t *sm = base + tb + db;
    int32_t *dtok = reinterpret_cast<int32_t *>(sm);
    float *du = reinterpret_cast<float *>(sm + kAlign);
    float *dur = reinterpret_cast<float *>(sm + 2 * kAlign);
    int32_t *dout = reinterpret_cast<int32_t *>(sm + 3 * kAlign);  // [accepted, tokens...]
    TQF_HIP(ctx, hipMemcpyAsync(dt, target, (size_t)(k + 1) * vocab * 4, hipMemcpyHostToDevice, ctx->stream));
    if (!greedy) {
        TQF_HIP(ctx, hipMemcpyAsync(dd, draft, (size_t)k * vocab * 4, hipMemcpyHostToDevice, ctx->stream));
        if (k) TQF_HIP(ctx, hipMemcpyAsync(du, u, k * 4, hipMemcpyHostToDevice, ctx->stream));
        TQF_HIP(ctx, hipMemcpyAsync(dur, u_resample, (k + 1) * 4, hipMemcpyHostToDevice, ctx->stream));
    }
    if (k) TQF_HIP(ctx, hipMemcpyAsync(dtok, draft_tokens, k * 4, hipMemcpyHostToDevice, ctx->stream));
    const bool rec = recovering(ctx) && accept_one_launch(k, vocab);
    if (int32_t rc = enqueue_accept(ctx, dt, dd, k ? dtok : nullptr, k, vocab, temperature, greedy,
                                    greedy ? nullptr : du, greedy ? nullptr : dur, dout, dout + 1, rec))
        return rc;
    std::vector<int32_t> res(k + 2);
    TQF_HIP(ctx, hipMemcpyAsync(res.data(), dout, (k + 2) * 4, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (rec && ctx->h_flags[kFlagAccept] != 0) {
        if (int32_t rc = rerun_accept(ctx, dt, dd, k ? dtok : nullptr, k, vocab, temperature, greedy,
                                      greedy ? nullptr : du, greedy ? nullptr : dur, dout, dout + 1))
            return rc;
        TQF_HIP(ctx, hipMemcpyAsync(res.data(), dout, (k + 2) * 4, hipMemcpyDeviceToHost, ctx->stream));
        TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    }
    *accepted = res[0];
    std::memcpy(tokens_out, res.data() + 1, (k + 1) * 4);
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_sampler_select_device(tqf_hip_ctx *ctx, const float *d_logits, uint32_t rows,
                                                 uint32_t vocab, float temperature, const float *d_u,
                                                 int32_t *d_tokens, float *d_sums) {
    TQF_ENTER(ctx);
    if (!d_logits || !d_tokens || (temperature != 0.0f && !d_u))
        return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (rows == 0 || rows > (uint32_t)kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "rows must be in 1..8");
    if (vocab == 0 || vocab > (1u << 22)) return fail(ctx, TQF_HIP_ERR_INVALID, "vocab must be in 1..4194304");
    if (!(temperature >= 0.0f) || !(temperature <= 3.402823466e38f))
        return fail(ctx, TQF_HIP_ERR_INVALID, "temperature must be finite and >= 0");
    const size_t need = sample_scratch_bytes(rows, vocab);
    if (!ctx->d_sample || ctx->sample_bytes < need) {
        TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
        TQF_HIP(ctx, grow(ctx->d_sample, ctx->sample_bytes, need));
    }
    Prof p(ctx);
    hipError_t e = launch_sample_select(ctx->stream, d_logits, rows, vocab, temperature, d_u, d_tokens, d_sums,
                                        ctx->d_sample);
    if (e != hipSuccess) return hip_fail(ctx, "sampler launch", e);
    p.end(TQF_HIP_KERNEL_SAMPLE, (double)rows * vocab * 4, 0.0, nullptr);
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_top_logit_candidates(tqf_hip_ctx *ctx, const float *logits,
                                                uint32_t rows, uint32_t vocab, uint32_t *tokens4,
                                                float *logits4) {
    TQF_ENTER(ctx);
    if (!logits || !tokens4 || !logits4 || rows == 0 || vocab == 0)
        return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer or empty logits");
    if (rows > 65535) return fail(ctx, TQF_HIP_ERR_INVALID, "rows must be <= 65535");
    const size_t lb = align_up((size_t)rows * vocab * 4, kAlign);
    const size_t ob = align_up((size_t)rows * 16, kAlign);
    if (int32_t rc = ensure_stage(ctx, lb + 2 * ob)) return rc;
    uint8_t *base = static_cast<uint8_t *>(ctx->d_stage);
    float *dl = reinterpret_cast<float *>(base);
    uint32_t *dtok = reinterpret_cast<uint32_t *>(base + lb);
    float *dval = reinterpret_cast<float *>(base + lb + ob);
    TQF_HIP(ctx, hipMemcpyAsync(dl, logits, (size_t)rows * vocab * 4, hipMemcpyHostToDevice, ctx->stream));
    hipError_t e = launch_top4(ctx->stream, dl, rows, vocab, dtok, dval);
    if (e != hipSuccess) return hip_fail(ctx, "top-4 kernel launch", e);
    TQF_HIP(ctx, hipMemcpyAsync(tokens4, dtok, (size_t)rows * 16, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipMemcpyAsync(logits4, dval, (size_t)rows * 16, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TQF_HIP_OK;
}

// ===========================================================================
// grouped expert GEMM (prefill)
// ===========================================================================
namespace {
int32_t check_grouped(tqf_hip_ctx *ctx, const tqf_hip_layer *layer, uint32_t t) {
    if (!layer) return fail(ctx, TQF_HIP_ERR_INVALID, "null layer");
    if (t == 0 || t > TQF_HIP_GROUPED_MAX_TOKENS)
        return fail(ctx, TQF_HIP_ERR_INVALID, "t must be in 1..TQF_HIP_GROUPED_MAX_TOKENS");
    const LayerDev &L = layer->dev;
    if (layer->format != TQF_HIP_FORMAT_Q4_0)
        return fail(ctx, TQF_HIP_ERR_INVALID, "the grouped GEMM reads Q4_0 expert matrices");
    if (L.hidden % 256 || L.width % 256 || L.n_experts == 0 || L.n_experts > 256)
        return fail(ctx, TQF_HIP_ERR_INVALID, "layer geometry unsupported by the grouped GEMM");
    return TQF_HIP_OK;
}

int32_t enqueue_grouped(tqf_hip_ctx *ctx, const LayerDev &L, const uint16_t *x, uint32_t t,
                        const uint16_t *ids, const float *w, float *y, int32_t *status) {
    const size_t need = grouped_scratch_bytes(t, L.n_experts, L.hidden, L.width);
    if (!ctx->d_grouped || ctx->grouped_bytes < need) {
        TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
        TQF_HIP(ctx, grow(ctx->d_grouped, ctx->grouped_bytes, need));
    }
    const GroupedBuffers g = grouped_buffers(ctx->d_grouped, t, L.n_experts, L.hidden, L.width);
    const double pairs = (double)t * kTopK;
    {
        Prof p(ctx);
        hipError_t e = launch_grouped_plan(ctx->stream, ids, t, L.n_experts, g, status);
        if (e != hipSuccess) return hip_fail(ctx, "grouped plan kernel launch", e);
        p.end(TQF_HIP_KERNEL_GROUPED_AUX, pairs * 2, 0, nullptr);
    }
    {
        Prof p(ctx);
        hipError_t e = launch_grouped_gate_up(ctx->stream, L, x, g);
        if (e != hipSuccess) return hip_fail(ctx, "grouped gate/up kernel launch", e);
        p.end(TQF_HIP_KERNEL_GROUPED_GATE_UP, 0, 0, nullptr);
    }
    {
        Prof p(ctx);
        hipError_t e = launch_grouped_down(ctx->stream, L, g);
        if (e != hipSuccess) return hip_fail(ctx, "grouped down kernel launch", e);
        p.end(TQF_HIP_KERNEL_GROUPED_DOWN, 0, 0, nullptr);
    }
    {
        Prof p(ctx);
        hipError_t e = launch_grouped_combine(ctx->stream, g, w, t, L.hidden, y);
        if (e != hipSuccess) return hip_fail(ctx, "grouped combine kernel launch", e);
        p.end(TQF_HIP_KERNEL_GROUPED_AUX, pairs * (L.hidden * 4.0 + 8) + t * L.hidden * 4.0, 0, nullptr);
    }
    return TQF_HIP_OK;
}
}  // namespace

extern "C" int32_t tqf_hip_grouped_gemm_device(tqf_hip_ctx *ctx, const tqf_hip_layer *layer,
                                               const uint16_t *d_x_bf16, uint32_t t,
                                               const uint16_t *d_ids, const float *d_w,
                                               float *d_y, int32_t *d_status) {
    TQF_ENTER(ctx);
    if (!d_x_bf16 || !d_ids || !d_w || !d_y) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (int32_t rc = check_grouped(ctx, layer, t)) return rc;
    return enqueue_grouped(ctx, layer->dev, d_x_bf16, t, d_ids, d_w, d_y, d_status);
}

extern "C" int32_t tqf_hip_grouped_gemm(tqf_hip_ctx *ctx, const tqf_hip_layer *layer,
                                        const uint16_t *x_bf16, uint32_t t, const uint16_t *ids,
                                        const float *w, float *y) {
    TQF_ENTER(ctx);
    if (!x_bf16 || !ids || !w || !y) return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (int32_t rc = check_grouped(ctx, layer, t)) return rc;
    const LayerDev &L = layer->dev;
    for (size_t i = 0; i < (size_t)t * kTopK; ++i)
        if (ids[i] >= L.n_experts) return fail(ctx, TQF_HIP_ERR_INVALID, "expert id out of range");
    const size_t xb = align_up((size_t)t * L.hidden * 2, kAlign);
    const size_t ib = align_up((size_t)t * kTopK * 2, kAlign);
    const size_t wb = align_up((size_t)t * kTopK * 4, kAlign);
    const size_t yb = align_up((size_t)t * L.hidden * 4, kAlign);
    if (int32_t rc = ensure_stage(ctx, xb + ib + wb + yb + kAlign)) return rc;
    uint8_t *base = static_cast<uint8_t *>(ctx->d_stage);
    uint16_t *dx = reinterpret_cast<uint16_t *>(base);
    uint16_t *dids = reinterpret_cast<uint16_t *>(base + xb);
    float *dw = reinterpret_cast<float *>(base + xb + ib);
    float *dy = reinterpret_cast<float *>(base + xb + ib + wb);
    int32_t *dstatus = reinterpret_cast<int32_t *>(base + xb + ib + wb + yb);
    const int32_t zero = 0;
    TQF_HIP(ctx, hipMemcpyAsync(dstatus, &zero, 4, hipMemcpyHostToDevice, ctx->stream));
    TQF_HIP(ctx, hipMemcpyAsync(dx, x_bf16, (size_t)t * L.hidden * 2, hipMemcpyHostToDevice, ctx->stream));
    TQF_HIP(ctx, hipMemcpyAsync(dids, ids, (size_t)t * kTopK * 2, hipMemcpyHostToDevice, ctx->stream));
    TQF_HIP(ctx, hipMemcpyAsync(dw, w, (size_t)t * kTopK * 4, hipMemcpyHostToDevice, ctx->stream));
    if (int32_t rc = enqueue_grouped(ctx, L, dx, t, dids, dw, dy, dstatus)) return rc;
    int32_t status = 0;
    TQF_HIP(ctx, hipMemcpyAsync(&status, dstatus, 4, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipMemcpyAsync(y, dy, (size_t)t * L.hidden * 4, hipMemcpyDeviceToHost, ctx->stream));
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (status != 0) return fail(ctx, status, "expert id out of range");
    return TQF_HIP_OK;
}

// ===========================================================================
// verify step
// ===========================================================================
extern "C" int32_t tqf_hip_verify_step_device(tqf_hip_ctx *ctx, const tqf_hip_stack *stack,
                                              const float *d_h_in, float *d_h, uint32_t m,
                                              const float *d_target,
                                              const float *d_draft, const int32_t *d_dtok,
                                              uint32_t vocab, float temperature, int32_t greedy,
                                              const float *d_u, const float *d_ures,
                                              int32_t *d_accepted, int32_t *d_tokens,
                                              int32_t *d_status) {
    TQF_ENTER(ctx);
    if (!stack || !d_h || !d_target || !d_accepted || !d_tokens)
        return fail(ctx, TQF_HIP_ERR_INVALID, "null pointer");
    if (m == 0 || m > kMaxTokens) return fail(ctx, TQF_HIP_ERR_INVALID, "m must be in 1..8");
    const uint32_t k = m - 1;
    if (k > 0 && !d_dtok) return fail(ctx, TQF_HIP_ERR_INVALID, "null draft tokens");
    if (int32_t rc = check_accept(ctx, k, vocab, temperature, greedy, d_draft != nullptr,
                                  d_u != nullptr && d_ures != nullptr))
        return rc;
    if (int32_t rc = ensure_accept_scratch(ctx, accept_scratch_bytes(k, vocab))) return rc;
    const bool rec_accept = recovering(ctx) && accept_one_launch(k, vocab);
    bool rec_stack = false;
    if (stack_persistent_ok(ctx, stack, m)) {
        rec_stack = recovering(ctx);
        if (int32_t rc = enqueue_stack_persistent(ctx, stack, d_h_in, d_h, m, nullptr, nullptr, d_status,
                                                  rec_stack))
            return rc;
        if (int32_t rc = enqueue_accept(ctx, d_target, d_draft, d_dtok, k, vocab, temperature, greedy, d_u,
                                        d_ures, d_accepted, d_tokens, rec_accept))
            return rc;
    } else {
        if (int32_t rc = ensure_layer_scratch(ctx, stack->layers[0]->dev, stack->format)) return rc;
        uint32_t tbits;
        std::memcpy(&tbits, &temperature, 4);
        std::vector<uint64_t> key = {2,          k64(stack), k64(d_h_in), k64(d_h), m, k64(d_target),
                                     k64(d_draft), k64(d_dtok), vocab,     tbits,       (uint64_t)greedy,
                                     k64(d_u),   k64(d_ures), k64(d_accepted), k64(d_tokens),
                                     k64(d_status), (uint64_t)rec_accept};
        // the captured acceptance reports to the same host flag at every replay
        if (rec_accept) ctx->h_flags[kFlagAccept] = 0;
        if (int32_t rc = run_graphed(ctx, key, [&]() {
                if (int32_t rc = enqueue_stack(ctx, stack, d_h_in, d_h, m, nullptr, nullptr, d_status)) return rc;
                return enqueue_accept(ctx, d_target, d_draft, d_dtok, k, vocab, temperature, greedy, d_u,
                                      d_ures, d_accepted, d_tokens, rec_accept);
            }))
            return rc;
    }
    if (!rec_stack && !rec_accept) return TQF_HIP_OK;
    TQF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    // the acceptance reads only the logits, so each part re-runs on its own
    if (rec_stack && ctx->h_flags[kFlagStack] != 0)
        if (int32_t rc = rerun_stack(ctx, stack, d_h, m, nullptr, nullptr, d_status)) return rc;
    if (rec_accept && ctx->h_flags[kFlagAccept] != 0)
        return rerun_accept(ctx, d_target, d_draft, d_dtok, k, vocab, temperature, greedy, d_u, d_ures, d_accepted,
                            d_tokens);
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_recovery_counts(tqf_hip_ctx *ctx, uint64_t *stack_reruns, uint64_t *accept_reruns) {
    TQF_ENTER(ctx);
    if (stack_reruns) *stack_reruns = ctx->reruns[kFlagStack];
    if (accept_reruns) *accept_reruns = ctx->reruns[kFlagAccept];
    return TQF_HIP_OK;
}

// ===========================================================================
// profiling
// ===========================================================================
extern "C" int32_t tqf_hip_profile_enable(tqf_hip_ctx *ctx, int32_t enable) {
    TQF_ENTER(ctx);
    resolve_profile(ctx);
    ctx->profiling = enable != 0;
    for (int i = 0; i < TQF_HIP_KERNEL_KINDS; ++i) {
        ctx->prof_launches[i] = 0;
        ctx->prof_ms[i] = 0.0;
        ctx->prof_bytes[i] = 0.0;
    }
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_profile_read(tqf_hip_ctx *ctx, int32_t kind, uint64_t *launches,
                                        double *total_ms, double *algorithmic_bytes) {
    TQF_ENTER(ctx);
    if (kind < 0 || kind >= TQF_HIP_KERNEL_KINDS) return fail(ctx, TQF_HIP_ERR_INVALID, "unknown kernel kind");
    resolve_profile(ctx);
    if (launches) *launches = ctx->prof_launches[kind];
    if (total_ms) *total_ms = ctx->prof_ms[kind];
    if (algorithmic_bytes) *algorithmic_bytes = ctx->prof_bytes[kind];
    return TQF_HIP_OK;
}
