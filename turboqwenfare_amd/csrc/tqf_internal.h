// tqf_internal.h -- shared definitions of the gfx950 HIP backend (not ABI).
//
// Device layout of one Q4_0 matrix ("row-lane layout").  A GGML Q4_0 matrix
// is rows x B blocks of 18 bytes (f16 scale d, 16 nibble bytes qs; element j
// of a block is (qs[j] & 15) - 8, element j + 16 is (qs[j] >> 4) - 8;
// format/quant/dequant.rs:110-123).  The backend pads B to Bp (16, 32 or a
// multiple of 64) and the rows to a multiple of 64, and stores every octet of
// rows 8o..8o+7 as one contiguous chunk of 9 * Bp * 16 bytes:
//   [8 rows][Bp blocks][16 nibble bytes]   then   [Bp blocks][8 rows x f16]
// A row's blocks are spread across lanes: lane l of a 64-wide wavefront owns
// block (l mod LPR) (LPR = min(Bp, 64) lanes per row, Bp/LPR blocks per
// lane), so one 128-bit load per lane reads 64/LPR whole rows = 1 KiB
// contiguously, one 16-byte scale load gives a lane the scales of eight rows,
// and a wavefront that owns whole octets reads one contiguous 9 KiB stretch
// per octet (DRAM-page friendly).  Padding has zero scale (products exactly
// zero).  The bytes are the GGML bytes moved, never re-encoded: the repack is
// lossless and tqf_hip_weights_download() inverts it.
//
// Activation prep ("xprep").  A Q4_0 dot is evaluated with exact integer
// arithmetic: each 32-element activation block is written as
//   x_j = X_j * 2^e,  |X_j| <= 2^22,  e chosen per block from max |x_j|
// and X_j is split into six balanced base-16 digits D_kj in [-8, 7]
// (X = sum_k D_k 16^k).  The weights enter as signed nibbles q - 8 (q ^ 8 is
// their 4-bit two's complement), so sum_j (q_j - 8) X_j is six chains of
// four v_dot8_i32_i4, recombined exactly in int32, and the block contributes
// d * 2^e * (float)that.  The representation keeps 22 bits of every block
// relative to its largest element, so the only rounding beyond the fp32
// accumulation is 2^-23 of each block's max |x|.  One xprep record per
// (token, block) is 28 dwords:
//   dw[4k .. 4k+4)  digit k (k < 6): the nibble of element j sits in dword
//                   (j mod 16) / 4 at bit 4 (2 (j mod 4) + j / 16), mirroring
//                   the Q4_0 nibble order of qs
//   dw[24]          2^e (float);  dw[25..28) unused
// The records of one activation row (a token, or a pair slot's h) are stored
// as 7 planes of 16 bytes per block: plane q = [Bp blocks][dwords 4q..4q+3],
// so the seven loads of a wavefront whose lane b needs block b are each one
// contiguous 1 KiB access.  Row stride: 28 * Bp dwords.  Records of padding
// blocks are never written; readers zero their scale word (dw 24), so a
// padding block contributes exactly 0 whatever the scratch held before.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/tqf_hip.h"

namespace tqf {

constexpr int kWave = 64;
constexpr int kRowsPerGroup = 64;  // row padding unit
constexpr int kXprepDwords = 28;  // per block
constexpr int kTopK = TQF_HIP_TOP_K;
constexpr int kMaxTokens = TQF_HIP_MAX_TOKENS;
constexpr int kMaxExperts = 256;
// One slot per (expert, token) pair: M shared-expert pairs + 8M routed pairs.
constexpr int kMaxSlots = kMaxTokens * (kTopK + 1);
// Algorithmic bytes of one GGML Q4_0 block.
constexpr int kQ4Block = 18;

struct MatrixDims {
    uint32_t rows, cols;
    uint32_t rows_padded;    // multiple of 64
    uint32_t blocks;         // cols / 32
    uint32_t blocks_padded;  // Bp: 16, 32 or a multiple of 64
    uint32_t lpr;            // lanes per row: min(Bp, 64)
};

inline uint32_t padded_blocks(uint32_t blocks) {
    if (blocks <= 16) return 16;
    if (blocks <= 32) return 32;
    return (blocks + 63) / 64 * 64;
}

inline MatrixDims matrix_dims(uint32_t rows, uint32_t cols) {
    MatrixDims d;
    d.rows = rows;
    d.cols = cols;
    d.rows_padded = (rows + kRowsPerGroup - 1) / kRowsPerGroup * kRowsPerGroup;
    d.blocks = cols / 32;
    d.blocks_padded = padded_blocks(d.blocks);
    d.lpr = d.blocks_padded < 64 ? d.blocks_padded : 64;
    return d;
}
// Byte offsets of nibble (row, block) and of the f16 scale of (row, block).
__host__ __device__ inline size_t nibble_offset(const MatrixDims &d, size_t row, size_t block) {
    return (((row >> 3) * 9 + (row & 7)) * d.blocks_padded + block) * 16;
}
__host__ __device__ inline size_t scale_offset(const MatrixDims &d, size_t row, size_t block) {
    return (((row >> 3) * 9 + 8) * d.blocks_padded + block) * 16 + (row & 7) * 2;
}
inline size_t layout_bytes(const MatrixDims &d) {
    return (size_t)d.rows_padded * d.blocks_padded * kQ4Block;
}

// Q4_K row-lane layout.  A GGML Q4_K matrix is rows x (cols / 256)
// super-blocks of 144 bytes: f16 d, f16 dmin, 12 bytes packing eight 6-bit
// (scale, min) pairs, 128 nibble bytes (format/quant/dequant.rs:139-184).
// Element i of sub-block j (32 elements) decodes to d sc_j q_i - dmin m_j.
// The device copy keeps the Q4_0 geometry with 32-element sub-blocks in
// place of Q4_0 blocks (MatrixDims.blocks = cols / 32):
//   nibble slot (row, sub-block)   16 bytes at nibble_offset(); byte 4i + t
//                                  holds element 2i + 8t (low nibble) and
//                                  2i + 1 + 8t (high nibble) ("class order":
//                                  class c = elements c, c+8, c+16, c+24)
//   scale slot (octet, sub-block)  16 bytes at scale_offset(): per row the
//                                  bytes (sc, m) of that sub-block
// Within an octet, the eight rows of sub-block b sit in permuted positions:
// position p of the nibble and scale slots holds row p ^ (b mod 8)
// (q4k_slot_row), so that the lane that owns sub-block b reads row p ^ k
// (k = b mod 8) into register slot p with the same contiguous wavefront
// loads as the Q4_0 layout, and the eight lanes of a super-block can be
// summed with a select-free butterfly (lane k keeps row k).
//   (d, dmin) table                after the octet chunks: per (octet,
//                                  super-block) 32 bytes, per row f16 d then
//                                  f16 dmin
// 148 bytes per 256 elements and row (GGML: 144); every bit is kept and
// tqf_hip_q4k_weights_download() re-packs the GGML bytes.
constexpr int kQ4KBlock = 144;
// The nibble_offset()/scale_offset() row argument under which row r of
// sub-block b is stored.
__host__ __device__ inline size_t q4k_slot_row(size_t row, size_t block) {
    return (row & ~(size_t)7) | ((row ^ block) & 7);
}
__host__ __device__ inline size_t q4k_dm_base(const MatrixDims &d) {
    return (size_t)(d.rows_padded >> 3) * 9 * d.blocks_padded * 16;
}
__host__ __device__ inline size_t q4k_dm_offset(const MatrixDims &d, size_t row, size_t sb) {
    return q4k_dm_base(d) + (((row >> 3) * (d.blocks_padded >> 3) + sb) * 8 + (row & 7)) * 4;
}
inline size_t q4k_layout_bytes(const MatrixDims &d) {
    return q4k_dm_base(d) + (size_t)d.rows_padded * (d.blocks_padded >> 3) * 4;
}

// Q6_K row-lane layout.  A GGML Q6_K super-block holds 256 weights in 210
// bytes: ql[128] low nibbles, qh[64] two high bits each, sixteen int8 scales
// of 16-element groups, f16 d (format/quant/dequant.rs:190-218); weight i
// decodes to d * scale[i / 16] * (q_i - 32).  The device copy uses 32-element
// sub-blocks (MatrixDims.blocks = cols / 32) and one contiguous chunk of
// 13 * Bp * 16 bytes per row octet:
//   planes 0..7   nibble slot p: [Bp][16 bytes] (class order)
//   planes 8..11  high-bit slots 2q, 2q + 1: [Bp][8 + 8 bytes]
//   plane 12      scales: [Bp][8 positions x 2 int8]
// with the rows of sub-block b in the XOR-permuted positions of the Q4_K
// layout (position p holds row p ^ (b mod 8)), then a d table of 16 bytes per
// (octet, super-block) (8 rows x f16, row order).  210 bytes per 256 weights
// and row, as GGML; tqf_hip_q6k_weights_download() re-packs the GGML bytes.
constexpr int kQ6KBlock = 210;
__host__ __device__ inline size_t q6k_slot_row(size_t row, size_t block) {
    return (row & ~(size_t)7) | ((row ^ block) & 7);
}
__host__ __device__ inline size_t q6k_nibble_offset(const MatrixDims &d, size_t prow, size_t b) {
    return (((prow >> 3) * 13 + (prow & 7)) * d.blocks_padded + b) * 16;
}
__host__ __device__ inline size_t q6k_high_offset(const MatrixDims &d, size_t prow, size_t b) {
    return (((prow >> 3) * 13 + 8 + ((prow & 7) >> 1)) * d.blocks_padded + b) * 16 + (prow & 1) * 8;
}
__host__ __device__ inline size_t q6k_scale_offset(const MatrixDims &d, size_t prow, size_t b) {
    return (((prow >> 3) * 13 + 12) * d.blocks_padded + b) * 16 + (prow & 7) * 2;
}
__host__ __device__ inline size_t q6k_d_base(const MatrixDims &d) {
    return (size_t)(d.rows_padded >> 3) * 13 * d.blocks_padded * 16;
}
__host__ __device__ inline size_t q6k_d_offset(const MatrixDims &d, size_t row, size_t sb) {
    return q6k_d_base(d) + (((row >> 3) * (d.blocks_padded >> 3) + sb) * 8 + (row & 7)) * 2;
}
inline size_t q6k_layout_bytes(const MatrixDims &d) {
    return q6k_d_base(d) + (size_t)(d.rows_padded >> 3) * (d.blocks_padded >> 3) * 16;
}

// Route plan written by the route kernel and read by the expert kernels.
// Work is planned per (expert, token) pair so that every workgroup carries
// the same arithmetic: slots [0, M) are the shared expert for tokens 0..M-1
// (coefficient sigmoid(shared gate logit), experts/mod.rs:1614-1615); then,
// for each distinct routed expert in first-demand order (the union of
// experts/mod.rs:268-275 BatchExpertPlan), one slot per token routed to it
// (coefficient = that token's route weight).  Slots of one expert are
// adjacent, so its second reads come from L2 / Infinity Cache.
// One pair slot as the expert kernels read it: a single 32-byte scalar load.
struct SlotRec {
    const uint8_t *mat[3];  // gate, up, down matrices of the slot's expert
    int32_t token;          // < 0: no work (routing failed)
    float coef;
};
static_assert(sizeof(SlotRec) == 32, "slot record is one s_load_dwordx8");

// Reads a slot record with one 32-byte load, ahead of any use of its fields.
__device__ __forceinline__ SlotRec load_slot(const SlotRec *p) {
    typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
    const u32x8 v = *reinterpret_cast<const u32x8 *>(p);
    return __builtin_bit_cast(SlotRec, v);
}

struct Plan {
    int32_t n_slots;  // 9 * M when routing succeeded, 0 otherwise
    int32_t status;   // 0 or TQF_HIP_ERR_ROUTER
    int32_t n_union;  // distinct routed experts (HBM bytes = (n_union + 1) experts)
    int32_t m;
    int32_t pad[4];
    SlotRec slots[kMaxSlots];
    int32_t slot_expert[kMaxSlots];  // expert index; n_experts = shared
    uint16_t ids[kMaxTokens][kTopK];
    float weights[kMaxTokens][kTopK];
    float gate_logit[kMaxTokens];
    int32_t union_ids[kMaxTokens * kTopK];
    int32_t pair_slot[kMaxTokens * kTopK];  // slot of route (t, k) at index t * kTopK + k
};

// Device-side description of one MoE layer (passed by value to kernels).
struct LayerDev {
    const float *router;             // [n_experts x hidden]
    const float *shared_input_gate;  // [hidden]
    const uint8_t *const *mats;      // [(n_experts + 1) x 3]: gate, up, down
    uint32_t n_experts, hidden, width;
};

// Per-context device scratch (allocated once, grown on demand).
struct Scratch {
    uint32_t *xprep = nullptr;   // [kMaxTokens x padded(hidden/32) x 32]
    uint32_t *hprep = nullptr;   // [kMaxSlots x padded(width/32) x 32]
    uint64_t *logits = nullptr;  // [kMaxTokens x (n_experts + 1)] tagged words (tag << 32 | f32 bits)
    Plan *plan = nullptr;
    float *partial = nullptr;    // [slot groups x kMaxTokens x hidden]
    uint32_t *counters = nullptr;  // last-arriver counters (see kCounter*)
    void *accept = nullptr;      // acceptance partials
    size_t accept_bytes = 0;
    uint32_t hidden = 0, width = 0, experts = 0;
};

struct ProfileSlot {
    hipEvent_t start, stop;
    int kind;
    double fixed_bytes;     // algorithmic bytes independent of the route
    double per_slot_bytes;  // algorithmic bytes per expert slot of the plan
    int ring_index;         // pinned-host copy of plan->n_slots, or -1
};

// Weights arena: large slabs sub-allocated with a bump pointer, released when
// their last allocation is freed (few large hipMallocs for an 18 GB model).
struct Slab {
    uint8_t *base;
    size_t size, used, live;
};

}  // namespace tqf

struct tqf_hip_weights {
    tqf::MatrixDims dims;
    int32_t format;              // TQF_HIP_FORMAT_Q4_0, _Q4_K or _Q6_K
    uint8_t *tiles;              // device: nibble plane, then scale plane
    size_t bytes;
    const uint8_t **d_self;      // device: one-entry table {tiles}
};

struct tqf_hip_tensor {
    float *data;  // device
    size_t count;
};

struct tqf_hip_layer {
    tqf::LayerDev dev;
    const uint8_t **d_mats;  // device array owned by the layer
    int32_t format;          // TQF_HIP_FORMAT_Q4_0 or _Q4_K (every expert of the layer)
};

namespace tqf {
// ---- persistent stack kernel (tqf_stack.hip) -------------------------------
// One launch runs every layer of a stack: per layer three grid-wide phases
// (A: RMSNorm + router logits + activation records; B: routing, computed
// identically by every workgroup, then gate/up per (expert, 32-row block)
// for all of that expert's tokens; C: down per 64-row team with a
// deterministic in-team combine and the residual), separated by grid
// barriers whose waits are time-bounded (a timeout sets `abort`, every
// workgroup then leaves and the launch reports TQF_HIP_ERR_DEVICE).
struct StackLayer {
    const float *router;         // [E x H]
    const float *gate_vec;       // [H]
    const float *norm;           // [H]
    const uint8_t *const *mats;  // [(E + 1) x 3]
};
constexpr int kStackMT = 4;        // tokens of one persistent launch (k <= 3)
constexpr int kStackHidden = 2048; // the persistent kernel's hidden size
constexpr int kStackTeams = kStackHidden / 64;
// Grid-barrier arrivals go through two levels of counters: 256 same-address
// atomics from every compute unit serialise at the coherence point, and
// groups of workgroups (blockIdx mod 8 is one XCD under the round-robin
// dispatch) counting on lines of their own first shorten that chain.
constexpr int kStackBarrierGroups = 8;
struct StackSync {
    uint32_t barrier;  // arrivals (atomic adds only)
    uint32_t exit;
    uint32_t pad0[30];
    uint32_t release;  // epoch released by the last arrival, and the abort flag:
    uint32_t abort;    // one 64-bit poll load, on its own cache line
    uint32_t pad1[30];
    uint32_t step_base;  // layer steps of the launches completed (mod 2^31; the tags' base, tqf_tags.h)
    uint32_t xcd_bad;    // set by a workgroup that is not on XCD blockIdx % 8 (this launch)
    uint32_t pad2[30];
    // first-level arrivals: workgroup b counts on line b % kStackBarrierGroups
    // (one line per group; the last arrival of a group counts on `barrier`)
    uint32_t group[kStackBarrierGroups][32];
};
struct StackArgs {
    const StackLayer *layers;
    uint32_t n_layers, E, F, m;
    const float *h_in;
    float *h;
    uint16_t *ids_out;
    float *w_out;
    int32_t *status;
    uint64_t *lacc;     // [2][kLaccWords] router logits (2^-32 fixed point), by layer parity
    uint32_t *xprep;    // [kStackMT rows of 28 x 64 dwords]
    uint32_t *hprep;    // [9 kStackMT pair rows of 28 x bp_down dwords]
    float *hshared;     // [kStackMT x F] the shared expert's silu(g) * u rows
    uint64_t *partial;  // [teams x members x kStackMT x 64] tagged words (tag << 32 | f32 bits)
    float *ssq;         // [teams x kStackMT] 64-bit words: layer-step tag << 32 | f32 sum of squares
    StackSync *sync;
    uint32_t members;   // workgroups per 64-row team in phase C
    uint32_t fail_at;   // layer whose barrier-B wait workgroup 0 takes as timed out (~0u: none)
    int32_t *dev_status;  // receives TQF_HIP_ERR_DEVICE after a timed-out wait (may be null)
    float *h_save;        // [kStackMT x kStackHidden]: a copy of h_in, written by the prologue
    int32_t *host_flag;   // pinned host word: the last workgroup out writes 1 after an
                          // abort, 0 otherwise (may be null)
};
// Words of one parity of the logit accumulator: kStackMT rows of the 256
// routed experts and the shared-expert gate, then a non-finite flag.
constexpr uint32_t kLaccWords = kStackMT * (256 + 1) + 1;
struct StackScratch {
    StackSync *sync = nullptr;
    uint64_t *lacc = nullptr;
    uint32_t *xprep = nullptr;
    uint32_t *hprep = nullptr;
    float *hshared = nullptr;
    uint64_t *partial = nullptr;
    float *ssq = nullptr;
    float *h_save = nullptr;  // [kStackMT x kStackHidden]
    uint32_t experts = 0, bp_down = 0, members = 0;
};
// Workgroups of a persistent launch (0 if the device cannot co-schedule it)
// and the launcher; `grid` workgroups must be co-resident (they are when the
// device runs nothing else; a grid-barrier wait that times out reports an error).
uint32_t stack_grid(int device, uint32_t bp_down);
hipError_t launch_stack(hipStream_t s, const StackArgs &a, uint32_t grid, uint32_t bp_down);
size_t stack_lds_bytes(uint32_t bp_down, uint32_t members);
}  // namespace tqf

struct tqf_hip_stack {
    std::vector<const tqf_hip_layer *> layers;
    std::vector<const float *> norms;
    uint32_t hidden, width, experts;
    int32_t format;                       // the layers' expert format
    tqf::StackLayer *d_layers = nullptr;  // device copy for the persistent kernel
};

namespace tqf {
struct GraphEntry;
}

struct tqf_hip_ctx {
    int device;
    hipStream_t stream;
    std::string last_error;
    tqf::Scratch scratch;
    // profiling
    bool profiling = false;
    std::vector<tqf::ProfileSlot> prof_pending;
    std::vector<hipEvent_t> event_pool;
    uint64_t prof_launches[TQF_HIP_KERNEL_KINDS] = {};
    double prof_ms[TQF_HIP_KERNEL_KINDS] = {};
    double prof_bytes[TQF_HIP_KERNEL_KINDS] = {};
    int32_t *prof_ring = nullptr;  // pinned host ring of n_slots copies
    int prof_ring_next = 0;
    bool capturing = false;
    std::vector<tqf::GraphEntry *> graphs;
    std::vector<tqf::Slab> slabs;
    // device pointer table for batched GEMV (+ host shadow to skip re-copies)
    const uint8_t **d_table = nullptr;
    std::vector<const uint8_t *> table_shadow;
    size_t table_cap = 0;
    uint32_t *d_gemv_xprep = nullptr;
    size_t gemv_xprep_bytes = 0;
    // Q4_K expert forward: Q8_K records of x and h, gate/up outputs, h
    uint8_t *d_q4k = nullptr;
    size_t q4k_bytes = 0;
    // LM head: Q8_K records of x, per-workgroup top-4 candidates
    uint8_t *d_lm = nullptr;
    size_t lm_bytes = 0;
    // host staging for the synchronous host-pointer entry points
    void *d_stage = nullptr;
    size_t stage_bytes = 0;
    // one-matrix / one-expert layer tables reused by the non-MoE entry points
    const uint8_t **d_adhoc_mats = nullptr;
    tqf::Plan *d_adhoc_plan = nullptr;
    // persistent stack kernel
    tqf::StackScratch stack;
    uint32_t stack_grid = 0;  // 0: not determined yet
    // grouped expert GEMM scratch
    void *d_grouped = nullptr;
    size_t grouped_bytes = 0;
    // reference-exact sampler scratch
    void *d_sample = nullptr;
    size_t sample_bytes = 0;
    // this device's copy of the allocation-free acceptance scratch
    void *noalloc_scratch = nullptr;
    // kernel variant selectors (TQF_HIP_VARIANT_*), from the environment at
    // creation, changed by tqf_hip_set_variant
    int32_t variant[TQF_HIP_VARIANTS] = {1, 1, 1, 1};
    // recovery from a timed-out cross-workgroup wait: pinned host words the
    // kernels report an abort in ([0] the persistent stack, [1] the one-launch
    // acceptance), their device addresses, and the reruns so far
    int32_t *h_flags = nullptr;
    int32_t *d_flags = nullptr;
    uint64_t reruns[2] = {0, 0};
};

namespace tqf {

// Counter array layout: [route launch count (slot 1) | pad | down (one per
// row group, at most hidden / 16)].  The down counters return to zero in the
// workgroup that finishes its kernel; the route kernel's launch count only
// grows (it tags that launch's logit words).
constexpr int kCounterDown = 64;
// [0, 64) route; [64, 64 + hidden / 16) the Q4_0 down kernel; then the Q4_K
// down launch's combine fold, kMaxTokens x (hidden / 64) (token, row tile)
inline size_t counter_fold_offset(uint32_t hidden) { return kCounterDown + hidden / 16; }
inline size_t counter_count(uint32_t hidden) {
    return counter_fold_offset(hidden) + (size_t)kMaxTokens * (hidden / 64);
}

// ---- launchers (defined in the .hip translation units) -------------------
// All are asynchronous on ctx->stream and return a hipError_t.
hipError_t launch_repack(hipStream_t s, const uint8_t *d_aos, const MatrixDims &d,
                         uint8_t *tiles);
hipError_t launch_synth_q4_0(hipStream_t s, const MatrixDims &d, uint32_t tensor_id,
                             uint32_t seed, uint32_t recipe, uint8_t *tiles);
hipError_t launch_prep(hipStream_t s, const float *x, uint32_t m, uint32_t cols,
                       uint32_t blocks_padded, uint32_t *xprep);
hipError_t launch_gemv(hipStream_t s, const uint8_t *const *d_tiles, uint32_t count,
                       const MatrixDims &d, const uint32_t *xprep, uint32_t m, float *y);
// status_out (may be null) is set to TQF_HIP_ERR_ROUTER when routing fails and
// left untouched otherwise (a sticky flag the caller zeroes).
// records = false skips the Q4_0 activation records (xprep), which only the
// Q4_0 gate/up kernel reads; q8 (with its record stride bp8 = the gate/up
// matrices' padded block count) asks for the Q8_K records of the (normed)
// rows as well, which the Q4_K gate/up reads.
hipError_t launch_route(hipStream_t s, const LayerDev &L, const float *h, const float *norm,
                        uint32_t m, Scratch &sc, uint16_t *ids_out, float *w_out,
                        int32_t *status_out, bool records = true, uint32_t *q8 = nullptr,
                        uint32_t bp8 = 0);
// gate/up needs the gate/up matrices' padded block count (hidden / 32) and the
// down matrix's (width / 32) in {16, 32, 64}; other shapes return
// hipErrorInvalidValue (callers validate first).
// `slots` is the number of pair slots the grid covers (9 M for a MoE layer);
// a slot whose record has token < 0 does no work.
hipError_t launch_gate_up(hipStream_t s, const LayerDev &L, uint32_t slots, const Plan *plan,
                          const uint32_t *xprep, uint32_t *hprep);
hipError_t launch_down(hipStream_t s, const LayerDev &L, uint32_t m, uint32_t slots, Scratch &sc,
                       const Plan *plan, const uint32_t *hprep, const float *resid, float *out);
size_t accept_scratch_bytes(uint32_t k, uint32_t vocab);
void accept_warm();
hipError_t launch_embed_rows(hipStream_t s, const uint8_t *tiles, const MatrixDims &d, const int32_t *tokens,
                             uint32_t n, const float *add, float *out, int32_t *status);
hipError_t launch_rmsnorm_rows(hipStream_t s, const float *x, uint32_t n, uint32_t cols, const float *w,
                               float *out);
// multi = true takes the three-kernel path (no wait between workgroups) even
// where the one-launch kernel applies; scratch must then hold
// accept_multi_scratch_bytes.  host_flag (pinned host word, may be null): the
// one-launch kernel writes 1 there when a wait times out.
hipError_t launch_accept(hipStream_t s, const float *target, const float *draft,
                         const int32_t *dtok, uint32_t k, uint32_t vocab, float temperature,
                         int32_t greedy, const float *u, const float *ures, int32_t *accepted,
                         int32_t *tokens, void *scratch, hipEvent_t ev_start, hipEvent_t ev_stop,
                         bool multi = false, int32_t *host_flag = nullptr);
size_t accept_multi_scratch_bytes(uint32_t k, uint32_t vocab);
// Whether launch_accept takes the one-launch kernel (whose workgroups wait on
// one another) for k and vocab.
bool accept_one_launch(uint32_t k, uint32_t vocab);
hipError_t launch_top4(hipStream_t s, const float *logits, uint32_t rows, uint32_t vocab,
                       uint32_t *tokens4, float *logits4);
// Sampler::select (tqf_sample.hip): one token per row of logits [rows x
// vocab] from the uniform u[row]; temperature 0 takes the argmax.  sums (may
// be null) receives each row's two folds.  scratch holds
// sample_scratch_bytes(rows, vocab).
size_t sample_scratch_bytes(uint32_t rows, uint32_t vocab);
hipError_t launch_sample_select(hipStream_t s, const float *logits, uint32_t rows, uint32_t vocab,
                                float temperature, const float *u, int32_t *tokens, float *sums, void *scratch);

// ---- Q4_K (tqf_q4k.hip) ----------------------------------------------------
// Activation records: q4k_prep writes the fp32-semantics GEMV's records
// (28 dwords per (token, sub-block), row stride 28 Bp); q8k_quantize writes
// Q8_K records (12 dwords per (token, sub-block), row stride 12 Bp) for
// cols a multiple of 256.
constexpr int kQ8KRecDwords = 12;
hipError_t launch_q4k_repack(hipStream_t s, const uint8_t *d_aos, const MatrixDims &d,
                             uint8_t *tiles);
hipError_t launch_q4k_prep(hipStream_t s, const float *x, uint32_t m, uint32_t cols, uint32_t bp,
                           uint32_t *xprep);
hipError_t launch_q4k_gemv(hipStream_t s, const uint8_t *const *tables, uint32_t count,
                           const MatrixDims &d, const uint32_t *xprep, uint32_t m, float *y);
hipError_t launch_q8k_quantize(hipStream_t s, const float *x, uint32_t m, uint32_t cols,
                               uint32_t bp, uint32_t *q8);
hipError_t launch_q4k_q8k_gemv(hipStream_t s, const uint8_t *const *tables, uint32_t count,
                               const MatrixDims &d, const uint32_t *q8, uint32_t m, float *y);
// quantize_q8_k of h = silu_mul(gate, up) for m rows, gu = [gate rows | up
// rows] ([2 x m x cols]).
hipError_t launch_q8k_swiglu_quantize(hipStream_t s, const float *gu, uint32_t m, uint32_t cols,
                                      uint32_t bp, uint32_t *q8);
// The Q4_K MoE layer over a route plan (n_slots = 9 M slots of launch_route):
// gate and up of every slot (y [2 x n_slots x rows]: gate rows, then up rows;
// the records of the slot's token, q8 [M x 12 Bp]), or down of every slot
// (records of the slot's own h, q8 [n_slots x 12 Bp]; y [n_slots x rows]).
// Down with gu (the gate/up output, [2 x n_slots x cols]) makes each slot's
// records of h = silu_mul(gate, up) in the workgroup instead (q8 unused).
// With out (and counters [M x q4k_fold_tiles(d)], zero between launches),
// the down form also folds in launch_q4k_moe_combine's work (+ resid), so
// out receives the layer output without a combine launch.
hipError_t launch_q4k_q8k_slots(hipStream_t s, const Plan *plan, uint32_t n_slots, bool down,
                                const MatrixDims &d, const uint32_t *q8, float *y,
                                const float *gu = nullptr, float *out = nullptr,
                                const float *resid = nullptr, uint32_t *counters = nullptr);
uint32_t q4k_fold_tiles(const MatrixDims &d);
bool q4k_fold_ok(const MatrixDims &d);  // the down matrix's shape allows the fold
// y[t] = resid[t] (if given) + (shared slot t's down x its coefficient, then
// + route (t, k) down x weight for k = 0..7); nothing when routing failed.
hipError_t launch_q4k_moe_combine(hipStream_t s, const Plan *plan, const float *dn, uint32_t m,
                                  uint32_t hidden, const float *resid, float *y);

// ---- Q6_K (tqf_q6k.hip) ----------------------------------------------------
hipError_t launch_q6k_repack(hipStream_t s, const uint8_t *d_aos, const MatrixDims &d,
                             uint8_t *tiles);
// Q8_K matvec over q8k_quantize records; with top4_scratch (count must be 1,
// q6k_top4_scratch_bytes of it) also the per-row top-4 candidates
// (tokens4 / logits4 [m x 4]).
size_t q6k_top4_scratch_bytes(const MatrixDims &d, uint32_t m);
hipError_t launch_q6k_q8k_gemv(hipStream_t s, const uint8_t *const *tables, uint32_t count,
                               const MatrixDims &d, const uint32_t *q8, uint32_t m, float *y,
                               void *top4_scratch, uint32_t *tokens4, float *logits4);

// ---- grouped expert GEMM (tqf_grouped.hip) --------------------------------
// Scratch views of one call over T tokens (P = 8 T pairs): the expert-sorted
// positions, the tile list, h (bf16 hi and lo, [P x width]) and the
// per-pair expert outputs ([P x hidden] f32).  Shapes: hidden and width
// multiples of 256, at most 256 experts.
struct GroupedBuffers {
    int32_t *pos_of_pair, *pair_of_pos, *n_tiles;
    uint2 *tiles;
    uint16_t *h_hi, *h_lo;
    float *out;
    uint32_t tokens, max_tiles;
};
size_t grouped_scratch_bytes(uint32_t T, uint32_t E, uint32_t H, uint32_t F);
GroupedBuffers grouped_buffers(void *scratch, uint32_t T, uint32_t E, uint32_t H, uint32_t F);
// status (may be null) is set to TQF_HIP_ERR_INVALID when an id is >= E; the
// later kernels then do nothing.
hipError_t launch_grouped_plan(hipStream_t s, const uint16_t *ids, uint32_t T, uint32_t E,
                               const GroupedBuffers &g, int32_t *status);
hipError_t launch_grouped_gate_up(hipStream_t s, const LayerDev &L, const uint16_t *x_bf16,
                                  const GroupedBuffers &g);
hipError_t launch_grouped_down(hipStream_t s, const LayerDev &L, const GroupedBuffers &g);
hipError_t launch_grouped_combine(hipStream_t s, const GroupedBuffers &g, const float *w,
                                  uint32_t T, uint32_t H, float *y);

}  // namespace tqf
