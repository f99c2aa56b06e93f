// tqf_grouped.hip -- prefill-shaped grouped expert GEMM on the matrix cores.
//
// T tokens, each routed to 8 experts with weights (ids/w given), through one
// prepared MoE layer's routed experts:
//   y[t] = sum_k w[t,k] * down_e(silu(gate_e x_t) * up_e x_t),  e = ids[t,k]
// which is the routed part of Qwen36ResidentMoe::forward
// (experts/mod.rs:1617-1630) over LoadedQwen36Expert::forward
// (model/qwen36/weights.rs:566-610), batched over tokens the way
// Qwen36StreamingMoe::forward_batch (experts/mod.rs:1540-1577) serves a
// prefill chunk.
//
// Kernels (stream-ordered, no host round trip):
//   plan     one workgroup: counting sort of the T*8 (token, k) pairs by
//            expert (stable in pair order), the tile list of 32-pair tiles;
//   gate_up  grid (F / 128 column blocks, tiles): gate and up on bf16 MFMA,
//            SwiGLU, h stored as bf16 hi + lo;
//   down     grid (H / 256 column blocks, tiles): down on bf16 MFMA;
//   combine  y[t] = sum_k w[t,k] * out[pos(t,k)] in route order.
// (Dealing a tile's column blocks to one XCD, so that they share its
// activation rows in one L2, measured no faster: the GEMM kernels are bound
// by per-workgroup latency, not by fetch bandwidth.)
//
// Exactness of the weights.  A Q4_0 block is (q - 8) * d with a per-row,
// per-32-column f16 scale d.  Rounding (q - 8) * d to bf16 would cost 8 bits,
// so the MFMA B operand is the exact bf16 value 128 + q (bit pattern 0x43,q:
// one v_perm_b32 per two elements), the bias is removed by starting each
// block's accumulation from sum_k x_k * (-136) (MFMAs against a constant
// operand, shared by every column tile of the wavefront), and the block's
// fp32 result is scaled by d and accumulated in fp32.  Every product is exact
// (bf16 x bf16 fits fp32); rounding happens only in the fp32 sums.
// Activations: x is bf16 on entry (exact); h is split into bf16 hi + lo
// (16 significant bits), so down runs two MFMAs per 16 k.
//
// v_mfma_f32_32x32x16_bf16 lane layout (l = lane, h = l / 32): A holds row
// l % 32, k = 8h .. 8h + 7; B holds column l % 32, the same k; D holds column
// l % 32, rows 8 (v / 4) + 4h + v % 4 for v = 0..15.  For a Q4 block the two
// MFMAs take k 0..15 (low nibbles of qs bytes 8h..8h+7) and k 16..31 (high
// nibbles of the same bytes).
#include <hip/hip_runtime.h>

#include "tqf_device.h"
#include "tqf_internal.h"

namespace tqf {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTileM = 32;          // pairs per tile (MFMA rows)
constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / kWave;
constexpr uint32_t kNeg136 = 0xC308C308u;  // bf16 pair (-136, -136)

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t *p) {
    const u32x4 v = *(const __attribute__((address_space(1))) u32x4 *)(p);
    return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// This lane's 8 qs bytes of one block (c0 = bytes 0..3, c1 = bytes 4..7 of
// its half) -> B operands 128 + q for k 0..15 (lo) and k 16..31 (hi).
__device__ __forceinline__ void biased_operands(uint32_t c0, uint32_t c1, bf16x8 &lo, bf16x8 &hi) {
    constexpr uint32_t kExp = 0x43434343u, kSel01 = 0x04010400u, kSel23 = 0x04030402u;
    const uint32_t l0 = c0 & 0x0F0F0F0Fu, l1 = c1 & 0x0F0F0F0Fu;
    const uint32_t h0 = (c0 >> 4) & 0x0F0F0F0Fu, h1 = (c1 >> 4) & 0x0F0F0F0Fu;
    const u32x4 a = {__builtin_amdgcn_perm(kExp, l0, kSel01), __builtin_amdgcn_perm(kExp, l0, kSel23),
                     __builtin_amdgcn_perm(kExp, l1, kSel01), __builtin_amdgcn_perm(kExp, l1, kSel23)};
    const u32x4 b = {__builtin_amdgcn_perm(kExp, h0, kSel01), __builtin_amdgcn_perm(kExp, h0, kSel23),
                     __builtin_amdgcn_perm(kExp, h1, kSel01), __builtin_amdgcn_perm(kExp, h1, kSel23)};
    lo = __builtin_bit_cast(bf16x8, a);
    hi = __builtin_bit_cast(bf16x8, b);
}

// Row of D[v] for this lane.
__device__ __forceinline__ int d_row(int v, int half) { return 8 * (v / 4) + 4 * half + (v % 4); }

}  // namespace

// ---- plan: counting sort of the (token, k) pairs by expert ------------------
// Positions are stable in pair order (p = 8 t + k).  The pairs go in batches
// of kPlanRounds x 1024: in each round a wavefront ranks equal experts with
// ballots and the first lane of each peer group writes the group's size to
// the count slot (round, wavefront) of its expert; one thread per expert
// then turns its slots into exclusive prefixes (slot order is pair order),
// so a pair's position is base[e] + the positions of e in earlier batches +
// its slot's prefix + its rank, with three workgroup barriers per batch.
// base[e] is the exclusive scan of the expert counts: with one batch these
// are the slot totals; with more, a first pass counts every pair (one count
// per peer group).  Tile i of expert e covers positions off[e] + 32 i ..
// + rows; a tile entry is {first position, e | rows << 16}.
constexpr int kPlanRounds = 4;
constexpr uint32_t kPlanBatch = kPlanRounds * kPlanThreads;
constexpr int kPlanSlots = kPlanRounds * kPlanWaves;
__global__ __launch_bounds__(kPlanThreads) void gg_plan_kernel(
    const uint16_t *__restrict__ ids, uint32_t pairs, uint32_t E, int32_t *__restrict__ pos_of_pair,
    int32_t *__restrict__ pair_of_pos, uint2 *__restrict__ tiles, int32_t *__restrict__ n_tiles,
    int32_t *__restrict__ status) {
    __shared__ uint16_t cnt[kPlanSlots][256];  // per slot: count of expert e, then its prefix
    __shared__ int32_t hist[256], base[256], tbase[256], done[256], total[256];
    __shared__ int32_t s_bad;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const uint64_t below = (1ull << lane) - 1;
    const bool one = pairs <= kPlanBatch;
    if (tid < 256) {
        hist[tid] = 0;
        done[tid] = 0;
    }
    if (tid == 0) s_bad = 0;
    __syncthreads();
    if (!one) {
        for (uint32_t r = 0; r < pairs; r += kPlanThreads) {
            const uint32_t p = r + tid;
            uint32_t key = 256u;  // no expert
            if (p < pairs) {
                const uint32_t e = ids[p];
                if (e < E) key = e;
                else s_bad = 1;
            }
            const uint64_t peers = match_peers(key);
            if (key < 256u && (peers & below) == 0) atomicAdd(&hist[key], (int)__popcll(peers));
        }
    }
    bool planned = false;
    for (uint32_t b0 = 0; b0 < pairs; b0 += kPlanBatch) {
        uint32_t key[kPlanRounds];
        int rank[kPlanRounds];
#pragma unroll
        for (int i = 0; i < kPlanRounds; ++i) {
            const uint32_t p = b0 + (uint32_t)i * kPlanThreads + tid;
            key[i] = 256u;
            if (p < pairs) {
                const uint32_t e = ids[p];
                if (e < E) key[i] = e;
                else s_bad = 1;
            }
        }
        for (int i = tid; i < kPlanSlots * 256 / 8; i += kPlanThreads)
            reinterpret_cast<uint4 *>(&cnt[0][0])[i] = make_uint4(0, 0, 0, 0);
        __syncthreads();
        if (s_bad) {
            if (tid == 0) {
                *n_tiles = 0;
                if (status) *status = TQF_HIP_ERR_INVALID;
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < kPlanRounds; ++i) {
            const uint64_t peers = match_peers(key[i]);
            rank[i] = __popcll(peers & below);
            if (key[i] < 256u && rank[i] == 0) cnt[i * kPlanWaves + wave][key[i]] = (uint16_t)__popcll(peers);
        }
        __syncthreads();
        if (tid < (int)E) {
            int s = 0;
            for (int v = 0; v < kPlanSlots; ++v) {
                const int c = cnt[v][tid];
                cnt[v][tid] = (uint16_t)s;
                s += c;
            }
            total[tid] = s;
            if (one) hist[tid] = s;
        }
        __syncthreads();
        if (!planned) {
            planned = true;
            if (wave == 0) {  // exclusive scans of pair and tile counts, 4 experts per lane
                int c[4], tc[4], s = 0, ts = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t e = 4 * lane + j;
                    c[j] = e < E ? hist[e] : 0;
                    tc[j] = (c[j] + kTileM - 1) / kTileM;
                    s += c[j];
                    ts += tc[j];
                }
                int is = s, its = ts;
#pragma unroll
                for (int d = 1; d < kWave; d *= 2) {
                    const int a = __shfl_up(is, d), b = __shfl_up(its, d);
                    if (lane >= d) {
                        is += a;
                        its += b;
                    }
                }
                int o = is - s, to = its - ts;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t e = 4 * lane + j;
                    base[e] = o;
                    tbase[e] = to;
                    o += c[j];
                    to += tc[j];
                }
                if (lane == kWave - 1) *n_tiles = its;
            }
            __syncthreads();
            for (uint32_t e = tid; e < E; e += kPlanThreads) {
                const int c = hist[e];
                for (int i = 0; i * kTileM < c; ++i) {
                    const int rows = c - i * kTileM < kTileM ? c - i * kTileM : kTileM;
                    tiles[tbase[e] + i] = make_uint2((uint32_t)(base[e] + i * kTileM), e | ((uint32_t)rows << 16));
                }
            }
        }
#pragma unroll
        for (int i = 0; i < kPlanRounds; ++i) {
            if (key[i] < 256u) {
                const uint32_t p = b0 + (uint32_t)i * kPlanThreads + tid;
                const int pos = base[key[i]] + done[key[i]] + cnt[i * kPlanWaves + wave][key[i]] + rank[i];
                pos_of_pair[p] = pos;
                pair_of_pos[pos] = (int32_t)p;
            }
        }
        __syncthreads();
        if (tid < (int)E) done[tid] += total[tid];
    }
}

// ---- the tiled GEMMs -----------------------------------------------------------
// A workgroup (8 wavefronts) owns one tile (<= 32 pairs of one expert) and 256
// weight rows: gate/up takes 128 width columns of gate (wavefronts 0-3) and
// the same 128 of up (4-7); down takes 256 hidden columns.  Each wavefront
// runs the full K for its own 32 rows (one 32x32 MFMA tile), so there is no
// cross-wave reduction, and the workgroup shares every staged byte.
// K advances in chunks of 4 Q4 blocks (128 k): the workgroup loads chunk
// c + 2 with coalesced 16 B buffer loads into registers while chunk c, in
// LDS, feeds the MFMAs and chunk c + 1 waits in the other register set; one
// barrier per chunk flips the two LDS stages.  While staging, four adjacent
// lanes sum each activation row's 32-element block, so the bias correction
// -136 * sum_k a_k enters the MFMA as its accumulator input (no extra MFMA).
// LDS images of a chunk (pitches padded so that MFMA fragment reads are free
// of bank conflicts):
//   weights  [row][pair p][half h][block of pair][8 B]   (64 B + 16 B pad): a
//            lane's 16 B read for (row n, pair p, half h) is its B operand
//            bytes of both blocks of the pair;
//   scales   [octet][block][8 rows x f16]                (as in HBM);
//   acts     [set][row][128 x bf16]                      (256 B + 16 B pad);
//   xs       [block][half h][16] f32: -136 * block sum over all activation
//            sets of row 8 (v / 4) + 4 h + v % 4 at position v, i.e. already in
//            the D-register order of the lanes of half h (one 64 B read).
constexpr int kChunk = 4;            // Q4 blocks per K chunk
constexpr int kGemmThreads = 512;
constexpr int kGemmWaves = kGemmThreads / kWave;
constexpr int kImgRows = 32 * kGemmWaves;  // weight rows per workgroup
constexpr int kWPitch = 80;
constexpr int kAPitch = 272;
constexpr int kGUCols = kImgRows / 2;      // gate/up: width columns per workgroup
constexpr int kDnCols = kImgRows;          // down: hidden columns per workgroup

template <int NA>
struct GemmStage {
    uint8_t w[kImgRows * kWPitch];
    uint8_t sc[(kImgRows / 8) * kChunk * 16];
    uint8_t a[NA][kTileM * kAPitch];
    float xs[kChunk][2][16];
};
template <int NA>
constexpr size_t gemm_lds_bytes() { return 2 * sizeof(GemmStage<NA>); }

__device__ __forceinline__ uint4 lds_u4(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }
__device__ __forceinline__ bf16x8 lds_bf16x8(const uint8_t *p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
}

// Loads go through buffer descriptors (base and byte range in SGPRs): each
// thread keeps a 32-bit offset per piece for the whole K loop and the chunk
// advances a scalar offset.  A load outside the descriptor's range returns
// zero instead of touching memory.
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_u4(Rsrc r, uint32_t voff, uint32_t soff) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// One chunk in registers.  Thread t stages weight pieces (row, block j) t and
// t + 512 of the 1024, scale piece t % 128 (duplicates write identical bytes:
// no divergent branch, so the pipeline stays in one basic block) and the 16 B
// piece (row t / 16, elements 8 (t % 16) ..) of every activation set.
template <int NA>
struct Chunk {
    uint4 q[2];
    uint4 s;
    uint4 a[NA];
};
// Per-thread offsets of those pieces at k = 0 (the chunk adds b0 * 16 bytes
// to weights and scales, k0 * 2 bytes to activations).
template <int NA>
struct ChunkOffsets {
    uint32_t q[2], s, a;
    int s_mat;  // matrix of the scale piece (uniform per wavefront)
};

template <int MATS, int NA>
__device__ __forceinline__ ChunkOffsets<NA> chunk_offsets(const MatrixDims &dm, uint32_t n0, uint32_t a_row_off,
                                                          int tid) {
    constexpr int kPerMat = kImgRows / MATS;
    ChunkOffsets<NA> o;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int f = i * kGemmThreads + tid, r = f / kChunk, j = f % kChunk;
        o.q[i] = (uint32_t)nibble_offset(dm, n0 + r % kPerMat, j);
    }
    const int sp = tid % ((kImgRows / 8) * kChunk), oct = sp / kChunk, j = sp % kChunk;
    o.s = (uint32_t)scale_offset(dm, n0 + (8 * oct) % kPerMat, j);
    o.s_mat = __builtin_amdgcn_readfirstlane((8 * oct) / kPerMat);
    o.a = a_row_off + (tid % 16) * 16;
    return o;
}

template <int MATS, int NA>
__device__ __forceinline__ void chunk_load(Chunk<NA> &c, const Rsrc (&ws)[MATS], const Rsrc (&as)[NA],
                                           const ChunkOffsets<NA> &o, uint32_t chunk) {
    constexpr int kPerMat = kImgRows / MATS;
    const uint32_t b0 = chunk * kChunk, k0 = b0 * 32;
#pragma unroll
    for (int i = 0; i < 2; ++i) c.q[i] = buf_u4(ws[(kImgRows / 2 * i) / kPerMat], o.q[i], b0 * 16);
    c.s = buf_u4(MATS == 1 || o.s_mat == 0 ? ws[0] : ws[MATS - 1], o.s, b0 * 16);
#pragma unroll
    for (int n = 0; n < NA; ++n) c.a[n] = buf_u4(as[n], o.a, k0 * 2);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

template <int NA>
__device__ __forceinline__ void chunk_store(const Chunk<NA> &c, GemmStage<NA> &st, int tid) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int f = i * kGemmThreads + tid, r = f / kChunk, j = f % kChunk;
        uint8_t *row = st.w + r * kWPitch + (j >> 1) * 32 + (j & 1) * 8;
        *reinterpret_cast<uint2 *>(row) = make_uint2(c.q[i].x, c.q[i].y);        // half 0
        *reinterpret_cast<uint2 *>(row + 16) = make_uint2(c.q[i].z, c.q[i].w);   // half 1
    }
    *reinterpret_cast<uint4 *>(st.sc + (tid % ((kImgRows / 8) * kChunk)) * 16) = c.s;
    const int m = tid / 16, u = tid % 16;
    float sum = 0.0f;
#pragma unroll
    for (int n = 0; n < NA; ++n) {
        *reinterpret_cast<uint4 *>(st.a[n] + m * kAPitch + u * 16) = c.a[n];
        const uint32_t w4[4] = {c.a[n].x, c.a[n].y, c.a[n].z, c.a[n].w};
#pragma unroll
        for (int d = 0; d < 4; ++d) sum += bf16_lo(w4[d]) + bf16_hi(w4[d]);
    }
    // the 4 lanes of one block (pieces 4j .. 4j + 3 of the row) are adjacent;
    // all four store the same sum (no divergent branch in the pipeline)
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    st.xs[u >> 2][(m >> 2) & 1][4 * (m >> 3) + (m & 3)] = -136.0f * sum;
}

// A fragments of block b (0..3 of the chunk) of set n for this lane (row = lane
// % 32, half h): k 0..15 and 16..31 of the block.
__device__ __forceinline__ void a_block(const uint8_t *img, int col, int half, int b, bf16x8 &lo, bf16x8 &hi) {
    const uint8_t *r = img + col * kAPitch + (32 * b + 8 * half) * 2;
    lo = lds_bf16x8(r);
    hi = lds_bf16x8(r + 32);
}

// The correction of every D row of this lane (rows of D[v] are
// 8 (v / 4) + 4 h + v % 4): one contiguous 64 B LDS read into the MFMA's
// accumulator input.
__device__ __forceinline__ f32x16 correction(const float (&xs)[2][16], int half) {
    return *reinterpret_cast<const f32x16 *>(&xs[half][0]);
}

// One chunk of this wavefront's 32-row tile: per block, B operands of its row
// from the weight image, MFMAs over every activation set starting from the
// correction, fp32 scaling by the block's scale.
template <int RG, int NA>
__device__ __forceinline__ void chunk_mma(const GemmStage<NA> &s, uint32_t row, int col, int half,
                                          float (&acc)[4 * RG]) {
#pragma unroll
    for (int p = 0; p < kChunk / 2; ++p) {
        const uint4 q = lds_u4(s.w + row * kWPitch + p * 32 + half * 16);
        const uint16_t *scp = reinterpret_cast<const uint16_t *>(s.sc + ((row >> 3) * kChunk + 2 * p) * 16) + (row & 7);
        const float s0 = f16_to_f32(scp[0]), s1 = f16_to_f32(scp[8]);
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
            const int b = 2 * p + bb;
            bf16x8 lo, hi;
            biased_operands(bb ? q.z : q.x, bb ? q.w : q.y, lo, hi);
            f32x16 t = correction(s.xs[b], half);
#pragma unroll
            for (int n = 0; n < NA; ++n) {
                bf16x8 alo, ahi;
                a_block(s.a[n], col, half, b, alo, ahi);
                t = mfma(alo, lo, t);
                t = mfma(ahi, hi, t);
            }
            const float sb = bb ? s1 : s0;
#pragma unroll
            for (int v = 0; v < 4 * RG; ++v) acc[v] = fmaf(sb, t[v], acc[v]);
            __builtin_amdgcn_sched_barrier(0);  // one block's operands live at a time
        }
    }
}

// The pipelined K loop of one workgroup (chunks even: K is a multiple of 256).
template <int RG, int MATS, int NA>
__device__ __forceinline__ void gemm_tile(GemmStage<NA> *sm, const Rsrc (&ws)[MATS], const Rsrc (&as)[NA],
                                          const ChunkOffsets<NA> &o, uint32_t chunks, uint32_t row,
                                          int tid, int col, int half, float (&acc)[4 * RG]) {
#pragma unroll
    for (int v = 0; v < 4 * RG; ++v) acc[v] = 0.0f;
    Chunk<NA> c0, c1;
    chunk_load<MATS, NA>(c0, ws, as, o, 0);
    chunk_store<NA>(c0, sm[0], tid);
    __syncthreads();
    chunk_load<MATS, NA>(c1, ws, as, o, 1);
    for (uint32_t c = 0; c + 2 < chunks; c += 2) {
        chunk_load<MATS, NA>(c0, ws, as, o, c + 2);
        chunk_mma<RG, NA>(sm[0], row, col, half, acc);
        chunk_store<NA>(c1, sm[1], tid);
        __syncthreads();
        chunk_load<MATS, NA>(c1, ws, as, o, c + 3);
        chunk_mma<RG, NA>(sm[1], row, col, half, acc);
        chunk_store<NA>(c0, sm[0], tid);
        __syncthreads();
    }
    chunk_mma<RG, NA>(sm[0], row, col, half, acc);
    chunk_store<NA>(c1, sm[1], tid);
    __syncthreads();
    chunk_mma<RG, NA>(sm[1], row, col, half, acc);
}

template <int MATS, int NA>
__device__ __forceinline__ void gemm_dispatch(int rg, GemmStage<NA> *sm, const Rsrc (&ws)[MATS],
                                              const Rsrc (&as)[NA], const ChunkOffsets<NA> &o,
                                              uint32_t chunks, uint32_t row, int tid, int col, int half,
                                              float (&acc)[16]) {
    switch (rg) {
        case 1: gemm_tile<1, MATS, NA>(sm, ws, as, o, chunks, row, tid, col, half,
                                       *reinterpret_cast<float(*)[4]>(acc)); break;
        case 2: gemm_tile<2, MATS, NA>(sm, ws, as, o, chunks, row, tid, col, half,
                                       *reinterpret_cast<float(*)[8]>(acc)); break;
        case 3: gemm_tile<3, MATS, NA>(sm, ws, as, o, chunks, row, tid, col, half,
                                       *reinterpret_cast<float(*)[12]>(acc)); break;
        default: gemm_tile<4, MATS, NA>(sm, ws, as, o, chunks, row, tid, col, half, acc); break;
    }
}

// ---- gate/up + SwiGLU --------------------------------------------------------
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(4))) void gg_gate_up_kernel(
    const uint8_t *const *__restrict__ mats, MatrixDims dg, uint32_t mat_bytes,
    const uint16_t *__restrict__ x, uint32_t x_bytes, const int32_t *__restrict__ pair_of_pos,
    const uint2 *__restrict__ tiles, const int32_t *__restrict__ n_tiles, uint32_t H, uint32_t F,
    uint16_t *__restrict__ h_hi, uint16_t *__restrict__ h_lo) {
    extern __shared__ uint4 gg_smem[];
    GemmStage<1> *sm = reinterpret_cast<GemmStage<1> *>(gg_smem);
    if ((int)blockIdx.y >= *n_tiles) return;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave, half = lane >> 5, col = lane & 31;
    const uint2 tl = tiles[blockIdx.y];
    const uint32_t pos0 = tl.x, e = tl.y & 0xFFFFu, rows = tl.y >> 16;
    const Rsrc ws[2] = {make_rsrc(load_global_ptr(mats + e * 3 + 0), mat_bytes),
                        make_rsrc(load_global_ptr(mats + e * 3 + 1), mat_bytes)};
    const Rsrc as[1] = {make_rsrc(x, x_bytes)};
    const uint32_t n0 = blockIdx.x * kGUCols;
    const uint32_t m = tid / 16;  // the activation row this thread stages (clamped to a real row)
    const uint32_t tok = (uint32_t)pair_of_pos[pos0 + (m < rows ? m : 0u)] / kTopK;
    const ChunkOffsets<1> o = chunk_offsets<2, 1>(dg, n0, tok * H * 2, tid);
    const int rg = __builtin_amdgcn_readfirstlane((int)(rows + 7) / 8);
    float acc[16];
    gemm_dispatch<2, 1>(rg, sm, ws, as, o, H / 32 / kChunk, (uint32_t)(32 * wave + col), tid, col, half, acc);
    // SwiGLU: the up wavefronts hand their tile to the gate wavefronts in LDS
    __syncthreads();
    float *xu = reinterpret_cast<float *>(gg_smem);  // [4 waves][16][64]
    if (wave >= kGemmWaves / 2) {
#pragma unroll
        for (int v = 0; v < 16; ++v)
            if (v < 4 * rg) xu[((wave - kGemmWaves / 2) * 16 + v) * kWave + lane] = acc[v];
    }
    __syncthreads();
    if (wave >= kGemmWaves / 2) return;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        if (v >= 4 * rg) break;
        const uint32_t r = (uint32_t)d_row(v, half);
        if (r < rows) {
            const float g = acc[v], u = xu[(wave * 16 + v) * kWave + lane];
            const float hv = (g / (1.0f + expf(-g))) * u;
            const __bf16 hb = (__bf16)hv;
            const __bf16 lb = (__bf16)(hv - (float)hb);
            const size_t off = (size_t)(pos0 + r) * F + n0 + 32 * wave + col;
            h_hi[off] = __builtin_bit_cast(uint16_t, hb);
            h_lo[off] = __builtin_bit_cast(uint16_t, lb);
        }
    }
}

// ---- down ------------------------------------------------------------------
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(4))) void gg_down_kernel(
    const uint8_t *const *__restrict__ mats, MatrixDims dd, uint32_t mat_bytes,
    const uint16_t *__restrict__ h_hi, const uint16_t *__restrict__ h_lo, uint32_t h_bytes,
    const uint2 *__restrict__ tiles, const int32_t *__restrict__ n_tiles, uint32_t H, uint32_t F,
    float *__restrict__ out) {
    extern __shared__ uint4 gg_smem[];
    GemmStage<2> *sm = reinterpret_cast<GemmStage<2> *>(gg_smem);
    if ((int)blockIdx.y >= *n_tiles) return;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave, half = lane >> 5, col = lane & 31;
    const uint2 tl = tiles[blockIdx.y];
    const uint32_t pos0 = tl.x, e = tl.y & 0xFFFFu, rows = tl.y >> 16;
    const Rsrc ws[1] = {make_rsrc(load_global_ptr(mats + e * 3 + 2), mat_bytes)};
    const Rsrc as[2] = {make_rsrc(h_hi, h_bytes), make_rsrc(h_lo, h_bytes)};
    const uint32_t n0 = blockIdx.x * kDnCols;
    const uint32_t m = tid / 16;
    const ChunkOffsets<2> o = chunk_offsets<1, 2>(dd, n0, (pos0 + (m < rows ? m : 0u)) * F * 2, tid);
    const int rg = __builtin_amdgcn_readfirstlane((int)(rows + 7) / 8);
    float acc[16];
    gemm_dispatch<1, 2>(rg, sm, ws, as, o, F / 32 / kChunk, (uint32_t)(32 * wave + col), tid, col, half, acc);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        if (v >= 4 * rg) break;
        const uint32_t r = (uint32_t)d_row(v, half);
        if (r < rows) out[(size_t)(pos0 + r) * H + n0 + 32 * wave + col] = acc[v];
    }
}

// ---- combine: y[t] = sum_k w[t,k] * out[pos(t,k)], k in route order ----------
__global__ __launch_bounds__(256) void gg_combine_kernel(const float *__restrict__ out,
                                                         const int32_t *__restrict__ pos_of_pair,
                                                         const int32_t *__restrict__ n_tiles,
                                                         const float *__restrict__ w, uint32_t T,
                                                         uint32_t H, float *__restrict__ y) {
    if (*n_tiles == 0) return;  // the plan rejected the routes (status is set)
    const uint32_t per_row = H / 4;
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)T * per_row) return;
    const uint32_t t = (uint32_t)(idx / per_row), c = (uint32_t)(idx % per_row) * 4;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
        const int pos = pos_of_pair[t * kTopK + k];
        const float wk = w[t * kTopK + k];
        const float4 v = load_global_f4(out + (size_t)pos * H + c);
        acc.x = acc.x + wk * v.x;
        acc.y = acc.y + wk * v.y;
        acc.z = acc.z + wk * v.z;
        acc.w = acc.w + wk * v.w;
    }
    *reinterpret_cast<float4 *>(y + (size_t)t * H + c) = acc;
}

// ---- host side ----------------------------------------------------------------
namespace {
size_t round256(size_t v) { return (v + 255) / 256 * 256; }
uint32_t max_tiles_for(uint32_t T, uint32_t E) {
    const uint32_t P = T * kTopK;
    return (P + kTileM - 1) / kTileM + (E < P ? E : P);
}
}  // namespace

size_t grouped_scratch_bytes(uint32_t T, uint32_t E, uint32_t H, uint32_t F) {
    const size_t P = (size_t)T * kTopK;
    return 2 * round256(P * 4) + round256((size_t)max_tiles_for(T, E) * 8) + 256 +
           2 * round256(P * F * 2) + round256(P * H * 4);
}

GroupedBuffers grouped_buffers(void *scratch, uint32_t T, uint32_t E, uint32_t H, uint32_t F) {
    const size_t P = (size_t)T * kTopK;
    uint8_t *p = static_cast<uint8_t *>(scratch);
    auto take = [&](size_t bytes) {
        uint8_t *r = p;
        p += round256(bytes);
        return r;
    };
    GroupedBuffers g;
    g.pos_of_pair = reinterpret_cast<int32_t *>(take(P * 4));
    g.pair_of_pos = reinterpret_cast<int32_t *>(take(P * 4));
    g.tokens = T;
    g.max_tiles = max_tiles_for(T, E);
    g.tiles = reinterpret_cast<uint2 *>(take((size_t)g.max_tiles * 8));
    g.n_tiles = reinterpret_cast<int32_t *>(take(256));
    g.h_hi = reinterpret_cast<uint16_t *>(take(P * F * 2));
    g.h_lo = reinterpret_cast<uint16_t *>(take(P * F * 2));
    g.out = reinterpret_cast<float *>(take(P * H * 4));
    return g;
}

hipError_t launch_grouped_plan(hipStream_t s, const uint16_t *ids, uint32_t T, uint32_t E,
                               const GroupedBuffers &g, int32_t *status) {
    hipLaunchKernelGGL(gg_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, ids, T * kTopK, E,
                       g.pos_of_pair, g.pair_of_pos, g.tiles, g.n_tiles, status);
    return hipGetLastError();
}

hipError_t launch_grouped_gate_up(hipStream_t s, const LayerDev &L, const uint16_t *x,
                                  const GroupedBuffers &g) {
    static const hipError_t attr = hipFuncSetAttribute(
        (const void *)gg_gate_up_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_lds_bytes<1>());
    if (attr != hipSuccess) return attr;
    const MatrixDims dg = matrix_dims(L.width, L.hidden);
    hipLaunchKernelGGL(gg_gate_up_kernel, dim3(L.width / kGUCols, g.max_tiles), dim3(kGemmThreads),
                       gemm_lds_bytes<1>(), s, L.mats, dg, (uint32_t)layout_bytes(dg), x,
                       g.tokens * L.hidden * 2, g.pair_of_pos, g.tiles, g.n_tiles, L.hidden,
                       L.width, g.h_hi, g.h_lo);
    return hipGetLastError();
}

hipError_t launch_grouped_down(hipStream_t s, const LayerDev &L, const GroupedBuffers &g) {
    static const hipError_t attr = hipFuncSetAttribute(
        (const void *)gg_down_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_lds_bytes<2>());
    if (attr != hipSuccess) return attr;
    const MatrixDims dd = matrix_dims(L.hidden, L.width);
    hipLaunchKernelGGL(gg_down_kernel, dim3(L.hidden / kDnCols, g.max_tiles), dim3(kGemmThreads),
                       gemm_lds_bytes<2>(), s, L.mats, dd, (uint32_t)layout_bytes(dd), g.h_hi,
                       g.h_lo, g.tokens * kTopK * L.width * 2, g.tiles, g.n_tiles, L.hidden,
                       L.width, g.out);
    return hipGetLastError();
}

hipError_t launch_grouped_combine(hipStream_t s, const GroupedBuffers &g, const float *w,
                                  uint32_t T, uint32_t H, float *y) {
    const uint64_t threads = (uint64_t)T * (H / 4);
    hipLaunchKernelGGL(gg_combine_kernel, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, s,
                       g.out, g.pos_of_pair, g.n_tiles, w, T, H, y);
    return hipGetLastError();
}

}  // namespace tqf
