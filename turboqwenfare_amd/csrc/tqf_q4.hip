// tqf_q4.hip -- Q4_0 tile layout, activation prep, GEMV and the three MoE
// layer kernels (route, gate/up + SwiGLU, down + weighted combine) for gfx950.
//
// The matrix tile layout and the integer-dot activation format are described
// in tqf_internal.h.  Every kernel here is HBM-bound: the weight bytes are
// read exactly once with 128-bit loads (one row per lane, 1 KiB per
// wavefront load), all of a wavefront's loads are issued before any math,
// and partial sums are combined through LDS in a fixed order, so results are
// deterministic run to run.
#include <hip/hip_runtime.h>

#include "tqf_device.h"
#include "tqf_internal.h"

namespace tqf {

// ---------------------------------------------------------------------------
// Repack: GGML Q4_0 (rows x B x 18 bytes) -> tile layout.  One thread per
// block; the destination was zero-filled (padding rows/blocks keep scale 0).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t *__restrict__ aos,
                                                     uint32_t rows, uint32_t blocks,
                                                     uint32_t chunks,
                                                     uint8_t *__restrict__ tiles) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)rows * blocks) return;
    const uint32_t r = (uint32_t)(idx / blocks), b = (uint32_t)(idx % blocks);
    const uint8_t *src = aos + idx * kQ4Block;
    uint8_t *tile = tiles + ((size_t)(r / kRowsPerGroup) * chunks + b / kChunkBlocks) * kTileBytes;
    const uint32_t lane = r % kRowsPerGroup, j = b % kChunkBlocks;
    uint8_t *nib = tile + j * 1024 + lane * 16;
#pragma unroll
    for (int i = 0; i < 16; ++i) nib[i] = src[2 + i];
    uint8_t *sc = tile + kTileNibbleBytes + lane * 16 + j * 2;
    sc[0] = src[0];
    sc[1] = src[1];
}

hipError_t launch_repack(hipStream_t s, const uint8_t *d_aos, const MatrixDims &d,
                         uint8_t *tiles) {
    const uint64_t n = (uint64_t)d.rows * (d.cols / 32);
    if (n == 0) return hipSuccess;
    const uint32_t grid = (uint32_t)((n + 255) / 256);
    hipLaunchKernelGGL(repack_kernel, dim3(grid), dim3(256), 0, s, d_aos, d.rows, d.cols / 32,
                       d.chunks, tiles);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Activation prep: x [m x cols] f32 -> xprep [m x blocks_padded x 32 dwords].
// One wavefront handles two blocks (32 lanes each).  Blocks past `cols` are
// written as zero records.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prep_kernel(const float *__restrict__ x, uint32_t cols,
                                                   uint32_t blocks_padded,
                                                   uint32_t *__restrict__ xprep) {
    const uint32_t t = blockIdx.y;
    const uint32_t kb = (blockIdx.x * blockDim.x + threadIdx.x) / 32;
    if (kb >= blocks_padded) return;
    const uint32_t j = threadIdx.x & 31;
    const uint32_t col = kb * 32 + j;
    float v[1] = {col < cols ? x[(size_t)t * cols + col] : 0.0f};
    prep_block<1>(v, (int)j, xprep + ((size_t)t * blocks_padded + kb) * kXprepDwords);
}

hipError_t launch_prep(hipStream_t s, const float *x, uint32_t m, uint32_t cols,
                       uint32_t blocks_padded, uint32_t *xprep) {
    const uint32_t threads = blocks_padded * 32;
    const uint32_t grid = (threads + 255) / 256;
    hipLaunchKernelGGL(prep_kernel, dim3(grid, m), dim3(256), 0, s, x, cols, blocks_padded,
                       xprep);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Shared wavefront body: one tile (64 rows x 8 blocks) of one matrix against
// up to MT tokens.  acc[t] accumulates for token tok[t] (t < m_tok).
// ---------------------------------------------------------------------------
template <int MT>
__device__ __forceinline__ void tile_accumulate(const uint4 (&nib)[kChunkBlocks], const uint4 scl,
                                                uint32_t chunk, const uint32_t *__restrict__ xprep,
                                                uint32_t blocks_per_token,
                                                const int (&tok)[MT], int m_tok,
                                                float (&acc)[MT]) {
#pragma unroll
    for (int j = 0; j < kChunkBlocks; ++j) {
        const float d = tile_scale(scl, j);
        const uint32_t kb = chunk * kChunkBlocks + j;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (t < m_tok) {
                const uint32_t *xp =
                    xprep + ((size_t)tok[t] * blocks_per_token + kb) * kXprepDwords;
                acc[t] = fmaf(d, q4_block_dot(nib[j], xp), acc[t]);
            }
        }
    }
}

__device__ __forceinline__ void load_tile(const uint8_t *tile, int lane,
                                          uint4 (&nib)[kChunkBlocks], uint4 &scl) {
    const uint8_t *p = tile + lane * 16;
#pragma unroll
    for (int j = 0; j < kChunkBlocks; ++j) nib[j] = load_u4(p + j * 1024);
    scl = load_u4(p + kTileNibbleBytes);
}

// ---------------------------------------------------------------------------
// Standalone GEMV / small-M GEMM: y[mat][t][row] for `count` matrices of one
// shape.  Grid (row groups, count); block = W wavefronts, wavefront w takes
// chunks w, w + W, ...; partials meet in LDS and are summed in wave order.
// ---------------------------------------------------------------------------
template <int MT>
__global__ __launch_bounds__(512) void gemv_kernel(const uint8_t *const *__restrict__ tables,
                                                   MatrixDims d,
                                                   const uint32_t *__restrict__ xprep,
                                                   uint32_t m, float *__restrict__ y) {
    __shared__ float red[8][MT][kWave];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int waves = blockDim.x / kWave;
    const uint32_t g = blockIdx.x, mat = blockIdx.y;
    const uint8_t *tiles = tables[mat];
    const uint32_t bpt = d.chunks * kChunkBlocks;
    int tok[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) tok[t] = t;
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
    for (uint32_t c = wave; c < d.chunks; c += waves) {
        uint4 nib[kChunkBlocks], scl;
        load_tile(tiles + ((size_t)g * d.chunks + c) * kTileBytes, lane, nib, scl);
        tile_accumulate<MT>(nib, scl, c, xprep, bpt, tok, (int)m, acc);
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();
    const uint32_t row = g * kRowsPerGroup + lane;
    for (int t = wave; t < (int)m; t += waves) {
        float s = red[0][t][lane];
        for (int w = 1; w < waves; ++w) s += red[w][t][lane];
        if (row < d.rows) y[((size_t)mat * m + t) * d.rows + row] = s;
    }
}

hipError_t launch_gemv(hipStream_t s, const uint8_t *const *d_tiles, uint32_t count,
                       const MatrixDims &d, const uint32_t *xprep, uint32_t m, float *y) {
    const uint32_t waves = d.chunks < 8 ? d.chunks : 8;
    dim3 grid(d.groups, count), block(waves * kWave);
    if (m <= 1)
        hipLaunchKernelGGL(gemv_kernel<1>, grid, block, 0, s, d_tiles, d, xprep, m, y);
    else if (m <= 2)
        hipLaunchKernelGGL(gemv_kernel<2>, grid, block, 0, s, d_tiles, d, xprep, m, y);
    else if (m <= 4)
        hipLaunchKernelGGL(gemv_kernel<4>, grid, block, 0, s, d_tiles, d, xprep, m, y);
    else
        hipLaunchKernelGGL(gemv_kernel<8>, grid, block, 0, s, d_tiles, d, xprep, m, y);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Cross-workgroup hand-off without whole-L2 write-back/invalidate fences.
// Values that another workgroup will read are stored with agent-scope
// atomic stores (coherent at device scope, i.e. not left dirty in one XCD's
// L2), each thread waits for its stores to complete, and only then is the
// device-scope counter incremented; the workgroup that sees the final count
// reads the values back with agent-scope atomic loads.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void store_coherent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// ---------------------------------------------------------------------------
// Route kernel.  One workgroup per two router rows (row n_experts is the
// shared-expert input gate, experts/mod.rs:1614).  Each workgroup
//   1. loads h [m x hidden], applies RMSNorm when `norm` is given
//      (weights.rs:216-239: x * (1/sqrt(mean(x^2) + 1e-6)) * w),
//   2. writes the xprep records of the blocks assigned to it,
//   3. computes its router logits (experts/mod.rs:1491 router matvec).
// The last workgroup to finish turns the logits into routes
// (RouterResult::from_logits, experts/mod.rs:134-167: softmax, stable
// descending top-8 with ties to the lower id, renormalise) and the pair plan.
// ---------------------------------------------------------------------------
constexpr int kRouteRows = 2;

template <int MT>
__global__ __launch_bounds__(256) void route_kernel(LayerDev L, const float *__restrict__ h,
                                                    const float *__restrict__ norm, uint32_t m,
                                                    uint32_t *__restrict__ xprep,
                                                    float *__restrict__ logits,
                                                    Plan *__restrict__ plan,
                                                    uint32_t *__restrict__ counter,
                                                    uint16_t *__restrict__ ids_out,
                                                    float *__restrict__ w_out,
                                                    int32_t *__restrict__ status_out) {
    __shared__ float lds_red[4][MT * kRouteRows];
    __shared__ float lds_norm[4][MT];
    __shared__ int s_last;
    __shared__ int s_bad;
    __shared__ int s_ids[kMaxTokens * kTopK];
    __shared__ float s_w[kMaxTokens * kTopK];

    const int tid = threadIdx.x;
    const uint32_t H = L.hidden, E = L.n_experts;
    const int vpt = (int)(H / 256);  // 1..8 elements per thread
    const uint32_t col0 = (uint32_t)tid * vpt;

    float x[MT][8];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int v = 0; v < 8; ++v)
            x[t][v] = (t < (int)m && v < vpt) ? h[(size_t)t * H + col0 + v] : 0.0f;

    if (norm != nullptr) {
        float ss[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            ss[t] = 0.0f;
#pragma unroll
            for (int v = 0; v < 8; ++v) ss[t] += x[t][v] * x[t][v];
        }
        block_sum_256<MT>(ss, lds_norm);
        float wv[8];
#pragma unroll
        for (int v = 0; v < 8; ++v) wv[v] = v < vpt ? norm[col0 + v] : 0.0f;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const float inv = 1.0f / sqrtf(ss[t] / (float)H + 1e-6f);
#pragma unroll
            for (int v = 0; v < 8; ++v) x[t][v] = x[t][v] * inv * wv[v];
        }
    }

    // 2. xprep of block kb is held by threads [kb * 32/vpt, (kb+1) * 32/vpt).
    const uint32_t KB = H / 32;
    for (uint32_t kb = blockIdx.x; kb < KB; kb += gridDim.x) {
        const int lpb = 32 / vpt;
        const int first = (int)kb * lpb;
        if (tid >= first && tid < first + lpb) {
            for (int t = 0; t < (int)m; ++t) {
                uint32_t *rec = xprep + ((size_t)t * KB + kb) * kXprepDwords;
                if (vpt == 8) {
                    float v8[8];
#pragma unroll
                    for (int v = 0; v < 8; ++v) v8[v] = x[t][v];
                    prep_block<8>(v8, tid - first, rec);
                } else if (vpt == 4) {
                    float v4[4];
#pragma unroll
                    for (int v = 0; v < 4; ++v) v4[v] = x[t][v];
                    prep_block<4>(v4, tid - first, rec);
                } else if (vpt == 2) {
                    float v2[2] = {x[t][0], x[t][1]};
                    prep_block<2>(v2, tid - first, rec);
                } else {
                    float v1[1] = {x[t][0]};
                    prep_block<1>(v1, tid - first, rec);
                }
            }
        }
    }

    // 3. logits of this workgroup's rows.
    float dots[MT * kRouteRows];
#pragma unroll
    for (int rr = 0; rr < kRouteRows; ++rr) {
        const uint32_t r = blockIdx.x * kRouteRows + rr;
        float wv[8];
        const float *wrow = (r < E) ? L.router + (size_t)r * H : L.shared_input_gate;
#pragma unroll
        for (int v = 0; v < 8; ++v) wv[v] = (r <= E && v < vpt) ? wrow[col0 + v] : 0.0f;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            float s = 0.0f;
#pragma unroll
            for (int v = 0; v < 8; ++v) s = fmaf(x[t][v], wv[v], s);
            dots[rr * MT + t] = s;
        }
    }
    block_sum_256<MT * kRouteRows>(dots, lds_red);
    if (tid == 0) {
#pragma unroll
        for (int rr = 0; rr < kRouteRows; ++rr) {
            const uint32_t r = blockIdx.x * kRouteRows + rr;
            if (r <= E)
                for (int t = 0; t < (int)m; ++t)
                    store_coherent(&logits[(size_t)t * (E + 1) + r], dots[rr * MT + t]);
        }
        wait_own_stores();
        s_last = (counter_arrive(counter) == gridDim.x - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;

    // ---- last workgroup: routes and the pair plan --------------------------
    const int wave = tid / kWave, lane = tid % kWave;
    if (tid == 0) s_bad = 0;
    __syncthreads();
    for (int t = wave; t < (int)m; t += 4) {
        const float *lt = logits + (size_t)t * (E + 1);
        float lv[4];
        bool fin = true;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t e = (uint32_t)lane + 64u * i;
            lv[i] = e < E ? load_coherent(lt + e) : -INFINITY;
            if (e < E && !(fabsf(lv[i]) <= 3.402823466e38f)) fin = false;
        }
        if (__any(!fin)) {
            if (lane == 0) s_bad = 1;
            continue;
        }
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
        float psel[kTopK];
        int idsel[kTopK];
#pragma unroll
        for (int k = 0; k < kTopK; ++k) {
            // lane's best: highest p, then lowest id (ids ascend with i)
            float bp = p[0];
            int bid = lane;
#pragma unroll
            for (int i = 1; i < 4; ++i)
                if (p[i] > bp) { bp = p[i]; bid = lane + 64 * i; }
            const float best = group_reduce<64>(bp, MaxOp());
            const int win = group_reduce<64>(bp == best ? bid : 0x7FFFFFFF, MinOp());
            psel[k] = best;
            idsel[k] = win;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (lane + 64 * i == win) p[i] = -1.0f;
        }
        if (lane == 0) {
            float total = -0.0f;
            for (int k = 0; k < kTopK; ++k) total += psel[k];
            float wsum = 0.0f;
            for (int k = 0; k < kTopK; ++k) {
                const float wk = psel[k] / total;
                s_ids[t * kTopK + k] = idsel[k];
                s_w[t * kTopK + k] = wk;
                wsum += wk;
            }
            if (!(fabsf(wsum - 1.0f) <= 1e-4f)) s_bad = 1;
        }
    }
    __syncthreads();
    const int n = (int)m * kTopK;
    if (s_bad) {
        if (tid == 0) {
            plan->n_slots = 0;
            plan->n_union = 0;
            plan->status = TQF_HIP_ERR_ROUTER;
            plan->m = (int)m;
            if (status_out) *status_out = TQF_HIP_ERR_ROUTER;
            counter_reset(counter);
        }
        return;
    }
    // Pair plan, one route entry i = (t, k) per lane of wave 0 (n <= 64).
    if (wave == 0) {
        const int e_i = lane < n ? s_ids[lane] : -1;
        int first = lane, cnt = 0, rank = 0;
        for (int j = 0; j < n; ++j) {
            const int ej = readlane_i(e_i, j);
            if (ej == e_i) {
                ++cnt;
                if (j < lane) ++rank;
                if (j < first) first = j;
            }
        }
        const bool flag = lane < n && first == lane;
        const int fc = flag ? cnt : 0;
        int base = 0, upos = 0;
        for (int j = 0; j < n; ++j) {
            const int fcj = readlane_i(fc, j);
            if (j < first) {
                base += fcj;
                upos += fcj ? 1 : 0;
            }
        }
        const int nu = __builtin_popcountll(__ballot(flag));
        if (lane < n) {
            const int slot = (int)m + base + rank;
            const int t = lane / kTopK, k = lane % kTopK;
            const float wv = s_w[lane];
            plan->slot_expert[slot] = e_i;
            plan->slot_token[slot] = t;
            plan->slot_coef[slot] = wv;
            plan->ids[t][k] = (uint16_t)e_i;
            plan->weights[t][k] = wv;
            if (flag) plan->union_ids[upos] = e_i;
            if (ids_out) ids_out[lane] = (uint16_t)e_i;
            if (w_out) w_out[lane] = wv;
        }
        if (lane < (int)m) {
            const float gl = load_coherent(logits + (size_t)lane * (E + 1) + E);
            plan->gate_logit[lane] = gl;
            plan->slot_expert[lane] = (int)E;
            plan->slot_token[lane] = lane;
            plan->slot_coef[lane] = 1.0f / (1.0f + expf(-gl));
        }
        if (lane == 0) {
            plan->n_union = nu;
            plan->n_slots = (int)m * (kTopK + 1);
            plan->status = 0;
            plan->m = (int)m;
            counter_reset(counter);
        }
    }
}

hipError_t launch_route(hipStream_t s, const LayerDev &L, const float *h, const float *norm,
                        uint32_t m, Scratch &sc, uint16_t *ids_out, float *w_out,
                        int32_t *status_out) {
    const uint32_t grid = (L.n_experts + 1 + kRouteRows - 1) / kRouteRows;
    uint32_t *counter = sc.counters;
#define TQF_ROUTE(MT)                                                                        \
    hipLaunchKernelGGL(route_kernel<MT>, dim3(grid), dim3(256), 0, s, L, h, norm, m, sc.xprep, \
                       sc.logits, sc.plan, counter, ids_out, w_out, status_out)
    if (m <= 1) TQF_ROUTE(1);
    else if (m <= 2) TQF_ROUTE(2);
    else if (m <= 4) TQF_ROUTE(4);
    else TQF_ROUTE(8);
#undef TQF_ROUTE
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// One wavefront's share of a pair slot: chunks [c_begin, c_end) step `step`
// of one matrix for one token.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float slot_dot(const uint8_t *tiles, int lane, uint32_t c_begin,
                                          uint32_t c_end, uint32_t step,
                                          const uint32_t *__restrict__ xp_token) {
    float acc = 0.0f;
    int tok[1] = {0};
    float a[1] = {0.0f};
    for (uint32_t c = c_begin; c < c_end; c += step) {
        uint4 nib[kChunkBlocks], scl;
        load_tile(tiles + (size_t)c * kTileBytes, lane, nib, scl);
        a[0] = 0.0f;
        tile_accumulate<1>(nib, scl, c, xp_token, 0, tok, 1, a);
        acc += a[0];
    }
    return acc;
}

// ---------------------------------------------------------------------------
// Gate/up kernel.  Grid (width/64 row groups, pair slots, K parts).  A
// workgroup holds 2 * W wavefronts: W read the gate matrix and W the up
// matrix, each wavefront one 9 KiB tile (64 rows x 256 columns) at a time.
// Partials meet in LDS; with one K part the workgroup forms
// h = silu(gate) * up (weights.rs:241-259) for its 64 rows and writes h as
// xprep records for the down kernel.  With several K parts (small M, so the
// grid still covers every CU) the parts hand off through device-coherent
// partials and the last part to finish forms h.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void gate_up_kernel(LayerDev L, const Plan *__restrict__ plan,
                                                       const uint32_t *__restrict__ xprep,
                                                       uint32_t *__restrict__ hprep,
                                                       float *__restrict__ gu_partial,
                                                       uint32_t *__restrict__ counters) {
    __shared__ float red[16][kWave];
    __shared__ int s_last;
    const int slot = blockIdx.y;
    if (slot >= plan->n_slots) return;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int waves = blockDim.x / kWave;
    const int wpm = waves / 2;
    const uint32_t g = blockIdx.x, kpart = blockIdx.z, kp = gridDim.z;
    const uint32_t G = gridDim.x;
    const int expert = __builtin_amdgcn_readfirstlane(plan->slot_expert[slot]);
    const int tok = __builtin_amdgcn_readfirstlane(plan->slot_token[slot]);
    const int mat = wave / wpm, wi = wave % wpm;
    const uint32_t chunks = L.hidden / kChunkCols;
    const uint32_t cpk = chunks / kp;
    const uint32_t bpt = L.hidden / 32;
    const uint8_t *tiles = L.mats[expert * 3 + mat] + (size_t)g * chunks * kTileBytes;
    const uint32_t *xp = xprep + (size_t)tok * bpt * kXprepDwords;
    red[wave][lane] = slot_dot(tiles, lane, kpart * cpk + wi, (kpart + 1) * cpk, wpm, xp);
    __syncthreads();
    float gate = 0.0f, up = 0.0f;
    if (wave == 0) {
        for (int w = 0; w < wpm; ++w) {
            gate += red[w][lane];
            up += red[wpm + w][lane];
        }
    }
    if (kp > 1) {
        float *part = gu_partial + ((size_t)(slot * G + g) * 4) * 2 * kWave;
        if (wave == 0) {
            store_coherent(&part[(kpart * 2 + 0) * kWave + lane], gate);
            store_coherent(&part[(kpart * 2 + 1) * kWave + lane], up);
            wait_own_stores();
        }
        __syncthreads();
        uint32_t *ctr = counters + slot * G + g;
        if (threadIdx.x == 0) s_last = (counter_arrive(ctr) == kp - 1) ? 1 : 0;
        __syncthreads();
        if (!s_last) return;
        if (wave == 0) {
            gate = 0.0f;
            up = 0.0f;
            for (uint32_t q = 0; q < kp; ++q) {
                gate += load_coherent(&part[(q * 2 + 0) * kWave + lane]);
                up += load_coherent(&part[(q * 2 + 1) * kWave + lane]);
            }
            if (lane == 0) counter_reset(ctr);
        }
    }
    if (wave == 0) {
        const float hv = (gate / (1.0f + expf(-gate))) * up;
        const uint32_t hb = L.width / 32;
        const uint32_t blk = g * 2 + (uint32_t)(lane >> 5);
        uint32_t *rec = hprep + ((size_t)slot * hb + blk) * kXprepDwords;
        float v1[1] = {hv};
        prep_block<1>(v1, lane & 31, rec);
    }
}

hipError_t launch_gate_up(hipStream_t s, const LayerDev &L, uint32_t m, Scratch &sc,
                          const Plan *plan, const uint32_t *xprep) {
    const uint32_t kp = gate_up_kparts(m, L.hidden);
    const uint32_t cpk = (L.hidden / kChunkCols) / kp;
    const uint32_t wpm = cpk < 8 ? cpk : 8;
    dim3 grid(L.width / kRowsPerGroup, m * (kTopK + 1), kp), block(2 * wpm * kWave);
    hipLaunchKernelGGL(gate_up_kernel, grid, block, 0, s, L, plan, xprep, sc.hprep, sc.gu_partial,
                       sc.counters + counter_gate_up_offset(L.hidden));
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Down kernel.  Grid (hidden/64 row groups, slot groups of `spg` pair
// slots); each wavefront takes one 9 KiB tile (one slot, one 256-column
// chunk of the width).  The workgroup weights each slot by its coefficient
// (shared: sigmoid gate; routed: route weight; experts/mod.rs:1609-1630) and
// sums per token; the last workgroup of a row group sums the slot groups in
// order and adds the residual (runtime.rs:802) when given.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void down_kernel(LayerDev L, const Plan *__restrict__ plan,
                                                    const uint32_t *__restrict__ hprep,
                                                    float *__restrict__ partial,
                                                    uint32_t *__restrict__ counters,
                                                    const float *resid, float *out, uint32_t m,
                                                    uint32_t spg) {
    __shared__ float red[16][kWave];
    __shared__ int s_tok[16];
    __shared__ int s_last;
    const int n_slots = plan->n_slots;
    const int n_sg = (n_slots + (int)spg - 1) / (int)spg;
    const int sg = blockIdx.y;
    if (sg >= n_sg) return;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int waves = blockDim.x / kWave;
    const uint32_t chunks = L.width / kChunkCols;
    const int slot = sg * (int)spg + wave / (int)chunks;
    const uint32_t c = (uint32_t)wave % chunks;
    const uint32_t g = blockIdx.x;
    const uint32_t H = L.hidden;
    const uint32_t hb = L.width / 32;
    float v = 0.0f;
    int tok = -1;
    if (slot < n_slots) {
        const int expert = __builtin_amdgcn_readfirstlane(plan->slot_expert[slot]);
        tok = __builtin_amdgcn_readfirstlane(plan->slot_token[slot]);
        const float coef = plan->slot_coef[slot];
        const uint8_t *tiles = L.mats[expert * 3 + 2] + (size_t)g * chunks * kTileBytes;
        const uint32_t *xp = hprep + (size_t)slot * hb * kXprepDwords;
        v = coef * slot_dot(tiles, lane, c, c + 1, 1, xp);
    }
    red[wave][lane] = v;
    if (lane == 0) s_tok[wave] = tok;
    __syncthreads();
    const uint32_t row = g * kRowsPerGroup + lane;
    for (int t = wave; t < (int)m; t += waves) {
        float p = 0.0f;
        for (int w = 0; w < waves; ++w)
            if (s_tok[w] == t) p += red[w][lane];
        store_coherent(&partial[((size_t)sg * kMaxTokens + t) * H + row], p);
    }
    wait_own_stores();
    __syncthreads();
    if (threadIdx.x == 0) s_last = (counter_arrive(&counters[g]) == (uint32_t)n_sg - 1) ? 1 : 0;
    __syncthreads();
    if (!s_last) return;
    for (int t = wave; t < (int)m; t += waves) {
        float s = 0.0f;
        for (int q = 0; q < n_sg; ++q) s += load_coherent(&partial[((size_t)q * kMaxTokens + t) * H + row]);
        const size_t o = (size_t)t * H + row;
        out[o] = resid ? resid[o] + s : s;
    }
    if (threadIdx.x == 0) counter_reset(&counters[g]);
}

hipError_t launch_down(hipStream_t s, const LayerDev &L, uint32_t m, Scratch &sc,
                       const Plan *plan, const float *resid, float *out) {
    const uint32_t chunks = L.width / kChunkCols;
    uint32_t spg = 16 / chunks;  // at most 16 wavefronts per workgroup
    if (spg > m) spg = m;        // M slots per group: 9 groups for any M
    if (spg == 0) spg = 1;
    const uint32_t n_sg = (m * (kTopK + 1) + spg - 1) / spg;
    dim3 grid(L.hidden / kRowsPerGroup, n_sg), block(spg * chunks * kWave);
    hipLaunchKernelGGL(down_kernel, grid, block, 0, s, L, plan, sc.hprep, sc.partial,
                       sc.counters + kCounterDown, resid, out, m, spg);
    return hipGetLastError();
}

}  // namespace tqf
