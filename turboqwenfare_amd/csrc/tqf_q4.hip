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
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
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
// Block-wide reduction of N floats per thread (256 threads); result valid in
// every thread.
// ---------------------------------------------------------------------------
template <int N>
__device__ __forceinline__ void block_sum_256(float (&v)[N], float (*lds)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v[i] += __shfl_xor(v[i], off);
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
// The last workgroup to finish (device-scope counter) turns the logits into
// routes (RouterResult::from_logits, experts/mod.rs:134-167: softmax, stable
// descending top-8 with ties to the lower id, renormalise) and the slot plan
// (union in first-demand order, slot 0 = shared expert with coefficient
// sigmoid(gate logit), routed coefficients = route weights).
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
    __shared__ uint16_t s_ids[kMaxTokens][kTopK];
    __shared__ float s_w[kMaxTokens][kTopK];
    __shared__ int s_slot_of[kMaxExperts];

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
                for (int t = 0; t < (int)m; ++t) logits[(size_t)t * (E + 1) + r] = dots[rr * MT + t];
        }
        __threadfence();
        const uint32_t prev = atomicAdd(counter, 1u);
        s_last = (prev == gridDim.x - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    // ---- last workgroup: routes ------------------------------------------
    const int wave = tid / kWave, lane = tid % kWave;
    if (tid == 0) s_bad = 0;
    for (int e = tid; e < kMaxExperts; e += 256) s_slot_of[e] = -1;
    __syncthreads();
    for (int t = wave; t < (int)m; t += 4) {
        const float *lt = logits + (size_t)t * (E + 1);
        float lv[4];
        bool fin = true;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t e = (uint32_t)lane + 64u * i;
            lv[i] = e < E ? __builtin_nontemporal_load(lt + e) : -INFINITY;
            if (e < E && !(fabsf(lv[i]) <= 3.402823466e38f)) fin = false;
        }
        if (__any(!fin)) {
            if (lane == 0) s_bad = 1;
            continue;
        }
        float mx = fmaxf(fmaxf(lv[0], lv[1]), fmaxf(lv[2], lv[3]));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        float p[4], ssum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t e = (uint32_t)lane + 64u * i;
            p[i] = e < E ? expf(lv[i] - mx) : 0.0f;
            ssum += p[i];
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ssum += __shfl_xor(ssum, off);
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = ((uint32_t)lane + 64u * i < E) ? p[i] / ssum : -1.0f;
        float psel[kTopK];
        int idsel[kTopK];
        for (int k = 0; k < kTopK; ++k) {
            // best of this lane: highest p, then lowest id (ids ascend with i)
            float bp = -1.0f;
            int bid = 0x7FFFFFFF;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (p[i] > bp) { bp = p[i]; bid = lane + 64 * i; }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                const float op = __shfl_xor(bp, off);
                const int oid = __shfl_xor(bid, off);
                if (op > bp || (op == bp && oid < bid)) { bp = op; bid = oid; }
            }
            psel[k] = bp;
            idsel[k] = bid;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (lane + 64 * i == bid) p[i] = -1.0f;
        }
        if (lane == 0) {
            float total = -0.0f;
            for (int k = 0; k < kTopK; ++k) total += psel[k];
            float wsum = 0.0f;
            for (int k = 0; k < kTopK; ++k) {
                const float wk = psel[k] / total;
                s_ids[t][k] = (uint16_t)idsel[k];
                s_w[t][k] = wk;
                wsum += wk;
            }
            if (!(fabsf(wsum - 1.0f) <= 1e-4f)) s_bad = 1;
        }
    }
    __syncthreads();
    if (tid == 0) {
        if (s_bad) {
            plan->n_slots = 0;
            plan->status = TQF_HIP_ERR_ROUTER;
        } else {
            int n = 1;
            plan->slot_expert[0] = (int)E;
            plan->slot_mask[0] = (1u << m) - 1u;
            for (int t = 0; t < kMaxTokens; ++t) {
                const float gl = (t < (int)m) ? logits[(size_t)t * (E + 1) + E] : 0.0f;
                plan->gate_logit[t] = gl;
                plan->coef[0][t] = (t < (int)m) ? 1.0f / (1.0f + expf(-gl)) : 0.0f;
            }
            for (int t = 0; t < (int)m; ++t) {
                for (int k = 0; k < kTopK; ++k) {
                    const int e = s_ids[t][k];
                    int s = s_slot_of[e];
                    if (s < 0) {
                        s = n++;
                        s_slot_of[e] = s;
                        plan->slot_expert[s] = e;
                        plan->slot_mask[s] = 0;
                        for (int tt = 0; tt < kMaxTokens; ++tt) plan->coef[s][tt] = 0.0f;
                    }
                    plan->slot_mask[s] |= 1u << t;
                    plan->coef[s][t] = s_w[t][k];
                    plan->ids[t][k] = (uint16_t)e;
                    plan->weights[t][k] = s_w[t][k];
                }
            }
            plan->n_slots = n;
            plan->status = 0;
        }
        if (status_out && plan->status) *status_out = plan->status;
        *counter = 0u;
    }
    if (ids_out != nullptr || w_out != nullptr) {
        __syncthreads();
        if (!s_bad) {
            for (int i = tid; i < (int)m * kTopK; i += 256) {
                if (ids_out) ids_out[i] = s_ids[i / kTopK][i % kTopK];
                if (w_out) w_out[i] = s_w[i / kTopK][i % kTopK];
            }
        }
    }
}

hipError_t launch_route(hipStream_t s, const LayerDev &L, const float *h, const float *norm,
                        uint32_t m, Scratch &sc, uint16_t *ids_out, float *w_out,
                        int32_t *status_out) {
    const uint32_t grid = (L.n_experts + 1 + kRouteRows - 1) / kRouteRows;
    uint32_t *counter = sc.counters;  // counters[0] belongs to the route kernel
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
// Token list of a slot from its mask (uniform per wavefront).
// ---------------------------------------------------------------------------
template <int MT>
__device__ __forceinline__ int mask_tokens(uint32_t mask, int (&tok)[MT]) {
    int n = 0;
#pragma unroll
    for (int t = 0; t < MT; ++t) tok[t] = 0;
    for (int t = 0; t < kMaxTokens; ++t)
        if ((mask >> t) & 1u) {
            if (n < MT) tok[n] = t;
            ++n;
        }
    return n;
}

// ---------------------------------------------------------------------------
// Gate/up kernel.  Grid (width/64 row groups, slots); 8 wavefronts per
// workgroup: waves 0-3 read the gate matrix, 4-7 the up matrix, each a
// quarter of the hidden dimension.  The epilogue forms
// h = silu(gate) * up (weights.rs:241-259) for 64 rows x the slot's tokens
// and writes h as xprep records for the down kernel.
// ---------------------------------------------------------------------------
template <int MT>
__global__ __launch_bounds__(512) void gate_up_kernel(LayerDev L, const Plan *__restrict__ plan,
                                                      const uint32_t *__restrict__ xprep,
                                                      uint32_t *__restrict__ hprep) {
    __shared__ float red[8][MT][kWave];
    const int slot = blockIdx.y;
    if (slot >= plan->n_slots) return;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const uint32_t g = blockIdx.x;
    const int expert = plan->slot_expert[slot];
    int tok[MT];
    const int m_tok = mask_tokens<MT>(plan->slot_mask[slot], tok);
    const int mat = wave >> 2, quarter = wave & 3;
    const uint32_t chunks = L.hidden / kChunkCols;
    const uint32_t bpt = L.hidden / 32;
    const uint8_t *tiles = L.mats[expert * 3 + mat] + (size_t)g * chunks * kTileBytes;

    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
    for (uint32_t c0 = quarter; c0 < chunks; c0 += 8) {
        const uint32_t c1 = c0 + 4;
        uint4 nib0[kChunkBlocks], scl0, nib1[kChunkBlocks], scl1;
        load_tile(tiles + (size_t)c0 * kTileBytes, lane, nib0, scl0);
        const bool has1 = c1 < chunks;
        if (has1) load_tile(tiles + (size_t)c1 * kTileBytes, lane, nib1, scl1);
        tile_accumulate<MT>(nib0, scl0, c0, xprep, bpt, tok, m_tok, acc);
        if (has1) tile_accumulate<MT>(nib1, scl1, c1, xprep, bpt, tok, m_tok, acc);
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();
    const int ti = wave;
    if (ti < m_tok && ti < MT) {
        const float gate = (red[0][ti][lane] + red[1][ti][lane]) + (red[2][ti][lane] + red[3][ti][lane]);
        const float up = (red[4][ti][lane] + red[5][ti][lane]) + (red[6][ti][lane] + red[7][ti][lane]);
        const float hv = (gate / (1.0f + expf(-gate))) * up;
        const uint32_t hb = L.width / 32;
        const uint32_t blk = g * 2 + (uint32_t)(lane >> 5);
        uint32_t *rec = hprep + (((size_t)slot * kMaxTokens + tok[ti]) * hb + blk) * kXprepDwords;
        float v1[1] = {hv};
        prep_block<1>(v1, lane & 31, rec);
    }
}

hipError_t launch_gate_up(hipStream_t s, const LayerDev &L, uint32_t m, Scratch &sc,
                          const Plan *plan, const uint32_t *xprep) {
    const uint32_t max_slots = m * kTopK + 1;
    dim3 grid(L.width / kRowsPerGroup, max_slots), block(8 * kWave);
    if (m <= 1)
        hipLaunchKernelGGL(gate_up_kernel<1>, grid, block, 0, s, L, plan, xprep, sc.hprep);
    else if (m <= 2)
        hipLaunchKernelGGL(gate_up_kernel<2>, grid, block, 0, s, L, plan, xprep, sc.hprep);
    else if (m <= 4)
        hipLaunchKernelGGL(gate_up_kernel<4>, grid, block, 0, s, L, plan, xprep, sc.hprep);
    else
        hipLaunchKernelGGL(gate_up_kernel<8>, grid, block, 0, s, L, plan, xprep, sc.hprep);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Down kernel.  Grid (hidden/64 row groups, slot groups of 4); wavefront w
// computes slot 4*sg + w over the whole width.  The workgroup combines its
// four slots with the plan coefficients (shared: sigmoid gate; routed: the
// route weight; experts/mod.rs:1609-1630) into one partial per token; the
// last workgroup of a row group (device-scope counter) sums the partials in
// slot-group order and adds the residual (runtime.rs:802) when given.
// ---------------------------------------------------------------------------
template <int MT>
__global__ __launch_bounds__(256) void down_kernel(LayerDev L, const Plan *__restrict__ plan,
                                                   const uint32_t *__restrict__ hprep,
                                                   float *__restrict__ partial,
                                                   uint32_t *__restrict__ counters,
                                                   const float *resid, float *out, uint32_t m) {
    __shared__ float red[4][kMaxTokens][kWave];
    __shared__ int s_last;
    const int n_slots = plan->n_slots;
    const int n_sg = (n_slots + 3) / 4;
    const int sg = blockIdx.y;
    if (sg >= n_sg) return;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const uint32_t g = blockIdx.x;
    const uint32_t H = L.hidden;
    const int slot = sg * 4 + wave;
    const bool active = slot < n_slots;
    for (int t = 0; t < (int)m; ++t) red[wave][t][lane] = 0.0f;
    if (active) {
        const int expert = plan->slot_expert[slot];
        int tok[MT];
        const int m_tok = mask_tokens<MT>(plan->slot_mask[slot], tok);
        const uint32_t chunks = L.width / kChunkCols;
        const uint32_t hb = L.width / 32;
        const uint8_t *tiles = L.mats[expert * 3 + 2] + (size_t)g * chunks * kTileBytes;
        const uint32_t *hp = hprep + (size_t)slot * kMaxTokens * hb * kXprepDwords;
        float acc[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
        for (uint32_t c0 = 0; c0 < chunks; c0 += 2) {
            uint4 nib0[kChunkBlocks], scl0, nib1[kChunkBlocks], scl1;
            load_tile(tiles + (size_t)c0 * kTileBytes, lane, nib0, scl0);
            const bool has1 = c0 + 1 < chunks;
            if (has1) load_tile(tiles + (size_t)(c0 + 1) * kTileBytes, lane, nib1, scl1);
            tile_accumulate<MT>(nib0, scl0, c0, hp, hb, tok, m_tok, acc);
            if (has1) tile_accumulate<MT>(nib1, scl1, c0 + 1, hp, hb, tok, m_tok, acc);
        }
#pragma unroll
        for (int t = 0; t < MT; ++t)
            if (t < m_tok) red[wave][tok[t]][lane] = plan->coef[slot][tok[t]] * acc[t];
    }
    __syncthreads();
    const uint32_t row = g * kRowsPerGroup + lane;
    for (int t = wave; t < (int)m; t += 4) {
        const float p = (red[0][t][lane] + red[1][t][lane]) + (red[2][t][lane] + red[3][t][lane]);
        partial[((size_t)sg * kMaxTokens + t) * H + row] = p;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        const uint32_t prev = atomicAdd(&counters[g], 1u);
        s_last = (prev == (uint32_t)n_sg - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int t = wave; t < (int)m; t += 4) {
        float s = 0.0f;
        for (int q = 0; q < n_sg; ++q)
            s += __builtin_nontemporal_load(&partial[((size_t)q * kMaxTokens + t) * H + row]);
        const size_t o = (size_t)t * H + row;
        out[o] = resid ? resid[o] + s : s;
    }
    if (threadIdx.x == 0) counters[g] = 0u;
}

hipError_t launch_down(hipStream_t s, const LayerDev &L, uint32_t m, Scratch &sc,
                       const Plan *plan, const float *resid, float *out) {
    const uint32_t max_slots = m * kTopK + 1;
    dim3 grid(L.hidden / kRowsPerGroup, (max_slots + 3) / 4), block(4 * kWave);
    uint32_t *counters = sc.counters + 64;  // counters[0..64) belong to the route kernel
#define TQF_DOWN(MT)                                                                          \
    hipLaunchKernelGGL(down_kernel<MT>, grid, block, 0, s, L, plan, sc.hprep, sc.partial,     \
                       counters, resid, out, m)
    if (m <= 1) TQF_DOWN(1);
    else if (m <= 2) TQF_DOWN(2);
    else if (m <= 4) TQF_DOWN(4);
    else TQF_DOWN(8);
#undef TQF_DOWN
    return hipGetLastError();
}

}  // namespace tqf
