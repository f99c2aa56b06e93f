// tqf_q4.hip -- Q4_0 row-lane layout, activation prep, GEMV and the three MoE
// layer kernels (route, gate/up + SwiGLU, down + weighted combine) for gfx950.
//
// The matrix layout and the integer-dot activation format are described in
// tqf_internal.h.  Every kernel here is HBM-bound: the weight bytes are read
// exactly once with 128-bit loads (a row's blocks spread over the lanes, 1 KiB
// per wavefront load), all of a wavefront's loads are issued before any
// math, and partial sums are combined in a fixed order (DPP / permlane
// transposes, then LDS), so results are deterministic run to run.
#include <hip/hip_runtime.h>

#include "tqf_device.h"
#include "tqf_internal.h"

namespace tqf {

// ---------------------------------------------------------------------------
// Repack: GGML Q4_0 (rows x B x 18 bytes) -> row-lane layout.  One thread per
// block; the destination was zero-filled (padding rows/blocks keep scale 0).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t *__restrict__ aos,
                                                     MatrixDims d, uint8_t *__restrict__ dst) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)d.rows * d.blocks) return;
    const uint32_t r = (uint32_t)(idx / d.blocks), b = (uint32_t)(idx % d.blocks);
    const uint8_t *src = aos + idx * kQ4Block;
    uint8_t *nib = dst + nibble_offset(d, r, b);
#pragma unroll
    for (int i = 0; i < 16; ++i) nib[i] = src[2 + i];
    uint8_t *sc = dst + scale_offset(d, r, b);
    sc[0] = src[0];
    sc[1] = src[1];
}

hipError_t launch_repack(hipStream_t s, const uint8_t *d_aos, const MatrixDims &d,
                         uint8_t *dst) {
    const uint64_t n = (uint64_t)d.rows * d.blocks;
    if (n == 0) return hipSuccess;
    const uint32_t grid = (uint32_t)((n + 255) / 256);
    hipLaunchKernelGGL(repack_kernel, dim3(grid), dim3(256), 0, s, d_aos, d, dst);
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
    prep_block<1>(v, (int)j, xprep + (size_t)t * blocks_padded * kXprepDwords, blocks_padded, kb);
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
// Standalone GEMV / small-M GEMM: y[mat][t][row] for `count` matrices of one
// shape.  Grid (row groups, count), eight wavefronts per workgroup.  Lane
// group j (LPR lanes) of a wavefront owns 8 consecutive rows (one octet);
// lane b reads block b (+ LPR, + 2 LPR, ... for long rows) of each of them.
// Per chunk of LPR blocks, every load (8 nibble vectors, the octet's scales
// and the activation records of up to four tokens) is issued before any
// arithmetic; the row sums come out of transpose_reduce, one row per lane.
// Tokens beyond four reuse the weights held in registers.
// ---------------------------------------------------------------------------
constexpr int kGemvWaves = 8;
constexpr int kGemvRows = 8;  // rows per lane group

template <int LPR, int TG>
__global__ __launch_bounds__(kGemvWaves * kWave) void gemv_kernel(
    const uint8_t *const *__restrict__ tables, MatrixDims d, const uint32_t *__restrict__ xprep,
    uint32_t m, float *__restrict__ y) {
    constexpr int G = kWave / LPR;
    constexpr int RW = kGemvRows * G;  // rows per wavefront
    constexpr int NL = kGemvRows;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const uint32_t j = (uint32_t)lane / LPR, b = (uint32_t)lane % LPR;
    const uint32_t mat = blockIdx.y;
    const uint32_t r0 = (blockIdx.x * kGemvWaves + wave) * RW;
    if (r0 >= d.rows_padded) return;
    const RowLane W = row_lane(tables[mat], d.blocks_padded);
    const uint32_t rl = r0 + j * NL;
    const uint32_t row = rl + reduced_index<LPR, NL>(lane);
    const bool writer = reduced_first_copy<LPR, NL>(lane) && row < d.rows;
    const uint32_t chunks = d.blocks_padded / LPR;
    const size_t xstride = (size_t)d.blocks_padded * kXprepDwords;
    for (uint32_t t0 = 0; t0 < m; t0 += TG) {
        float acc[TG][NL];
#pragma unroll
        for (int t = 0; t < TG; ++t)
#pragma unroll
            for (int n = 0; n < NL; ++n) acc[t][n] = 0.0f;
        for (uint32_t c = 0; c < chunks; ++c) {
            const uint32_t blk = c * LPR + b;
            uint4 nib[NL];
#pragma unroll
            for (int n = 0; n < NL; ++n) nib[n] = q4_signed(load_nibbles(W, rl + n, blk));
            const uint4 sc = load_scales(W, rl / 8, blk);
            uint32_t x[TG][28];
#pragma unroll
            for (int t = 0; t < TG; ++t) {
                const uint32_t tt = t0 + t < m ? t0 + t : 0;  // loads stay unconditional
                load_xrec(xprep + tt * xstride, d.blocks_padded, blk, x[t]);
                if (blk >= d.blocks) x[t][24] = 0;  // padding: exactly 0 whatever it holds
            }
            __builtin_amdgcn_sched_barrier(0);  // every load in flight before any math
#pragma unroll
            for (int t = 0; t < TG; ++t)
#pragma unroll
                for (int n = 0; n < NL; ++n)
                    acc[t][n] = fmaf(octet_scale(sc, n), q4_block_dot(nib[n], x[t]), acc[t][n]);
        }
#pragma unroll
        for (int t = 0; t < TG; ++t) {
            const float s = transpose_reduce<LPR, NL>(acc[t]);
            if (writer && t0 + t < m) y[((size_t)mat * m + t0 + t) * d.rows + row] = s;
        }
    }
}

template <int LPR>
hipError_t launch_gemv_lpr(hipStream_t s, const uint8_t *const *d_tables, uint32_t count,
                           const MatrixDims &d, const uint32_t *xprep, uint32_t m, float *y) {
    constexpr uint32_t rows_per_group = kGemvWaves * kGemvRows * (kWave / LPR);
    const dim3 grid((d.rows_padded + rows_per_group - 1) / rows_per_group, count);
    const dim3 block(kGemvWaves * kWave);
    if (m <= 1) hipLaunchKernelGGL((gemv_kernel<LPR, 1>), grid, block, 0, s, d_tables, d, xprep, m, y);
    else if (m <= 2) hipLaunchKernelGGL((gemv_kernel<LPR, 2>), grid, block, 0, s, d_tables, d, xprep, m, y);
    else hipLaunchKernelGGL((gemv_kernel<LPR, 4>), grid, block, 0, s, d_tables, d, xprep, m, y);
    return hipGetLastError();
}

hipError_t launch_gemv(hipStream_t s, const uint8_t *const *d_tables, uint32_t count,
                       const MatrixDims &d, const uint32_t *xprep, uint32_t m, float *y) {
    if (d.lpr == 16) return launch_gemv_lpr<16>(s, d_tables, count, d, xprep, m, y);
    if (d.lpr == 32) return launch_gemv_lpr<32>(s, d_tables, count, d, xprep, m, y);
    return launch_gemv_lpr<64>(s, d_tables, count, d, xprep, m, y);
}

// ---------------------------------------------------------------------------
// Cross-workgroup hand-off without whole-L2 write-back/invalidate fences.
// Values that another workgroup will read are stored with agent-scope
// atomic stores (coherent at device scope, i.e. not left dirty in one XCD's
// L2), each thread waits for its stores to complete, and only then is the
// device-scope counter incremented; the workgroup that sees the final count
// reads the values back with agent-scope atomic loads (store_coherent,
// load_coherent, wait_own_stores, counter_arrive in tqf_device.h).
// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// Route kernel.  One workgroup per two router rows (row n_experts is the
// shared-expert input gate, experts/mod.rs:1614).  Each workgroup
//   1. loads h [m x hidden], applies RMSNorm when `norm` is given
//      (weights.rs:216-239: x * (1/sqrt(mean(x^2) + 1e-6)) * w),
//   2. computes its router logits (experts/mod.rs:1491 router matvec) and
//      stores them as tagged words (tag << 32 | f32 bits; the tag is the
//      launch count with the high bit set, so a word of an earlier launch,
//      or the zeroed allocation, never matches),
//   3. writes the xprep / Q8_K records of the blocks assigned to it
//      (workgroups 1..).
// Workgroup 0 polls every logit word of this launch, turns the logits into
// routes (RouterResult::from_logits, experts/mod.rs:134-167: softmax, stable
// descending top-8 with ties to the lower id, renormalise) and the pair
// plan, and advances the launch count.  The poll is bounded in time; a
// timeout writes a failed plan (TQF_HIP_ERR_DEVICE).
// ---------------------------------------------------------------------------
constexpr int kRouteRows = 2;
constexpr int64_t kRouteSpinLimit = 2000000;  // wall-clock ticks (100 MHz): 20 ms
constexpr int kRouteSeq = 1;                   // the launch count's counter slot

template <int MT>
__global__ __launch_bounds__(256) void route_kernel(LayerDev L, const float *__restrict__ h,
                                                    const float *__restrict__ norm, uint32_t m,
                                                    uint32_t bp, uint32_t *__restrict__ xprep,
                                                    uint64_t *__restrict__ logits,
                                                    Plan *__restrict__ plan,
                                                    uint32_t *__restrict__ counter,
                                                    uint16_t *__restrict__ ids_out,
                                                    float *__restrict__ w_out,
                                                    int32_t *__restrict__ status_out,
                                                    uint32_t *__restrict__ q8, uint32_t bp8) {
    __shared__ float lds_red[4][MT * kRouteRows];
    __shared__ float lds_norm[4][MT];
    __shared__ int s_last;
    __shared__ int s_bad;
    __shared__ int s_ids[kMaxTokens * kTopK];
    __shared__ float s_w[kMaxTokens * kTopK];
    __shared__ float s_gate[kMaxTokens];

    const int tid = threadIdx.x;
    const uint32_t seq = __hip_atomic_load(&counter[kRouteSeq], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t tag = 0x80000000u | (seq & 0x7FFFFFFFu);
    const uint32_t H = L.hidden, E = L.n_experts;
    const int vpt = (int)(H / 256);  // 1..8 elements per thread
    const uint32_t col0 = (uint32_t)tid * vpt;

    // this workgroup's router rows, loaded first so that their latency
    // overlaps the activation loads and the records below
    // (the model geometry, hidden 2048, loads 8 contiguous floats per thread
    // as two 16-byte loads; other widths element by element)
    float wv[kRouteRows][8];
    float x[MT][8];
    if (vpt == 8) {
#pragma unroll
        for (int rr = 0; rr < kRouteRows; ++rr) {
            const uint32_t r = blockIdx.x * kRouteRows + rr;
            const float *wrow = (r < E) ? L.router + (size_t)r * H : L.shared_input_gate;
            const float4 a = r <= E ? *reinterpret_cast<const float4 *>(wrow + col0) : make_float4(0, 0, 0, 0);
            const float4 b = r <= E ? *reinterpret_cast<const float4 *>(wrow + col0 + 4) : make_float4(0, 0, 0, 0);
            wv[rr][0] = a.x; wv[rr][1] = a.y; wv[rr][2] = a.z; wv[rr][3] = a.w;
            wv[rr][4] = b.x; wv[rr][5] = b.y; wv[rr][6] = b.z; wv[rr][7] = b.w;
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const float *xr = h + (size_t)t * H + col0;
            const float4 a = t < (int)m ? *reinterpret_cast<const float4 *>(xr) : make_float4(0, 0, 0, 0);
            const float4 b = t < (int)m ? *reinterpret_cast<const float4 *>(xr + 4) : make_float4(0, 0, 0, 0);
            x[t][0] = a.x; x[t][1] = a.y; x[t][2] = a.z; x[t][3] = a.w;
            x[t][4] = b.x; x[t][5] = b.y; x[t][6] = b.z; x[t][7] = b.w;
        }
    } else {
#pragma unroll
        for (int rr = 0; rr < kRouteRows; ++rr) {
            const uint32_t r = blockIdx.x * kRouteRows + rr;
            const float *wrow = (r < E) ? L.router + (size_t)r * H : L.shared_input_gate;
#pragma unroll
            for (int v = 0; v < 8; ++v) wv[rr][v] = (r <= E && v < vpt) ? wrow[col0 + v] : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int v = 0; v < 8; ++v)
                x[t][v] = (t < (int)m && v < vpt) ? h[(size_t)t * H + col0 + v] : 0.0f;
    }

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

    // 2. logits of this workgroup's rows.
    float dots[MT * kRouteRows];
#pragma unroll
    for (int rr = 0; rr < kRouteRows; ++rr) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            float s = 0.0f;
#pragma unroll
            for (int v = 0; v < 8; ++v) s = fmaf(x[t][v], wv[rr][v], s);
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
                    __hip_atomic_store(&logits[(size_t)t * (E + 1) + r],
                                       ((uint64_t)tag << 32) | __float_as_uint(dots[rr * MT + t]),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // 3. xprep (when asked for) of block kb is held by threads [kb * 32/vpt,
    //    (kb+1) * 32/vpt) of workgroup kb + 1 (workgroup 0 routes); records
    //    are strided by the gate/up matrices' padded block count bp.  The
    //    kernels that read them start after this one ends.
    const uint32_t KB = xprep ? H / 32 : 0;
    for (uint32_t kb = blockIdx.x - 1; blockIdx.x > 0 && kb < KB; kb += gridDim.x - 1) {
        const int lpb = 32 / vpt;
        const int first = (int)kb * lpb;
        if (tid >= first && tid < first + lpb) {
            for (int t = 0; t < (int)m; ++t) {
                uint32_t *rec = xprep + (size_t)t * bp * kXprepDwords;
                if (vpt == 8) {
                    float v8[8];
#pragma unroll
                    for (int v = 0; v < 8; ++v) v8[v] = x[t][v];
                    prep_block<8>(v8, tid - first, rec, bp, kb);
                } else if (vpt == 4) {
                    float v4[4];
#pragma unroll
                    for (int v = 0; v < 4; ++v) v4[v] = x[t][v];
                    prep_block<4>(v4, tid - first, rec, bp, kb);
                } else if (vpt == 2) {
                    float v2[2] = {x[t][0], x[t][1]};
                    prep_block<2>(v2, tid - first, rec, bp, kb);
                } else {
                    float v1[1] = {x[t][0]};
                    prep_block<1>(v1, tid - first, rec, bp, kb);
                }
            }
        }
    }

    // 4. Q8_K records (when asked for): chunk j < m * H / 256 (chunk c = j %
    //    (H / 256) of row t = j / (H / 256)) by workgroup (j + 1) % grid, so
    //    that workgroup 0, which routes, has one only when the grid has no
    //    other workgroup left for it; staged in LDS in the quantizer's lane
    //    order.
    const uint32_t cpr = H / 256;
    const uint32_t jq = blockIdx.x == 0 ? gridDim.x - 1 : blockIdx.x - 1;
    if (q8 != nullptr && jq < m * cpr) {
        __shared__ float s_chunk[256];
        const uint32_t t = jq / cpr, c = jq % cpr;
#pragma unroll
        for (int tt = 0; tt < MT; ++tt)
            if (tt == (int)t)
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                    const uint32_t e = col0 + (uint32_t)v;
                    if (v < vpt && e >= 256 * c && e < 256 * c + 256) s_chunk[e - 256 * c] = x[tt][v];
                }
        __syncthreads();
        if (tid < kWave) {
            const int k = tid >> 3, cc = tid & 7;
            float v4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v4[i] = s_chunk[32 * k + cc + 8 * i];
            q8k_quantize_values(v4, q8 + (size_t)t * bp8 * kQ8KRecDwords, bp8, c);
        }
    }

    if (blockIdx.x != 0) return;

    // ---- workgroup 0: routes and the pair plan ------------------------------
    const int wave = tid / kWave, lane = tid % kWave;
    if (tid == 0) {
        s_bad = 0;
        s_last = 0;  // 1: the poll timed out
    }
    __syncthreads();
    for (int t = wave; t < (int)m; t += 4) {
        // this token's E + 1 words: lane l takes experts l + 64 i, lane 0 also
        // the gate word; until every word carries this launch's tag
        const uint64_t *lt = logits + (size_t)t * (E + 1);
        uint64_t w[5];
        uint32_t need = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if ((uint32_t)lane + 64u * i < E) need |= 1u << i;
        if (lane == 0) need |= 1u << 4;
        int64_t t0 = 0;
        for (uint32_t spin = 1;; ++spin) {
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                if ((need >> i) & 1u) {
                    const uint32_t e = i < 4 ? (uint32_t)lane + 64u * i : E;
                    w[i] = __hip_atomic_load(const_cast<uint64_t *>(lt + e), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
                    if ((uint32_t)(w[i] >> 32) == tag) need &= ~(1u << i);
                }
            }
            if (__all(need == 0)) break;
            if ((spin & 63) == 0) {
                const int64_t now = wall_clock64();
                if (t0 == 0) {
                    t0 = now;
                } else if (now - t0 > kRouteSpinLimit) {
                    if (lane == 0) s_last = 1;
                    break;
                }
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (s_last) continue;
        float lv[4];
        bool fin = true;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t e = (uint32_t)lane + 64u * i;
            lv[i] = e < E ? __uint_as_float((uint32_t)w[i]) : -INFINITY;
            if (e < E && !(fabsf(lv[i]) <= 3.402823466e38f)) fin = false;
        }
        if (lane == 0) s_gate[t] = __uint_as_float((uint32_t)w[4]);
        if (__any(!fin)) {
            if (lane == 0) s_bad = 1;
            continue;
        }
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
        // top-8 by (probability descending, id ascending)
        float psel[kTopK];
        int idsel[kTopK];
        top8_by_probability(p, lane, E, psel, idsel);
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
    if (tid == 0)  // every word of this launch has been read
        __hip_atomic_store(&counter[kRouteSeq], seq + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (s_bad || s_last) {
        const int32_t err = s_last ? TQF_HIP_ERR_DEVICE : TQF_HIP_ERR_ROUTER;
        if (wave == 0)
            for (int i = lane; i < (int)m * (kTopK + 1); i += kWave) plan->slots[i].token = -1;
        if (tid == 0) {
            plan->n_slots = 0;
            plan->n_union = 0;
            plan->status = err;
            plan->m = (int)m;
            if (status_out) *status_out = err;
        }
        return;
    }
    // Pair plan, one route entry i = (t, k) per lane of wave 0 (n <= 64).
    // The entries of one expert as the bits of one mask (broadcast LDS reads):
    // a group starts at its lowest entry; base = the entries of the groups
    // that start earlier, upos = those groups' count.
    if (wave == 0) {
        __shared__ int s_first[kMaxTokens * kTopK];
        const int e_i = lane < n ? s_ids[lane] : -1;
        uint64_t eq = 0;
#pragma unroll
        for (int j = 0; j < MT * kTopK; ++j) eq |= (j < n && s_ids[j] == e_i) ? (1ull << j) : 0ull;
        const int rank = __builtin_popcountll(eq & ((1ull << lane) - 1ull));
        const int first = lane < n ? (int)__builtin_ctzll(eq) : lane;
        const bool flag = lane < n && first == lane;
        const uint64_t F = __ballot(flag);
        const int upos = __builtin_popcountll(F & ((1ull << first) - 1ull));
        s_first[lane] = first;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        int base = 0;
#pragma unroll
        for (int j = 0; j < MT * kTopK; ++j) base += (j < n && s_first[j] < first) ? 1 : 0;
        const int nu = __builtin_popcountll(F);
        if (lane < n) {
            const int slot = (int)m + base + rank;
            const int t = lane / kTopK, k = lane % kTopK;
            const float wv = s_w[lane];
            SlotRec rec;
            rec.mat[0] = L.mats[e_i * 3 + 0];
            rec.mat[1] = L.mats[e_i * 3 + 1];
            rec.mat[2] = L.mats[e_i * 3 + 2];
            rec.token = t;
            rec.coef = wv;
            plan->slots[slot] = rec;
            plan->slot_expert[slot] = e_i;
            plan->pair_slot[lane] = slot;
            plan->ids[t][k] = (uint16_t)e_i;
            plan->weights[t][k] = wv;
            if (flag) plan->union_ids[upos] = e_i;
            if (ids_out) ids_out[lane] = (uint16_t)e_i;
            if (w_out) w_out[lane] = wv;
        }
        if (lane < (int)m) {
            const float gl = s_gate[lane];
            plan->gate_logit[lane] = gl;
            SlotRec rec;
            rec.mat[0] = L.mats[E * 3 + 0];
            rec.mat[1] = L.mats[E * 3 + 1];
            rec.mat[2] = L.mats[E * 3 + 2];
            rec.token = lane;
            rec.coef = 1.0f / (1.0f + expf(-gl));
            plan->slots[lane] = rec;
            plan->slot_expert[lane] = (int)E;
        }
        if (lane == 0) {
            plan->n_union = nu;
            plan->n_slots = (int)m * (kTopK + 1);
            plan->status = 0;
            plan->m = (int)m;
        }
    }
}

hipError_t launch_route(hipStream_t s, const LayerDev &L, const float *h, const float *norm,
                        uint32_t m, Scratch &sc, uint16_t *ids_out, float *w_out,
                        int32_t *status_out, bool records, uint32_t *q8, uint32_t bp8) {
    if (q8 && (m * (L.hidden / 256) > (L.n_experts + 1 + kRouteRows - 1) / kRouteRows || bp8 < L.hidden / 32))
        return hipErrorInvalidValue;
    const uint32_t grid = (L.n_experts + 1 + kRouteRows - 1) / kRouteRows;
    const uint32_t bp = padded_blocks(L.hidden / 32);
    uint32_t *counter = sc.counters;
#define TQF_ROUTE(MT)                                                                        \
    hipLaunchKernelGGL(route_kernel<MT>, dim3(grid), dim3(256), 0, s, L, h, norm, m, bp,          \
                       records ? sc.xprep : nullptr,                                               \
                       sc.logits, sc.plan, counter, ids_out, w_out, status_out, q8, bp8)
    if (m <= 1) TQF_ROUTE(1);
    else if (m <= 2) TQF_ROUTE(2);
    else if (m <= 4) TQF_ROUTE(4);
    else TQF_ROUTE(8);
#undef TQF_ROUTE
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Gate/up kernel.  Grid (width / (64 G) row groups, pair slots), eight
// wavefronts per workgroup; G = 64 / LPR lane groups per wavefront, LPR =
// the gate/up matrices' padded block count (hidden / 32 <= 64).  Lane group
// j of a wavefront owns 8 rows of both matrices: lane b loads block b of each
// row (16 nibble loads), the scales of its block for the 8 rows (one 16-byte
// load per matrix) and the activation record of block b of the slot's token,
// then reduces the 16 block products across the group (value 2n + u: row n,
// u = 0 gate, 1 up).  h = silu(gate) * up (weights.rs:241-259) meets in LDS
// and the first G wavefronts write it as xprep records for the down kernel.
// ---------------------------------------------------------------------------
constexpr int kGateUpWaves = 8;
constexpr int kGateUpRows = 8;  // rows per lane group per matrix

template <int LPR>
__global__ __launch_bounds__(kGateUpWaves * kWave) void gate_up_kernel(
    LayerDev L, const Plan *__restrict__ plan, const uint32_t *__restrict__ xprep,
    uint32_t *__restrict__ hprep, uint32_t rows_padded, uint32_t bp_down) {
    constexpr int G = kWave / LPR;
    constexpr int RW = kGateUpRows * G;  // rows per wavefront per matrix
    constexpr int R = LPR / 16;          // copies of each reduced value
    __shared__ float s_h[kGateUpWaves * RW];
    const int slot = blockIdx.y;
    const SlotRec rec = load_slot(&plan->slots[slot]);
    if (rec.token < 0) return;  // routing failed: no work
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const uint32_t j = (uint32_t)lane / LPR, b = (uint32_t)lane % LPR;
    const int tok = rec.token;
    const uint32_t r0 = (blockIdx.x * kGateUpWaves + wave) * RW;
    if (r0 < rows_padded) {
        const RowLane Wg = row_lane(rec.mat[0], LPR);
        const RowLane Wu = row_lane(rec.mat[1], LPR);
        const uint32_t rl = r0 + j * kGateUpRows;
        uint4 ng[kGateUpRows], nu[kGateUpRows];
#pragma unroll
        for (int n = 0; n < kGateUpRows; ++n) {
            ng[n] = q4_signed(load_nibbles(Wg, rl + n, b));
            nu[n] = q4_signed(load_nibbles(Wu, rl + n, b));
        }
        const uint4 sg = load_scales(Wg, rl / 8, b), su = load_scales(Wu, rl / 8, b);
        uint32_t x[28];
        load_xrec(xprep + (size_t)tok * LPR * kXprepDwords, LPR, b, x);
        if (b >= L.hidden / 32) x[24] = 0;  // padding block: contributes exactly 0
        __builtin_amdgcn_sched_barrier(0);  // every load in flight before any math
        float v[2 * kGateUpRows];
#pragma unroll
        for (int n = 0; n < kGateUpRows; ++n) {
            v[2 * n] = octet_scale(sg, n) * q4_block_dot(ng[n], x);
            v[2 * n + 1] = octet_scale(su, n) * q4_block_dot(nu[n], x);
        }
        const float gate = transpose_reduce<LPR, 2 * kGateUpRows>(v);
        const float up = dpp_f<0x100 + R>(gate);  // row_shl:R -> the up value
        const uint32_t q = (uint32_t)lane % LPR;
        if (q % (2 * R) == 0)
            s_h[wave * RW + j * kGateUpRows + q / (2 * R)] = (gate / (1.0f + expf(-gate))) * up;
    }
    __syncthreads();
    if (wave < G) {
        const uint32_t blk = blockIdx.x * (2 * G) + 2 * wave + (uint32_t)(lane >> 5);
        if (blk < L.width / 32) {
            float hv[1] = {s_h[(2 * wave + (lane >> 5)) * 32 + (lane & 31)]};
            prep_block<1>(hv, lane & 31, hprep + (size_t)slot * bp_down * kXprepDwords, bp_down,
                          blk);
        }
    }
}

hipError_t launch_gate_up(hipStream_t s, const LayerDev &L, uint32_t slots, const Plan *plan,
                          const uint32_t *xprep, uint32_t *hprep) {
    const MatrixDims g = matrix_dims(L.width, L.hidden);
    const MatrixDims dn = matrix_dims(L.hidden, L.width);
    const uint32_t G = kWave / g.lpr;
    const uint32_t rows_per_group = kGateUpWaves * kGateUpRows * G;
    dim3 grid((g.rows_padded + rows_per_group - 1) / rows_per_group, slots);
    dim3 block(kGateUpWaves * kWave);
#define TQF_GU(LPR)                                                                         \
    hipLaunchKernelGGL(gate_up_kernel<LPR>, grid, block, 0, s, L, plan, xprep, hprep,          \
                       g.rows_padded, dn.blocks_padded)
    if (g.blocks_padded == 16) TQF_GU(16);
    else if (g.blocks_padded == 32) TQF_GU(32);
    else if (g.blocks_padded == 64) TQF_GU(64);
    else return hipErrorInvalidValue;
#undef TQF_GU
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Down kernel.  Grid (hidden / (16 G) row groups, slot groups of four pair
// slots), one wavefront per slot.  Lane group j owns 16 consecutive rows of
// the slot's down matrix; lane b reads block b of each (LPR = the padded
// block count of the width, <= 64) against block b of the slot's h records.
// The workgroup weights each slot by its coefficient (shared: sigmoid gate;
// routed: route weight; experts/mod.rs:1609-1630) and sums per token in slot
// order; the last workgroup of a row group sums the slot groups in order and
// adds the residual (runtime.rs:802) when given.
// ---------------------------------------------------------------------------
constexpr int kDownSlots = 4;
constexpr int kDownRows = 16;  // rows per lane group

template <int LPR>
__global__ __launch_bounds__(kDownSlots * kWave) void down_kernel(
    LayerDev L, const Plan *__restrict__ plan, const uint32_t *__restrict__ hprep,
    uint32_t rows_padded, float *__restrict__ partial, uint32_t *__restrict__ counters,
    const float *resid, float *out, uint32_t m, int n_slots) {
    constexpr int G = kWave / LPR;
    constexpr int RW = kDownRows * G;  // rows per workgroup
    __shared__ float red[kDownSlots][RW];
    __shared__ int s_tok[kDownSlots];
    __shared__ int s_last;
    const int n_sg = gridDim.y;  // every workgroup arrives, with or without work
    const int sg = blockIdx.y;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const uint32_t j = (uint32_t)lane / LPR, b = (uint32_t)lane % LPR;
    const int slot = sg * kDownSlots + wave;
    const uint32_t r0 = blockIdx.x * RW;
    const uint32_t H = L.hidden;
    float v = 0.0f;
    const SlotRec rec = load_slot(&plan->slots[slot < n_slots ? slot : 0]);
    const int tok = slot < n_slots ? rec.token : -1;
    if (tok >= 0) {
        const float coef = rec.coef;
        const RowLane W = row_lane(rec.mat[2], LPR);
        const uint32_t rl = r0 + j * kDownRows;
        uint4 nib[kDownRows];
#pragma unroll
        for (int n = 0; n < kDownRows; ++n) nib[n] = q4_signed(load_nibbles(W, rl + n, b));
        const uint4 s0 = load_scales(W, rl / 8, b), s1 = load_scales(W, rl / 8 + 1, b);
        uint32_t x[28];
        load_xrec(hprep + (size_t)slot * LPR * kXprepDwords, LPR, b, x);
        if (b >= L.width / 32) x[24] = 0;  // padding block: contributes exactly 0
        __builtin_amdgcn_sched_barrier(0);  // every load in flight before any math
        float a[kDownRows];
#pragma unroll
        for (int n = 0; n < kDownRows; ++n)
            a[n] = octet_scale(n < 8 ? s0 : s1, n % 8) * q4_block_dot(nib[n], x);
        v = coef * transpose_reduce<LPR, kDownRows>(a);
    }
    if (reduced_first_copy<LPR, kDownRows>(lane))
        red[wave][j * kDownRows + reduced_index<LPR, kDownRows>(lane)] = v;
    if (lane == 0) s_tok[wave] = tok;
    __syncthreads();
    for (int i = threadIdx.x; i < (int)m * RW; i += kDownSlots * kWave) {
        const int t = i / RW, r = i % RW;
        float p = 0.0f;
#pragma unroll
        for (int w = 0; w < kDownSlots; ++w)
            if (s_tok[w] == t) p += red[w][r];
        if (r0 + r < H) store_coherent(&partial[((size_t)sg * kMaxTokens + t) * H + r0 + r], p);
    }
    wait_own_stores();
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = (counter_arrive(&counters[blockIdx.x]) == (uint32_t)n_sg - 1) ? 1 : 0;
    __syncthreads();
    if (!s_last) return;
    for (int i = threadIdx.x; i < (int)m * RW; i += kDownSlots * kWave) {
        const int t = i / RW, r = i % RW;
        if (r0 + r >= H) continue;
        float sum = 0.0f;
        for (int q = 0; q < n_sg; ++q)
            sum += load_coherent(&partial[((size_t)q * kMaxTokens + t) * H + r0 + r]);
        const size_t o = (size_t)t * H + r0 + r;
        out[o] = resid ? resid[o] + sum : sum;
    }
    if (threadIdx.x == 0) counter_reset(&counters[blockIdx.x]);
}

hipError_t launch_down(hipStream_t s, const LayerDev &L, uint32_t m, uint32_t slots, Scratch &sc,
                       const Plan *plan, const uint32_t *hprep, const float *resid, float *out) {
    const MatrixDims dn = matrix_dims(L.hidden, L.width);
    const uint32_t G = kWave / dn.lpr;
    const uint32_t rows_per_group = kDownRows * G;
    const uint32_t n_sg = (slots + kDownSlots - 1) / kDownSlots;
    dim3 grid((dn.rows_padded + rows_per_group - 1) / rows_per_group, n_sg);
    dim3 block(kDownSlots * kWave);
#define TQF_DOWN(LPR)                                                                      \
    hipLaunchKernelGGL(down_kernel<LPR>, grid, block, 0, s, L, plan, hprep, dn.rows_padded, \
                       sc.partial, sc.counters + kCounterDown, resid, out, m, (int)slots)
    if (dn.blocks_padded == 16) TQF_DOWN(16);
    else if (dn.blocks_padded == 32) TQF_DOWN(32);
    else if (dn.blocks_padded == 64) TQF_DOWN(64);
    else return hipErrorInvalidValue;
#undef TQF_DOWN
    return hipGetLastError();
}

}  // namespace tqf
