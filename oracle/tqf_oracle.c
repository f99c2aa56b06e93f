/*
 * tqf_oracle.c -- TEST INFRASTRUCTURE ONLY (see tqf_oracle.h).
 *
 * CPU restatement of the reference crate's scalar semantics for the MTP
 * speculative-verify path, plus the new k-token acceptance algorithm that the
 * HIP kernels implement.  Built with -O2 -ffp-contract=off so that no a*b+c
 * is fused (Rust never contracts); explicit fmaf() is used only inside the
 * acceptance exponential, whose definition asks for a fused multiply-add.
 *
 * Citations are path:line in the reference checkout.
 */
#include "tqf_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_TOP_K 8
#define ORC_Q4_0_BLOCK_BYTES 18
#define ORC_Q4_0_BLOCK_ELEMS 32
#define ORC_Q4_K_BLOCK_BYTES 144
#define ORC_Q4_K_BLOCK_ELEMS 256

static inline uint32_t f32_bits(float v) { uint32_t b; memcpy(&b, &v, 4); return b; }
static inline float bits_f32(uint32_t b) { float v; memcpy(&v, &b, 4); return v; }

/* ======================================================================= */
/* a1: dequant.rs:19-48 -- binary16 -> binary32 by bit composition.         */
/* ======================================================================= */
float orc_f16_to_f32(uint16_t bits)
{
    uint32_t sign = (bits >> 15) & 0x1u;
    uint32_t exp = (bits >> 10) & 0x1Fu;
    uint32_t frac = bits & 0x3FFu;
    uint32_t out;
    if (exp == 0) {
        if (frac == 0) {
            out = sign << 31;
        } else {
            /* subnormal half: shift until the implicit bit lands */
            int32_t e = -1;
            uint32_t m = frac;
            while ((m & 0x400u) == 0) { m <<= 1; e += 1; }
            m &= 0x3FFu;
            uint32_t exp32 = (uint32_t)(127 - 15 - e);
            out = (sign << 31) | (exp32 << 23) | (m << 13);
        }
    } else if (exp == 0x1F) {
        out = (sign << 31) | (0xFFu << 23) | (frac << 13);
    } else {
        out = (sign << 31) | ((exp + (127 - 15)) << 23) | (frac << 13);
    }
    return bits_f32(out);
}

/* validate.rs:48-69 -- arithmetic twin (deliberately a different method). */
float orc_f16_to_f32_indep(uint16_t bits)
{
    float sign = (bits & 0x8000u) ? -1.0f : 1.0f;
    int exp = (bits >> 10) & 0x1F;
    float frac = (float)(bits & 0x3FF);
    if (exp == 0x1F) {
        return frac == 0.0f ? sign * INFINITY : NAN;
    }
    if (exp == 0) {
        if (frac == 0.0f) return sign * 0.0f;
        return sign * (frac / 1024.0f) * powf(2.0f, -14.0f);
    }
    return sign * (1.0f + frac / 1024.0f) * powf(2.0f, (float)(exp - 15));
}

/* dequant.rs:54-100 -- binary32 -> binary16, round to nearest, ties even. */
uint16_t orc_f32_to_f16(float value)
{
    uint32_t bits = f32_bits(value);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t exponent = (int32_t)((bits >> 23) & 0xFFu);
    uint32_t mantissa = bits & 0x7FFFFFu;

    if (exponent == 0xFF) {
        return (uint16_t)(sign | (mantissa == 0 ? 0x7C00u
                                                : (0x7E00u | ((mantissa >> 13) & 0x01FFu))));
    }
    int32_t half_exponent = exponent - 127 + 15;
    if (half_exponent >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (half_exponent <= 0) {
        if (half_exponent < -10) return sign;
        uint32_t significand = mantissa | 0x800000u;
        uint32_t shift = (uint32_t)(14 - half_exponent);
        uint32_t truncated = significand >> shift;
        uint32_t remainder = significand & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        uint32_t rounded = truncated +
            ((remainder > halfway || (remainder == halfway && (truncated & 1u))) ? 1u : 0u);
        return (uint16_t)(sign | rounded);
    }
    uint32_t truncated = mantissa >> 13;
    uint32_t remainder = mantissa & 0x1FFFu;
    uint32_t rounded = truncated +
        ((remainder > 0x1000u || (remainder == 0x1000u && (truncated & 1u))) ? 1u : 0u);
    uint32_t encoded_exponent = (uint32_t)half_exponent;
    uint32_t encoded_mantissa = rounded;
    if (encoded_mantissa == 0x400u) {
        encoded_exponent += 1;
        encoded_mantissa = 0;
        if (encoded_exponent >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    }
    return (uint16_t)(sign | (encoded_exponent << 10) | encoded_mantissa);
}

/* ======================================================================= */
/* a2: dequant.rs:110-123 -- element j = (qs[j] & 0xF) - 8, j+16 = hi - 8.  */
/* ======================================================================= */
void orc_dequantize_q4_0(const uint8_t *block, float *out)
{
    float d = orc_f16_to_f32((uint16_t)(block[0] | (block[1] << 8)));
    const uint8_t *qs = block + 2;
    for (int j = 0; j < 16; ++j) {
        int x0 = (int)(qs[j] & 0x0F) - 8;
        int x1 = (int)(qs[j] >> 4) - 8;
        out[j] = (float)x0 * d;
        out[j + 16] = (float)x1 * d;
    }
}

/* validate.rs:71-87 -- arithmetic nibble extraction, independent f16. */
void orc_dequantize_q4_0_indep(const uint8_t *block, float *out)
{
    float d = orc_f16_to_f32_indep((uint16_t)(block[0] | (block[1] << 8)));
    const uint8_t *qs = block + 2;
    for (int i = 0; i < 32; ++i) {
        uint8_t byte = qs[i % 16];
        uint8_t nibble = (uint8_t)(i < 16 ? byte % 16 : byte / 16);
        out[i] = ((float)nibble - 8.0f) * d;
    }
}

/* ======================================================================= */
/* a3: weights.rs:617-750 + :827-843 -- Q4_0 matvec_row.                    */
/* ======================================================================= */
static float q4_0_row_dot(const uint8_t *row, uint32_t blocks, const float *x)
{
    float output = 0.0f; /* `let mut output = 0.0;` */
    float decoded[ORC_Q4_0_BLOCK_ELEMS];
    for (uint32_t b = 0; b < blocks; ++b) {
        orc_dequantize_q4_0(row + (size_t)b * ORC_Q4_0_BLOCK_BYTES, decoded);
        const float *v = x + (size_t)b * ORC_Q4_0_BLOCK_ELEMS;
        float partial = -0.0f; /* Iterator::sum::<f32>() seed */
        for (int j = 0; j < ORC_Q4_0_BLOCK_ELEMS; ++j) partial += decoded[j] * v[j];
        output += partial;
    }
    return output;
}

int orc_q4_0_matvec(const uint8_t *w, size_t len, uint32_t rows, uint32_t cols,
                    const float *x, float *y)
{
    if (cols % ORC_Q4_0_BLOCK_ELEMS != 0) return -1;
    size_t blocks = cols / ORC_Q4_0_BLOCK_ELEMS;
    if (len != (size_t)rows * blocks * ORC_Q4_0_BLOCK_BYTES) return -1;
    for (uint32_t r = 0; r < rows; ++r)
        y[r] = q4_0_row_dot(w + (size_t)r * blocks * ORC_Q4_0_BLOCK_BYTES, (uint32_t)blocks, x);
    return 0;
}

/* ======================================================================= */
/* a5: weights.rs:802-808 -- F32 matvec_row (sum seeded with -0.0).          */
/* ======================================================================= */
static float f32_row_dot(const float *row, uint32_t cols, const float *x)
{
    float acc = -0.0f;
    for (uint32_t c = 0; c < cols; ++c) acc += row[c] * x[c];
    return acc;
}

void orc_f32_matvec(const float *w, uint32_t rows, uint32_t cols, const float *x, float *y)
{
    for (uint32_t r = 0; r < rows; ++r) y[r] = f32_row_dot(w + (size_t)r * cols, cols, x);
}

/* ======================================================================= */
/* a6: experts/mod.rs:134-197 -- RouterResult::from_logits + validate.       */
/* ======================================================================= */
int orc_router_validate(const uint16_t *ids, const float *weights)
{
    unsigned char seen[256];
    memset(seen, 0, sizeof seen);
    float total = 0.0f;
    for (int k = 0; k < ORC_TOP_K; ++k) {
        uint32_t index = ids[k];
        if (index >= 256 || seen[index]) return -1;
        float weight = weights[k];
        if (!isfinite(weight) || weight < 0.0f) return -1;
        seen[index] = 1;
        total += weight;
    }
    if (!isfinite(total) || fabsf(total - 1.0f) > 1e-4f) return -1;
    return 0;
}

typedef struct { uint32_t id; float p; } ranked_t;

/* IEEE total order key (f32::total_cmp). */
static inline int32_t total_key(float v)
{
    int32_t b = (int32_t)f32_bits(v);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

int orc_router_from_logits(const float *logits, uint32_t n, uint16_t *ids, float *weights)
{
    if (n != 256) return -1;
    for (uint32_t i = 0; i < n; ++i)
        if (!isfinite(logits[i])) return -1;
    float max = -INFINITY;
    for (uint32_t i = 0; i < n; ++i) max = fmaxf(max, logits[i]);
    float probabilities[256];
    for (uint32_t i = 0; i < n; ++i) probabilities[i] = expf(logits[i] - max);
    float normalizer = -0.0f;
    for (uint32_t i = 0; i < n; ++i) normalizer += probabilities[i];
    ranked_t ranked[256];
    for (uint32_t i = 0; i < n; ++i) { ranked[i].id = i; ranked[i].p = probabilities[i] / normalizer; }
    /* Stable insertion sort: right.total_cmp(left) then left_id < right_id. */
    for (uint32_t i = 1; i < n; ++i) {
        ranked_t cur = ranked[i];
        int32_t key = total_key(cur.p);
        int32_t j = (int32_t)i - 1;
        while (j >= 0) {
            int32_t kj = total_key(ranked[j].p);
            int before = (key > kj) || (key == kj && cur.id < ranked[j].id);
            if (!before) break;
            ranked[j + 1] = ranked[j];
            --j;
        }
        ranked[j + 1] = cur;
    }
    float selected_total = -0.0f;
    for (int k = 0; k < ORC_TOP_K; ++k) selected_total += ranked[k].p;
    for (int k = 0; k < ORC_TOP_K; ++k) {
        ids[k] = (uint16_t)ranked[k].id;
        weights[k] = ranked[k].p / selected_total;
    }
    return orc_router_validate(ids, weights);
}

/* ======================================================================= */
/* a7 / a21 / sigmoid                                                       */
/* ======================================================================= */
void orc_silu_mul(const float *g, const float *u, float *out, uint32_t n)
{
    for (uint32_t i = 0; i < n; ++i) out[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

void orc_qwen_rmsnorm(const float *x, const float *w, uint32_t n, float *out)
{
    float ss = -0.0f;
    for (uint32_t i = 0; i < n; ++i) ss += x[i] * x[i];
    float inv_rms = 1.0f / sqrtf(ss / (float)n + 1e-6f);
    for (uint32_t i = 0; i < n; ++i) out[i] = x[i] * inv_rms * w[i];
}

float orc_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

/* ======================================================================= */
/* a10: weights.rs:566-610 -- gate, up, silu_mul, down.                     */
/* ======================================================================= */
static size_t q4_bytes(uint32_t rows, uint32_t cols)
{
    return (size_t)rows * (cols / ORC_Q4_0_BLOCK_ELEMS) * ORC_Q4_0_BLOCK_BYTES;
}

static void expert_forward_nocheck(const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                                   uint32_t hidden, uint32_t width, const float *x, float *y,
                                   float *scratch /* 3*width */)
{
    float *g = scratch, *u = scratch + width, *h = scratch + 2 * width;
    orc_q4_0_matvec(gate, q4_bytes(width, hidden), width, hidden, x, g);
    orc_q4_0_matvec(up, q4_bytes(width, hidden), width, hidden, x, u);
    orc_silu_mul(g, u, h, width);
    orc_q4_0_matvec(down, q4_bytes(hidden, width), hidden, width, h, y);
}

int orc_expert_forward(const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                       uint32_t hidden, uint32_t width, const float *x, float *y)
{
    if (hidden % ORC_Q4_0_BLOCK_ELEMS || width % ORC_Q4_0_BLOCK_ELEMS) return -1;
    float *scratch = (float *)malloc(sizeof(float) * 3 * width);
    if (!scratch) return -1;
    expert_forward_nocheck(gate, up, down, hidden, width, x, y, scratch);
    free(scratch);
    return 0;
}

/* ======================================================================= */
/* a11 / a12: experts/mod.rs:1540-1577 with the row arithmetic of           */
/* :1600-1634 (shared -> scale -> add_scaled per route in route order).      */
/* ======================================================================= */
uint32_t orc_batch_union(const uint16_t *ids, uint32_t m, uint16_t *out_union)
{
    uint32_t count = 0;
    for (uint32_t t = 0; t < m; ++t) {
        for (int k = 0; k < ORC_TOP_K; ++k) {
            uint16_t e = ids[t * ORC_TOP_K + k];
            int found = 0;
            for (uint32_t i = 0; i < count; ++i) if (out_union[i] == e) { found = 1; break; }
            if (!found) out_union[count++] = e;
        }
    }
    return count;
}

/* Rows of one Q4_0 matrix computed in parallel (OpenMP over rows).  Each
 * row's dot is q4_0_row_dot unchanged, so any thread count is bit-exact. */
static void q4_0_matvec_par(const uint8_t *w, uint32_t rows, uint32_t cols, const float *x,
                            float *y, int nthreads)
{
    uint32_t blocks = cols / ORC_Q4_0_BLOCK_ELEMS;
    size_t row_bytes = (size_t)blocks * ORC_Q4_0_BLOCK_BYTES;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads) if (nthreads > 1)
#endif
    for (int64_t r = 0; r < (int64_t)rows; ++r)
        y[r] = q4_0_row_dot(w + (size_t)r * row_bytes, blocks, x);
    (void)nthreads;
}

typedef int (*moe_matvec_fn)(const uint8_t *w, uint32_t rows, uint32_t cols, const float *x,
                             float *y, int nthreads);

static int q4_0_matvec_fn(const uint8_t *w, uint32_t rows, uint32_t cols, const float *x, float *y,
                          int nthreads)
{
    q4_0_matvec_par(w, rows, cols, x, y, nthreads);
    return 0;
}

/* matvec_payload's Q4_K arm (weights.rs:680-735): quantize_q8_k of x once,
 * then q4_k_dot_pre per row (rows in parallel; each row's arithmetic is
 * that of orc_q4_k_matvec). */
static int q4_k_matvec_fn(const uint8_t *w, uint32_t rows, uint32_t cols, const float *x, float *y,
                          int nthreads)
{
    if (cols % ORC_Q4_K_BLOCK_ELEMS != 0) return -1;
    const uint32_t nb = cols / ORC_Q4_K_BLOCK_ELEMS;
    int8_t *q8 = (int8_t *)malloc((size_t)nb * 256);
    int16_t *sums = (int16_t *)malloc((size_t)nb * 16 * sizeof(int16_t));
    float *scales = (float *)malloc((size_t)nb * sizeof(float));
    if (!q8 || !sums || !scales) {
        free(q8);
        free(sums);
        free(scales);
        return -1;
    }
    for (uint32_t b = 0; b < nb; ++b)
        orc_quantize_q8_k(x + (size_t)b * 256, q8 + (size_t)b * 256, sums + (size_t)b * 16, &scales[b]);
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads) if (nthreads > 1)
#endif
    for (int64_t r = 0; r < (int64_t)rows; ++r)
        y[r] = orc_q4_k_dot_pre(w + (size_t)r * nb * ORC_Q4_K_BLOCK_BYTES, nb, q8, sums, scales);
    (void)nthreads;
    free(q8);
    free(sums);
    free(scales);
    return 0;
}

static int moe_forward_batch_fmt(const orc_moe_layer *L, moe_matvec_fn matvec, const float *x,
                                 uint32_t m, float *y, uint16_t *ids_out, float *w_out,
                                 int nthreads)
{
    const uint32_t H = L->hidden, F = L->width, E = L->n_experts;
    if (nthreads < 1) nthreads = 1;
    float *logits = (float *)malloc(sizeof(float) * E);
    float *g = (float *)malloc(sizeof(float) * F);
    float *u = (float *)malloc(sizeof(float) * F);
    float *h = (float *)malloc(sizeof(float) * F);
    float *routed = (float *)malloc(sizeof(float) * H);
    uint16_t *ids = (uint16_t *)malloc(sizeof(uint16_t) * ORC_TOP_K * (m ? m : 1));
    float *wts = (float *)malloc(sizeof(float) * ORC_TOP_K * (m ? m : 1));
    int rc = 0;
    if (!logits || !g || !u || !h || !routed || !ids || !wts) { rc = -1; goto done; }

    /* Route every row first (forward_batch :1549-1553). */
    for (uint32_t t = 0; t < m; ++t) {
        const float *xt = x + (size_t)t * H;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads) if (nthreads > 1)
#endif
        for (int64_t e = 0; e < (int64_t)E; ++e)
            logits[e] = f32_row_dot(L->router + (size_t)e * H, H, xt);
        if (orc_router_from_logits(logits, E, ids + t * ORC_TOP_K, wts + t * ORC_TOP_K) != 0) {
            rc = -1;
            goto done;
        }
    }
    /* Per row: shared expert, gate scale, routed accumulate in route order. */
    for (uint32_t t = 0; t < m; ++t) {
        const float *xt = x + (size_t)t * H;
        float *out = y + (size_t)t * H;
        if (matvec(L->shared_gate, F, H, xt, g, nthreads) || matvec(L->shared_up, F, H, xt, u, nthreads)) {
            rc = -1;
            goto done;
        }
        orc_silu_mul(g, u, h, F);
        if (matvec(L->shared_down, H, F, h, out, nthreads)) {
            rc = -1;
            goto done;
        }
        float shared_gate_logit = f32_row_dot(L->shared_input_gate, H, xt);
        float scale = 1.0f / (1.0f + expf(-shared_gate_logit));
        for (uint32_t i = 0; i < H; ++i) out[i] *= scale;
        for (int k = 0; k < ORC_TOP_K; ++k) {
            uint32_t e = ids[t * ORC_TOP_K + k];
            float weight = wts[t * ORC_TOP_K + k];
            if (matvec(L->routed_gate[e], F, H, xt, g, nthreads) ||
                matvec(L->routed_up[e], F, H, xt, u, nthreads)) {
                rc = -1;
                goto done;
            }
            orc_silu_mul(g, u, h, F);
            if (matvec(L->routed_down[e], H, F, h, routed, nthreads)) {
                rc = -1;
                goto done;
            }
            for (uint32_t i = 0; i < H; ++i) out[i] += routed[i] * weight;
        }
    }
    if (ids_out) memcpy(ids_out, ids, sizeof(uint16_t) * ORC_TOP_K * m);
    if (w_out) memcpy(w_out, wts, sizeof(float) * ORC_TOP_K * m);
done:
    free(logits); free(g); free(u); free(h); free(routed); free(ids); free(wts);
    return rc;
}

int orc_moe_forward_batch(const orc_moe_layer *L, const float *x, uint32_t m, float *y,
                          uint16_t *ids_out, float *w_out, int nthreads)
{
    return moe_forward_batch_fmt(L, q4_0_matvec_fn, x, m, y, ids_out, w_out, nthreads);
}

int orc_moe_forward_batch_q4k(const orc_moe_layer *L, const float *x, uint32_t m, float *y,
                              uint16_t *ids_out, float *w_out, int nthreads)
{
    return moe_forward_batch_fmt(L, q4_k_matvec_fn, x, m, y, ids_out, w_out, nthreads);
}

int orc_routed_combine(const orc_moe_layer *L, const float *x, uint32_t t, const uint16_t *ids,
                       const float *w, float *y, int nthreads)
{
    const uint32_t H = L->hidden, F = L->width;
    if (nthreads < 1) nthreads = 1;
    for (size_t i = 0; i < (size_t)t * ORC_TOP_K; ++i)
        if (ids[i] >= L->n_experts) return -1;
    int bad = 0;
#ifdef _OPENMP
#pragma omp parallel num_threads(nthreads) if (nthreads > 1)
#endif
    {
        float *scratch = (float *)malloc(sizeof(float) * (3 * (size_t)F + H));
        if (!scratch) {
#ifdef _OPENMP
#pragma omp atomic write
#endif
            bad = 1;
        } else {
            float *routed = scratch + 3 * (size_t)F;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
            for (int64_t r = 0; r < (int64_t)t; ++r) {
                const float *xt = x + (size_t)r * H;
                float *out = y + (size_t)r * H;
                for (uint32_t i = 0; i < H; ++i) out[i] = 0.0f;
                for (int k = 0; k < ORC_TOP_K; ++k) {
                    uint32_t e = ids[(size_t)r * ORC_TOP_K + k];
                    float weight = w[(size_t)r * ORC_TOP_K + k];
                    expert_forward_nocheck(L->routed_gate[e], L->routed_up[e], L->routed_down[e], H,
                                           F, xt, routed, scratch);
                    for (uint32_t i = 0; i < H; ++i) out[i] += routed[i] * weight;
                }
            }
            free(scratch);
        }
    }
    return bad ? -1 : 0;
}

/* ======================================================================= */
/* a16: runtime/decode.rs:48-64 -- top_logit_candidates.                    */
/* ======================================================================= */
void orc_top_logit_candidates(const float *logits, uint32_t n, uint32_t *tokens, float *vals)
{
    uint32_t tok[4] = {0, 0, 0, 0};
    float lg[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    for (uint32_t i = 0; i < n; ++i) {
        float logit = logits[i];
        int position = -1;
        for (int s = 0; s < 4; ++s) if (logit > lg[s]) { position = s; break; }
        if (position < 0) continue;
        for (int s = 3; s > position; --s) { tok[s] = tok[s - 1]; lg[s] = lg[s - 1]; }
        tok[position] = i;
        lg[position] = logit;
    }
    for (int s = 0; s < 4; ++s) { tokens[s] = tok[s]; vals[s] = lg[s]; }
}

/* ======================================================================= */
/* a17: sampling/mod.rs:166-190 softmax + :227-248 draw + :258-266 order.   */
/* ======================================================================= */
typedef struct { uint32_t token; float value; } cand_t;

/* compare_desc(a, b).then(a.token.cmp(&b.token)) as a qsort comparator. */
static int cand_cmp(const void *pa, const void *pb)
{
    const cand_t *a = (const cand_t *)pa, *b = (const cand_t *)pb;
    int an = isnan(a->value), bn = isnan(b->value);
    int ord;
    if (an && bn) ord = 0;
    else if (an) ord = 1;
    else if (bn) ord = -1;
    else ord = (b->value < a->value) ? -1 : (b->value > a->value ? 1 : 0);
    if (ord != 0) return ord;
    return (a->token < b->token) ? -1 : (a->token > b->token ? 1 : 0);
}

uint32_t orc_softmax_draw(const float *logits, uint32_t n, float temperature, float u)
{
    return orc_softmax_draw_sums(logits, n, temperature, u, NULL, NULL);
}

/* The same draw, also returning its two sums: *total, the token-order sum of
 * the exponentials (sampling/mod.rs:176-178), and *psum, the sorted-order sum
 * of the probabilities (:236); either pointer may be NULL. */
uint32_t orc_softmax_draw_sums(const float *logits, uint32_t n, float temperature, float u, float *total_out,
                               float *psum_out)
{
    if (n == 0) return 0;
    float max = -INFINITY;
    for (uint32_t i = 0; i < n; ++i) max = fmaxf(max, logits[i]);
    cand_t *c = (cand_t *)malloc(sizeof(cand_t) * n);
    if (!c) return 0;
    for (uint32_t i = 0; i < n; ++i) { c[i].token = i; c[i].value = expf((logits[i] - max) / temperature); }
    float total = -0.0f;
    for (uint32_t i = 0; i < n; ++i) total += c[i].value;
    if (total > 0.0f)
        for (uint32_t i = 0; i < n; ++i) c[i].value /= total;
    qsort(c, n, sizeof(cand_t), cand_cmp);
    float psum = -0.0f;
    for (uint32_t i = 0; i < n; ++i) psum += c[i].value;
    if (total_out) *total_out = total;
    if (psum_out) *psum_out = psum;
    uint32_t result;
    if (!isfinite(psum) || psum <= 0.0f) {
        result = c[0].token;
    } else {
        float target = u * psum;
        float cumulative = 0.0f;
        result = c[n - 1].token;
        for (uint32_t i = 0; i < n; ++i) {
            cumulative += c[i].value;
            if (cumulative >= target) { result = c[i].token; break; }
        }
    }
    free(c);
    return result;
}

/* ======================================================================= */
/* a18: sampling/mod.rs:283-298 (SplitMix64 seeding), :311-326, :328-330.   */
/* ======================================================================= */
static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

void orc_xoshiro_seed(orc_xoshiro *rng, uint64_t seed)
{
    uint64_t z = seed;
    for (int i = 0; i < 4; ++i) {
        z += 0x9E3779B97F4A7C15ull;
        uint64_t x = z;
        x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
        x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
        rng->s[i] = x ^ (x >> 31);
    }
}

uint64_t orc_xoshiro_next_u64(orc_xoshiro *rng)
{
    uint64_t *s = rng->s;
    uint64_t result = rotl64(s[0] + s[3], 23) + s[0];
    uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}

float orc_xoshiro_next_f32(orc_xoshiro *rng)
{
    return (float)(orc_xoshiro_next_u64(rng) >> 40) / (float)(1u << 24);
}

/* ======================================================================= */
/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11).                        */
/* ======================================================================= */
void orc_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4])
{
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int round = 0; round < 10; ++round) {
        if (round) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* ======================================================================= */
/* a22: k-token speculative acceptance (new; no reference code).            */
/*                                                                          */
/* Definition (the HIP kernels implement exactly this; every sum is an      */
/* exact unsigned-integer sum, so the result is independent of the order    */
/* in which a parallel machine adds):                                        */
/*                                                                          */
/*  texp(z): 0 if !(z >= -87); else n = rint(z*LOG2E), r = fma(-n, LN2_HI,   */
/*   z), r = fma(-n, LN2_LO, r), p = degree-7 Taylor polynomial of e^r by    */
/*   Horner with fma, result = p * 2^n (Cody & Waite range reduction).       */
/*  Row statistics, for every target row i <= k and draft row i < k:          */
/*   M = max of the non-NaN logits (-inf if none); e_x = 0 for a NaN logit,   */
/*   1 when l_x == M, else texp((l_x - M) / T);  E_x = floor(e_x * 2^40);     */
/*   S_fix = sum E_x (u64);  S = rn_f32(S_fix) * 2^-40.                       */
/*  ftz(v) = 0 when |v| < FLT_MIN (subnormals count as zero probability).    */
/*  Greedy: a_i = argmax of target row i (strict '>', lowest index wins,     */
/*   NaN never wins; decode.rs:48-64).  Accept draft i iff a_i == d_i.       */
/*  Stochastic: p = ftz(e_p[d_i] / S_p) (0 if S_p == 0), q likewise from the */
/*   draft row; accept iff (q > 0 ? u_i < p / q : p > 0).                    */
/*  i* = first rejected position, or k.  Tokens 0..i*-1 are the drafts.      */
/*  Token i*: greedy -> a_{i*}.  Stochastic, i* < k -> inverse CDF over      */
/*   w_x = floor(ftz(max(0, ftz(e_p/S_p) - ftz(e_q/S_q))) * 2^62) with        */
/*   uniform u_resample[i*]; if sum w == 0 it falls back to w_x = E_x of     */
/*   target row i*.  i* == k -> inverse CDF over E_x of target row k with   */
/*   u_resample[k] (argmax if that row's S_fix == 0).                        */
/*  Inverse CDF: t = floor(W * u) (exact), token = smallest x with           */
/*   sum_{y<=x} w_y > t.  This picks only tokens with w_x > 0.               */
/* ======================================================================= */
/* log2(e), ln2 split as Cody & Waite (the high part has 9 trailing zero
 * bits, so n * LN2_HI is exact for |n| <= 127), and the Taylor coefficients
 * 1/k! rounded to binary32. */
#define ACC_LOG2E 0x1.715476p+0f
#define ACC_LN2_HI 0x1.62e4p-1f
#define ACC_LN2_LO 0x1.7f7d1cp-20f
#define ACC_C7 0x1.a01a02p-13f /* 1/5040 */
#define ACC_C6 0x1.6c16c2p-10f /* 1/720  */
#define ACC_C5 0x1.111112p-7f  /* 1/120  */
#define ACC_C4 0x1.555556p-5f  /* 1/24   */
#define ACC_C3 0x1.555556p-3f  /* 1/6    */

float orc_accept_exp(float z)
{
    if (!(z >= -87.0f)) return 0.0f;
    if (z > 88.0f) return INFINITY;
    float n = rintf(z * ACC_LOG2E);
    float r = fmaf(-n, ACC_LN2_HI, z);
    r = fmaf(-n, ACC_LN2_LO, r);
    float p = ACC_C7;
    p = fmaf(p, r, ACC_C6);
    p = fmaf(p, r, ACC_C5);
    p = fmaf(p, r, ACC_C4);
    p = fmaf(p, r, ACC_C3);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int32_t ni = (int32_t)n;
    float scale = bits_f32((uint32_t)(ni + 127) << 23);
    return p * scale;
}

/* floor(v * 2^shift) for v in [0, 1] (NaN/negative/subnormal -> 0). */
static uint64_t fix_shift(float v, int shift)
{
    uint32_t b = f32_bits(v);
    if (b & 0x80000000u) return 0;
    uint32_t ex = (b >> 23) & 0xFFu;
    if (ex == 0 || ex == 0xFF) return 0;
    uint64_t m = (uint64_t)((b & 0x7FFFFFu) | 0x800000u);
    int s = (int)ex - 127 - 23 + shift;
    if (s >= 0) return m << s;
    if (s <= -24) return 0;
    return m >> (-s);
}

uint64_t orc_fix40(float v) { return fix_shift(v, 40); }
uint64_t orc_fix62(float v) { return fix_shift(v, 62); }

float orc_u64_to_f32(uint64_t v)
{
    if (v == 0) return 0.0f;
    int lz = __builtin_clzll(v);
    uint64_t norm = v << lz;                 /* top bit at 63 */
    uint32_t mant = (uint32_t)(norm >> 40);  /* 24 bits incl. implicit one */
    uint64_t rest = norm & ((1ull << 40) - 1);
    uint64_t half = 1ull << 39;
    int exp = 63 - lz;
    if (rest > half || (rest == half && (mant & 1u))) {
        mant += 1;
        if (mant == (1u << 24)) { mant >>= 1; exp += 1; }
    }
    return bits_f32(((uint32_t)(exp + 127) << 23) | (mant & 0x7FFFFFu));
}

uint64_t orc_scale_floor(uint64_t total, float u)
{
    uint32_t b = f32_bits(u);
    uint32_t ex = (b >> 23) & 0xFFu;
    if ((b & 0x80000000u) || ex == 0) return 0;     /* u <= 0 or subnormal */
    uint64_t m = (uint64_t)((b & 0x7FFFFFu) | 0x800000u);
    int s = (int)ex - 127 - 23;                       /* u = m * 2^s, s <= -24 */
    if (s >= 0) return total;                         /* u >= 1: caller rejects */
    unsigned __int128 prod = (unsigned __int128)total * m;
    int sh = -s;
    if (sh >= 128) return 0;
    return (uint64_t)(prod >> sh);
}

static inline float ftz(float v) { return (fabsf(v) < 1.17549435e-38f) ? 0.0f : v; }

typedef struct { float max; uint64_t sfix; float s; } row_stat_t;

static float row_e(const float *row, uint32_t x, float M, float T)
{
    float l = row[x];
    if (isnan(l)) return 0.0f;
    if (l == M) return 1.0f;
    return orc_accept_exp((l - M) / T);
}

static row_stat_t row_stats(const float *row, uint32_t V, float T)
{
    row_stat_t st;
    float M = -INFINITY;
    for (uint32_t x = 0; x < V; ++x) if (!isnan(row[x]) && row[x] > M) M = row[x];
    uint64_t s = 0;
    for (uint32_t x = 0; x < V; ++x) s += orc_fix40(row_e(row, x, M, T));
    st.max = M;
    st.sfix = s;
    st.s = orc_u64_to_f32(s) * 9.094947017729282379150390625e-13f; /* 2^-40 */
    return st;
}

static uint32_t argmax_row(const float *row, uint32_t V)
{
    uint32_t best = 0;
    float bv = -INFINITY;
    for (uint32_t x = 0; x < V; ++x) if (row[x] > bv) { bv = row[x]; best = x; }
    return best;
}

static float prob_of(float e, float s) { return s == 0.0f ? 0.0f : ftz(e / s); }

int orc_accept(const float *target, const float *draft, const int32_t *dtok, uint32_t k,
               uint32_t V, float T, int greedy, const float *u, const float *ures,
               int32_t *accepted, int32_t *tokens)
{
    if (V == 0 || !target || !tokens || !accepted) return -1;
    if (k > 0 && !dtok) return -1;
    for (uint32_t i = 0; i < k; ++i) if (dtok[i] < 0 || (uint32_t)dtok[i] >= V) return -1;
    for (uint32_t i = 0; i <= k; ++i) tokens[i] = -1;
    if (greedy) {
        uint32_t i = 0;
        for (; i < k; ++i) {
            uint32_t a = argmax_row(target + (size_t)i * V, V);
            if ((int32_t)a != dtok[i]) break;
            tokens[i] = dtok[i];
        }
        tokens[i] = (int32_t)argmax_row(target + (size_t)i * V, V);
        *accepted = (int32_t)i;
        return 0;
    }
    if (!(T > 0.0f) || !isfinite(T) || !draft || !u || !ures) return -1;
    for (uint32_t i = 0; i < k; ++i) if (!(u[i] >= 0.0f && u[i] < 1.0f)) return -1;
    for (uint32_t i = 0; i <= k; ++i) if (!(ures[i] >= 0.0f && ures[i] < 1.0f)) return -1;

    uint32_t istar = k;
    row_stat_t sp_star = {0}, sq_star = {0};
    for (uint32_t i = 0; i < k; ++i) {
        const float *tr = target + (size_t)i * V, *dr = draft + (size_t)i * V;
        row_stat_t sp = row_stats(tr, V, T), sq = row_stats(dr, V, T);
        uint32_t d = (uint32_t)dtok[i];
        float p = prob_of(row_e(tr, d, sp.max, T), sp.s);
        float q = prob_of(row_e(dr, d, sq.max, T), sq.s);
        int acc = (q > 0.0f) ? (u[i] < p / q) : (p > 0.0f);
        if (!acc) { istar = i; sp_star = sp; sq_star = sq; break; }
        tokens[i] = dtok[i];
    }
    const float *tr = target + (size_t)istar * V;
    uint64_t *w = (uint64_t *)malloc(sizeof(uint64_t) * V);
    if (!w) return -1;
    uint64_t W = 0;
    float uu = ures[istar];
    row_stat_t st;
    if (istar < k) {
        const float *dr = draft + (size_t)istar * V;
        st = sp_star;
        for (uint32_t x = 0; x < V; ++x) {
            float p = prob_of(row_e(tr, x, sp_star.max, T), sp_star.s);
            float q = prob_of(row_e(dr, x, sq_star.max, T), sq_star.s);
            float r = ftz(fmaxf(0.0f, p - q));
            w[x] = orc_fix62(r);
            W += w[x];
        }
    } else {
        st = row_stats(tr, V, T);
    }
    if (W == 0) {
        for (uint32_t x = 0; x < V; ++x) w[x] = orc_fix40(row_e(tr, x, st.max, T));
        W = st.sfix;
    }
    int32_t token;
    if (W == 0) {
        token = (int32_t)argmax_row(tr, V);
    } else {
        uint64_t t = orc_scale_floor(W, uu), cum = 0;
        token = (int32_t)(V - 1);
        for (uint32_t x = 0; x < V; ++x) {
            cum += w[x];
            if (cum > t) { token = (int32_t)x; break; }
        }
    }
    free(w);
    tokens[istar] = token;
    *accepted = (int32_t)istar;
    return 0;
}


/* ======================================================================== */
/* f1 / a4 / a20: Q4_K                                                      */
/* ======================================================================== */

/* dequant.rs:139-148 -- get_scale_min_k4: the 6-bit (scale, min) of
 * sub-block j from the 12 packed bytes. */
static void q4k_scale_min(int j, const uint8_t *q, int *sc, int *mn)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        *mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* dequant.rs:154-184 -- pairs of sub-blocks per 64 elements: low nibbles of
 * 32 bytes, then their high nibbles; value = (d sc) q - (dmin m). */
void orc_dequantize_q4_k(const uint8_t *block, float *out)
{
    const float d = orc_f16_to_f32((uint16_t)(block[0] | (block[1] << 8)));
    const float dmin = orc_f16_to_f32((uint16_t)(block[2] | (block[3] << 8)));
    const uint8_t *scales = block + 4, *qs = block + 16;
    int is = 0, out_idx = 0, q_idx = 0;
    for (int g = 0; g < 4; ++g) {
        int sc1, m1, sc2, m2;
        q4k_scale_min(is, scales, &sc1, &m1);
        const float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
        q4k_scale_min(is + 1, scales, &sc2, &m2);
        const float d2 = d * (float)sc2, mm2 = dmin * (float)m2;
        for (int l = 0; l < 32; ++l) out[out_idx + l] = d1 * (float)(qs[q_idx + l] & 0x0F) - mm1;
        for (int l = 0; l < 32; ++l) out[out_idx + 32 + l] = d2 * (float)(qs[q_idx + l] >> 4) - mm2;
        out_idx += 64;
        q_idx += 32;
        is += 2;
    }
}

/* validate.rs:97-126 -- each sub-block j located from j alone (group j / 2,
 * nibble half j % 2), with the independent f16 decoder. */
void orc_dequantize_q4_k_indep(const uint8_t *block, float *out)
{
    const float d = orc_f16_to_f32_indep((uint16_t)(block[0] | (block[1] << 8)));
    const float dmin = orc_f16_to_f32_indep((uint16_t)(block[2] | (block[3] << 8)));
    const uint8_t *s = block + 4, *qs = block + 16;
    for (int j = 0; j < 8; ++j) {
        const int sc = j < 4 ? (s[j] & 63) : ((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        const int m = j < 4 ? (s[j + 4] & 63) : ((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
        const float dj = d * (float)sc, mj = dmin * (float)m;
        const int group = j / 2, half = j % 2;
        for (int l = 0; l < 32; ++l) {
            const uint8_t byte = qs[group * 32 + l];
            const int nib = half == 0 ? (byte & 0x0F) : (byte >> 4);
            out[group * 64 + half * 32 + l] = dj * (float)nib - mj;
        }
    }
}

/* backend/reference.rs:49-67 -- acc starts at 0.0 and takes every element
 * of the row in order (a plain loop, not an iterator sum). */
int orc_q4k_gemv(const uint8_t *w, uint32_t rows, uint32_t cols, const float *x, float *y)
{
    if (cols % ORC_Q4_K_BLOCK_ELEMS != 0) return -1;
    const uint32_t bpr = cols / ORC_Q4_K_BLOCK_ELEMS;
    float dq[ORC_Q4_K_BLOCK_ELEMS];
    for (uint32_t r = 0; r < rows; ++r) {
        float acc = 0.0f;
        for (uint32_t b = 0; b < bpr; ++b) {
            orc_dequantize_q4_k(w + ((size_t)r * bpr + b) * ORC_Q4_K_BLOCK_BYTES, dq);
            const float *v = x + (size_t)b * ORC_Q4_K_BLOCK_ELEMS;
            for (int i = 0; i < ORC_Q4_K_BLOCK_ELEMS; ++i) acc += dq[i] * v[i];
        }
        y[r] = acc;
    }
    return 0;
}

/* weights.rs:898-931 -- the signed value of largest magnitude (first on
 * ties) maps to -127; values round half to even; .min(127) then `as i8`. */
void orc_quantize_q8_k(const float *values, int8_t *q, int16_t *sums, float *scale)
{
    float smax = 0.0f, amax = 0.0f;
    for (int i = 0; i < 256; ++i) {
        const float a = fabsf(values[i]);
        if (a > amax) {
            amax = a;
            smax = values[i];
        }
    }
    if (amax == 0.0f) {
        memset(q, 0, 256);
        memset(sums, 0, 16 * sizeof(int16_t));
        *scale = 0.0f;
        return;
    }
    const float inv = -127.0f / smax;
    *scale = 1.0f / inv;
    for (int i = 0; i < 256; ++i) {
        float t = nearbyintf(values[i] * inv); /* round_ties_even (default mode) */
        if (!(t <= 127.0f)) t = 127.0f;        /* f32::min(127): NaN gives 127 */
        if (t < -128.0f) t = -128.0f;          /* `as i8` saturates */
        q[i] = (int8_t)t;
    }
    for (int j = 0; j < 16; ++j) {
        int s = 0;
        for (int i = 0; i < 16; ++i) s += q[16 * j + i];
        sums[j] = (int16_t)s;
    }
}

/* weights.rs:944-1021 -- integer lane sums (lane = element index mod 8 within
 * each quarter of a sub-block), then the f32 combination in the reference's
 * order: sums[lane] += (d * q8scale) * lane_sum; minimum_sum -= (dmin *
 * q8scale) * block_minimum_sum; result = minimum_sum + sum(sums). */
float orc_q4_k_dot_pre(const uint8_t *row, uint32_t nblocks, const int8_t *q8, const int16_t *sums,
                       const float *scales)
{
    float lane_acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float minimum_sum = 0.0f;
    for (uint32_t b = 0; b < nblocks; ++b) {
        const uint8_t *w = row + (size_t)b * ORC_Q4_K_BLOCK_BYTES;
        const float ws = orc_f16_to_f32((uint16_t)(w[0] | (w[1] << 8)));
        const float ms = orc_f16_to_f32((uint16_t)(w[2] | (w[3] << 8)));
        const uint8_t *packed = w + 4, *vals = w + 16;
        const int8_t *qb = q8 + (size_t)b * 256;
        const int16_t *sb = sums + (size_t)b * 16;
        int32_t bms = 0;
        for (int k = 0; k < 8; ++k) {
            int sc, mn;
            q4k_scale_min(k, packed, &sc, &mn);
            bms += mn * ((int32_t)sb[2 * k] + (int32_t)sb[2 * k + 1]);
        }
        int8_t unp[256];
        for (int c = 0; c < 4; ++c)
            for (int i = 0; i < 32; ++i) {
                unp[c * 64 + i] = (int8_t)(vals[c * 32 + i] & 0x0F);
                unp[c * 64 + 32 + i] = (int8_t)(vals[c * 32 + i] >> 4);
            }
        int32_t lane_sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int k = 0; k < 8; ++k) {
            int sc, mn;
            q4k_scale_min(k, packed, &sc, &mn);
            for (int quarter = 0; quarter < 4; ++quarter)
                for (int lane = 0; lane < 8; ++lane) {
                    const int idx = k * 32 + quarter * 8 + lane;
                    lane_sums[lane] += sc * (int32_t)qb[idx] * (int32_t)unp[idx];
                }
        }
        const float combined = ws * scales[b];
        for (int lane = 0; lane < 8; ++lane) lane_acc[lane] += combined * (float)lane_sums[lane];
        minimum_sum -= ms * scales[b] * (float)bms;
    }
    float total = -0.0f; /* Iterator::sum::<f32>() seed */
    for (int lane = 0; lane < 8; ++lane) total += lane_acc[lane];
    return minimum_sum + total;
}

/* weights.rs:680-735 -- quantize x once per 256-element chunk, then one
 * q4_k_dot_pre per row. */
int orc_q4_k_matvec(const uint8_t *w, uint32_t rows, uint32_t cols, const float *x, float *y)
{
    if (cols % ORC_Q4_K_BLOCK_ELEMS != 0) return -1;
    const uint32_t nb = cols / ORC_Q4_K_BLOCK_ELEMS;
    int8_t *q8 = (int8_t *)malloc((size_t)nb * 256);
    int16_t *sums = (int16_t *)malloc((size_t)nb * 16 * sizeof(int16_t));
    float *scales = (float *)malloc((size_t)nb * sizeof(float));
    if (!q8 || !sums || !scales) {
        free(q8);
        free(sums);
        free(scales);
        return -1;
    }
    for (uint32_t b = 0; b < nb; ++b) orc_quantize_q8_k(x + (size_t)b * 256, q8 + (size_t)b * 256, sums + (size_t)b * 16, &scales[b]);
    for (uint32_t r = 0; r < rows; ++r)
        y[r] = orc_q4_k_dot_pre(w + (size_t)r * nb * ORC_Q4_K_BLOCK_BYTES, nb, q8, sums, scales);
    free(q8);
    free(sums);
    free(scales);
    return 0;
}

/* ======================================================================= */
/* f3: Q6_K, the canonical LM head format                                   */
/* ======================================================================= */
#define ORC_Q6_K_BLOCK_BYTES 210

/* The signed 6-bit value q - 32 of element e (0..255) of one block: the two
 * 128-element halves each interleave four 32-element groups, low nibbles
 * from ql, two high bits from qh (dequant.rs:198-216). */
static int q6k_value(const uint8_t *b, int e)
{
    const int half = e / 128, r = e % 128, grp = r / 32, i = r % 32;
    const uint8_t *ql = b + 64 * half, *qh = b + 128 + 32 * half;
    const uint8_t low = (grp & 1) ? ql[i + 32] : ql[i];
    const int lo = (grp < 2) ? (low & 0x0F) : (low >> 4);
    const int hi = (qh[i] >> (2 * grp)) & 3;
    return (lo | (hi << 4)) - 32;
}

/* dequant.rs:190-218: (d * scale) * q in that order. */
void orc_dequantize_q6_k(const uint8_t *b, float *out)
{
    const float d = orc_f16_to_f32((uint16_t)(b[208] | (b[209] << 8)));
    for (int e = 0; e < 256; ++e) {
        const int8_t sc = (int8_t)b[192 + e / 16];
        out[e] = d * (float)sc * (float)q6k_value(b, e);
    }
}

/* weights.rs:1023-1101: integer lane sums (lane = element index mod 8),
 * sums[lane] += (d * q8scale) * lane_sum block after block, then the
 * iterator sum from -0.0. */
float orc_q6_k_dot_pre(const uint8_t *row, uint32_t nblocks, const int8_t *q8, const float *scales)
{
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t b = 0; b < nblocks; ++b) {
        const uint8_t *w = row + (size_t)b * ORC_Q6_K_BLOCK_BYTES;
        const int8_t *qb = q8 + (size_t)b * 256;
        const float d = orc_f16_to_f32((uint16_t)(w[208] | (w[209] << 8)));
        int32_t lane_sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int group = 0; group < 16; ++group) {
            const int32_t sc = (int8_t)w[192 + group];
            for (int half = 0; half < 2; ++half)
                for (int lane = 0; lane < 8; ++lane) {
                    const int idx = group * 16 + half * 8 + lane;
                    lane_sums[lane] += sc * (int32_t)qb[idx] * q6k_value(w, idx);
                }
        }
        const float combined = d * scales[b];
        for (int lane = 0; lane < 8; ++lane) sums[lane] += combined * (float)lane_sums[lane];
    }
    float total = -0.0f;
    for (int lane = 0; lane < 8; ++lane) total += sums[lane];
    return total;
}

int orc_q6_k_matvec(const uint8_t *w, uint32_t rows, uint32_t cols, const float *x, float *y)
{
    if (cols % 256 != 0) return -1;
    const uint32_t nb = cols / 256;
    int8_t *q8 = (int8_t *)malloc((size_t)nb * 256);
    int16_t *sums = (int16_t *)malloc((size_t)nb * 16 * sizeof(int16_t));
    float *scales = (float *)malloc((size_t)nb * sizeof(float));
    if (!q8 || !sums || !scales) {
        free(q8);
        free(sums);
        free(scales);
        return -1;
    }
    for (uint32_t b = 0; b < nb; ++b)
        orc_quantize_q8_k(x + (size_t)b * 256, q8 + (size_t)b * 256, sums + (size_t)b * 16, &scales[b]);
#pragma omp parallel for schedule(static) if (rows >= 4096)
    for (uint32_t r = 0; r < rows; ++r)
        y[r] = orc_q6_k_dot_pre(w + (size_t)r * nb * ORC_Q6_K_BLOCK_BYTES, nb, q8, scales);
    free(q8);
    free(sums);
    free(scales);
    return 0;
}
