/*
 * tqf_oracle.h -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C CPU restatement of the reference crate's scalar path for the
 * MTP speculative-verify hot path (Q4_0 MoE expert FFN + acceptance).  It is
 * the checker the HIP backend is compared against.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library never links or calls it.
 *
 * Every function names the reference file:line whose semantics it restates
 * (paths relative to the reference checkout).  Rust semantics reproduced:
 *   - no FMA contraction (build with -ffp-contract=off);
 *   - `Iterator::sum::<f32>()` is a sequential left fold seeded with -0.0;
 *   - `f32::exp` is the platform libm expf;
 *   - `sort_by` is stable, `total_cmp` is IEEE total order.
 *
 * Pinning status (what checks each function against something other than
 * itself) is listed beside each declaration and enforced in
 * tests/test_oracle.py.
 */
#ifndef TQF_ORACLE_H
#define TQF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- a1: binary16 <-> binary32 ---------------------------------------- */
/* dequant.rs:19-48.  Pinned: dequant.rs:244-251 known values; exhaustive
 * agreement with the arithmetic twin below over all 65,536 patterns
 * (simd/mod.rs:459-475 does the same). */
float orc_f16_to_f32(uint16_t bits);
/* validate.rs:48-69 (independent arithmetic decoder). */
float orc_f16_to_f32_indep(uint16_t bits);
/* dequant.rs:54-100 (round to nearest, ties to even).  Pinned: dequant.rs:
 * 279-284 round-trip set; numpy float16 conversion over a dense sweep. */
uint16_t orc_f32_to_f16(float value);

/* ---- a2: Q4_0 block decode -------------------------------------------- */
/* dequant.rs:110-123.  Pinned: dequant.rs:253-264 KAT; validate.rs:270-299
 * byte pattern i*37+11 against the independent decoder below. */
void orc_dequantize_q4_0(const uint8_t *block18, float *out32);
/* validate.rs:71-87 (arithmetic nibble extraction, independent f16). */
void orc_dequantize_q4_0_indep(const uint8_t *block18, float *out32);

/* ---- a3: Q4_0 matvec -------------------------------------------------- */
/* weights.rs:617-750 (matvec_payload shape checks) and :827-843 (matvec_row
 * Q4_0: per-block iterator sum, then sequential row accumulate).
 * `w` is rows x (cols/32) row-major 18-byte blocks.  Returns 0, or -1 on a
 * shape error (the reference returns ModelError::Shape).  Pinned:
 * weights.rs:2500-2508 (224.0), :2458-2480 (7.0 x32 / 0.0 x32), :2511-2530;
 * a float64 brute-force dot on random shapes. */
int orc_q4_0_matvec(const uint8_t *w, size_t len, uint32_t rows, uint32_t cols,
                    const float *x, float *y);

/* ---- a5: F32 matvec (router) ------------------------------------------ */
/* weights.rs:802-808 (F32 matvec_row) and :306-323 (dot = 1-row matvec).
 * Pinned: weights.rs:2440-2456 ([14, 32]); float64 brute force. */
void orc_f32_matvec(const float *w, uint32_t rows, uint32_t cols, const float *x,
                    float *y);

/* ---- a6: router softmax / stable top-8 / renormalise ------------------ */
/* experts/mod.rs:134-197.  n must be 256 (require_len).  Returns 0, or -1 on
 * a wrong length, a non-finite logit, or a failed validate().  Pinned:
 * experts/mod.rs:1639-1673 KATs; invariants (ids descend by probability,
 * ties to lower id, sum of weights within 1e-4 of one). */
int orc_router_from_logits(const float *logits, uint32_t n, uint16_t *ids8,
                           float *weights8);
/* validate() alone (experts/mod.rs:169-197), for the duplicate-id KAT. */
int orc_router_validate(const uint16_t *ids8, const float *weights8);

/* ---- a7 / a21: activation algebra ------------------------------------- */
/* weights.rs:241-259: out = (g / (1 + exp(-g))) * u.  Pinned: silu(0)=0
 * (reference.rs:124-128), sign/limit closed forms. */
void orc_silu_mul(const float *g, const float *u, float *out, uint32_t n);
/* weights.rs:216-239 (eps 1e-6).  Pinned: unit-RMS KAT (weights.rs:2483). */
void orc_qwen_rmsnorm(const float *x, const float *w, uint32_t n, float *out);
/* reference.rs:116-118 / experts/mod.rs:1514: 1 / (1 + exp(-v)). */
float orc_sigmoid(float v);

/* ---- a10: one routed/shared expert ------------------------------------ */
/* weights.rs:566-610: gate [width x hidden], up [width x hidden], down
 * [hidden x width], all Q4_0; y = down(silu(gate x) * up x).  Returns 0 or
 * -1 on a shape error.  Pinned: one-hot-expert and linearity invariants,
 * float64 brute force. */
int orc_expert_forward(const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                       uint32_t hidden, uint32_t width, const float *x, float *y);

/* ---- a11 / a12: MoE layer over M rows --------------------------------- */
typedef struct orc_moe_layer {
    const float *router;            /* f32 [n_experts x hidden]          */
    const float *shared_input_gate; /* f32 [hidden]                      */
    const uint8_t *shared_gate;     /* Q4_0 [width x hidden]             */
    const uint8_t *shared_up;       /* Q4_0 [width x hidden]             */
    const uint8_t *shared_down;     /* Q4_0 [hidden x width]             */
    const uint8_t *const *routed_gate; /* [n_experts] -> Q4_0 planes     */
    const uint8_t *const *routed_up;
    const uint8_t *const *routed_down;
    uint32_t n_experts;             /* 256 (router requires it)          */
    uint32_t hidden;                /* 2048                              */
    uint32_t width;                 /* 512                               */
} orc_moe_layer;

/* experts/mod.rs:1540-1577 (forward_batch) with the per-row arithmetic of
 * :1600-1634: route every row; shared expert (gate/up/SwiGLU/down) scaled by
 * sigmoid(shared_input_gate . x); then add_scaled_in_place (weights.rs:
 * 267-281) for each route in route order.  x, y are [m x hidden]; ids/w are
 * [m x 8] (may be NULL).  nthreads > 1 parallelises over output rows with
 * OpenMP; each row's arithmetic is unchanged, so results are bit-identical
 * to nthreads == 1.  Returns 0, or -1 on a router error. */
int orc_moe_forward_batch(const orc_moe_layer *layer, const float *x, uint32_t m,
                          float *y, uint16_t *ids, float *w, int nthreads);

/* The same layer with Q4_K expert matrices (GGML super-blocks; the plane
 * pointers of orc_moe_layer then point at rows x cols/256 x 144 bytes):
 * every expert matvec is matvec_payload's Q4_K arm (weights.rs:680-735,
 * orc_q4_k_matvec's arithmetic), everything else as orc_moe_forward_batch.
 * Pinned through its parts (router, orc_q4_k_matvec, silu_mul) and the
 * composition tests of the oracle suite.  Returns 0, or -1 on a router
 * error, a cols % 256 shape or an allocation failure. */
int orc_moe_forward_batch_q4k(const orc_moe_layer *layer, const float *x, uint32_t m,
                              float *y, uint16_t *ids, float *w, int nthreads);

/* The routed accumulate of forward_batch (experts/mod.rs:1562-1566) for
 * given routes: y[t] = 0, then for k = 0..7 in route order
 * y[t] += expert_{ids[t,k]}(x_t) * w[t,k] (add_scaled_in_place, weights.rs:
 * 267-281; expert as weights.rs:566-610).  x, y are [t x hidden]; ids, w
 * [t x 8].  nthreads > 1 parallelises over tokens (bit-identical).  Returns
 * 0, or -1 on an id >= n_experts or an allocation failure. */
int orc_routed_combine(const orc_moe_layer *layer, const float *x, uint32_t t,
                       const uint16_t *ids, const float *w, float *y, int nthreads);

/* Distinct-expert union of M routes in first-demand order (experts/mod.rs:
 * 268-275 BatchExpertPlan, :937 prepare_batch_route).  Returns the count. */
uint32_t orc_batch_union(const uint16_t *ids, uint32_t m, uint16_t *out_union);

/* ---- a16: top_logit_candidates ---------------------------------------- */
/* runtime/decode.rs:48-64: 4 slots, strict '>' (ties to the lower index, NaN
 * never enters).  Pinned: sampling/mod.rs:412-452 KATs. */
void orc_top_logit_candidates(const float *logits, uint32_t n, uint32_t *tokens4,
                              float *logits4);

/* ---- a17 / a18: stochastic draw and xoshiro256++ ---------------------- */
/* sampling/mod.rs:166-190 (softmax, sorted descending, ties to lower token,
 * NaN last) then :227-248 (inverse CDF with u*total, first cum >= target;
 * top-token fallback on a non-finite/zero total).  `u` is the uniform that
 * rng.next_f32() would supply.  Pinned: sampling/mod.rs:476-499 frequency
 * test, :500-519 temperature test, NaN tests. */
uint32_t orc_softmax_draw(const float *logits, uint32_t n, float temperature, float u);
uint32_t orc_softmax_draw_sums(const float *logits, uint32_t n, float temperature, float u, float *total_out,
                               float *psum_out);

typedef struct orc_xoshiro { uint64_t s[4]; } orc_xoshiro;
/* sampling/mod.rs:283-298 SplitMix64 seeding. */
void orc_xoshiro_seed(orc_xoshiro *rng, uint64_t seed);
/* sampling/mod.rs:311-326.  Pinned: sampling/mod.rs:662-669 (16,777,217). */
uint64_t orc_xoshiro_next_u64(orc_xoshiro *rng);
/* sampling/mod.rs:328-330. */
float orc_xoshiro_next_f32(orc_xoshiro *rng);

/* ---- Philox4x32-10 (Salmon et al., SC'11) ----------------------------- */
/* No reference code (the configs name a seeded Philox stream).  Pinned:
 * Random123 known-answer vectors and ROCm's open-source
 * rocrand_philox4x32_10.h (vectors committed under tests/golden/). */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* ---- a22: k-token speculative acceptance (no reference code) ---------- */
/* The exact, order-independent algorithm the HIP kernels implement (see the
 * definition in oracle/tqf_oracle.c above orc_accept).  target [k+1 x V],
 * draft [k x V] (unused when greedy), draft_tokens [k], u [k],
 * u_resample [k+1].  Writes *accepted and tokens_out[k+1] (entries past
 * accepted are -1).  Returns 0, or -1 on invalid arguments.  Pinned: greedy
 * k=1 == verify_pair (mtp.rs:98-104, 212-221); closed forms (p == q always
 * accepts, p(d)=0<q(d) always rejects, one-hot target accepts); chi-square
 * test that emitted tokens are distributed as the target softmax. */
int orc_accept(const float *target, const float *draft, const int32_t *draft_tokens,
               uint32_t k, uint32_t vocab, float temperature, int greedy,
               const float *u, const float *u_resample, int32_t *accepted,
               int32_t *tokens_out);

/* Building blocks of orc_accept, exported so tests can pin them. */
float orc_accept_exp(float z);               /* Cody-Waite + degree-7 Taylor */
uint64_t orc_fix40(float v);                 /* floor(v * 2^40), v in [0,1]  */
uint64_t orc_fix62(float v);                 /* floor(v * 2^62), v in [0,1]  */
float orc_u64_to_f32(uint64_t v);            /* round to nearest even        */
uint64_t orc_scale_floor(uint64_t total, float u); /* floor(total * u) exact */

/* ---- f1 / a4 / a20: Q4_K (144-byte super-blocks of 256) --------------- */
/* dequant.rs:139-184 (get_scale_min_k4, dequantize_q4_k).  Pinned:
 * dequant.rs:287-306 KAT; validate.rs:289-298 byte pattern i*19+3 against the
 * independent decoder below; one-hot probes through orc_q4k_gemv. */
void orc_dequantize_q4_k(const uint8_t *block144, float *out256);
/* validate.rs:97-126 (sub-blocks walked directly, independent f16). */
void orc_dequantize_q4_k_indep(const uint8_t *block144, float *out256);
/* backend/reference.rs:49-67 q4k_gemv: rows x (cols/256) blocks row-major;
 * one fp32 accumulator per row over every dequantized element in order.
 * Returns 0, or -1 if cols is not a multiple of 256.  Pinned: float64 brute
 * force on the reference's LCG fixture (backend/metal/kernels.rs:1118-1138)
 * and random blocks; one-hot columns recover orc_dequantize_q4_k exactly
 * (kernels.rs:1168-1196). */
int orc_q4k_gemv(const uint8_t *w, uint32_t rows, uint32_t cols, const float *x, float *y);
/* weights.rs:898-931 quantize_q8_k over one 256-element chunk: values q[256],
 * per-16 sums[16], scale.  Pinned: closed forms (the largest |v| maps to
 * -127, ties round to even, a zero chunk gives scale 0), numpy sums. */
void orc_quantize_q8_k(const float *values256, int8_t *q256, int16_t *sums16, float *scale);
/* weights.rs:933-1021 q4_k_dot_pre (the scalar lane loop; the NEON path is
 * bit-identical to it) of one row of nblocks blocks against pre-quantized
 * chunks (q8 [nblocks x 256], sums [nblocks x 16], scales [nblocks]).
 * Pinned: float64 evaluation of the same integer terms. */
float orc_q4_k_dot_pre(const uint8_t *row, uint32_t nblocks, const int8_t *q8, const int16_t *sums,
                       const float *scales);
/* weights.rs:680-735: Q8_K quantization of x per 256-element chunk (hoisted
 * out of the row loop), then q4_k_dot_pre per row.  Returns 0, or -1 if cols
 * is not a multiple of 256.  Pinned: composition of the two above; agrees
 * with orc_q4k_gemv to the Q8_K quantization error. */
int orc_q4_k_matvec(const uint8_t *w, uint32_t rows, uint32_t cols, const float *x, float *y);

/* ---- f3: Q6_K (210-byte super-blocks of 256), the canonical LM head -------- */
/* dequant.rs:190-218 dequantize_q6_k: ql[128], qh[64], 16 signed group
 * scales, f16 d; value = (d * scale) * (q - 32).  Pinned: the all -32 KAT
 * (dequant.rs:308-315); every value equals the exact float64 decode rounded
 * once; a vectorised numpy decoder. */
void orc_dequantize_q6_k(const uint8_t *block210, float *out256);
/* weights.rs:1023-1101 q6_k_dot_pre (scalar lane loop) over nblocks blocks
 * of one row against Q8_K values / scales of the same chunks.  Pinned:
 * float64 evaluation of the same integer terms; lane sums against a numpy
 * restatement. */
float orc_q6_k_dot_pre(const uint8_t *row, uint32_t nblocks, const int8_t *q8, const float *scales);
/* weights.rs:680-735 for GgmlType::Q6K: Q8_K per chunk, then q6_k_dot_pre per
 * row.  Returns 0, or -1 if cols is not a multiple of 256.  Pinned: the
 * -8192 KAT (weights.rs:2532-2543); the Q8_K rounding bound against the
 * float64 GEMV of the decoded weights. */
int orc_q6_k_matvec(const uint8_t *w, uint32_t rows, uint32_t cols, const float *x, float *y);

#ifdef __cplusplus
}
#endif
#endif /* TQF_ORACLE_H */
