/*
 * tqf_hip.h -- C ABI of the MI355X (gfx950) HIP backend for TurboQwenFare's
 * MTP speculative-verify hot path.
 *
 * The reference crate has no backend trait in code; its seams are free
 * functions plus the ExpertValue {Cpu, Gpu} dispatch.  Each entry point below
 * names the reference seam it replaces (paths relative to the reference
 * checkout).  The Rust side binds these through a thin `extern "C"` module and
 * maps a non-zero status plus tqf_hip_last_error() to BackendError::Gpu(String)
 * (src/error.rs:285-288) or, for shape violations, ModelError::Shape.
 *
 * Conventions
 *   - Every function returns int32_t status: TQF_HIP_OK (0) or an error code.
 *     Shape violations are reported, never asserted (the reference asserts in
 *     backend/metal/kernels.rs:565-593; a panic may not cross FFI).
 *   - Host pointers are caller-owned and borrowed for the call; those calls
 *     are synchronous on return.  `_device` entry points take device pointers,
 *     are stream-ordered on the context's stream and return before the GPU
 *     finishes (tqf_hip_synchronize() waits).
 *   - Device weights are owned by opaque handles until their *_free call, the
 *     analogue of BufferLease's Drop (backend/metal/buffer.rs:16-24).  Scratch
 *     is a context-owned arena that is reused across calls (no per-token
 *     allocation; the reference allocates per call in kernels.rs:694-697).
 *   - A context is not thread-safe: the reference serialises the GPU behind
 *     Mutex<GpuExecutionState> (experts/mod.rs:320, 905-917).
 *   - Weights use GGML Q4_0 (18-byte blocks of 32: f16 scale, 16 nibble bytes;
 *     element j = (qs[j] & 15) - 8, element j+16 = (qs[j] >> 4) - 8,
 *     format/quant/dequant.rs:110-123).  Upload repacks them losslessly into a
 *     device row-lane layout (8-row chunks: nibble rows, then their scales);
 *     tqf_hip_weights_download() inverts it.
 */
#ifndef TQF_HIP_H
#define TQF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TQF_HIP_OK 0
#define TQF_HIP_ERR_INVALID 1 /* shape/argument violation (ModelError::Shape)      */
#define TQF_HIP_ERR_DEVICE 2  /* HIP runtime failure (BackendError::Gpu)           */
#define TQF_HIP_ERR_NOMEM 3   /* device allocation failed; nothing was allocated   */
#define TQF_HIP_ERR_ROUTER 4  /* non-finite router logits / invalid route
                                 (ModelError::Unsupported, experts/mod.rs:136-141) */

#define TQF_HIP_TOP_K 8        /* Qwen36Geometry::ROUTED_EXPERTS_PER_TOKEN        */
#define TQF_HIP_MAX_TOKENS 8   /* largest M (= k+1 verify rows) per MoE call      */

typedef struct tqf_hip_ctx tqf_hip_ctx;
typedef struct tqf_hip_weights tqf_hip_weights; /* one Q4_0 matrix in HBM      */
typedef struct tqf_hip_tensor tqf_hip_tensor;   /* one f32 tensor in HBM       */
typedef struct tqf_hip_layer tqf_hip_layer;     /* prepared MoE layer          */
typedef struct tqf_hip_stack tqf_hip_stack;     /* prepared stack of layers    */

/* ---- context: GpuExecutionState::init (backend/metal/expert.rs:77-95) --- */
int32_t tqf_hip_create(int32_t device, tqf_hip_ctx **out);
int32_t tqf_hip_destroy(tqf_hip_ctx *ctx);
/* Last error text of this context ("" if none); valid until the next call. */
const char *tqf_hip_last_error(const tqf_hip_ctx *ctx);
int32_t tqf_hip_synchronize(tqf_hip_ctx *ctx);
/* Device name and compute-unit count, for logs. */
int32_t tqf_hip_device_info(tqf_hip_ctx *ctx, char *name, size_t name_len, int32_t *cu_count);

/* ---- plain device buffers: MetalContext::allocate_broker_buffer_with_data
 *      (backend/metal/context.rs:84-125) without the broker ---------------- */
int32_t tqf_hip_buffer_alloc(tqf_hip_ctx *ctx, size_t bytes, void **dptr);
int32_t tqf_hip_buffer_free(tqf_hip_ctx *ctx, void *dptr);
int32_t tqf_hip_memcpy_h2d(tqf_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
int32_t tqf_hip_memcpy_d2h(tqf_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Device-to-device copy ordered on the context's stream (not waited for):
 * the copies a decode loop makes between stages (the MTP loop's h_prev row). */
int32_t tqf_hip_memcpy_d2d(tqf_hip_ctx *ctx, void *dst, const void *src, size_t bytes);

/* ---- Q4_0 weights: GpuResidentExpert::upload (backend/metal/expert.rs:
 *      110-147) ------------------------------------------------------------- */
/* Device bytes an upload of this shape occupies, so the caller can reserve
 * them with its broker *before* uploading (context.rs:84-125).  0 on a shape
 * the backend cannot hold (cols not a multiple of 32). */
uint64_t tqf_hip_weights_bytes_for(uint32_t rows, uint32_t cols);
/* `q4_0` is rows x (cols/32) row-major 18-byte blocks, len must equal
 * rows*(cols/32)*18.  On failure nothing stays allocated. */
int32_t tqf_hip_weights_upload(tqf_hip_ctx *ctx, const uint8_t *q4_0, size_t len,
                               uint32_t rows, uint32_t cols, tqf_hip_weights **out);
/* Same, from a device-resident Q4_0 byte buffer (a loader that has already
 * placed the .tqf payload in HBM). */
int32_t tqf_hip_weights_upload_device(tqf_hip_ctx *ctx, const void *d_q4_0, size_t len,
                                      uint32_t rows, uint32_t cols, tqf_hip_weights **out);
/* Inverse repack back to GGML Q4_0 bytes (validation, spec's "reorder only
 * if the values are proven unchanged"; format/quant/validate.rs:148-250). */
int32_t tqf_hip_weights_download(tqf_hip_ctx *ctx, const tqf_hip_weights *w, uint8_t *q4_0,
                                 size_t len);
/* GpuResidentExpert::stored_bytes (expert.rs:152-154) for one matrix. */
uint64_t tqf_hip_weights_bytes(const tqf_hip_weights *w);
int32_t tqf_hip_weights_free(tqf_hip_ctx *ctx, tqf_hip_weights *w);

/* f32 tensors (router [n_experts x hidden], shared input gate [hidden], norm
 * scales [hidden]): LoadedQwen36Tensor with GgmlType::F32 (weights.rs:802). */
int32_t tqf_hip_tensor_upload(tqf_hip_ctx *ctx, const float *data, size_t count,
                              tqf_hip_tensor **out);
int32_t tqf_hip_tensor_free(tqf_hip_ctx *ctx, tqf_hip_tensor *t);

/* ---- Q4_0 GEMV / small-M GEMM ------------------------------------------- */
/* Replaces backend::reference::q4k_gemv/q4k_gemm (backend/reference.rs:49-81)
 * and metal::kernels::q4k_gemv_persistent_weights (kernels.rs:565-593) for
 * Q4_0 (matvec_row, model/qwen36/weights.rs:827-843).  x is [m x cols] f32,
 * y is [m x rows] f32, 1 <= m <= TQF_HIP_MAX_TOKENS. */
int32_t tqf_hip_q4_gemv(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *x, uint32_t m,
                        float *y);
int32_t tqf_hip_q4_gemv_device(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *d_x,
                               uint32_t m, float *d_y);
/* `count` same-shape matrices against one shared x [cols] in one launch;
 * d_y is [count x rows].  The rotating-pool bandwidth probe of the GEMV. */
int32_t tqf_hip_q4_gemv_batched_device(tqf_hip_ctx *ctx, const tqf_hip_weights *const *ws,
                                       uint32_t count, const float *d_x, float *d_y);

/* ---- one expert: LoadedQwen36Expert::forward (weights.rs:566-610) and
 *      GpuResidentExpert::forward (backend/metal/expert.rs:162-172) -------- */
/* gate/up are [width x hidden], down is [hidden x width]; x [m x hidden],
 * y [m x hidden].  SwiGLU is fused; no host round trip between GEMVs. */
int32_t tqf_hip_expert_forward(tqf_hip_ctx *ctx, const tqf_hip_weights *gate,
                               const tqf_hip_weights *up, const tqf_hip_weights *down,
                               const float *x, uint32_t m, float *y);

/* ---- one MoE layer over M rows: Qwen36StreamingMoe::forward_batch
 *      (experts/mod.rs:1540-1577) with the arithmetic of
 *      Qwen36ResidentMoe::forward (:1600-1634) ---------------------------- */
typedef struct tqf_hip_moe_weights {
    const tqf_hip_tensor *router;            /* f32 [n_experts x hidden]   */
    const tqf_hip_tensor *shared_input_gate; /* f32 [hidden]               */
    const tqf_hip_weights *shared_gate;      /* Q4_0|Q4_K [width x hidden] */
    const tqf_hip_weights *shared_up;        /* Q4_0|Q4_K [width x hidden] */
    const tqf_hip_weights *shared_down;      /* Q4_0|Q4_K [hidden x width] */
    const tqf_hip_weights *const *routed_gate; /* [n_experts]              */
    const tqf_hip_weights *const *routed_up;   /* [n_experts]              */
    const tqf_hip_weights *const *routed_down; /* [n_experts]              */
    uint32_t n_experts; /* 256: RouterResult::from_logits requires it      */
    uint32_t hidden;    /* 2048 (multiple of 256)                          */
    uint32_t width;     /* 512  (multiple of 256)                          */
} tqf_hip_moe_weights;

/* Builds the device-side expert table once (the analogue of pinning every
 * expert resident: experts/mod.rs:512-545 stage_expert_values).  All
 * 3 (n_experts + 1) expert matrices share one format: TQF_HIP_FORMAT_Q4_0
 * (the group-32 configs) or TQF_HIP_FORMAT_Q4_K (the canonical checkpoint's
 * experts, LoadedQwen36Expert::payload_parts, model/qwen36/weights.rs:
 * 552-561), else TQF_HIP_ERR_INVALID.  A Q4_K layer runs every expert matvec
 * on the Q8_K path of matvec_payload (weights.rs:680-735; bit-identical per
 * matvec to tqf_hip_q4k_matvec), through the same layer, stack and
 * verify-step entry points; tqf_hip_grouped_gemm reads Q4_0 layers only. */
int32_t tqf_hip_moe_layer_prepare(tqf_hip_ctx *ctx, const tqf_hip_moe_weights *weights,
                                  tqf_hip_layer **out);
int32_t tqf_hip_moe_layer_free(tqf_hip_ctx *ctx, tqf_hip_layer *layer);
/* x [m x hidden] f32 -> y [m x hidden]; ids [m x 8] and w [m x 8] receive the
 * routes (RouterResult; may be NULL), for RouterTrace parity
 * (runtime/decode.rs:14-17).  TQF_HIP_ERR_ROUTER if a router logit is not
 * finite. */
int32_t tqf_hip_moe_layer(tqf_hip_ctx *ctx, const tqf_hip_layer *layer, const float *x,
                          uint32_t m, float *y, uint16_t *ids, float *w);
/* Same with bf16 activations (converted exactly to f32 on entry). */
int32_t tqf_hip_moe_layer_bf16(tqf_hip_ctx *ctx, const tqf_hip_layer *layer,
                               const uint16_t *x_bf16, uint32_t m, float *y, uint16_t *ids,
                               float *w);
/* Device-pointer form; d_status (may be NULL) receives 0 or TQF_HIP_ERR_ROUTER. */
int32_t tqf_hip_moe_layer_device(tqf_hip_ctx *ctx, const tqf_hip_layer *layer, const float *d_x,
                                 uint32_t m, float *d_y, uint16_t *d_ids, float *d_w,
                                 int32_t *d_status);

/* ---- stacked layers: the layer wrapper of bounded_layer_forward
 *      (model/qwen36/runtime.rs:777-802): h <- h + MoE_l(rmsnorm_l(h)) ------ */
int32_t tqf_hip_stack_prepare(tqf_hip_ctx *ctx, const tqf_hip_layer *const *layers,
                              const tqf_hip_tensor *const *ffn_norms, uint32_t n_layers,
                              tqf_hip_stack **out);
int32_t tqf_hip_stack_free(tqf_hip_ctx *ctx, tqf_hip_stack *stack);
/* d_h_in [m x hidden] f32 is the layer-0 input (the verify rows' hidden
 * state); the result is written to d_h [m x hidden].  d_h_in may be NULL or
 * equal d_h to update d_h in place.  d_ids/d_w ([n_layers x m x 8], may be
 * NULL) receive every layer's route; *d_status (may be NULL, zeroed by the
 * caller) is set to TQF_HIP_ERR_ROUTER if any layer's routing fails.
 * Every layer of a stack has one expert format.  For Q4_0 layers with
 * m <= 4 on the model geometry (hidden 2048, width <= 2048, <= 256
 * experts) the whole stack runs as one persistent launch of one workgroup
 * per CU, which needs every workgroup resident at once.  If other work on
 * the device keeps it from being co-scheduled, its waits time out after
 * 20 ms; with TQF_HIP_VARIANT_RECOVER (the default) the call then re-runs the
 * stack through the per-layer kernels and returns their result (counted by
 * tqf_hip_recovery_counts), for which it waits for the persistent launch
 * before returning; with the variant off the call stays asynchronous and a
 * timed-out launch reports TQF_HIP_ERR_DEVICE in *d_status, d_h undefined.
 * Otherwise the per-layer kernels are captured once into a HIP graph per
 * argument set and replayed. */
int32_t tqf_hip_stack_forward_device(tqf_hip_ctx *ctx, const tqf_hip_stack *stack,
                                     const float *d_h_in, float *d_h, uint32_t m,
                                     uint16_t *d_ids, float *d_w, int32_t *d_status);

/* ---- acceptance: Sampler::select (sampling/mod.rs:68-74) and
 *      mtp::verify_pair (runtime/mtp.rs:98-104) generalised to k drafts ------
 * target [k+1 x vocab], draft [k x vocab] (ignored when greedy), draft_tokens
 * [k].  Greedy (the temperature == 0 identity path, sampling/mod.rs:43-50):
 * accept while argmax(target_i) == draft_i (argmax as
 * top_logit_candidates, runtime/decode.rs:48-64); k == 1 is verify_pair.
 * Stochastic: accept draft i iff u[i] < p_i(d)/q_i(d) with p, q the softmax of
 * logits/temperature; on the first rejection resample from
 * norm(max(0, p - q)) with u_resample[i]; if all k are accepted the bonus
 * token is drawn from p_k with u_resample[k].  Writes *accepted (0..k) and
 * tokens_out[k+1] (tokens_out[0..accepted] are emitted, the rest are -1).
 * Bit-exact with the CPU definition for identical inputs.  Vocabularies up
 * to about one million run as one launch whose workgroups exchange partials
 * and so must all be resident at once.  An exchange that does not complete
 * within 20 ms (other work holding compute units) makes that launch write
 * *accepted = -1; with TQF_HIP_VARIANT_RECOVER (the default) the call then
 * re-runs the acceptance through the three-kernel path (no waits between
 * workgroups; the same bits) and returns its result, for which the device
 * form waits for the launch before returning; with the variant off the -1
 * stays and the next call runs normally. */
int32_t tqf_hip_accept(tqf_hip_ctx *ctx, const float *target, const float *draft,
                       const int32_t *draft_tokens, uint32_t k, uint32_t vocab, float temperature,
                       int32_t greedy, const float *u, const float *u_resample, int32_t *accepted,
                       int32_t *tokens_out);
int32_t tqf_hip_accept_device(tqf_hip_ctx *ctx, const float *d_target, const float *d_draft,
                              const int32_t *d_draft_tokens, uint32_t k, uint32_t vocab,
                              float temperature, int32_t greedy, const float *d_u,
                              const float *d_u_resample, int32_t *d_accepted,
                              int32_t *d_tokens_out);
/* tqf_hip_accept_device without any allocation: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * same kernels and results as tqf_hip_accept_device, with their scratch in a
 * fixed per-GPU array of 256 KiB (held until the process ends) instead of a
 * context allocation.  It holds the one-launch acceptance kernel's scratch
 * (vocab up to 1,048,576 at k <= 3 and 524,288 at k >= 4 on MI355X); larger
 * vocabularies, whose kernels need more, are TQF_HIP_ERR_INVALID.  Every call on one GPU
 * shares that array, so calls that overlap on one GPU (from two contexts or
 * two streams) race; calls ordered on one stream do not.  The entry point
 * calls no hipMalloc, hipFree or other allocating routine, and records no
 * profiling events. */
int32_t tqf_hip_accept_device_noalloc(tqf_hip_ctx *ctx, const float *d_target,
                                      const float *d_draft, const int32_t *d_draft_tokens,
                                      uint32_t k, uint32_t vocab, float temperature,
                                      int32_t greedy, const float *d_u,
                                      const float *d_u_resample, int32_t *d_accepted,
                                      int32_t *d_tokens_out);
/* Sampler::select (sampling/mod.rs:68-74) for each of `rows` (<= 8) rows of
 * vocab logits (device pointers), bit-identical to the reference: with
 * temperature 0, Sampler::Greedy's argmax (top_logit_candidates'); otherwise
 * the stochastic path with the default filters (no penalties, top_k, top_p or
 * min_p): softmax(logits / temperature) with f32::exp and the token-order f32
 * total (softmax, :166-190), the stable descending sort with ties to the
 * lower token (compare_desc, :258-266), then draw's inverse CDF (:227-248)
 * with d_u[row] in the place of rng.next_f32().  d_tokens [rows] receives
 * the tokens.  The two sums are the reference's sequential f32 folds, bit for
 * bit, computed in parallel: integer sums on the running sum's grid, with the
 * crossings of a binade and the exact ties as single f32 adds.  d_sums (may
 * be NULL; not written at temperature 0) receives [rows x 2]: the token-order
 * total of the exponentials and the sorted-order total of the probabilities
 * (NaN when a probability is NaN), for callers that check the softmax's
 * normalisation.  For callers that need the reference's token for the same
 * uniform; the acceptance's draw (exact fixed-point sums, no sort) is the
 * faster pick. */
int32_t tqf_hip_sampler_select_device(tqf_hip_ctx *ctx, const float *d_logits, uint32_t rows, uint32_t vocab,
                                      float temperature, const float *d_u, int32_t *d_tokens, float *d_sums);
/* top_logit_candidates (runtime/decode.rs:48-64) over `rows` rows of vocab
 * logits: tokens4/logits4 are [rows x 4]. */
int32_t tqf_hip_top_logit_candidates(tqf_hip_ctx *ctx, const float *logits, uint32_t rows,
                                     uint32_t vocab, uint32_t *tokens4, float *logits4);

/* ---- prefill-shaped grouped expert GEMM: the routed loop of
 *      Qwen36StreamingMoe::forward_batch (experts/mod.rs:1562-1566, one
 *      forward_batch_expert :1079-1131 GEMV chain per row and route) over a
 *      prefill chunk (prefill_chunk, model/qwen36/runtime.rs:265-366), and
 *      the unused Metal tqf_q4k_gemm (backend/metal/kernels.rs:311-336) -----
 * x_bf16 [t x hidden], ids [t x 8] (< n_experts), w [t x 8] f32 ->
 * y [t x hidden] f32 = sum_k w[t,k] * expert_{ids[t,k]}(x_t), summed in route
 * order (the routed part only: the caller adds the shared expert).  The
 * (token, k) pairs are sorted by expert on the device and each expert's
 * gate/up/down run as bf16 matrix-core GEMMs with exact Q4_0 weights and
 * fp32 accumulation.  1 <= t <= TQF_HIP_GROUPED_MAX_TOKENS. */
#define TQF_HIP_GROUPED_MAX_TOKENS 4096
int32_t tqf_hip_grouped_gemm(tqf_hip_ctx *ctx, const tqf_hip_layer *layer, const uint16_t *x_bf16,
                             uint32_t t, const uint16_t *ids, const float *w, float *y);
/* Device-pointer form; *d_status (may be NULL, zeroed by the caller) is set
 * to TQF_HIP_ERR_INVALID if an id is out of range (y is then not written). */
int32_t tqf_hip_grouped_gemm_device(tqf_hip_ctx *ctx, const tqf_hip_layer *layer,
                                    const uint16_t *d_x_bf16, uint32_t t, const uint16_t *d_ids,
                                    const float *d_w, float *d_y, int32_t *d_status);

/* ---- canonical Q4_K matrices (GGML 144-byte super-blocks of 256 elements,
 *      format/quant/dequant.rs:139-184): the format of the checkpoint's
 *      routed experts (LoadedQwen36Expert::payload_parts, model/qwen36/
 *      weights.rs:552-561) ------------------------------------------------- */
/* A handle from these uploads is a tqf_hip_weights of format Q4_K: only the
 * q4k entry points accept it (the Q4_0 ones reject it, and vice versa). */
#define TQF_HIP_FORMAT_Q4_0 0
#define TQF_HIP_FORMAT_Q4_K 1
#define TQF_HIP_FORMAT_Q6_K 2
/* Device bytes of a Q4_K upload of this shape; 0 unless cols is a positive
 * multiple of 256. */
uint64_t tqf_hip_q4k_weights_bytes_for(uint32_t rows, uint32_t cols);
/* `q4_k` is rows x (cols/256) row-major 144-byte super-blocks; len must equal
 * rows*(cols/256)*144.  Lossless repack (GpuResidentExpert::upload,
 * backend/metal/expert.rs:110-147, for one matrix). */
int32_t tqf_hip_q4k_weights_upload(tqf_hip_ctx *ctx, const uint8_t *q4_k, size_t len,
                                   uint32_t rows, uint32_t cols, tqf_hip_weights **out);
int32_t tqf_hip_q4k_weights_upload_device(tqf_hip_ctx *ctx, const void *d_q4_k, size_t len,
                                          uint32_t rows, uint32_t cols, tqf_hip_weights **out);
/* Inverse repack back to the GGML Q4_K bytes (format/quant/validate.rs:
 * 148-250's "reorder only if the values are proven unchanged"). */
int32_t tqf_hip_q4k_weights_download(tqf_hip_ctx *ctx, const tqf_hip_weights *w, uint8_t *q4_k,
                                     size_t len);

/* ---- routed-expert superextents of a .tqf container -> device ----------------
 * The expert-index half of TqfReader (format/tqf/reader.rs:170-247, 312-327)
 * and the staging path of Qwen36WeightLoader::expert_stored_bytes /
 * load_expert (model/qwen36/weights.rs:1387-1444) with
 * WholeExpertLfuCache::stage_expert_values (experts/mod.rs:512-545), over a
 * container region the caller supplies (it reads or maps the file; file I/O
 * and the BLAKE3 digests of the checksum table stay on its side).
 * Decoded forms of the spec's section-124 records (the on-disk 32- and
 * 24-byte little-endian layouts of format/tqf/records.rs:221-313).  The
 * table functions run on the host only; their ctx may be NULL (it receives
 * the last-error message). */
#define TQF_HIP_MATRIX_GATE_UP 0
#define TQF_HIP_MATRIX_DOWN 1
typedef struct tqf_hip_expert_index {
    uint8_t layer;
    uint16_t expert;
    uint16_t flags;          /* bit 0: per-tile checksums follow the expert's digest */
    uint16_t layout_id;      /* quant layout; 2 = Q4_K passthrough */
    uint64_t file_offset;    /* the superextent, from the start of the container */
    uint32_t stored_bytes;
    uint32_t tile_first;     /* into the tile table */
    uint16_t tile_count;
    uint32_t checksum_index;
} tqf_hip_expert_index;
typedef struct tqf_hip_expert_tile {
    uint8_t matrix;          /* TQF_HIP_MATRIX_GATE_UP or _DOWN */
    uint16_t tile_id;
    uint16_t neuron_start, neuron_count;
    uint32_t relative_offset, stored_bytes;  /* within the superextent */
    uint16_t quant_layout_id;
    uint16_t flags;
} tqf_hip_expert_tile;
typedef struct tqf_hip_expert_table tqf_hip_expert_table;
/* Parses the expert-index blob (superblock expert_index_offset /
 * expert_index_bytes): expert_count index records, then tile records to the
 * end of the blob; expert_count is the ExpertIndex section's element_count,
 * file_len the container's length, checksum_entries the checksum table's
 * entry count.  TQF_HIP_ERR_INVALID (nothing allocated) unless, as TqfReader
 * requires: the records fit, the tile part holds whole records with known
 * matrices, every superextent lies inside the container, every tile range
 * inside the tile table and exactly partitioning its superextent in order,
 * and per-tile checksum ranges inside the checksum table. */
int32_t tqf_hip_expert_table_open(tqf_hip_ctx *ctx, const uint8_t *blob, size_t blob_len, uint64_t expert_count,
                                  uint64_t file_len, uint64_t checksum_entries, tqf_hip_expert_table **out);
int32_t tqf_hip_expert_table_free(tqf_hip_ctx *ctx, tqf_hip_expert_table *table);
int32_t tqf_hip_expert_table_counts(const tqf_hip_expert_table *table, uint64_t *experts, uint64_t *tiles);
/* TqfReader::expert(layer, expert): the index record and its tiles
 * (tiles_out may be NULL to ask for *n_tiles). */
int32_t tqf_hip_expert_lookup(tqf_hip_ctx *ctx, const tqf_hip_expert_table *table, uint8_t layer, uint16_t expert,
                              tqf_hip_expert_index *index_out, tqf_hip_expert_tile *tiles_out, size_t tiles_cap,
                              size_t *n_tiles);
/* The reservations to make before staging (expert_stored_bytes, the broker's
 * reserve-before-allocate): the superextent's stored bytes (host staging),
 * and the device bytes of its three Q4_K uploads. */
int32_t tqf_hip_expert_reserve_bytes(tqf_hip_ctx *ctx, const tqf_hip_expert_table *table, uint8_t layer,
                                     uint16_t expert, uint64_t *stored_bytes, uint64_t *device_bytes);
/* load_expert's checks (layout Q4_K passthrough, 3 x 589,824 stored bytes,
 * every tile Q4_K, classify_partition over the gate+up and down regions),
 * then payload_parts and one Q4_K upload each of gate [512 x 2048], up
 * [512 x 2048] and down [2048 x 512] from container[file_offset ..].  On
 * failure nothing stays allocated. */
int32_t tqf_hip_expert_upload(tqf_hip_ctx *ctx, const tqf_hip_expert_table *table, uint8_t layer, uint16_t expert,
                              const uint8_t *container, size_t container_len, tqf_hip_weights **gate,
                              tqf_hip_weights **up, tqf_hip_weights **down);
/* fp32 semantics of backend::reference::q4k_gemv / q4k_gemm (backend/
 * reference.rs:49-81) and of the Metal tqf_q4k_gemv (backend/metal/
 * kernels.rs:535-593): y[t][r] = sum_i dequant(w[r])_i x[t][i].  x [m x cols],
 * y [m x rows] f32, 1 <= m <= TQF_HIP_MAX_TOKENS.  Within 2^-22 of each
 * 32-element block's largest |x| per product; fp32 accumulation. */
int32_t tqf_hip_q4k_gemv(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *x, uint32_t m,
                         float *y);
int32_t tqf_hip_q4k_gemv_device(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *d_x,
                                uint32_t m, float *d_y);
/* `count` same-shape Q4_K matrices against one x [cols]: d_y [count x rows]. */
int32_t tqf_hip_q4k_gemv_batched_device(tqf_hip_ctx *ctx, const tqf_hip_weights *const *ws,
                                        uint32_t count, const float *d_x, float *d_y);
/* The checkpoint's CPU matvec, matvec_payload for GgmlType::Q4K (model/
 * qwen36/weights.rs:680-735): quantize_q8_k per 256-element chunk of each x
 * row (:898-931), then q4_k_dot_pre per output row (:944-1021).  Bit-identical
 * to that scalar code (NaN as NaN).  Shapes as tqf_hip_q4k_gemv. */
int32_t tqf_hip_q4k_matvec(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *x, uint32_t m,
                           float *y);
int32_t tqf_hip_q4k_matvec_device(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *d_x,
                                  uint32_t m, float *d_y);
int32_t tqf_hip_q4k_matvec_batched_device(tqf_hip_ctx *ctx, const tqf_hip_weights *const *ws,
                                          uint32_t count, const float *d_x, float *d_y);
/* LoadedQwen36Expert::forward (weights.rs:566-610) over m rows: gate and up
 * Q4_K matvecs ([width x hidden]), silu_mul (weights.rs:241-260), down
 * matvec ([hidden x width]), each matvec with the Q8_K semantics above.
 * x [m x hidden], y [m x hidden] f32. */
int32_t tqf_hip_q4k_expert_forward(tqf_hip_ctx *ctx, const tqf_hip_weights *gate,
                                   const tqf_hip_weights *up, const tqf_hip_weights *down,
                                   const float *x, uint32_t m, float *y);
int32_t tqf_hip_q4k_expert_forward_device(tqf_hip_ctx *ctx, const tqf_hip_weights *gate,
                                          const tqf_hip_weights *up,
                                          const tqf_hip_weights *down, const float *d_x,
                                          uint32_t m, float *d_y);

/* ---- the LM head: canonical Q6_K matrices (GGML 210-byte super-blocks of
 *      256, format/quant/dequant.rs:190-218), the checkpoint's lm_head
 *      (model/qwen36/weights.rs:1744, runtime.rs:435) ---------------------- */
/* Device bytes of a Q6_K upload of this shape (the GGML size, 210 bytes per
 * 256 weights, plus padding); 0 unless cols is a positive multiple of 256. */
uint64_t tqf_hip_q6k_weights_bytes_for(uint32_t rows, uint32_t cols);
/* `q6_k` is rows x (cols/256) row-major 210-byte super-blocks; lossless
 * repack.  Handles are format TQF_HIP_FORMAT_Q6_K (only the q6k / lm_head
 * entry points accept them). */
int32_t tqf_hip_q6k_weights_upload(tqf_hip_ctx *ctx, const uint8_t *q6_k, size_t len,
                                   uint32_t rows, uint32_t cols, tqf_hip_weights **out);
int32_t tqf_hip_q6k_weights_upload_device(tqf_hip_ctx *ctx, const void *d_q6_k, size_t len,
                                          uint32_t rows, uint32_t cols, tqf_hip_weights **out);
int32_t tqf_hip_q6k_weights_download(tqf_hip_ctx *ctx, const tqf_hip_weights *w, uint8_t *q6_k,
                                     size_t len);
/* matvec_payload for GgmlType::Q6K (weights.rs:680-735): quantize_q8_k per
 * 256-element chunk of each x row, then q6_k_dot_pre per output row
 * (:1023-1101).  Bit-identical to that scalar code.  x [m x cols], y
 * [m x rows] f32, 1 <= m <= TQF_HIP_MAX_TOKENS. */
int32_t tqf_hip_q6k_matvec(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *x, uint32_t m,
                           float *y);
int32_t tqf_hip_q6k_matvec_device(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *d_x,
                                  uint32_t m, float *d_y);
/* The LM head with the fused greedy candidates: logits [m x V] =
 * tqf_hip_q6k_matvec(w [V x hidden], x [m x hidden]) (lm_head.matvec,
 * runtime.rs:435; the Metal lm_head_logits, backend/metal/kernels.rs:
 * 1080-1098, for Q6_K), and per row the four candidates of
 * top_logit_candidates (runtime/decode.rs:48-64) -- tokens4 / logits4
 * [m x 4], descending, ties to the lower token, NaN and -inf never taken
 * (empty slots: token 0, -inf) -- from the same pass over the weights. */
int32_t tqf_hip_lm_head_logits(tqf_hip_ctx *ctx, const tqf_hip_weights *w, const float *x,
                               uint32_t m, float *logits, uint32_t *tokens4, float *logits4);
int32_t tqf_hip_lm_head_logits_device(tqf_hip_ctx *ctx, const tqf_hip_weights *w,
                                      const float *d_x, uint32_t m, float *d_logits,
                                      uint32_t *d_tokens4, float *d_logits4);

/* ---- the decode loop's row kernels ------------------------------------------
 * Embedding rows (Qwen36Runtime::decode_step's embedding.row,
 * model/qwen36/runtime.rs:403; the row decoded per its dtype as
 * LoadedQwen36Tensor::row, model/qwen36/weights.rs:346-379): d_out[i] =
 * dequantize_q4_0(row d_tokens[i] of emb) (+ d_add[i] when d_add is given),
 * [n x cols] f32.  emb is a Q4_0 handle [V x cols].  A token outside [0, V)
 * gives a NaN row and, when d_status is given, TQF_HIP_ERR_INVALID there
 * (the reference's ModelError::Shape, runtime.rs:392-399).  d_add may be
 * d_out (in place: each element is read, then written, by the same thread);
 * any other overlap of d_add and d_out is not allowed. */
int32_t tqf_hip_embed_rows_device(tqf_hip_ctx *ctx, const tqf_hip_weights *emb, const int32_t *d_tokens,
                                  uint32_t n, const float *d_add, float *d_out, int32_t *d_status);
/* RMSNorm rows: the final norm ahead of the LM head (runtime.rs:430-431,
 * Qwen36Activation::qwen_rmsnorm): d_out[i] = d_x[i] * (1 / sqrt(mean(d_x[i]^2)
 * + 1e-6)) * w, [n x cols] f32, w a tensor of cols floats.  The sum of squares
 * is a block reduction (its order is not the scalar loop's). */
int32_t tqf_hip_rmsnorm_rows_device(tqf_hip_ctx *ctx, const float *d_x, uint32_t n, uint32_t cols,
                                    const tqf_hip_tensor *w, float *d_out);

/* ---- one MTP verify step: the stack over the k+1 verify rows, then the
 *      acceptance, as one stream-ordered (graph-replayed) unit.  The verify
 *      loop the reference leaves unwired (runtime/mtp.rs:1-20).
 *      d_status (device int32, may be null): the stack's device status, as
 *      tqf_hip_stack_forward_device writes it -- TQF_HIP_ERR_ROUTER for a
 *      non-finite router logit (RouterResult::from_logits, experts/mod.rs:
 *      140-145), TQF_HIP_ERR_DEVICE for a timed-out grid barrier when
 *      TQF_HIP_VARIANT_RECOVER is off (with it on, the library re-runs the
 *      timed-out part itself, as tqf_hip_stack_forward_device and
 *      tqf_hip_accept_device do, and the call returns once the step is
 *      complete); never cleared by the library, so the caller zeroes it and
 *      checks it after the step.  A step that sets it has left d_h
 *      undefined; the acceptance, which reads only the logits, still runs. */
int32_t tqf_hip_verify_step_device(tqf_hip_ctx *ctx, const tqf_hip_stack *stack,
                                   const float *d_h_in, float *d_h, uint32_t m,
                                   const float *d_target, const float *d_draft,
                                   const int32_t *d_draft_tokens, uint32_t vocab,
                                   float temperature, int32_t greedy, const float *d_u,
                                   const float *d_u_resample, int32_t *d_accepted,
                                   int32_t *d_tokens_out, int32_t *d_status);

/* ---- kernel variants: the counterpart of GpuKernelKind::from_env and
 *      GpuExecutionState::kernel_kind (backend/metal/expert.rs:56-92).  Each
 *      selector starts from the environment when the context is created
 *      (TQF_HIP_PERSISTENT, TQF_HIP_Q4K_FOLD, TQF_HIP_GRAPHS,
 *      TQF_HIP_RECOVER: "0" selects 0, anything else or unset 1) and is
 *      changed per context here; a change drops the context's captured
 *      graphs, so no replay keeps an old choice. ------------------------- */
#define TQF_HIP_VARIANT_PERSISTENT 0 /* 1: the persistent stack kernel where it applies;
                                        0: per-layer kernels (graph-replayed)          */
#define TQF_HIP_VARIANT_Q4K_FOLD 1   /* 1: a Q4_K layer's combine folded into its down
                                        launch; 0: the separate combine launch          */
#define TQF_HIP_VARIANT_GRAPHS 2     /* 1: multi-launch paths replay HIP graphs;
                                        0: eager launches of the same kernels           */
#define TQF_HIP_VARIANT_RECOVER 3    /* 1: a persistent launch whose cross-workgroup
                                        wait times out is re-run through kernels that
                                        do not wait on one another (the entry points
                                        that launch one wait for it); 0: asynchronous,
                                        the timeout reported as an error            */
#define TQF_HIP_VARIANTS 4
int32_t tqf_hip_set_variant(tqf_hip_ctx *ctx, int32_t variant, int32_t value);
int32_t tqf_hip_get_variant(tqf_hip_ctx *ctx, int32_t variant, int32_t *value);
/* Re-runs so far on this context after a timed-out persistent launch: of the
 * stack (per-layer kernels) and of the acceptance (three-kernel path).  The
 * counterpart of the reference's fallback when the GPU path cannot run
 * (experts/mod.rs:480-497), reported the way ExpertCacheStats reports cache
 * events (experts/mod.rs:201-234). */
int32_t tqf_hip_recovery_counts(tqf_hip_ctx *ctx, uint64_t *stack_reruns, uint64_t *accept_reruns);

/* ---- profiling: the HIP counterpart of backend/metal/timing.rs:23-80 ----- */
#define TQF_HIP_KERNEL_ROUTE 0    /* rmsnorm + router + top-8 + union plan    */
#define TQF_HIP_KERNEL_GATE_UP 1  /* union-expert gate/up GEMV + SwiGLU       */
#define TQF_HIP_KERNEL_DOWN 2     /* union-expert down GEMV + weighted combine */
#define TQF_HIP_KERNEL_GEMV 3     /* standalone Q4_0 GEMV                     */
#define TQF_HIP_KERNEL_ACCEPT 4   /* the acceptance kernels, summed           */
#define TQF_HIP_KERNEL_STACK 5    /* the persistent whole-stack MoE kernel     */
#define TQF_HIP_KERNEL_GROUPED_GATE_UP 6 /* grouped GEMM: gate/up + SwiGLU    */
#define TQF_HIP_KERNEL_GROUPED_DOWN 7    /* grouped GEMM: down                */
#define TQF_HIP_KERNEL_GROUPED_AUX 8     /* grouped GEMM: sort plan + combine */
#define TQF_HIP_KERNEL_Q4K_GEMV 9        /* Q4_K GEMV, fp32 semantics         */
#define TQF_HIP_KERNEL_Q4K_MATVEC 10     /* Q4_K matvec, Q8_K semantics       */
#define TQF_HIP_KERNEL_Q6K_MATVEC 11     /* Q6_K matvec / LM head (+ top-4)   */
#define TQF_HIP_KERNEL_SAMPLE 12         /* Sampler::select, reference-exact  */
#define TQF_HIP_KERNEL_KINDS 13
/* While enabled, eager (non-graph) launches of each kind are bracketed by HIP
 * events on the context stream.  Enabling clears the totals. */
int32_t tqf_hip_profile_enable(tqf_hip_ctx *ctx, int32_t enable);
/* Synchronises, then reports launches, summed kernel milliseconds and the
 * summed algorithmic HBM bytes of those launches for one kind (0 for the
 * grouped GEMM kinds, whose bytes depend on the routes: the caller, who holds
 * the ids, counts the distinct experts). */
int32_t tqf_hip_profile_read(tqf_hip_ctx *ctx, int32_t kind, uint64_t *launches,
                             double *total_ms, double *algorithmic_bytes);

#ifdef __cplusplus
}
#endif
#endif /* TQF_HIP_H */
