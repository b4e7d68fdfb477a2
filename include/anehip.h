/*
 * anehip.h — C ABI of the MI355X (gfx950) decode-step library.
 *
 * This library replaces the Metal decode path of ane-infer
 * (crates/engine/src/{metal_graph.rs, gpu_decode.rs, gpu_full_decode.rs} and
 * crates/engine/metal/{q8_gemv,q4_gemv,deltanet,attention}.metal) with hand-written HIP kernels for gfx950 that
 * are captured as one hipGraph per decode step.  The interface style follows
 * the reference's own C ABI precedent (crates/ane-bridge/objc/ane_runtime.h:
 * opaque handle, int status, explicit free), with these rules:
 *
 *   - every entry point is `extern "C"`, takes plain pointers and sizes, and
 *     returns an int status: ANEHIP_OK (0) or a negative ANEHIP_E* code;
 *   - after a failure `anehip_last_error(ctx)` returns a message
 *     (`anehip_last_error(NULL)` reports failures that had no context);
 *   - host buffers passed in are copied; the caller keeps ownership;
 *   - one context is used by one host thread at a time; all GPU work of a
 *     context is ordered on the context's stream.
 *
 * Quantised weight bytes are accepted exactly in the GGUF block layouts the
 * reference uses (crates/gguf/src/dequant.rs:12-38, parser.rs:127,131):
 *   Q8_0 (ggml type 8): 34-byte blocks = fp16 scale (LE) + 32 x int8
 *   Q4_0 (ggml type 2): 18-byte blocks = fp16 scale (LE) + 16 bytes; element i
 *                       is the low nibble of byte i, element i+16 the high
 *                       nibble; value = (nibble - 8) * scale
 * stored row-major: row r of an [m x n] tensor is n/32 consecutive blocks.
 */
#ifndef ANEHIP_H
#define ANEHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define ANEHIP_OK 0
#define ANEHIP_EINVAL (-1)       /* bad argument (null pointer, zero size, ...) */
#define ANEHIP_ESHAPE (-2)       /* sizes disagree (q8_gemv.rs:41-50 asserts)   */
#define ANEHIP_EUNSUPPORTED (-3) /* valid but not supported by these kernels     */
#define ANEHIP_ENOMEM (-4)       /* device allocation failed                     */
#define ANEHIP_EHIP (-5)         /* HIP runtime error (message has the detail)   */
#define ANEHIP_ESTATE (-6)       /* call out of order (no weights/state yet)     */
#define ANEHIP_ERANGE (-7)       /* position or token out of range               */
#define ANEHIP_ENODEV (-8)       /* no usable gfx950 device                      */

/* GGML type codes, as in QuantType (crates/engine/src/q8_gemv.rs:10-14). */
#define ANEHIP_GGML_Q4_0 2u
#define ANEHIP_GGML_Q8_0 8u

/* Layer types, as in LayerType (crates/engine/src/model.rs:100-104). */
#define ANEHIP_LAYER_DELTANET 0u
#define ANEHIP_LAYER_FULL_ATTENTION 1u

/*
 * Tensor kinds: one per field of DeltaNetLayerWeights / FullAttnLayerWeights /
 * FfnWeights / Qwen35ModelWeights (crates/engine/src/model.rs:108-157).
 * Per-layer kinds are uploaded with layer = 0..n_layers-1, model-level kinds
 * with layer = -1.  Shapes are [rows x cols] row-major, d = dim, F = hidden_dim,
 * H = ssm_group_count, C = 3*d conv channels, hd = head_dim.
 */
typedef enum anehip_tensor_kind {
    ANEHIP_T_ATTN_NORM = 0,       /* f32 [d]                                    */
    ANEHIP_T_POST_ATTN_NORM = 1,  /* f32 [d]                                    */
    ANEHIP_T_FFN_GATE = 2,        /* quant [F x d]                              */
    ANEHIP_T_FFN_UP = 3,          /* quant [F x d]                              */
    ANEHIP_T_FFN_DOWN = 4,        /* quant [d x F]                              */
    ANEHIP_T_QKV = 5,             /* DeltaNet: quant [C x d]                    */
    ANEHIP_T_ATTN_GATE = 6,       /* DeltaNet: quant [d x d]                    */
    ANEHIP_T_SSM_A = 7,           /* DeltaNet: f32 [H]                          */
    ANEHIP_T_SSM_ALPHA = 8,       /* DeltaNet: quant [H x d]                    */
    ANEHIP_T_SSM_BETA = 9,        /* DeltaNet: quant [H x d]                    */
    ANEHIP_T_SSM_CONV1D = 10,     /* DeltaNet: f32 [C x conv_kernel]            */
    ANEHIP_T_SSM_DT_BIAS = 11,    /* DeltaNet: f32 [H]                          */
    ANEHIP_T_SSM_NORM = 12,       /* DeltaNet: f32 [ssm_state_size]             */
    ANEHIP_T_SSM_OUT = 13,        /* DeltaNet: quant [d x d]                    */
    ANEHIP_T_WQ = 14,             /* attention: quant [2*n_heads*hd x d]        */
    ANEHIP_T_WK = 15,             /* attention: quant [n_kv_heads*hd x d]       */
    ANEHIP_T_WV = 16,             /* attention: quant [n_kv_heads*hd x d]       */
    ANEHIP_T_WO = 17,             /* attention: quant [d x n_heads*hd]          */
    ANEHIP_T_Q_NORM = 18,         /* attention: f32 [hd]                        */
    ANEHIP_T_K_NORM = 19,         /* attention: f32 [hd]                        */
    ANEHIP_T_EMBEDDING = 20,      /* model: f32 [vocab x d]                     */
    ANEHIP_T_FINAL_NORM = 21,     /* model: f32 [d]                             */
    ANEHIP_T_LM_HEAD = 22,        /* model: quant [vocab x d]                   */
    ANEHIP_T_COUNT = 23
} anehip_tensor_kind;

/*
 * Model description: the fields of ModelConfig + Qwen35Config
 * (crates/engine/src/model.rs:7-18, 59-67).  The DeltaNet mixer uses
 * 3*dim conv channels and dim/ssm_group_count key/value dims per head, exactly
 * as HybridCache::new (crates/engine/src/deltanet_cache.rs:81-83) and
 * deltanet_decode_step (crates/engine/src/deltanet.rs:452-457) derive them.
 */
typedef struct anehip_model_desc {
    uint32_t dim;               /* hidden size d                               */
    uint32_t hidden_dim;        /* FFN size F                                  */
    uint32_t n_layers;
    uint32_t n_heads;           /* attention query heads                       */
    uint32_t n_kv_heads;        /* attention key/value heads                   */
    uint32_t head_dim;          /* attention head dim                          */
    uint32_t vocab_size;
    uint32_t ssm_state_size;    /* DeltaNet key dim == value dim               */
    uint32_t ssm_conv_kernel;   /* depthwise conv width                        */
    uint32_t ssm_group_count;   /* DeltaNet heads                              */
    float rope_freq_base;
    float rms_norm_eps;
    const uint8_t *layer_types; /* n_layers entries of ANEHIP_LAYER_*         */
} anehip_model_desc;

typedef struct anehip_ctx anehip_ctx;

/* ---- runtime ------------------------------------------------------------ */

/* Checks that a gfx950 device is present.  Returns ANEHIP_OK or ANEHIP_ENODEV.
 * Replaces GpuContext::new's device probe (crates/engine/src/metal_graph.rs:79). */
int anehip_init(void);

/* Message for the last failure on ctx (or of a context-free call if ctx is
 * NULL).  The string stays valid until the next call on the same ctx. */
const char *anehip_last_error(const anehip_ctx *ctx);

/* Creates a context on HIP device `device`.  desc may be NULL for a bare
 * context that only runs the kernel-level entry points.  The context owns
 * a HIP stream.  Replaces GpuContext::new (metal_graph.rs:79-138) and the
 * constant setup of GpuConstantPool::new (gpu_full_decode.rs:104-159). */
int anehip_ctx_create(int device, const anehip_model_desc *desc, anehip_ctx **out);
void anehip_ctx_destroy(anehip_ctx *ctx);

/* Blocks until all work queued on the context's stream is done. */
int anehip_sync(anehip_ctx *ctx);

/* ---- device memory helpers (for callers that have no HIP runtime) -------- */
int anehip_dev_alloc(anehip_ctx *ctx, size_t nbytes, void **dptr);
int anehip_dev_free(anehip_ctx *ctx, void *dptr);
int anehip_h2d(anehip_ctx *ctx, void *dst, const void *src, size_t nbytes);
int anehip_d2h(anehip_ctx *ctx, void *dst, const void *src, size_t nbytes);
/* anehip_dev_memset enqueues on the context stream; it returns ANEHIP_ESTATE
 * while that stream is being captured (no memset nodes in graphs). */
int anehip_dev_memset(anehip_ctx *ctx, void *dst, int value, size_t nbytes);
int anehip_d2d(anehip_ctx *ctx, void *dst, const void *src, size_t nbytes);

/* ---- timing on the context's stream (hipEvent pairs) -------------------- */
/* Records a start event; anehip_timer_stop records the stop event, waits for
 * it and returns the elapsed milliseconds between the two. */
int anehip_timer_start(anehip_ctx *ctx);
int anehip_timer_stop(anehip_ctx *ctx, float *ms);

/* ---- graph capture of kernel-level calls -------------------------------- */
/* anehip_capture_begin starts capturing the context stream: the kernel-level
 * entry points called until anehip_capture_end are recorded, not run, into a
 * graph that anehip_graph_launch replays on the stream (same pointers, same
 * sizes).  Calls that would have to grow the context workspace fail during
 * capture: make each call once before capturing.  The decode-step entry
 * points keep their own per-step graph and are not capturable.  Replaces the
 * per-token command-buffer encoding of the reference (metal_graph.rs:79-138)
 * for callers that chain kernel-level calls themselves. */
typedef struct anehip_graph anehip_graph;
int anehip_capture_begin(anehip_ctx *ctx);
int anehip_capture_end(anehip_ctx *ctx, anehip_graph **out);
int anehip_graph_launch(anehip_ctx *ctx, anehip_graph *graph);
void anehip_graph_destroy(anehip_graph *graph);

/* ---- kernel-level entry points (device pointers, context stream) ------- */

/*
 * y[b][r] = sum_k W[r][k] * x[b][k]  for b < batch, r < m, k < n.
 * W: m*(n/32) quant blocks (ggml_type Q8_0 or Q4_0), x: [batch][n] fp32 packed,
 * y: [batch][m] fp32 packed.  batch is 1..32 and need not be a multiple of any
 * tile size (rows are read exactly as given: "ragged" small batches).
 * batch == 1 is the GEMV of q8_gemv / q4_gemv_cpu
 * (crates/engine/src/q8_gemv.rs:130-148, 67-98) and of the q8_gemv / q4_gemv
 * Metal kernels (crates/engine/metal/q8_gemv.metal:15-87, q4_gemv.metal:25-98);
 * batch > 1 computes `batch` independent GEMVs with one pass over W.
 * n must be a multiple of 256 (whole 8-block super-blocks per row).
 */
int anehip_quant_gemm(anehip_ctx *ctx, uint32_t ggml_type, const void *w, uint32_t m,
                      uint32_t n, const float *x, uint32_t batch, float *y);

/*
 * Panel layout: a GPU-native permutation of the same Q8_0 / Q4_0 bytes (rows
 * in tiles of 64, each cut into 256-column panels whose 16-byte quant chunks
 * are interleaved across the 64 rows, the rows' block scales after them) that
 * lets every lane of a wave stream its own row with fully coalesced loads.
 * No counterpart in the reference, which reads the GGUF blocks directly
 * (q8_gemv.metal:15-87); the decode step builds it itself, these entry points
 * expose it to callers that run their own batch-1 GEMVs over resident weights.
 *
 * anehip_quant_packed_bytes: size of the panel copy of an [m x n] matrix
 * (n a multiple of 256), or 0 for an unsupported type / shape.
 * anehip_quant_pack: dst <- panel copy of the m*(n/32) GGUF blocks at w.
 * anehip_quant_gemv_packed: y[r] = W[r] . x for r < m from the panel copy wp
 * (same result as anehip_quant_gemm with batch 1, up to fp32 summation order).
 */
size_t anehip_quant_packed_bytes(uint32_t ggml_type, uint32_t m, uint32_t n);
int anehip_quant_pack(anehip_ctx *ctx, uint32_t ggml_type, const void *w, uint32_t m, uint32_t n, void *dst);
int anehip_quant_gemv_packed(anehip_ctx *ctx, uint32_t ggml_type, const void *wp, uint32_t m, uint32_t n,
                             const float *x, float *y);
/* anehip_quant_gemm_packed: y[b][r] = W[r] . x[b] for b < batch (1..256), from
 * the panel copy wp; x [batch][n] fp32.  batch 1 is
 * anehip_quant_gemv_packed; batch > 1 runs on MFMA (the small-batch form of
 * anehip_quant_gemm, same tolerance; above 32 the GEMM anehip_prefill runs
 * its chunks of up to 256 tokens on) and needs m % 4 == 0
 * (ANEHIP_EUNSUPPORTED otherwise); above 32 rows the panels must stay
 * under 2 GiB (ANEHIP_ESHAPE otherwise). */
int anehip_quant_gemm_packed(anehip_ctx *ctx, uint32_t ggml_type, const void *wp, uint32_t m, uint32_t n,
                             const float *x, uint32_t batch, float *y);

/* Row-wise RMSNorm: out[r] = x[r] * 1/sqrt(mean(x[r]^2) + eps) * w, rows x n.
 * rmsnorm_simple (deltanet.metal:239-272) / rmsnorm_vec (main.rs:1106-1113). */
int anehip_rmsnorm(anehip_ctx *ctx, const float *x, const float *w, float *out, uint32_t rows, uint32_t n,
                   float eps);

/* a[i] = SiLU(a[i]) * b[i]: silu_mul (q8_gemv.metal:89-97) /
 * vec_silu_mul_inplace (scratch.rs:181-186). */
int anehip_silu_mul(anehip_ctx *ctx, float *a, const float *b, size_t n);

/* x[i] += y[i]: residual_add (deltanet.metal:227-235) / main.rs:983-985. */
int anehip_residual_add(anehip_ctx *ctx, float *x, const float *y, size_t n);

/*
 * Gated DeltaNet core for `batch` independent sequences: conv1d_silu +
 * l2_normalize_scale + compute_beta_decay + deltanet_recurrence
 * (deltanet.metal:16-177) = deltanet.rs:444-512 of deltanet_decode_step.
 * Layouts (C = 3 * n_heads * 128, head dims 128, conv width 4):
 *   qkv [batch][C], beta_raw / alpha_raw [batch][n_heads], conv_w [C][4],
 *   ssm_a / dt_bias [n_heads], conv_state [batch][C][4] (updated),
 *   S [batch][n_heads][128][128] (updated), out_heads [batch][n_heads*128].
 */
int anehip_deltanet_step(anehip_ctx *ctx, uint32_t batch, uint32_t n_heads, const float *qkv,
                         const float *beta_raw, const float *alpha_raw, const float *conv_w, const float *ssm_a,
                         const float *dt_bias, float *conv_state, float *S, float *out_heads);

/* Per-head RMSNorm with norm_w[128], then * SiLU(gate): rmsnorm_gated with a
 * gate (deltanet.metal:184-220) = deltanet.rs:517-533.  heads, gate, out:
 * [batch][n_heads*128]. */
int anehip_gated_rmsnorm(anehip_ctx *ctx, uint32_t batch, uint32_t n_heads, const float *heads,
                         const float *gate, const float *norm_w, float eps, float *out);

/*
 * Full-attention core for `batch` sequences: q/gate split, q/k RMSNorm
 * (eps 1e-6), RoPE, KV append at pos[b], softmax attention over 0..pos[b],
 * * sigmoid(gate): q_gate_split + rmsnorm_gated + rope_apply + gpu_memcpy +
 * sdpa_causal + sigmoid_gate (attention.metal:9-121) = deltanet.rs:565-669.
 * head_dim is 256; n_heads / n_kv_heads in {1, 2, 4}.
 *   qkv [batch][n_heads*512 + 2*n_kv_heads*256]: per sequence the wq output
 *       ([n_heads][q(256) | gate(256)]), then k, then v (wk, wv outputs);
 *   pos: device array [batch] (must be < max_seq);
 *   k_cache, v_cache: fp16 bits, [batch][n_kv_heads][max_seq][256] (written
 *       at pos);  out [batch][n_heads*256].
 */
int anehip_attention_step(anehip_ctx *ctx, uint32_t batch, uint32_t n_heads, uint32_t n_kv_heads,
                          uint32_t max_seq, const float *qkv, const float *q_norm, const float *k_norm,
                          float rope_base, const uint32_t *pos, uint16_t *k_cache, uint16_t *v_cache,
                          float *out);

/*
 * anehip_attention_step that allocates nothing: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as anehip_attention_step.  The RoPE table and
 * the chunk partials live in a static device array of 4 MiB per GPU, held
 * until the process ends; a call whose partials do not fit (more than
 * 1,048,320 floats: batch x n_kv_heads x chunks x (n_heads / n_kv_heads) x 258,
 * about 4 MB whatever max_seq at batch x n_kv_heads <= 256) returns
 * ANEHIP_ERANGE and launches nothing.  Every call on one GPU shares that
 * array: calls that overlap on one GPU (other streams or contexts on the same
 * device) race.  Each call writes its own RoPE table into the array with a
 * kernel launch ahead of the attention kernels (the table is a kernel
 * argument), so the call never synchronises, copies from host memory or
 * allocates, may be captured into a graph as its first use on a device, and a
 * replayed graph uses the rope_base it was captured with.  The array's address
 * on a device is looked up once, when the first context on that device is
 * created.
 */
int anehip_attention_step_noalloc(anehip_ctx *ctx, uint32_t batch, uint32_t n_heads, uint32_t n_kv_heads,
                                  uint32_t max_seq, const float *qkv, const float *q_norm, const float *k_norm,
                                  float rope_base, const uint32_t *pos, uint16_t *k_cache, uint16_t *v_cache,
                                  float *out);

/* Greedy sampling per row: index of the maximum under f32::total_cmp, the
 * last of equal maxima (greedy_sample, main.rs:1767-1775).  logits
 * [rows][n], out [rows] (device). */
int anehip_argmax(anehip_ctx *ctx, const float *logits, uint32_t rows, uint32_t n, uint32_t *out);

/* Set-up utilities for synthetic weights and states (no counterpart in the
 * reference, which loads GGUF files): fill n device values (fp32, or fp16
 * bits if is_f16) with seeded, counter-based draws, dist 0 = N(a, b^2),
 * dist 1 = U(a, b); and quantise a device fp32 [m x n] matrix into Q8_0
 * (d = absmax/127) or Q4_0 (d = absmax/7, +8 offset) blocks. */
int anehip_fill_random(anehip_ctx *ctx, void *dptr, size_t n, uint32_t dist, uint32_t is_f16, uint64_t seed,
                       float a, float b);
int anehip_quantize(anehip_ctx *ctx, uint32_t ggml_type, const float *w, uint32_t m, uint32_t n, void *out);

/* ---- model-level decode step (context created with a model desc) -------- */

/* Uploads one quantised tensor (host bytes, copied).  Checks ggml_type, the
 * byte count m*(n/32)*{34|18} as Q8Tensor::from_raw does (q8_gemv.rs:33-57)
 * and the [m x n] shape the kind has in this model.  Replaces
 * GpuContext::upload_q8_weights (metal_graph.rs:208-221) inside
 * upload_model_weights (gpu_decode.rs:152-283). */
int anehip_upload_quant(anehip_ctx *ctx, int32_t layer, uint32_t kind, const uint8_t *blocks, size_t nbytes,
                        uint32_t m, uint32_t n, uint32_t ggml_type);

/* Uploads one fp32 tensor (norm weights, conv1d, ssm_a, dt_bias, embedding). */
int anehip_upload_f32(anehip_ctx *ctx, int32_t layer, uint32_t kind, const float *data, size_t n);

/* Device address where tensor `kind` of `layer` lives (allocated on first
 * use, with ggml_type for quantised kinds, ignored for fp32 kinds), so a
 * caller can write it in place (e.g. with anehip_quantize); the tensor then
 * counts as uploaded.  *nbytes receives its size.  The decode step reads a
 * panel copy of quantised weights that is rebuilt at the first step after
 * this call (or after anehip_upload_quant): write before that step. */
int anehip_tensor_ptr(anehip_ctx *ctx, int32_t layer, uint32_t kind, uint32_t ggml_type, void **dptr,
                      size_t *nbytes);

/* Allocates zeroed per-sequence state for `batch` (1..32) sequences with KV
 * capacity max_seq, all positions 0: HybridCache::new (deltanet_cache.rs:
 * 76-136) and the state buffers of upload_model_weights (gpu_decode.rs:
 * 205-256).  Frees any previous state.  batch > 1 needs vocab_size % 4 == 0
 * (ANEHIP_EUNSUPPORTED otherwise). */
int anehip_alloc_state(anehip_ctx *ctx, uint32_t batch, uint32_t max_seq);

/* Zeroes all state and sets every position to 0. */
int anehip_reset_state(anehip_ctx *ctx);

/* Position of one sequence (HybridCache::pos, deltanet_cache.rs:71). */
int anehip_set_pos(anehip_ctx *ctx, uint32_t seq, uint32_t pos);
int anehip_get_pos(anehip_ctx *ctx, uint32_t seq, uint32_t *pos);

/* Device pointer and size of one state buffer of layer `layer`:
 * which 0: conv window [batch][3*dim][4] f32      (DeltaNet layers)
 *       1: recurrent S [batch][H][128][128] f32    (DeltaNet layers)
 *       2: K cache [batch][n_kv][max_seq][256] f16 (attention layers)
 *       3: V cache, same layout.
 * Lets a caller load state produced elsewhere or read it back. */
int anehip_state_ptr(anehip_ctx *ctx, uint32_t layer, uint32_t which, void **dptr, size_t *nbytes);

/* Enables (default) or disables replay of the captured step graph; with it
 * disabled the same kernels are launched one by one. */
int anehip_set_graph(anehip_ctx *ctx, int enabled);

/*
 * One decode step for every sequence: token_ids[batch] (ids >= vocab give a
 * zero embedding, main.rs:960-963), positions advance by one.  Writes the
 * logits [batch][vocab] to logits_out if not NULL and returns when the step
 * is done.  Fails with ANEHIP_ERANGE if a position reached max_seq.
 * Replaces encode_full_token_gpu (gpu_full_decode.rs:221-1044) and, as a
 * computation, qwen35_forward_token (main.rs:953-1023).
 */
int anehip_decode_step(anehip_ctx *ctx, const uint32_t *token_ids, uint32_t batch, float *logits_out);

/* Same, but only enqueues the step on the context stream. */
int anehip_decode_step_async(anehip_ctx *ctx, const uint32_t *token_ids, uint32_t batch);

/*
 * Prefill: tokens[n_tokens] of sequence `seq`, from its current position, in
 * chunks of up to 32 tokens -- the projections on the MFMA GEMM with one row
 * per token, the DeltaNet recurrence as a scan over each chunk's tokens with
 * the state held on chip, attention causal within the chunk.  Leaves the
 * sequence's state and position as n_tokens decode steps would (the other
 * sequences untouched) and writes the last token's logits [vocab] to
 * logits_out if not NULL.  Synchronous; ANEHIP_ERANGE if the tokens do not
 * fit in the KV capacity.  Replaces the reference's token-serial prefill
 * (ane_prefill_tokens, main.rs:1168-1429, with the ANE projections of
 * ane_prefill.rs:301 and the CPU recurrence / attention per token).
 */
int anehip_prefill(anehip_ctx *ctx, uint32_t seq, const uint32_t *tokens, uint32_t n_tokens, float *logits_out);

/* Device pointer of the last step's logits [batch][vocab]. */
int anehip_logits_ptr(anehip_ctx *ctx, const float **dptr);

/* Greedy tokens of the last step (argmax of its logits), [batch]. */
int anehip_sampled_tokens(anehip_ctx *ctx, uint32_t *out);

/* `steps` greedy decode steps with on-device token feedback: step 0 consumes
 * first_tokens, step i consumes the argmax of step i-1.  out_tokens
 * [steps][batch].  The reference's host loop (main.rs:473-487) with
 * greedy_sample moved on device. */
int anehip_generate(anehip_ctx *ctx, const uint32_t *first_tokens, uint32_t batch, uint32_t steps,
                    uint32_t *out_tokens);

#ifdef __cplusplus
}
#endif

#endif /* ANEHIP_H */
