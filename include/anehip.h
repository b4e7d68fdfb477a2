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
int anehip_dev_memset(anehip_ctx *ctx, void *dst, int value, size_t nbytes);

/* ---- timing on the context's stream (hipEvent pairs) -------------------- */
/* Records a start event; anehip_timer_stop records the stop event, waits for
 * it and returns the elapsed milliseconds between the two. */
int anehip_timer_start(anehip_ctx *ctx);
int anehip_timer_stop(anehip_ctx *ctx, float *ms);

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

#ifdef __cplusplus
}
#endif

#endif /* ANEHIP_H */
