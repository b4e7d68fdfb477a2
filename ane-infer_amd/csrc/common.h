// common.h — shared definitions of libanehip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/anehip.h"

namespace anehip {

// Per-context error slot.  Context-free failures use a thread-local slot.
struct ErrorSlot {
    std::string msg;
};

ErrorSlot &global_error();

int set_error(ErrorSlot &slot, int code, const char *fmt, ...) __attribute__((format(printf, 3, 4)));

#define ANEHIP_HIP_TRY(slot, expr)                                                            \
    do {                                                                                      \
        hipError_t _e = (expr);                                                               \
        if (_e != hipSuccess)                                                                 \
            return ::anehip::set_error((slot), ANEHIP_EHIP, "%s failed: %s (%s:%d)", #expr,   \
                                       hipGetErrorString(_e), __FILE__, __LINE__);            \
    } while (0)

// A device buffer owned by a context.
struct DevBuf {
    void *ptr = nullptr;
    size_t bytes = 0;
};

// Device workspace used by split-K reductions: partial sums and per-tile
// arrival counters.  Counters are returned to zero by the kernel that uses
// them, so the workspace needs clearing only once, at allocation.
struct Workspace {
    float *partial = nullptr;      // split-K partial sums
    size_t partial_floats = 0;
    uint32_t *counters = nullptr;  // per-row-tile arrival counters
    size_t n_counters = 0;
};

}  // namespace anehip

struct anehip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
    anehip::ErrorSlot err;
    anehip::Workspace ws;
    std::vector<void *> user_allocs;
    struct Model *model = nullptr;  // decode-step state (decode.hip)
    int cu_count = 0;
    float *inv_freq = nullptr;      // RoPE table of the kernel-level attention entry
    float inv_freq_base = 0.0f;
};

namespace anehip {

// Ensures the split-K workspace holds at least `floats` partials and
// `counters` counters (grown with hipMalloc, cleared once).
int ensure_workspace(anehip_ctx *ctx, size_t floats, size_t counters);

// ---- kernel launchers (all pointers are device pointers; work is queued on
// `stream`; they return ANEHIP_OK or set ctx->err) ---------------------------

// gemv.hip.  y[b][r] = W[r] . x[b].  launch_quant_gemm writes final values;
// launch_gemm_raw writes part[ks][batch][m] for ks < ksplit (final values when
// ksplit == 1), with ksplit from gemm_ksplit().
int launch_quant_gemm(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w,
                      uint32_t m, uint32_t n, const float *x, uint32_t batch, float *y);
int gemm_ksplit(const anehip_ctx *ctx, uint32_t m, uint32_t n);
// xsplit: device scratch of batch * n floats (x split into fp16 hi / lo
// planes for the MFMA path); may be null when batch == 1.
int launch_gemm_raw(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w, uint32_t m,
                    uint32_t n, const float *x, uint32_t batch, float *out, int ksplit, void *xsplit);
int launch_sum_partials(anehip_ctx *ctx, hipStream_t stream, const float *part, float *y, size_t count,
                        int ksplit);

// deltanet.hip
int launch_deltanet_step(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, const float *qkv,
                         int qkv_stride, const float *beta_raw, const float *alpha_raw, int ba_stride,
                         const float *conv_w, const float *ssm_a, const float *dt_bias, float *conv_state,
                         float *S, float *out);
int launch_dn_finish(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, const float *qkv,
                     int qkv_stride, float *conv_state, const float *heads, const float *gate, int gate_stride,
                     const float *norm_w, float *out, float eps);

// attention.hip
size_t attn_partial_floats(int batch, int n_kv, int max_seq, int G);
int launch_attention(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, int n_kv, int max_seq,
                     const float *qkv, int stride, const float *q_norm, const float *k_norm,
                     const float *inv_freq, const uint32_t *pos, __half *k_cache, __half *v_cache,
                     float *part, float *out);

// elementwise.hip
int launch_rmsnorm(anehip_ctx *ctx, hipStream_t s, int rows, int n, const float *x, const float *w, float *out,
                   float eps);
int launch_embed_rmsnorm(anehip_ctx *ctx, hipStream_t s, int rows, int n, const uint32_t *tokens,
                         const float *emb, uint32_t vocab, float *x, const float *w, float *xn, float eps);
int launch_residual_rmsnorm(anehip_ctx *ctx, hipStream_t s, int rows, int n, float *x, const float *part,
                            int ksplit, const float *w, float *xn, float eps);
int launch_silu_mul_stacked(anehip_ctx *ctx, hipStream_t s, int rows, int F, const float *gu, int ksplit,
                            float *h);
int launch_silu_mul(anehip_ctx *ctx, hipStream_t s, float *a, const float *b, size_t n);
int launch_residual_add(anehip_ctx *ctx, hipStream_t s, float *x, const float *y, size_t n);
size_t argmax_workspace_bytes(int rows);
int launch_argmax(anehip_ctx *ctx, hipStream_t s, int rows, uint32_t n, const float *logits, void *ws,
                  uint32_t *out);

// Host helper: inv_freq[p] = 1 / base^(2p / head_dim), the
// reference's formula (deltanet.rs:601-603) evaluated once on the host.
void rope_inv_freq(float base, int head_dim, float *out);

}  // namespace anehip
