// api.hip — kernel-level C-ABI entry points (device pointers, context stream).
//
// Each wraps one hot-path kernel of the decode step so it can be driven and
// checked on its own, as the reference's CPU functions can
// (crates/engine/src/deltanet.rs, scratch.rs, crates/cli/src/main.rs).
#include "common.h"

#include <mutex>
#include <vector>

using namespace anehip;

namespace {

bool bad_ctx(anehip_ctx *ctx) { return ctx == nullptr; }

#define NEED_CTX(ctx, name)                                                                    \
    do {                                                                                       \
        if (bad_ctx(ctx)) return set_error(global_error(), ANEHIP_EINVAL, name ": ctx is NULL"); \
    } while (0)

uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t dmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Counter-based fill: value i of a normal fill uses the pair (2j, 2j+1),
// j = i/2, of SplitMix64(key + c) with Box-Muller (fp32 on device); a uniform
// fill uses SplitMix64(key + i) alone.
__global__ void fill_random_kernel(void *dst, size_t n, int uniform, int is_f16, uint64_t key, float a, float b) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        float v;
        if (uniform) {
            const float u = ((float)(dmix64(key + i) >> 40) + 0.5f) * (1.0f / 16777216.0f);
            v = a + (b - a) * u;
        } else {
            const uint64_t j = i >> 1;
            const float u1 = ((float)(dmix64(key + 2 * j) >> 40) + 0.5f) * (1.0f / 16777216.0f);
            const float u2 = ((float)(dmix64(key + 2 * j + 1) >> 40) + 0.5f) * (1.0f / 16777216.0f);
            const float r = sqrtf(-2.0f * logf(u1));
            const float t = 6.2831853071795865f * u2;
            v = a + b * ((i & 1) ? r * sinf(t) : r * cosf(t));
        }
        if (is_f16) static_cast<__half *>(dst)[i] = __float2half_rn(v);
        else static_cast<float *>(dst)[i] = v;
    }
}

// One thread per 32-value block.  Q8_0: d = absmax/127, q = round(w/d) (half
// away from zero) clamped to +-127.  Q4_0: d = absmax/7, q = round(w/d) + 8
// clamped to 0..15, element i in the low nibble of byte i and element i+16 in
// the high nibble (dequant.rs:12-25).  d is stored as fp16 (RNE).
template <int Q8>
__global__ void quantize_kernel(const float *__restrict__ w, size_t nblocks, uint8_t *__restrict__ out) {
    const size_t blk = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= nblocks) return;
    const float *x = w + blk * 32;
    float v[32];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        v[i] = x[i];
        amax = fmaxf(amax, fabsf(v[i]));
    }
    const float d = amax / (Q8 ? 127.0f : 7.0f);
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const unsigned short dh = __half_as_ushort(__float2half_rn(d));
    uint8_t *o = out + blk * (Q8 ? 34 : 18);
    o[0] = (uint8_t)(dh & 0xff);
    o[1] = (uint8_t)(dh >> 8);
    if (Q8) {
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const float q = fminf(fmaxf(roundf(v[i] * id), -127.0f), 127.0f);
            o[2 + i] = (uint8_t)(int8_t)q;
        }
    } else {
        uint8_t q[32];
#pragma unroll
        for (int i = 0; i < 32; i++) q[i] = (uint8_t)fminf(fmaxf(roundf(v[i] * id) + 8.0f, 0.0f), 15.0f);
#pragma unroll
        for (int i = 0; i < 16; i++) o[2 + i] = (uint8_t)(q[i] | (q[i + 16] << 4));
    }
}

// Scratch of anehip_attention_step_noalloc: the RoPE table (first 256
// floats) and the attention's chunk partials, at most kScratchFloats floats
// (4 MiB) in all.  Each GPU the library runs on holds its own copy until the
// process ends.  In host code `scratch` names a host-side stand-in, never the
// device memory: host code uses the address hipGetSymbolAddress returned for
// the device (anehip_ctx::noalloc_scratch, set by noalloc_setup).
constexpr size_t kScratchFloats = (size_t)1 << 20;
constexpr size_t kScratchTable = 256;  // floats reserved for the RoPE table
__device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
float *g_noalloc[kMaxDevices];  // device address of `scratch` per device (null: not looked up yet)
std::mutex g_noalloc_mu;

// The RoPE table of one call, by value: a kernel argument is recorded in the
// graph node when the call is captured, so no host buffer has to outlive the
// launch and a replay writes its own table again.
struct RopeTab {
    float f[128];
};
__global__ __launch_bounds__(128) void rope_table_kernel(RopeTab tab, float *__restrict__ dst) {
    dst[threadIdx.x] = tab.f[threadIdx.x];
}

}  // namespace

namespace anehip {

// Set-up of the entry point that allocates nothing, at context creation with
// the context's device current: the scratch address on this device, looked
// up once per device.
int noalloc_setup(anehip_ctx *ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices) return ANEHIP_OK;  // the entry point refuses such devices
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc[ctx->device]) {
        void *p = nullptr;
        ANEHIP_HIP_TRY(ctx->err, hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return set_error(ctx->err, ANEHIP_EHIP, "noalloc: no device address for the scratch array");
        g_noalloc[ctx->device] = static_cast<float *>(p);
    }
    ctx->noalloc_scratch = g_noalloc[ctx->device];
    return ANEHIP_OK;
}

}  // namespace anehip

extern "C" {

int anehip_rmsnorm(anehip_ctx *ctx, const float *x, const float *w, float *out, uint32_t rows, uint32_t n,
                   float eps) {
    NEED_CTX(ctx, "rmsnorm");
    if (!x || !w || !out || !rows || !n) return set_error(ctx->err, ANEHIP_EINVAL, "rmsnorm: bad argument");
    return launch_rmsnorm(ctx, ctx->stream, (int)rows, (int)n, x, w, out, eps);
}

int anehip_silu_mul(anehip_ctx *ctx, float *a, const float *b, size_t n) {
    NEED_CTX(ctx, "silu_mul");
    if (!a || !b) return set_error(ctx->err, ANEHIP_EINVAL, "silu_mul: null pointer");
    if (!n) return ANEHIP_OK;
    return launch_silu_mul(ctx, ctx->stream, a, b, n);
}

int anehip_residual_add(anehip_ctx *ctx, float *x, const float *y, size_t n) {
    NEED_CTX(ctx, "residual_add");
    if (!x || !y) return set_error(ctx->err, ANEHIP_EINVAL, "residual_add: null pointer");
    if (!n) return ANEHIP_OK;
    return launch_residual_add(ctx, ctx->stream, x, y, n);
}

int anehip_deltanet_step(anehip_ctx *ctx, uint32_t batch, uint32_t n_heads, const float *qkv,
                         const float *beta_raw, const float *alpha_raw, const float *conv_w, const float *ssm_a,
                         const float *dt_bias, float *conv_state, float *S, float *out_heads) {
    NEED_CTX(ctx, "deltanet_step");
    if (!qkv || !beta_raw || !alpha_raw || !conv_w || !ssm_a || !dt_bias || !conv_state || !S || !out_heads)
        return set_error(ctx->err, ANEHIP_EINVAL, "deltanet_step: null pointer");
    if (!batch || !n_heads) return set_error(ctx->err, ANEHIP_EINVAL, "deltanet_step: batch and n_heads must be > 0");
    const int chunk = (int)n_heads * 128;
    MixIn mq, mb, ma;
    mq.p = qkv;
    mq.stride = 3 * chunk;
    mb.p = beta_raw;
    mb.stride = (int)n_heads;
    ma.p = alpha_raw;
    ma.stride = (int)n_heads;
    // batch > 1: one workgroup per head and sequence (commits every window)
    if (batch > 1)
        return launch_deltanet_head(ctx, ctx->stream, (int)batch, (int)n_heads, mq, mb, ma, conv_w, ssm_a, dt_bias,
                                    conv_state, S, out_heads, 0, nullptr, 0.0f, Planes{});
    // batch 1: one launch, the q / k windows committed in-kernel (256
    // counters per head); beyond the counters, dn_finish commits them
    if ((size_t)n_heads * 256 <= (size_t)kDnCounters)
        return launch_deltanet_step(ctx, ctx->stream, (int)batch, (int)n_heads, mq, mb, ma, conv_w, ssm_a, dt_bias,
                                    conv_state, S, out_heads, ctx->dn_count);
    int rc = launch_deltanet_step(ctx, ctx->stream, (int)batch, (int)n_heads, mq, mb, ma, conv_w, ssm_a, dt_bias,
                                  conv_state, S, out_heads);
    if (rc) return rc;
    return launch_dn_finish(ctx, ctx->stream, (int)batch, (int)n_heads, mq, conv_state, nullptr, 0, nullptr, nullptr,
                            Planes{}, 0.0f);
}

int anehip_gated_rmsnorm(anehip_ctx *ctx, uint32_t batch, uint32_t n_heads, const float *heads, const float *gate,
                         const float *norm_w, float eps, float *out) {
    NEED_CTX(ctx, "gated_rmsnorm");
    if (!heads || !gate || !norm_w || !out || !batch || !n_heads)
        return set_error(ctx->err, ANEHIP_EINVAL, "gated_rmsnorm: bad argument");
    MixIn mg;
    mg.p = gate;
    mg.stride = (int)n_heads * 128;
    return launch_dn_finish(ctx, ctx->stream, (int)batch, (int)n_heads, mg, nullptr, heads, 0, norm_w, out, Planes{},
                            eps);
}

int anehip_attention_step(anehip_ctx *ctx, uint32_t batch, uint32_t n_heads, uint32_t n_kv_heads, uint32_t max_seq,
                          const float *qkv, const float *q_norm, const float *k_norm, float rope_base,
                          const uint32_t *pos, uint16_t *k_cache, uint16_t *v_cache, float *out) {
    NEED_CTX(ctx, "attention_step");
    if (!qkv || !q_norm || !k_norm || !pos || !k_cache || !v_cache || !out)
        return set_error(ctx->err, ANEHIP_EINVAL, "attention_step: null pointer");
    if (!batch || !n_heads || !n_kv_heads || !max_seq || n_heads % n_kv_heads)
        return set_error(ctx->err, ANEHIP_EINVAL, "attention_step: bad shape");
    if (!(rope_base > 0.0f)) return set_error(ctx->err, ANEHIP_EINVAL, "attention_step: rope_base must be > 0");
    if (!ctx->inv_freq || ctx->inv_freq_base != rope_base) {
        std::vector<float> f(128);
        rope_inv_freq(rope_base, 256, f.data());
        if (!ctx->inv_freq && hipMalloc(&ctx->inv_freq, 128 * sizeof(float)) != hipSuccess) {
            ctx->inv_freq = nullptr;
            return set_error(ctx->err, ANEHIP_ENOMEM, "attention_step: table allocation failed");
        }
        ANEHIP_HIP_TRY(ctx->err, hipMemcpy(ctx->inv_freq, f.data(), 128 * sizeof(float), hipMemcpyHostToDevice));
        ctx->inv_freq_base = rope_base;
    }
    const int G = (int)(n_heads / n_kv_heads);
    int rc = ensure_workspace(ctx, attn_partial_floats((int)batch, (int)n_kv_heads, (int)max_seq, G));
    if (rc) return rc;
    MixIn mix;
    mix.p = qkv;
    mix.stride = (int)(n_heads * 2 * 256 + 2 * n_kv_heads * 256);
    return launch_attention(ctx, ctx->stream, (int)batch, (int)n_heads, (int)n_kv_heads, (int)max_seq, mix, q_norm,
                            k_norm, ctx->inv_freq, pos, reinterpret_cast<__half *>(k_cache),
                            reinterpret_cast<__half *>(v_cache), ctx->ws.partial, out, Planes{});
}

int anehip_attention_step_noalloc(anehip_ctx *ctx, uint32_t batch, uint32_t n_heads, uint32_t n_kv_heads,
                                  uint32_t max_seq, const float *qkv, const float *q_norm, const float *k_norm,
                                  float rope_base, const uint32_t *pos, uint16_t *k_cache, uint16_t *v_cache,
                                  float *out) {
    NEED_CTX(ctx, "attention_step_noalloc");
    if (!qkv || !q_norm || !k_norm || !pos || !k_cache || !v_cache || !out)
        return set_error(ctx->err, ANEHIP_EINVAL, "attention_step_noalloc: null pointer");
    if (!batch || !n_heads || !n_kv_heads || !max_seq || n_heads % n_kv_heads)
        return set_error(ctx->err, ANEHIP_EINVAL, "attention_step_noalloc: bad shape");
    if (!(rope_base > 0.0f))
        return set_error(ctx->err, ANEHIP_EINVAL, "attention_step_noalloc: rope_base must be > 0");
    const uint32_t G = n_heads / n_kv_heads;
    if (G != 1 && G != 2 && G != 4)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "attention_step_noalloc: %u query heads per kv head", G);
    const size_t need = attn_partial_floats((int)batch, (int)n_kv_heads, (int)max_seq, (int)G);
    if (need > kScratchFloats - kScratchTable)
        return set_error(ctx->err, ANEHIP_ERANGE,
                         "attention_step_noalloc: %zu partial floats needed, the static scratch holds %zu "
                         "(batch %u, %u kv heads, max_seq %u)",
                         need, kScratchFloats - kScratchTable, batch, n_kv_heads, max_seq);
    float *ptr = ctx->noalloc_scratch;
    if (!ptr)
        return set_error(ctx->err, ANEHIP_ESTATE, "attention_step_noalloc: no static scratch on device %d",
                         ctx->device);
    // the call's RoPE table goes to the scratch ahead of its attention launch
    // (same host formula as the allocating entry point, so the same bits)
    RopeTab tab;
    rope_inv_freq(rope_base, 256, tab.f);
    hipLaunchKernelGGL(rope_table_kernel, dim3(1), dim3(128), 0, ctx->stream, tab, ptr);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    MixIn mix;
    mix.p = qkv;
    mix.stride = (int)(n_heads * 2 * 256 + 2 * n_kv_heads * 256);
    return launch_attention(ctx, ctx->stream, (int)batch, (int)n_heads, (int)n_kv_heads, (int)max_seq, mix, q_norm,
                            k_norm, ptr, pos, reinterpret_cast<__half *>(k_cache),
                            reinterpret_cast<__half *>(v_cache), ptr + kScratchTable, out, Planes{});
}

int anehip_argmax(anehip_ctx *ctx, const float *logits, uint32_t rows, uint32_t n, uint32_t *out) {
    NEED_CTX(ctx, "argmax");
    if (!logits || !out || !rows || !n) return set_error(ctx->err, ANEHIP_EINVAL, "argmax: bad argument");
    int rc = ensure_workspace(ctx, (argmax_workspace_bytes((int)rows) + 3) / 4);
    if (rc) return rc;
    return launch_argmax(ctx, ctx->stream, (int)rows, n, logits, ctx->ws.partial, out);
}

int anehip_fill_random(anehip_ctx *ctx, void *dptr, size_t n, uint32_t dist, uint32_t is_f16, uint64_t seed,
                       float a, float b) {
    NEED_CTX(ctx, "fill_random");
    if (!dptr || dist > 1) return set_error(ctx->err, ANEHIP_EINVAL, "fill_random: bad argument");
    if (!n) return ANEHIP_OK;
    const uint64_t key = mix64(seed ^ 0x5DEECE66Dull);
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(fill_random_kernel, dim3(blocks), dim3(256), 0, ctx->stream, dptr, n, (int)dist,
                       is_f16 ? 1 : 0, key, a, b);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int anehip_quantize(anehip_ctx *ctx, uint32_t ggml_type, const float *w, uint32_t m, uint32_t n, void *out) {
    NEED_CTX(ctx, "quantize");
    if (!w || !out || !m) return set_error(ctx->err, ANEHIP_EINVAL, "quantize: bad argument");
    if (ggml_type != ANEHIP_GGML_Q8_0 && ggml_type != ANEHIP_GGML_Q4_0)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "quantize: ggml type %u", ggml_type);
    if (n == 0 || n % 32) return set_error(ctx->err, ANEHIP_ESHAPE, "quantize: n=%u not a multiple of 32", n);
    const size_t nblocks = (size_t)m * (n / 32);
    const unsigned grid = (unsigned)((nblocks + 255) / 256);
    if (ggml_type == ANEHIP_GGML_Q8_0)
        hipLaunchKernelGGL(quantize_kernel<1>, dim3(grid), dim3(256), 0, ctx->stream, w, nblocks,
                           static_cast<uint8_t *>(out));
    else
        hipLaunchKernelGGL(quantize_kernel<0>, dim3(grid), dim3(256), 0, ctx->stream, w, nblocks,
                           static_cast<uint8_t *>(out));
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

}  // extern "C"
