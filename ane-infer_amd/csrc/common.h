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

// Device scratch of the kernel-level entry points: split-K partial sums,
// fp16 input planes, attention partials, argmax candidates.
struct Workspace {
    float *partial = nullptr;
    size_t partial_floats = 0;
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
    float *noalloc_scratch = nullptr;  // this device's static scratch (api.hip, anehip_attention_step_noalloc)
    uint32_t *dn_count = nullptr;      // zeroed counters of anehip_deltanet_step's window commit
};

namespace anehip {

// Counters at anehip_ctx::dn_count for the q / k conv windows that
// anehip_deltanet_step commits in its kernel: 256 per (sequence, head), one
// per thread of its workgroups (256 heads at batch 1).
constexpr int kDnCounters = 65536;

// Ensures the workspace holds at least `floats` floats (grown with
// hipMalloc; refused while the context stream is being captured).
int ensure_workspace(anehip_ctx *ctx, size_t floats);
// Looks up the static scratch of anehip_attention_step_noalloc on the
// context's device (once per device; the device must be current).
int noalloc_setup(anehip_ctx *ctx);

// How a batch-1 GEMV forms its input vector from what the previous kernels
// left in memory (the element-wise step is fused into the GEMV's prologue, so
// it costs no launch of its own).  Each workgroup computes only the slice of
// the input its K range needs (plus any full-row reduction).
enum GemvInMode : int {
    GEMV_IN_PLAIN = 0,     // x
    GEMV_IN_RMSNORM,       // rmsnorm(x, w)
    GEMV_IN_RESID_RMSNORM, // r = x + sum_p part[p]; rmsnorm(r, w); r -> x_out
    GEMV_IN_EMBED_RMSNORM, // r = emb[token] (0 if token >= vocab); rmsnorm(r, w); r -> x_out
    GEMV_IN_GATED_NORM,    // per-128 head rmsnorm(x, w) * SiLU(gate), gate = sum_p part[p][gate_off..]
    GEMV_IN_SILU_MUL,      // SiLU(sum_p part[p][gu_index(k)]) * sum_p part[p][gu_index(k) + 32]
    GEMV_IN_ATTN_COMBINE,  // batch row 0's attention output of the slice's heads: the chunk partials
                           // merged (running max / sum) times sigmoid(gate), gate from part
};

struct GemvInput {
    int mode = GEMV_IN_PLAIN;
    const float *x = nullptr;
    const float *part = nullptr;  // partial slices, part_stride floats apart
    int kp = 0;
    size_t part_stride = 0;
    const float *w = nullptr;
    float eps = 0.0f;
    float *x_out = nullptr;       // new residual stream (written by workgroup (0, 0))
    const uint32_t *token = nullptr;
    const float *emb = nullptr;
    uint32_t vocab = 0;
    int gate_off = 0;
    // GATED_NORM only: the q/k conv windows [2n][4] are committed (shift left,
    // append part rows [0, 2n)) by the workgroups of this launch
    float *conv_state = nullptr;
    // ATTN_COMBINE only: attention partials of batch row 0 (launch_attention
    // without outputs), their chunk layout and the position; head h's gate is
    // part[h * 512 + 256 + d] (K-split slices as above)
    const float *att_o = nullptr, *att_ml = nullptr;
    int att_nch = 0, att_g = 0;
    const uint32_t *att_pos = nullptr;
};

// Decode attention split: a sequence of `len` positions has ceil(len / 64)
// live tiles of 64 positions, spread evenly over min(nch, tiles) chunks; the
// other chunks of the launch's nch are idle.  Shared by the attention kernels
// and the merges of their partials.
constexpr int kAttnTile = 64;
// Workgroups a decode attention launch aims for over the whole batch: one per
// CU of MI355X (256 CUs), the device this library is built for.
constexpr int kAttnWorkgroups = 256;
__host__ __device__ __forceinline__ int active_chunks(int len, int nch) {
    const int tiles = (len + kAttnTile - 1) / kAttnTile;
    return tiles < nch ? tiles : nch;
}
// Tiles [*tb, *te) of chunk c; false if the chunk is idle.
__host__ __device__ __forceinline__ bool chunk_tiles(int len, int nch, int c, int *tb, int *te) {
    const int tiles = (len + kAttnTile - 1) / kAttnTile;
    const int na = tiles < nch ? tiles : nch;
    if (c >= na) return false;
    // 32-bit: c < 128 and tiles < 2^15 (a cache row is below 1 GiB)
    *tb = (int)((uint32_t)(c * tiles) / (uint32_t)na);
    *te = (int)((uint32_t)((c + 1) * tiles) / (uint32_t)na);
    return true;
}

// A GEMV output read by a later kernel as kp partial slices: value (b, i) =
// sum over q < kp of p[q * split + b * stride + i], q ascending.
struct MixIn {
    const float *p = nullptr;
    int kp = 1;
    size_t split = 0;
    int stride = 0;
    // the same slices, starting `off` values into each row
    MixIn shifted(int off) const {
        MixIn m = *this;
        m.p = p + off;
        return m;
    }
    // The KP slices of value (b, i) loaded unconditionally (slices past kp
    // re-read the last one: an address the compiler cannot merge with another
    // load, which would make it wait for that load), so that a kernel can
    // issue all of its loads before it needs any; add() then sums them in
    // slice order, as at() does.
    template <int KP> __device__ __forceinline__ void load(int b, int i, float (&v)[KP]) const {
        const float *q0 = p + (size_t)b * stride + i;
#pragma unroll
        for (int q = 0; q < KP; q++) v[q] = q0[(size_t)min(q, kp - 1) * split];
    }
    template <int KP> __device__ __forceinline__ float add(const float (&v)[KP]) const {
        float s = v[0];
#pragma unroll
        for (int q = 1; q < KP; q++) s = q < kp ? s + v[q] : s;
        return s;
    }
    __host__ __device__ __forceinline__ float at(int b, int i) const {
        const float *q0 = p + (size_t)b * stride + i;
        float s = q0[0];
        for (int q = 1; q < kp; q++) s += q0[(size_t)q * split];
        return s;
    }
    __host__ __device__ __forceinline__ float4 at4(int b, int i) const {
        const float *q0 = p + (size_t)b * stride + i;
        float4 s = *reinterpret_cast<const float4 *>(q0);
        for (int q = 1; q < kp; q++) {
            const float4 v = *reinterpret_cast<const float4 *>(q0 + (size_t)q * split);
            s.x += v.x;
            s.y += v.y;
            s.z += v.z;
            s.w += v.w;
        }
        return s;
    }
};

// ---- kernel launchers (all pointers are device pointers; work is queued on
// `stream`; they return ANEHIP_OK or set ctx->err) ---------------------------

// gemv.hip.  y[b][r] = W[r] . x[b].  launch_quant_gemm writes final values;
// launch_gemm_raw writes part[ks][batch][m] for ks < ksplit (final values when
// ksplit == 1), with ksplit from gemm_ksplit().
int launch_quant_gemm(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w,
                      uint32_t m, uint32_t n, const float *x, uint32_t batch, float *y);
// Number of K splits for an [m x n] product: split ks covers super-blocks
// [ks * per, min(nsb, (ks + 1) * per)) with per = split_len(nsb, ksplit);
// max_k bounds the splits a consumer has to add (fused consumers take 8).
int gemm_ksplit(const anehip_ctx *ctx, uint32_t m, uint32_t n, int max_k = 8);
inline int split_len(int nsb, int ksplit) { return (nsb + ksplit - 1) / ksplit; }
// xsplit: device scratch of batch * n floats (x split into fp16 hi / lo
// planes for the MFMA path); may be null when batch == 1.
int launch_gemm_raw(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w, uint32_t m,
                    uint32_t n, const float *x, uint32_t batch, float *out, int ksplit, void *xsplit);
int launch_sum_partials(anehip_ctx *ctx, hipStream_t stream, const float *part, float *y, size_t count,
                        int ksplit);
// Panel layout (see gemv.hip): bytes of an [m x n] matrix, repack from GGUF
// blocks, and the batch-1 GEMV over panels.  il = F > 0 (m = 2 F, F % 32 ==
// 0): the rows of a stacked [gate; up] matrix are interleaved in groups of 32
// -- panel tile t holds gate rows 32 t .. 32 t + 31, then the up rows of the
// same features -- so every product over it leaves, per 64 output rows, 32
// gate sums followed by the 32 matching up sums (gu_index()).
size_t packed_bytes(uint32_t ggml_type, uint32_t m, uint32_t n);
int launch_repack(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *src, uint32_t m, uint32_t n,
                  void *dst, uint32_t il = 0);
// The inverse of launch_repack: panel bytes back to GGUF blocks (rows < m).
int launch_unpack(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *src, uint32_t m, uint32_t n,
                  void *dst, uint32_t il = 0);
// Output position of feature f's gate sum in a product over an interleaved
// [gate; up] panel matrix; its up sum follows 32 positions later.
__host__ __device__ __forceinline__ int gu_index(int f) { return 64 * (f >> 5) + (f & 31); }
// Input planes of the panel MFMA GEMM (batch 2..32): fp16 hi / lo planes of
// x in "fragment order", 32 rows (batch entries) x n columns per plane.
// Element (b, c) lies in the 1 KiB block of its 16-column step c / 16, at the
// lane that holds it in the A operand of v_mfma_f32_32x32x16_f16 (lane
// b + 32 * ((c / 8) % 2), 8 consecutive columns per lane), so a wave loads
// one step's operand with one fully contiguous 1 KiB load.  Rows past the
// batch are never read.  More than 32 rows (the prefill's chunks) are stored
// as consecutive 32-row planes, each xf_plane_len(n) halves: row b lies in
// plane b / 32 at row b % 32, and each 32-row group is one GEMM's input.
__host__ __device__ inline size_t xf_index(int b, int c, int n) {
    return (size_t)(b >> 5) * 32 * (size_t)n +
           ((size_t)(c >> 4) * 64 + (size_t)((b & 31) + 32 * ((c >> 3) & 1))) * 8 + (size_t)(c & 7);
}
__host__ __device__ inline size_t xf_plane_len(size_t n) { return 32 * n; }

// Range-safe planes.  fp16 alone covers 2^-24 .. 65504 and fp32 activations
// do not stay inside it, so each batch row is stored in groups of 128
// columns scaled by a power of two: group g of row b holds hi + lo of
// x * 2^-e, e = xe[b * xe_stride(n) + g] (int8), chosen so that the group's
// largest |x| scales into [2^14, 2^15) (hi cannot overflow; lo keeps the full
// 2^-22 relative accuracy down to 2^-17 of the group's largest value).
// Power-of-two scaling is exact.  A GEMM brings the groups it reads to one
// exponent per batch row (the largest) and scales its fp32 sums back.  e is
// kept in int8: it is clamped to -128 (groups whose largest |x| is below
// 2^-113 still scale into fp16's normal range by 2^128 down to |x| ~ 2^-142),
// an all-zero group has e = kXeEmpty (-128), a group holding inf / NaN e = 0
// (they propagate, as in fp32).  A row's exponents are padded to 16 bytes,
// so a GEMM reads those of the groups of its K split (2 per panel, splits
// aligned to their size) with one load.
constexpr int kXeGroup = 128;
constexpr int kXeEmpty = -128;
__host__ __device__ __forceinline__ int xe_stride(int n) { return ((n + kXeGroup - 1) / kXeGroup + 15) & ~15; }
inline size_t xe_bytes(size_t n) { return 32 * (size_t)xe_stride((int)n); }
struct Planes {
    _Float16 *hi = nullptr, *lo = nullptr;
    int8_t *xe = nullptr;
    // Deferred RMSNorm scale: when rs is set the planes hold r (.) w and the
    // GEMM multiplies batch row b's sums by 1 / sqrt(t / n + rs_eps), t the
    // row's rs_parts sums of squares rs[b * rs_parts + k] added in k order
    // (n = the GEMM's column count).  Only the x-stationary GEMM of 17..32
    // rows (gemm_xsh) applies it, and the launchers of the others refuse it;
    // kernels that write planes ignore it.
    float *rs = nullptr;
    int rs_parts = 0;
    float rs_eps = 0.0f;
    // the planes of rows 32 g .. 32 g + 31 for an n-column input
    __host__ __device__ Planes group(int g, int n) const {
        Planes p;
        p.hi = hi ? hi + (size_t)g * xf_plane_len((size_t)n) : nullptr;
        p.lo = lo ? lo + (size_t)g * xf_plane_len((size_t)n) : nullptr;
        p.xe = xe ? xe + (size_t)g * 32 * xe_stride(n) : nullptr;
        p.rs = rs ? rs + (size_t)g * 32 * rs_parts : nullptr;
        p.rs_parts = rs_parts;
        p.rs_eps = rs_eps;
        return p;
    }
    Planes without_scale() const {
        Planes p = *this;
        p.rs = nullptr;
        p.rs_parts = 0;
        return p;
    }
};
// 1 / sqrt(mean square + eps) of batch row b from its deferred-norm sums
// (the same additions, in the same order, as the full-row norm kernels).
// Non-temporal 16-byte load / store of 4 floats, for data streamed once per
// step that the caches cannot keep (the DeltaNet states).
typedef float nt_f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_nt4(const float *p) {
    return __builtin_bit_cast(float4, __builtin_nontemporal_load(reinterpret_cast<const nt_f32x4 *>(p)));
}
__device__ __forceinline__ void st_nt4(float *p, float4 v) {
    __builtin_nontemporal_store(__builtin_bit_cast(nt_f32x4, v), reinterpret_cast<nt_f32x4 *>(p));
}
// In two steps, so that the loads can be issued early and the arithmetic
// done later: rs_load (branch-free, rs_parts in 1..kMaxRsParts), rs_finish.
constexpr int kMaxRsParts = 8;
__device__ __forceinline__ void rs_load(const Planes &xp, int b, float (&v)[kMaxRsParts]) {
    const float *p = xp.rs + (size_t)b * xp.rs_parts;
#pragma unroll
    for (int k = 0; k < kMaxRsParts; k++) v[k] = p[min(k, xp.rs_parts - 1)];
}
__device__ __forceinline__ float rs_finish(const Planes &xp, const float (&v)[kMaxRsParts], int n) {
    float t = v[0];
#pragma unroll
    for (int k = 1; k < kMaxRsParts; k++) t = k < xp.rs_parts ? t + v[k] : t;
    return 1.0f / sqrtf(t / (float)n + xp.rs_eps);
}
__host__ __device__ __forceinline__ int xe_index(int b, int c, int n) { return b * xe_stride(n) + c / kXeGroup; }
// Group exponent from the group's largest |x|.
__device__ __forceinline__ int group_exp(float amax) {
    if (amax == 0.0f) return kXeEmpty;
    if (!(amax <= 3.402823466e38f)) return 0;  // inf / NaN
    int ex;
    (void)frexpf(amax, &ex);  // amax in [2^(ex-1), 2^ex)
    return ex - 15 < -128 ? -128 : ex - 15;
}
// hi + lo of v * 2^-e.
__device__ __forceinline__ void split_scaled(float v, int e, _Float16 &hi, _Float16 &lo) {
    const float s = ldexpf(v, -e);
    hi = (_Float16)s;
    lo = (_Float16)(s - (float)hi);
}
// Cross-lane sums on DPP (VALU, no LDS round trip).  Each step adds a lane's
// value to its partner's, and partners get the same two operands, so every
// lane of a group ends with the same bits.  All lanes of the wave must be
// active.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf,
                                                                     false));
}
// sum over each group of 8 lanes: quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror
__device__ __forceinline__ float sum8(float v) { return dpp_add<0x141>(dpp_add<0x4E>(dpp_add<0xB1>(v))); }
// sum over each 16-lane row: row_ror 8, 4, 2, 1
__device__ __forceinline__ float row_sum16(float v) {
    return dpp_add<0x121>(dpp_add<0x122>(dpp_add<0x124>(dpp_add<0x128>(v))));
}
// sum over the wave (the 4 row sums added through readlane; wave-uniform)
__device__ __forceinline__ float wave_sum(float v) {
    const int b = __builtin_bit_cast(int, row_sum16(v));
    const auto row = [&](int lane) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, lane)); };
    return (row(0) + row(16)) + (row(32) + row(48));
}
// sum over each 32-lane half of the wave
__device__ __forceinline__ float half_sum(float v) {
    const int b = __builtin_bit_cast(int, row_sum16(v));
    const auto row = [&](int lane) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, lane)); };
    return (threadIdx.x & 32) ? row(32) + row(48) : row(0) + row(16);
}
// Lane maxima on DPP (VALU, no LDS round trip).  dpp_max<CTRL>: the max of a
// lane's value and its DPP partner's; row_max16: every lane gets the max of
// its 16-lane row (xor 1, xor 2 by quad_perm, then row_half_mirror and
// row_mirror); half_max32: of its 32-lane half (two rows combined through
// readlane).  All lanes of the wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
    return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v),
                                                                        __builtin_bit_cast(int, v), CTRL, 0xf, 0xf,
                                                                        false)));
}
__device__ __forceinline__ float row_max16(float v) {
    return dpp_max<0x140>(dpp_max<0x141>(dpp_max<0x4E>(dpp_max<0xB1>(v))));
}
__device__ __forceinline__ float half_max32(float v) {
    const int b = __builtin_bit_cast(int, row_max16(v));
    const auto rd = [&](int lane) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, lane)); };
    return (threadIdx.x & 32) ? fmaxf(rd(32), rd(48)) : fmaxf(rd(0), rd(16));
}
__device__ __forceinline__ float wave_max64(float v) {
    const int b = __builtin_bit_cast(int, row_max16(v));
    const auto rd = [&](int lane) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, lane)); };
    return fmaxf(fmaxf(rd(0), rd(16)), fmaxf(rd(32), rd(48)));
}
// Max / sum over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane groups of
// a wave; every lane gets the result of its column) and max over l, l ^ 32:
// v_permlane16_swap / v_permlane32_swap, VALU lane exchanges with no LDS.
// Each swap takes two registers holding the same value and both of its
// results are used (checked in the gfx950 code these compile to).
__device__ __forceinline__ float lanes_max2(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto b = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)b[0]), __builtin_bit_cast(float, (uint32_t)b[1]));
}
__device__ __forceinline__ float lanes_max4(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return lanes_max2(fmaxf(__builtin_bit_cast(float, (uint32_t)a[0]), __builtin_bit_cast(float, (uint32_t)a[1])));
}
__device__ __forceinline__ float lanes_sum4(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float s1 = __builtin_bit_cast(float, (uint32_t)a[0]) + __builtin_bit_cast(float, (uint32_t)a[1]);
    const uint32_t u1 = __builtin_bit_cast(uint32_t, s1);
    const auto b = __builtin_amdgcn_permlane32_swap(u1, u1, false, false);
    return __builtin_bit_cast(float, (uint32_t)b[0]) + __builtin_bit_cast(float, (uint32_t)b[1]);
}
typedef _Float16 h4v __attribute__((ext_vector_type(4)));
// 4 values (consecutive columns of one fragment-order row) split at once.
__device__ __forceinline__ void split4_scaled(const float (&v)[4], int e, h4v &hi, h4v &lo) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
        _Float16 h, l;
        split_scaled(v[c], e, h, l);
        hi[c] = h;
        lo[c] = l;
    }
}
// Factor 2^(e - E) (e <= E) as fp16; 0 once below fp16's range.
__device__ __forceinline__ _Float16 xe_factor(int e, int E) { return (_Float16)ldexpf(1.0f, e - E); }
// Panel MFMA GEMM for batch 2..32: out[ks][b][r] (final values when ksplit
// is 1) from the fragment-order hi / lo planes of x (launch_split_x, or the
// hi / lo outputs of the element-wise kernels), ksplit from gemm_packed_ksplit.
// m must be a multiple of 4.
int gemm_packed_ksplit(const anehip_ctx *ctx, uint32_t m, uint32_t n, uint32_t batch);
// split_stride: floats between the K splits' outputs (0: batch * m).
int launch_gemm_packed(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *wp, uint32_t m,
                       uint32_t n, const Planes &xp, uint32_t batch, float *out, int ksplit, size_t split_stride = 0);
// The same for up to 256 rows: above 32 (the prefill's chunks) one gemm_tall
// launch over the 32-row groups of the planes (Planes::group), writing
// out[ks][row][r] with a split stride of rows * m; ksplit from
// gemm_rows_ksplit.
int gemm_rows_ksplit(const anehip_ctx *ctx, uint32_t m, uint32_t n, uint32_t rows);
int launch_gemm_rows(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *wp, uint32_t m, uint32_t n,
                     const Planes &xp, uint32_t rows, float *out, int ksplit);
// Whether gemm_packed_ksplit's split of [m x n] at this batch runs on an
// x-stationary kernel, which can also take x as fp32 rows [batch][n] (no
// planes needed): launch_gemm_xs_rows writes out[ks][b][r] for its
// gemm_packed_ksplit splits.
bool gemm_is_xs(const anehip_ctx *ctx, uint32_t m, uint32_t n, uint32_t batch);
// Whether launch_gemm_packed of this shape applies a deferred norm scale
// (Planes::rs): the 17..32-row x-stationary kernel, n <= 256 kMaxRsParts.
bool gemm_takes_norm_scale(const anehip_ctx *ctx, uint32_t m, uint32_t n, uint32_t batch);
// The FFN gate / up product (interleaved [gate; up] panel matrix, m = 2 F)
// with the SiLU-mul fused: h[b][f] as fp32 rows [batch][F], one launch, no
// partial sums; covered at batch 17..32 for K = 512, 1024 or 2048.
bool gemm_gate_up_silu_ok(const anehip_ctx *ctx, uint32_t m, uint32_t n, uint32_t batch);
int launch_gemm_gate_up_silu(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *wp, uint32_t m,
                             uint32_t n, const Planes &xp, uint32_t batch, float *h);
int launch_gemm_xs_rows(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *wp, uint32_t m,
                        uint32_t n, const float *x, uint32_t batch, float *out);
// x [batch][n] fp32 -> fragment-order hi / lo planes (xf_plane_len(n) halves each).
int launch_split_x(anehip_ctx *ctx, hipStream_t stream, const float *x, uint32_t batch, uint32_t n, const Planes &xp);
// K splits the batch-1 panel GEMV takes for an [m x n] matrix (<= 8) whose
// input is formed by prologue `mode` (a GEMV_IN_* value): norm prologues and
// the SiLU-mul prologue favour fewer splits.
int gemv_packed_ksplit(const anehip_ctx *ctx, uint32_t m, uint32_t n, int mode = GEMV_IN_PLAIN);
// One-launch batch-1 GEMV of a matrix with few row tiles (gemv.hip:
// gemv_rows); gemv_rows_split gives its row split, or 0 when it does not apply.
int gemv_rows_split(const anehip_ctx *ctx, uint32_t m, uint32_t n);
int launch_gemv_rows(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w, uint32_t m, uint32_t n,
                     const float *x, float *y, int H);
int launch_gemv_packed(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w, uint32_t m,
                       uint32_t n, const GemvInput &in, float *out, int ksplit);
// Batch-1 GEMV whose input is formed by `in` (see GemvInMode); writes
// out[ks][m] partials (final values if ksplit == 1).
int launch_gemv_fused(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w, uint32_t m,
                      uint32_t n, const GemvInput &in, float *out, int ksplit);

// Batch-1 DeltaNet step fused into the ssm_out GEMV (gemv.hip:
// dn_ssm_kernel).  The kernel reads the recurrent state and the conv windows
// but writes neither (the workgroups of a K split share each head's state):
// the head outputs are formed as o = S'^T q + delta (k . q) from the old
// state, and the update's inputs -- delta [H][128], the normalised k [H][128],
// decay [H], the new conv inputs [3 dim] -- go to a per-layer pending block of
// kDnPendFloats(dim, H) floats; launch_deltanet_apply commits every layer's
// update at the end of the step.
__host__ __device__ constexpr size_t kDnPendFloats(size_t dim, size_t n_heads) { return 5 * dim + n_heads; }
constexpr int kMaxDnApplyLayers = 64;
struct DnApplyTab {
    float *S[kMaxDnApplyLayers];
    float *conv[kMaxDnApplyLayers];
    const float *pend[kMaxDnApplyLayers];
    int n = 0;
};
// Whether the fused kernel covers this model at batch 1 (head dim 128, an
// even number of heads, one panel of ssm_out input per K split).
bool dn_ssm_fusable(const anehip_ctx *ctx, uint32_t dim, uint32_t n_heads);
// ssm_out partials [dim / 256][dim] of the batch-1 step; mix: the mixer-in
// projection [q | k | v (3 dim)][gate (dim)][beta (H)][alpha (H)].
int launch_dn_ssm(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w, uint32_t dim,
                  uint32_t n_heads, const MixIn &mix, const float *conv_w, const float *conv_state, const float *ssm_a,
                  const float *dt_bias, const float *S, const float *norm_w, float eps, float *pend, float *out);
// Commits the pending updates of tab's layers: S = decay S + k delta^T
// (deltanet.rs:485-512 order), conv windows shifted and the new inputs
// appended (deltanet_cache.rs:34-42).
int launch_deltanet_apply(anehip_ctx *ctx, hipStream_t stream, const DnApplyTab &tab, int n_heads, int dim);

// deltanet.hip.  mix: qkv [3*chunk]; beta, alpha: [n_heads] per sequence.
// With count (batch * n_heads zeroed counters, left zeroed) the q / k conv
// windows are committed too; without, launch_dn_finish (or the ssm_out
// GEMV's gated-norm prologue) commits them.
int launch_deltanet_step(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, const MixIn &mix,
                         const MixIn &beta, const MixIn &alpha, const float *conv_w, const float *ssm_a,
                         const float *dt_bias, float *conv_state, float *S, float *out, uint32_t *count = nullptr);
// Batch > 1: the whole DeltaNet step of a head in one workgroup -- conv +
// SiLU, L2 norms, beta / decay, recurrence, all conv windows committed -- and
// either the raw head outputs (out, fp32) or, with out == nullptr, the gated
// RMSNorm (gate from mix rows at gate_off, norm_w, eps) as range-safe
// fragment-order planes xp.
int launch_deltanet_head(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, const MixIn &mix,
                         const MixIn &beta, const MixIn &alpha, const float *conv_w, const float *ssm_a,
                         const float *dt_bias, float *conv_state, float *S, float *out, int gate_off,
                         const float *norm_w, float eps, const Planes &xp);
// Prefill: `rows` (<= 32) consecutive tokens of one sequence (mix row t =
// token t) through the DeltaNet step of every head, the state (the sequence's
// block S) kept in registers across the rows.  Three kernels: every token's
// normalised q, k, v, beta and decay to prep (scratch of rows * (3 * dim + 2 *
// n_heads) floats); the recurrence, raw head outputs to heads [rows][dim]
// (scratch); row t's gated RMSNorm to the planes and the conv windows (the
// sequence's block conv_state) advanced by the rows.
int launch_deltanet_scan(anehip_ctx *ctx, hipStream_t stream, int rows, int n_heads, const MixIn &mix,
                         const MixIn &beta, const MixIn &alpha, const float *conv_w, const float *ssm_a,
                         const float *dt_bias, float *conv_state, float *S, float *prep, float *heads,
                         int gate_off, const float *norm_w, float eps, const Planes &xp);
// Commits the q/k conv windows (if conv_state) and, if heads, writes the gated
// RMSNorm of the heads (gate from mix rows at gate_off) to out (fp32) or, if
// xp.hi, to range-safe fragment-order planes (Planes).
int launch_dn_finish(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, const MixIn &mix,
                     float *conv_state, const float *heads, int gate_off, const float *norm_w, float *out,
                     const Planes &xp, float eps);

// attention.hip.  mix per sequence: [q_full | k | v] rows.
size_t attn_partial_floats(int batch, int n_kv, int max_seq, int G);
// Chunks per (sequence, kv head) of the decode attention's partials for this
// state shape (the launch's grid.x).
int attn_chunks(int max_seq, int batch, int n_kv);
// With out == xp.hi == nullptr only the chunk partials are written (a
// batch-1 GEMV with GEMV_IN_ATTN_COMBINE merges them).
int launch_attention(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, int n_kv, int max_seq,
                     const MixIn &mix, const float *q_norm, const float *k_norm, const float *inv_freq,
                     const uint32_t *pos, __half *k_cache, __half *v_cache, float *part, float *out,
                     const Planes &xp);
// Prefill of `rows` consecutive tokens of one sequence (row t at position
// pos[t], q / k / v in mix row t): appends every row's k / v to the cache at
// cache_off (halves; the sequence's [kv_head][max_seq][256] block), then
// attends row t over positions [0, pos[t]] and writes fragment-order planes.
int launch_attention_prefill(anehip_ctx *ctx, hipStream_t stream, int rows, int n_heads, int n_kv, int max_seq,
                             const MixIn &mix, const float *q_norm, const float *k_norm, const float *inv_freq,
                             const uint32_t *pos, __half *k_cache, __half *v_cache, size_t cache_off, float *part,
                             const Planes &xp);

// elementwise.hip
int launch_rmsnorm(anehip_ctx *ctx, hipStream_t s, int rows, int n, const float *x, const float *w, float *out,
                   float eps);
// The next three write their result as fp32 (xn / h) or, when xp.hi is not
// null, as range-safe fragment-order planes (Planes) for the panel MFMA GEMM.
int launch_embed_rmsnorm(anehip_ctx *ctx, hipStream_t s, int rows, int n, const uint32_t *tokens,
                         const float *emb, uint32_t vocab, float *x, const float *w, float *xn, float eps,
                         const Planes &xp = Planes{});
int launch_residual_rmsnorm(anehip_ctx *ctx, hipStream_t s, int rows, int n, float *x, const float *part,
                            int ksplit, const float *w, float *xn, float eps, const Planes &xp = Planes{});
// x += sum of the ksplit slices; planes of x (.) w with the norm's scale
// deferred to the consumer (xp.rs: n / 256 sums of squares per row).
int launch_residual_rmsnorm_parts(anehip_ctx *ctx, hipStream_t s, int rows, int n, float *x, const float *part,
                                  int ksplit, const float *w, const Planes &xp);
// x = embedding rows of the tokens; planes of x (.) w, the scale deferred as above.
int launch_embed_rmsnorm_parts(anehip_ctx *ctx, hipStream_t s, int rows, int n, const uint32_t *tokens,
                               const float *emb, uint32_t vocab, float *x, const float *w, const Planes &xp);
// gu: the ksplit partial slices [rows][2F] of a product over the interleaved
// [gate; up] panel matrix (feature f's gate sum at gu_index(f), up + 32).
int launch_silu_mul_stacked(anehip_ctx *ctx, hipStream_t s, int rows, int F, const float *gu, int ksplit,
                            float *h, const Planes &xp = Planes{});
int launch_silu_mul(anehip_ctx *ctx, hipStream_t s, float *a, const float *b, size_t n);
int launch_residual_add(anehip_ctx *ctx, hipStream_t s, float *x, const float *y, size_t n);
size_t argmax_workspace_bytes(int rows);
// Greedy argmax of each row's n logits (f32::total_cmp order; equal keys:
// the last index, as Iterator::max_by) into out (and next, if given: the
// next step's input tokens); with pos, row r's position pos[r] is also
// advanced by one, after the token is recorded at hist[r * hist_stride +
// pos[r]] (if hist is given and pos[r] < hist_stride).
int launch_argmax(anehip_ctx *ctx, hipStream_t s, int rows, uint32_t n, const float *logits, void *ws,
                  uint32_t *out, uint32_t *pos = nullptr, uint32_t *next = nullptr, uint32_t *hist = nullptr,
                  uint32_t hist_stride = 0);

// Host helper: inv_freq[p] = 1 / base^(2p / head_dim), the
// reference's formula (deltanet.rs:601-603) evaluated once on the host.
void rope_inv_freq(float base, int head_dim, float *out);

}  // namespace anehip
