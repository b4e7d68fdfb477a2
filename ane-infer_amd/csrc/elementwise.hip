// elementwise.hip — row-wise norms, residuals, SiLU-mul, embedding gather and
// greedy argmax for gfx950.
//
// Replaces rmsnorm_simple, residual_add and silu_mul (crates/engine/metal/
// deltanet.metal:227-272, q8_gemv.metal:89-97) and their CPU forms
// (main.rs:983-992, 1106-1135; scratch.rs:174-186), plus the host-side
// embedding copy (gpu_full_decode.rs:273-278) and greedy_sample
// (main.rs:1767-1785), which move on-device.  GEMV outputs may arrive as
// K-split partial sums ([ksplit][rows][n]); the kernels here add them in split
// order, then apply the element-wise step, so a GEMV and its epilogue cost
// one extra launch at most.
#include "common.h"

namespace anehip {

namespace {

constexpr int kThreads = 256;

// Sum over a 256-thread block; every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return s;
}

// Largest |value| per 128-column group of a row, gathered in LDS by the
// threads of a workgroup (bit patterns of non-negative floats order as ints).
constexpr int kMaxGroups = 512;  // rows of up to 65536 columns

// out[b] = x[b] * (1/sqrt(mean(x[b]^2) + eps)) * w     (main.rs:1106-1113),
// written as fp32, or as row `brow` of range-safe fragment-order fp16 hi/lo
// planes (the input format of the panel MFMA GEMM, see Planes) when xp.hi is
// not null: a first pass takes each group's largest |value|, a second writes
// the planes.
__device__ __forceinline__ void rmsnorm_row(const float *x, const float *__restrict__ w, float *out, int n,
                                            float eps, float *red, Planes xp = Planes{}, int brow = 0) {
    __shared__ int gmax[kMaxGroups];
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kThreads) ss += x[i] * x[i];
    if (xp.hi)
        for (int g = threadIdx.x; g < (n + kXeGroup - 1) / kXeGroup; g += kThreads) gmax[g] = 0;
    ss = block_sum(ss, red);  // its barriers also order the gmax clearing
    const float inv_rms = 1.0f / sqrtf(ss / (float)n + eps);
    if (!xp.hi) {
        for (int i = threadIdx.x; i < n; i += kThreads) out[i] = (x[i] * inv_rms) * w[i];
        return;
    }
    for (int i = threadIdx.x; i < n; i += kThreads)
        atomicMax(&gmax[i / kXeGroup], __float_as_int(fabsf((x[i] * inv_rms) * w[i])));
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kThreads) {
        const float v = (x[i] * inv_rms) * w[i];
        const int e = group_exp(__int_as_float(gmax[i / kXeGroup]));
        split_scaled(v, e, xp.hi[xf_index(brow, i, n)], xp.lo[xf_index(brow, i, n)]);
        if (i % kXeGroup == 0) xp.xe[xe_index(brow, i, n)] = (int8_t)e;
    }
}

__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                           float *__restrict__ out, int n, float eps) {
    __shared__ float red[4];
    const size_t b = blockIdx.x;
    rmsnorm_row(x + b * n, w, out + b * n, n, eps, red);
}

// x[b] = embedding[token[b]] (zeros if token >= vocab, main.rs:960-963);
// xn[b] = rmsnorm(x[b], w).
__global__ __launch_bounds__(kThreads) void embed_rmsnorm_kernel(const uint32_t *__restrict__ tokens,
                                                                 const float *__restrict__ emb, uint32_t vocab,
                                                                 float *__restrict__ x, const float *__restrict__ w,
                                                                 float *__restrict__ xn, int n, float eps,
                                                                 Planes xp) {
    __shared__ float red[4];
    const size_t b = blockIdx.x;
    const uint32_t tok = tokens[b];
    float *xb = x + b * n;
    for (int i = threadIdx.x; i < n; i += kThreads) xb[i] = tok < vocab ? emb[(size_t)tok * n + i] : 0.0f;
    __syncthreads();
    rmsnorm_row(xb, w, xn ? xn + b * n : nullptr, n, eps, red, xp, (int)b);
}

// x[b] += sum_k part[k][b]; if w: xn[b] = rmsnorm(x[b], w).   part stride between
// splits = rows * n.
__global__ __launch_bounds__(kThreads) void residual_rmsnorm_kernel(float *__restrict__ x,
                                                                    const float *__restrict__ part, int ksplit,
                                                                    int rows, const float *__restrict__ w,
                                                                    float *__restrict__ xn, int n, float eps,
                                                                    Planes xp) {
    __shared__ float red[4];
    const size_t b = blockIdx.x;
    float *xb = x + b * n;
    const size_t split = (size_t)rows * n;
    for (int i = threadIdx.x; i < n; i += kThreads) {
        float s = part[b * n + i];
        for (int k = 1; k < ksplit; k++) s += part[k * split + b * n + i];
        xb[i] = xb[i] + s;
    }
    if (!w) return;
    __syncthreads();
    rmsnorm_row(xb, w, xn ? xn + b * n : nullptr, n, eps, red, xp, (int)b);
}

// The same for rows of n <= 2048 (n % 4 == 0) with one workgroup of 512
// threads per row: each thread owns one float4 and issues every load it needs
// (x, the KP partial slices, w) before any arithmetic, so the row costs one
// memory round trip instead of one per 256 elements and per pass.
template <int KP>
__global__ __launch_bounds__(512) void residual_rmsnorm_v4(float *__restrict__ x, const float *__restrict__ part,
                                                           int ksplit, int rows, const float *__restrict__ w,
                                                           float *__restrict__ xn, int n, float eps, Planes xp) {
    __shared__ float red[8];
    const int t = threadIdx.x;
    const size_t b = blockIdx.x;
    const int n4 = n >> 2, e4 = min(t, n4 - 1);
    float4 *x4 = reinterpret_cast<float4 *>(x) + b * n4;
    const float4 *p4 = reinterpret_cast<const float4 *>(part) + b * n4;
    const size_t split4 = (size_t)rows * n4;
    float4 r = x4[e4];
    float4 pv[KP];
#pragma unroll
    for (int k = 0; k < KP; k++) pv[k] = p4[(size_t)min(k, ksplit - 1) * split4 + e4];
    const float4 wv = w ? reinterpret_cast<const float4 *>(w)[e4] : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 s = pv[0];
#pragma unroll
    for (int k = 1; k < KP; k++) {
        const bool on = k < ksplit;
        s.x += on ? pv[k].x : 0.0f;
        s.y += on ? pv[k].y : 0.0f;
        s.z += on ? pv[k].z : 0.0f;
        s.w += on ? pv[k].w : 0.0f;
    }
    r = make_float4(r.x + s.x, r.y + s.y, r.z + s.z, r.w + s.w);
    const bool mine = t < n4;
    if (mine) x4[t] = r;
    if (!w) return;
    float ss = mine ? r.x * r.x + r.y * r.y + r.z * r.z + r.w * r.w : 0.0f;
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    // planes: the largest |r * w| of each 128-column group (32 consecutive
    // threads of one wave, all inside the row or all outside: n % 128 == 0),
    // taken while the sum of squares crosses the barrier; times inv_rms it
    // gives the group's binade (to a few ulps)
    const float gmax = xp.hi ? half_max32(mine ? fmaxf(fmaxf(fabsf(r.x * wv.x), fabsf(r.y * wv.y)),
                                                      fmaxf(fabsf(r.z * wv.z), fabsf(r.w * wv.w)))
                                               : 0.0f)
                             : 0.0f;
    __syncthreads();
    float tot = red[0];
#pragma unroll
    for (int i = 1; i < 8; i++) tot += red[i];
    const float inv_rms = 1.0f / sqrtf(tot / (float)n + eps);
    const float v[4] = {(r.x * inv_rms) * wv.x, (r.y * inv_rms) * wv.y, (r.z * inv_rms) * wv.z,
                        (r.w * inv_rms) * wv.w};
    if (xp.hi) {
        if (!mine) return;
        const int e = group_exp(gmax * inv_rms);
        // columns 4t .. 4t + 3 are consecutive in a fragment-order plane
        h4v vh, vl;
        split4_scaled(v, e, vh, vl);
        const size_t o = xf_index((int)b, 4 * t, n);
        *reinterpret_cast<h4v *>(xp.hi + o) = vh;
        *reinterpret_cast<h4v *>(xp.lo + o) = vl;
        if ((t & 31) == 0) xp.xe[xe_index((int)b, 4 * t, n)] = (int8_t)e;
    } else if (mine && xn) {
        reinterpret_cast<float4 *>(xn)[b * n4 + t] = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// The same residual add for a consumer that applies the RMSNorm's scale
// itself (Planes::rs, gemm_xsh): one wave per 256-column slice (grid n / 256
// x rows), so a row's partial slices are read by n / 256 CUs instead of one.
// The planes get r (.) w with each 128-column group's exponent from its own
// largest |r w|, and rs[b * (n / 256) + s] slice s's sum of squares -- the
// wave sums of residual_rmsnorm_v4, which its consumer adds in slice order
// as that kernel does; the scale (r * inv_rms) * w of main.rs:1106-1113 is
// then applied to the consumer's sums (reassociated).
template <int KP>
__global__ __launch_bounds__(64) void residual_rmsnorm_parts(float *__restrict__ x, const float *__restrict__ part,
                                                             int ksplit, int rows, const float *__restrict__ w,
                                                             int n, Planes xp) {
    const int t = threadIdx.x, sl = blockIdx.x;
    const size_t b = blockIdx.y;
    const int n4 = n >> 2, e4 = sl * 64 + t;
    float4 *x4 = reinterpret_cast<float4 *>(x) + b * n4;
    const float4 *p4 = reinterpret_cast<const float4 *>(part) + b * n4;
    const size_t split4 = (size_t)rows * n4;
    float4 r = x4[e4];
    float4 pv[KP];
#pragma unroll
    for (int k = 0; k < KP; k++) pv[k] = p4[(size_t)min(k, ksplit - 1) * split4 + e4];
    const float4 wv = reinterpret_cast<const float4 *>(w)[e4];
    float4 s = pv[0];
#pragma unroll
    for (int k = 1; k < KP; k++) {
        const bool on = k < ksplit;
        s.x += on ? pv[k].x : 0.0f;
        s.y += on ? pv[k].y : 0.0f;
        s.z += on ? pv[k].z : 0.0f;
        s.w += on ? pv[k].w : 0.0f;
    }
    r = make_float4(r.x + s.x, r.y + s.y, r.z + s.z, r.w + s.w);
    x4[e4] = r;
    const float ss = wave_sum(r.x * r.x + r.y * r.y + r.z * r.z + r.w * r.w);
    const float v[4] = {r.x * wv.x, r.y * wv.y, r.z * wv.z, r.w * wv.w};
    const int e = group_exp(half_max32(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])))));
    h4v vh, vl;
    split4_scaled(v, e, vh, vl);
    const size_t o = xf_index((int)b, 4 * e4, n);
    *reinterpret_cast<h4v *>(xp.hi + o) = vh;
    *reinterpret_cast<h4v *>(xp.lo + o) = vl;
    if ((t & 31) == 0) xp.xe[xe_index((int)b, 4 * e4, n)] = (int8_t)e;
    if (t == 0) xp.rs[b * (size_t)xp.rs_parts + sl] = ss;
}

// The embedding gather of embed_rmsnorm_kernel in the same form (grid n /
// 256 x rows, one wave per slice): x[b] = embedding[token[b]] (zeros if
// token >= vocab), the planes of x (.) w and the slices' sums of squares.
__global__ __launch_bounds__(64) void embed_rmsnorm_parts(const uint32_t *__restrict__ tokens,
                                                          const float *__restrict__ emb, uint32_t vocab,
                                                          float *__restrict__ x, const float *__restrict__ w, int n,
                                                          Planes xp) {
    const int t = threadIdx.x, sl = blockIdx.x;
    const size_t b = blockIdx.y;
    const int n4 = n >> 2, e4 = sl * 64 + t;
    const uint32_t tok = tokens[b];
    const float4 wv = reinterpret_cast<const float4 *>(w)[e4];
    const float4 r = tok < vocab ? reinterpret_cast<const float4 *>(emb + (size_t)tok * n)[e4]
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
    reinterpret_cast<float4 *>(x)[b * n4 + e4] = r;
    const float ss = wave_sum(r.x * r.x + r.y * r.y + r.z * r.z + r.w * r.w);
    const float v[4] = {r.x * wv.x, r.y * wv.y, r.z * wv.z, r.w * wv.w};
    const int e = group_exp(half_max32(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])))));
    h4v vh, vl;
    split4_scaled(v, e, vh, vl);
    const size_t o = xf_index((int)b, 4 * e4, n);
    *reinterpret_cast<h4v *>(xp.hi + o) = vh;
    *reinterpret_cast<h4v *>(xp.lo + o) = vl;
    if ((t & 31) == 0) xp.xe[xe_index((int)b, 4 * e4, n)] = (int8_t)e;
    if (t == 0) xp.rs[b * (size_t)xp.rs_parts + sl] = ss;
}

// Output of the GEMM over the interleaved [gate; up] panel matrix,
// gu[k][b][2F] with feature r's gate sum at gu_index(r) and its up sum 32
// positions on: h[b][r] = SiLU(gate) * up (scratch.rs:181-186: a = (a / (1 +
// exp(-a))) * b).
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const float *__restrict__ gu, int ksplit, int rows,
                                                            float *__restrict__ h, int F, Planes xp) {
    __shared__ float wm[kThreads / 64];
    const size_t b = blockIdx.y;
    const int r = blockIdx.x * kThreads + threadIdx.x;
    const bool in = r < F;
    const int rr = in ? r : F - 1;
    const size_t split = (size_t)rows * 2 * F;
    const size_t gi = b * 2 * F + gu_index(rr);
    float g = gu[gi], u = gu[gi + 32];
    for (int k = 1; k < ksplit; k++) {
        g += gu[k * split + gi];
        u += gu[k * split + gi + 32];
    }
    const float v = (g / (1.0f + expf(-g))) * u;
    if (xp.hi) {
        // a 128-column group is two waves of this workgroup
        float amax = in ? fabsf(v) : 0.0f;
        amax = wave_max64(amax);
        if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = amax;
        __syncthreads();
        const int w0 = (threadIdx.x >> 6) & ~1;
        const int e = group_exp(fmaxf(wm[w0], wm[w0 + 1]));
        if (!in) return;
        split_scaled(v, e, xp.hi[xf_index((int)b, r, F)], xp.lo[xf_index((int)b, r, F)]);
        if (r % kXeGroup == 0) xp.xe[xe_index((int)b, r, F)] = (int8_t)e;
    } else if (in) {
        h[b * F + r] = v;
    }
}

// The same for F % 4 == 0: one float4 of gate and of up per thread, with all
// KP (>= ksplit) slices loaded before any is added (slices past ksplit re-read
// the last one and are not added), so the row costs one memory round trip.
template <int KP>
__global__ __launch_bounds__(kThreads) void silu_mul_v4(const float *__restrict__ gu, int ksplit, int rows,
                                                        float *__restrict__ h, int F, Planes xp) {
    const int b = blockIdx.y;
    const int r = 4 * (blockIdx.x * kThreads + threadIdx.x);
    const bool in = r < F;
    if (!xp.hi && !in) return;
    const size_t split = (size_t)rows * 2 * F;
    // features r .. r + 3 lie in one group of 32 of the interleaved order
    const float *g0 = gu + (size_t)b * 2 * F + gu_index(in ? r : F - 4);
    float4 gv[KP], uv[KP];
#pragma unroll
    for (int k = 0; k < KP; k++) {
        const size_t o = (size_t)min(k, ksplit - 1) * split;
        gv[k] = *reinterpret_cast<const float4 *>(g0 + o);
        uv[k] = *reinterpret_cast<const float4 *>(g0 + 32 + o);
    }
    float g[4] = {gv[0].x, gv[0].y, gv[0].z, gv[0].w}, u[4] = {uv[0].x, uv[0].y, uv[0].z, uv[0].w};
#pragma unroll
    for (int k = 1; k < KP; k++) {
        const bool on = k < ksplit;
        const float ga[4] = {gv[k].x, gv[k].y, gv[k].z, gv[k].w}, ua[4] = {uv[k].x, uv[k].y, uv[k].z, uv[k].w};
#pragma unroll
        for (int c = 0; c < 4; c++) {
            g[c] = on ? g[c] + ga[c] : g[c];
            u[c] = on ? u[c] + ua[c] : u[c];
        }
    }
    float v[4];
#pragma unroll
    for (int c = 0; c < 4; c++) v[c] = (g[c] / (1.0f + expf(-g[c]))) * u[c];
    if (xp.hi) {
        // a 128-column group is 32 consecutive threads of one wave (all of
        // them inside the row or all outside: F % 128 == 0 for planes)
        const float amax =
            half_max32(in ? fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))) : 0.0f);
        if (!in) return;
        const int e = group_exp(amax);
        // columns r .. r + 3 (r % 4 == 0) are consecutive in a fragment-order plane
        h4v vh, vl;
        split4_scaled(v, e, vh, vl);
        const size_t o = xf_index(b, r, F);
        *reinterpret_cast<h4v *>(xp.hi + o) = vh;
        *reinterpret_cast<h4v *>(xp.lo + o) = vl;
        if ((threadIdx.x & 31) == 0) xp.xe[xe_index(b, r, F)] = (int8_t)e;
    } else {
        *reinterpret_cast<float4 *>(h + (size_t)b * F + r) = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// a[i] = silu(a[i]) * b[i]   (elementwise entry point)
__global__ __launch_bounds__(kThreads) void silu_mul_plain_kernel(float *__restrict__ a, const float *__restrict__ b,
                                                                  size_t n) {
    size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) a[i] = (a[i] / (1.0f + expf(-a[i]))) * b[i];
}

// x[i] += y[i]
__global__ __launch_bounds__(kThreads) void residual_add_kernel(float *__restrict__ x, const float *__restrict__ y,
                                                                size_t n) {
    size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) x[i] += y[i];
}

// f32::total_cmp order as a signed key (bit flip of negatives).
__device__ __forceinline__ int32_t total_key(float f) {
    int32_t b = __float_as_int(f);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

// (key, index) with the larger key; equal keys: the larger index (Iterator::max_by
// keeps the last maximum).
__device__ __forceinline__ void arg_better(int32_t &k, uint32_t &i, int32_t k2, uint32_t i2) {
    if (k2 > k || (k2 == k && i2 > i)) {
        k = k2;
        i = i2;
    }
}

// (key, index) as one unsigned 64-bit value (the key's sign bit flipped on
// top, the index below): the larger value is the better pair of arg_better.
__device__ __forceinline__ uint64_t arg_pack(int32_t k, uint32_t i) {
    return ((uint64_t)((uint32_t)k ^ 0x80000000u) << 32) | i;
}

// v and its DPP partner's value, the larger kept (both halves moved by DPP)
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_max_u64(uint64_t v) {
    const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
    const uint64_t o = ((uint64_t)(uint32_t)__builtin_amdgcn_update_dpp(hi, hi, CTRL, 0xf, 0xf, false) << 32) |
                       (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, CTRL, 0xf, 0xf, false);
    return o > v ? o : v;
}

// The wave's best (key, index) on DPP: quad_perm xor 1, xor 2, then the
// half-row and row mirrors (each lane ends with its 16-lane row's best), and
// the 4 rows through readlane.  Every lane of the wave must be active.
__device__ __forceinline__ void wave_argmax(int32_t &k, uint32_t &i) {
    uint64_t v = arg_pack(k, i);
    v = dpp_max_u64<0x140>(dpp_max_u64<0x141>(dpp_max_u64<0x4E>(dpp_max_u64<0xB1>(v))));
    const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
    uint64_t best = 0;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint64_t c = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, 16 * r) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane(lo, 16 * r);
        best = c > best ? c : best;
    }
    k = (int32_t)((uint32_t)(best >> 32) ^ 0x80000000u);
    i = (uint32_t)best;
}

__device__ __forceinline__ void block_argmax(int32_t &k, uint32_t &i, int32_t *rk, uint32_t *ri) {
    wave_argmax(k, i);
    if ((threadIdx.x & 63) == 0) {
        rk[threadIdx.x >> 6] = k;
        ri[threadIdx.x >> 6] = i;
    }
    __syncthreads();
    k = rk[0];
    i = ri[0];
    for (int w = 1; w < kThreads / 64; w++) arg_better(k, i, rk[w], ri[w]);
}

constexpr int kArgBlocks = 64;

// stage 1: grid (kArgBlocks, batch); each block scans a strided slice.
__global__ __launch_bounds__(kThreads) void argmax_stage1(const float *__restrict__ logits, uint32_t n,
                                                          int32_t *__restrict__ pk, uint32_t *__restrict__ pi) {
    __shared__ int32_t rk[4];
    __shared__ uint32_t ri[4];
    const size_t b = blockIdx.y;
    const float *row = logits + b * n;
    int32_t k = INT32_MIN;
    uint32_t idx = 0;
    bool any = false;
    // 8 strided values per trip, loaded before any is compared (the order of
    // the comparisons does not matter: arg_better is a total order on (key,
    // index)), so a 151936-entry row costs 2 round trips instead of 10
    constexpr uint32_t kStride = kArgBlocks * kThreads;
    for (uint32_t j0 = blockIdx.x * kThreads + threadIdx.x; j0 < n; j0 += 8 * kStride) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = row[min(j0 + u * kStride, n - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint32_t j = j0 + u * kStride;
            if (j < n) {
                const int32_t kk = total_key(v[u]);
                if (!any) {
                    k = kk;
                    idx = j;
                    any = true;
                } else {
                    arg_better(k, idx, kk, j);
                }
            }
        }
    }
    if (!any) {
        k = INT32_MIN;
        idx = 0;
    }
    block_argmax(k, idx, rk, ri);
    if (threadIdx.x == 0) {
        pk[b * kArgBlocks + blockIdx.x] = k;
        pi[b * kArgBlocks + blockIdx.x] = idx;
    }
}

// stage 2: one wave per row; with `pos`, row b's position is advanced too
// (the decode step's last operation, folded in to save a kernel boundary).
__global__ __launch_bounds__(64) void argmax_stage2(const int32_t *__restrict__ pk, const uint32_t *__restrict__ pi,
                                                    uint32_t *__restrict__ out, uint32_t *__restrict__ pos,
                                                    uint32_t *__restrict__ next, uint32_t *__restrict__ hist,
                                                    uint32_t hist_stride) {
    const size_t b = blockIdx.x;
    int32_t k = pk[b * kArgBlocks + threadIdx.x];
    uint32_t i = pi[b * kArgBlocks + threadIdx.x];
    wave_argmax(k, i);
    if (threadIdx.x == 0) {
        out[b] = i;
        if (next) next[b] = i;
        if (pos) {
            const uint32_t p = pos[b];
            if (hist && p < hist_stride) hist[b * hist_stride + p] = i;
            pos[b] = p + 1u;
        }
    }
}

}  // namespace

int launch_rmsnorm(anehip_ctx *ctx, hipStream_t s, int rows, int n, const float *x, const float *w, float *out,
                   float eps) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kThreads), 0, s, x, w, out, n, eps);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

static int check_planes(anehip_ctx *ctx, const Planes &xp, int n) {
    if (xp.hi && (!xp.lo || !xp.xe || n % kXeGroup || n > kMaxGroups * kXeGroup))
        return set_error(ctx->err, ANEHIP_EINVAL, "planes: incomplete, or n=%d not a multiple of %d up to %d", n,
                         kXeGroup, kMaxGroups * kXeGroup);
    return ANEHIP_OK;
}

int launch_embed_rmsnorm(anehip_ctx *ctx, hipStream_t s, int rows, int n, const uint32_t *tokens, const float *emb,
                         uint32_t vocab, float *x, const float *w, float *xn, float eps, const Planes &xp) {
    if (int rc = check_planes(ctx, xp, n)) return rc;
    hipLaunchKernelGGL(embed_rmsnorm_kernel, dim3(rows), dim3(kThreads), 0, s, tokens, emb, vocab, x, w, xn, n, eps,
                       xp);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_residual_rmsnorm(anehip_ctx *ctx, hipStream_t s, int rows, int n, float *x, const float *part,
                            int ksplit, const float *w, float *xn, float eps, const Planes &xp) {
    if (int rc = check_planes(ctx, xp, n)) return rc;
    if (n % 4 == 0 && n <= 2048 && ksplit >= 1 && ksplit <= 16) {
        if (ksplit <= 2)
            hipLaunchKernelGGL(residual_rmsnorm_v4<2>, dim3(rows), dim3(512), 0, s, x, part, ksplit, rows, w, xn, n,
                               eps, xp);
        else if (ksplit <= 8)
            hipLaunchKernelGGL(residual_rmsnorm_v4<8>, dim3(rows), dim3(512), 0, s, x, part, ksplit, rows, w, xn, n,
                               eps, xp);
        else
            hipLaunchKernelGGL(residual_rmsnorm_v4<16>, dim3(rows), dim3(512), 0, s, x, part, ksplit, rows, w, xn, n,
                               eps, xp);
    } else {
        hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(rows), dim3(kThreads), 0, s, x, part, ksplit, rows, w, xn,
                           n, eps, xp);
    }
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_residual_rmsnorm_parts(anehip_ctx *ctx, hipStream_t s, int rows, int n, float *x, const float *part,
                                  int ksplit, const float *w, const Planes &xp) {
    if (int rc = check_planes(ctx, xp, n)) return rc;
    if (!xp.hi || !xp.rs || !w || n % 256 || xp.rs_parts != n / 256 || xp.rs_parts > kMaxRsParts || ksplit < 1 ||
        ksplit > 16)
        return set_error(ctx->err, ANEHIP_EINVAL,
                         "residual_rmsnorm_parts: n=%d (multiple of 256), %d norm parts, K split %d (1..16)", n,
                         xp.rs_parts, ksplit);
    const dim3 grid(n / 256, rows);
    if (ksplit <= 8)
        hipLaunchKernelGGL(residual_rmsnorm_parts<8>, grid, dim3(64), 0, s, x, part, ksplit, rows, w, n, xp);
    else
        hipLaunchKernelGGL(residual_rmsnorm_parts<16>, grid, dim3(64), 0, s, x, part, ksplit, rows, w, n, xp);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_embed_rmsnorm_parts(anehip_ctx *ctx, hipStream_t s, int rows, int n, const uint32_t *tokens,
                               const float *emb, uint32_t vocab, float *x, const float *w, const Planes &xp) {
    if (int rc = check_planes(ctx, xp, n)) return rc;
    if (!xp.hi || !xp.rs || !w || n % 256 || xp.rs_parts != n / 256 || xp.rs_parts > kMaxRsParts)
        return set_error(ctx->err, ANEHIP_EINVAL, "embed_rmsnorm_parts: n=%d (multiple of 256), %d norm parts", n,
                         xp.rs_parts);
    hipLaunchKernelGGL(embed_rmsnorm_parts, dim3(n / 256, rows), dim3(64), 0, s, tokens, emb, vocab, x, w, n, xp);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_silu_mul_stacked(anehip_ctx *ctx, hipStream_t s, int rows, int F, const float *gu, int ksplit, float *h,
                            const Planes &xp) {
    if (int rc = check_planes(ctx, xp, F)) return rc;
    if (F % 4 == 0 && ksplit >= 1 && ksplit <= 16) {
        const dim3 grid((F / 4 + kThreads - 1) / kThreads, rows);
        if (ksplit == 1)
            hipLaunchKernelGGL(silu_mul_v4<1>, grid, dim3(kThreads), 0, s, gu, ksplit, rows, h, F, xp);
        else if (ksplit <= 4)
            hipLaunchKernelGGL(silu_mul_v4<4>, grid, dim3(kThreads), 0, s, gu, ksplit, rows, h, F, xp);
        else
            hipLaunchKernelGGL(silu_mul_v4<16>, grid, dim3(kThreads), 0, s, gu, ksplit, rows, h, F, xp);
    } else {
        hipLaunchKernelGGL(silu_mul_kernel, dim3((F + kThreads - 1) / kThreads, rows), dim3(kThreads), 0, s, gu,
                           ksplit, rows, h, F, xp);
    }
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_silu_mul(anehip_ctx *ctx, hipStream_t s, float *a, const float *b, size_t n) {
    hipLaunchKernelGGL(silu_mul_plain_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s,
                       a, b, n);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_residual_add(anehip_ctx *ctx, hipStream_t s, float *x, const float *y, size_t n) {
    hipLaunchKernelGGL(residual_add_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, x,
                       y, n);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

size_t argmax_workspace_bytes(int rows) { return (size_t)rows * kArgBlocks * 8; }

// ws: argmax_workspace_bytes(rows) bytes of device memory.
int launch_argmax(anehip_ctx *ctx, hipStream_t s, int rows, uint32_t n, const float *logits, void *ws,
                  uint32_t *out, uint32_t *pos, uint32_t *next, uint32_t *hist, uint32_t hist_stride) {
    int32_t *pk = static_cast<int32_t *>(ws);
    uint32_t *pi = reinterpret_cast<uint32_t *>(pk + (size_t)rows * kArgBlocks);
    hipLaunchKernelGGL(argmax_stage1, dim3(kArgBlocks, rows), dim3(kThreads), 0, s, logits, n, pk, pi);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    hipLaunchKernelGGL(argmax_stage2, dim3(rows), dim3(64), 0, s, pk, pi, out, pos, next, hist, hist_stride);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

}  // namespace anehip
