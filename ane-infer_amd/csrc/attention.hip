// attention.hip — GQA decode attention over an fp16 KV cache for gfx950.
//
// Replaces q_gate_split, rmsnorm_gated (q/k norm use), rope_apply, the KV
// append gpu_memcpys, sdpa_causal and sigmoid_gate (crates/engine/metal/
// attention.metal:9-121, deltanet.metal:184-220; dispatched at
// gpu_full_decode.rs:628-903) and the CPU core of full_attn_decode_step
// (crates/engine/src/deltanet.rs:565-669).
//
// Split-K ("flash-decoding"): the positions 0..pos of one sequence are cut
// into chunks of 64; one workgroup per (chunk, kv head, sequence) reads that
// chunk's K and V rows once for all G query heads that share the kv head,
// and writes an unnormalised partial output with its running max and sum.
// attn_combine_kernel merges the chunks with a log-sum-exp rescale and
// applies sigmoid(gate).  Chunks past the sequence's length exit at once, so
// one launch shape (sized for the cache capacity) serves every position and
// can be captured in a graph while pos lives in device memory.
//
// The KV cache keeps fp16 values (round-to-nearest-even) in the reference's
// per-sequence layout [kv_head][max_seq][head_dim] (kv_cache.rs:7-27).  The
// current position's k/v are rounded to fp16 before use, exactly as if they
// had been written to the cache and read back (the reference writes first,
// deltanet.rs:625, then reads every position).
#include "common.h"

namespace anehip {

namespace {

constexpr int kHd = 256;       // head_dim
constexpr int kCh = 64;        // positions per workgroup
constexpr int kThreads = 256;
constexpr int kRowH = kHd + 8; // LDS row stride in halfs (pad: conflict-free 16-byte reads)

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// RMSNorm (eps 1e-6, deltanet.rs:575-598) + RoPE (deltanet.rs:600-623) of one
// 256-dim head by one wave: lane l owns dims 4l..4l+3 = rotary pairs 2l, 2l+1.
__device__ __forceinline__ void norm_rope_head(const MixIn &mix, int b, int base, const float *__restrict__ w,
                                               const float *__restrict__ inv_freq, uint32_t pos, int lane,
                                               float *dst) {
    float4 x = mix.at4(b, base + 4 * lane);
    float ss = wave_sum(x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w);
    const float inv_rms = 1.0f / sqrtf(ss / (float)kHd + 1e-6f);
    float4 wv = *reinterpret_cast<const float4 *>(w + 4 * lane);
    float a0 = (x.x * inv_rms) * wv.x, a1 = (x.y * inv_rms) * wv.y;
    float a2 = (x.z * inv_rms) * wv.z, a3 = (x.w * inv_rms) * wv.w;
    const float fpos = (float)pos;
    const float t0 = fpos * inv_freq[2 * lane], t1 = fpos * inv_freq[2 * lane + 1];
    const float s0 = sinf(t0), c0 = cosf(t0), s1 = sinf(t1), c1 = cosf(t1);
    dst[0] = a0 * c0 - a1 * s0;
    dst[1] = a0 * s0 + a1 * c0;
    dst[2] = a2 * c1 - a3 * s1;
    dst[3] = a2 * s1 + a3 * c1;
}

// grid = (chunks, n_kv_heads, batch).  mix: per sequence [q_full | k | v]
// rows (K-split partial slices); q_full is [n_heads][q(256) | gate(256)].
template <int G>
__global__ __launch_bounds__(kThreads) void attn_partial_kernel(
    MixIn mix, const float *__restrict__ q_norm, const float *__restrict__ k_norm,
    const float *__restrict__ inv_freq, const uint32_t *__restrict__ pos_arr, __half *__restrict__ k_cache,
    __half *__restrict__ v_cache, int max_seq, int n_heads, int n_kv, float *__restrict__ part_o,
    float *__restrict__ part_ml) {
    __shared__ float qs[G][kHd];
    __shared__ __half tile[kCh * kRowH];
    __shared__ __half knew[kHd], vnew[kHd];
    __shared__ float probs[G][kCh];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int c = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const uint32_t pos = pos_arr[b];
    const int len = (int)pos + 1;
    const int start = c * kCh;
    if (start >= len) return;  // uniform exit: nothing of this sequence here
    const int nch = gridDim.x;
    const size_t cache_base = ((size_t)b * n_kv + kvh) * (size_t)max_seq * kHd;
    const bool has_new = (int)pos < start + kCh;  // this chunk holds the current position

    // K and V rows of the chunk (positions < pos) are loaded first, so their
    // memory latency overlaps the q / k preparation below.  Row pos comes from
    // this step's k / v (knew / vnew); rows past pos are zero.
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    constexpr int kPer = (kCh * kHd / 8) / kThreads;  // 16-byte vectors per thread and tile
    u32x4 kreg[kPer], vreg[kPer];
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int q = i * kThreads + t;
        const int r = q >> 5, part = q & 31;
        const int p = min(start + r, (int)pos - 1);  // in bounds; rows >= pos are replaced below
        const size_t off = cache_base + (size_t)max(p, 0) * kHd + part * 8;
        kreg[i] = *reinterpret_cast<const u32x4 *>(k_cache + off);
        vreg[i] = *reinterpret_cast<const u32x4 *>(v_cache + off);
    }

    // q heads of this kv group: wave w < G prepares head kvh*G + w
    if (wave < G) {
        const int h = kvh * G + wave;
        float q4[4];
        norm_rope_head(mix, b, h * 2 * kHd, q_norm, inv_freq, pos, lane, q4);
        *reinterpret_cast<float4 *>(&qs[wave][4 * lane]) = make_float4(q4[0], q4[1], q4[2], q4[3]);
    }
    if (has_new && wave == G % 4) {
        // k: RMSNorm + RoPE, v: as is; both rounded to fp16 and appended
        const int kin = n_heads * 2 * kHd + kvh * kHd;
        const int vin = n_heads * 2 * kHd + n_kv * kHd + kvh * kHd;
        float k4[4];
        norm_rope_head(mix, b, kin, k_norm, inv_freq, pos, lane, k4);
        float4 v4 = mix.at4(b, vin + 4 * lane);
        const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            knew[4 * lane + i] = __float2half_rn(k4[i]);
            vnew[4 * lane + i] = __float2half_rn(vv[i]);
        }
        __half *kd = k_cache + cache_base + (size_t)pos * kHd + 4 * lane;
        __half *vd = v_cache + cache_base + (size_t)pos * kHd + 4 * lane;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            kd[i] = knew[4 * lane + i];
            vd[i] = vnew[4 * lane + i];
        }
    }
    __syncthreads();

    // tile: 64 rows x 32 vectors of 16 bytes; vector q = i*256 + t
    auto store_tile = [&](const u32x4 *reg, const __half *fresh) {
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            const int q = i * kThreads + t;
            const int r = q >> 5, part = q & 31;
            const int p = start + r;
            u32x4 v = reg[i];
            if (p == (int)pos) v = *reinterpret_cast<const u32x4 *>(fresh + part * 8);
            if (p > (int)pos) v = u32x4{0u, 0u, 0u, 0u};
            *reinterpret_cast<u32x4 *>(&tile[r * kRowH + part * 8]) = v;
        }
    };
    store_tile(kreg, knew);
    __syncthreads();

    // scores: wave = query head of the group, lane = position in the chunk
    const float sdiv = sqrtf((float)kHd);
    if (wave < G) {
        const int p = start + lane;
        float dot = 0.0f;
        const __half *kr = &tile[lane * kRowH];
#pragma unroll 4
        for (int d = 0; d < kHd; d += 8) {
            u32x4 kv8 = *reinterpret_cast<const u32x4 *>(kr + d);
            const __half2 *h2 = reinterpret_cast<const __half2 *>(&kv8);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float2 kf = __half22float2(h2[e]);
                dot += qs[wave][d + 2 * e] * kf.x;
                dot += qs[wave][d + 2 * e + 1] * kf.y;
            }
        }
        const float s = p < len ? dot / sdiv : -INFINITY;
        const float m = wave_max(s);
        const float e = p < len ? expf(s - m) : 0.0f;
        const float l = wave_sum(e);
        probs[wave][lane] = e;
        if (lane == 0) {
            float *ml = part_ml + ((((size_t)b * n_kv + kvh) * nch + c) * G + wave) * 2;
            ml[0] = m;
            ml[1] = l;
        }
    }
    __syncthreads();
    store_tile(vreg, vnew);
    __syncthreads();

    // PV: wave = query head, lane = 4 consecutive dims
    if (wave < G) {
        float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
        const int nvalid = min(kCh, len - start);
        for (int p = 0; p < nvalid; p++) {
            const float pr = probs[wave][p];
            const __half2 *v2 = reinterpret_cast<const __half2 *>(&tile[p * kRowH + 4 * lane]);
            float2 a = __half22float2(v2[0]), bb = __half22float2(v2[1]);
            o0 += pr * a.x;
            o1 += pr * a.y;
            o2 += pr * bb.x;
            o3 += pr * bb.y;
        }
        float *po = part_o + ((((size_t)b * n_kv + kvh) * nch + c) * G + wave) * kHd + 4 * lane;
        *reinterpret_cast<float4 *>(po) = make_float4(o0, o1, o2, o3);
    }
}

// grid = (n_heads, batch), 256 threads (one per dim): merge the chunks of one
// head with a log-sum-exp rescale, normalise, multiply by sigmoid(gate)
// (deltanet.rs:667-669).  out: [batch][n_heads * 256] fp32, or fp16 hi/lo
// planes out_hi / out_lo when out_hi is not null.
template <int G>
__global__ __launch_bounds__(kThreads) void attn_combine_kernel(MixIn mix, const uint32_t *__restrict__ pos_arr,
                                                                const float *__restrict__ part_o,
                                                                const float *__restrict__ part_ml, int nch,
                                                                int n_heads, int n_kv, float *__restrict__ out,
                                                                _Float16 *__restrict__ out_hi,
                                                                _Float16 *__restrict__ out_lo) {
    __shared__ float wts[kThreads], red[4];
    const int d = threadIdx.x, h = blockIdx.x, b = blockIdx.y;
    const int kvh = h / G, hh = h % G;
    const int len = (int)pos_arr[b] + 1;
    const int nc = (len + kCh - 1) / kCh;
    const size_t base = ((size_t)b * n_kv + kvh) * nch;
    const float g = mix.at(b, h * 2 * kHd + kHd + d);  // issued early: independent of the partials
    // rounds of up to 256 chunks; the running maximum only grows, earlier
    // rounds are rescaled to it (log-sum-exp merge)
    float num = 0.f, den = 0.f, M = -INFINITY;
    for (int c0 = 0; c0 < nc; c0 += kThreads) {
        const int cc = c0 + d;
        const float m = cc < nc ? part_ml[((base + cc) * G + hh) * 2] : -INFINITY;
        float mx = m;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        if ((d & 63) == 0) red[d >> 6] = mx;
        __syncthreads();
        const float Mn = fmaxf(M, fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
        const float rescale = expf(M - Mn);  // 0 in the first round (num = den = 0)
        num *= rescale;
        den *= rescale;
        M = Mn;
        wts[d] = cc < nc ? expf(m - M) : 0.0f;
        __syncthreads();
        const int n = min(kThreads, nc - c0);
        int c = 0;
        for (; c + 4 <= n; c += 4) {  // 4 independent loads per trip
            float o4[4], l4[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                o4[i] = part_o[((base + c0 + c + i) * G + hh) * kHd + d];
                l4[i] = part_ml[((base + c0 + c + i) * G + hh) * 2 + 1];
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                num += wts[c + i] * o4[i];
                den += wts[c + i] * l4[i];
            }
        }
        for (; c < n; c++) {
            num += wts[c] * part_o[((base + c0 + c) * G + hh) * kHd + d];
            den += wts[c] * part_ml[((base + c0 + c) * G + hh) * 2 + 1];
        }
        __syncthreads();  // wts / red are rewritten by the next round
    }
    const float v = (num / den) * (1.0f / (1.0f + expf(-g)));
    if (out_hi) {
        const size_t o = xf_index(b, h * kHd + d);
        const _Float16 hi = (_Float16)v;
        out_hi[o] = hi;
        out_lo[o] = (_Float16)(v - (float)hi);
    } else {
        out[(size_t)b * n_heads * kHd + (size_t)h * kHd + d] = v;
    }
}

}  // namespace

size_t attn_partial_floats(int batch, int n_kv, int max_seq, int G) {
    const size_t nch = (size_t)(max_seq + kCh - 1) / kCh;
    return (size_t)batch * n_kv * nch * G * (kHd + 2);
}

// part: workspace of attn_partial_floats() floats.
int launch_attention(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, int n_kv, int max_seq,
                     const MixIn &mix, const float *q_norm, const float *k_norm, const float *inv_freq,
                     const uint32_t *pos, __half *k_cache, __half *v_cache, float *part, float *out,
                     _Float16 *out_hi, _Float16 *out_lo) {
    const int G = n_heads / n_kv;
    const int nch = (max_seq + kCh - 1) / kCh;
    float *part_o = part;
    float *part_ml = part + (size_t)batch * n_kv * nch * G * kHd;
    dim3 g1(nch, n_kv, batch), g2(n_heads, batch);
#define ANEHIP_ATTN_CASE(GG)                                                                                   \
    case GG:                                                                                                   \
        hipLaunchKernelGGL(attn_partial_kernel<GG>, g1, dim3(kThreads), 0, stream, mix, q_norm, k_norm,        \
                           inv_freq, pos, k_cache, v_cache, max_seq, n_heads, n_kv, part_o, part_ml);         \
        ANEHIP_HIP_TRY(ctx->err, hipGetLastError());                                                           \
        hipLaunchKernelGGL(attn_combine_kernel<GG>, g2, dim3(kThreads), 0, stream, mix, pos, part_o, part_ml,  \
                           nch, n_heads, n_kv, out, out_hi, out_lo);                                          \
        ANEHIP_HIP_TRY(ctx->err, hipGetLastError());                                                           \
        return ANEHIP_OK;
    switch (G) {
        ANEHIP_ATTN_CASE(1)
        ANEHIP_ATTN_CASE(2)
        ANEHIP_ATTN_CASE(4)
        default:
            return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "attention: %d query heads per kv head (1, 2 or 4)", G);
    }
#undef ANEHIP_ATTN_CASE
}

}  // namespace anehip
