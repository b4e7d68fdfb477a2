// attention.hip — GQA decode attention over an fp16 KV cache for gfx950.
//
// Replaces q_gate_split, rmsnorm_gated (q/k norm use), rope_apply, the KV
// append gpu_memcpys, sdpa_causal and sigmoid_gate (crates/engine/metal/
// attention.metal:9-121, deltanet.metal:184-220; dispatched at
// gpu_full_decode.rs:628-903) and the CPU core of full_attn_decode_step
// (crates/engine/src/deltanet.rs:565-669).
//
// Split-K ("flash-decoding"): the positions 0..pos of one sequence are cut
// into tiles of 64 and chunks of tiles_per_chunk() tiles (at most 128 chunks
// at the cache's capacity); one workgroup per (chunk, kv head, sequence)
// streams its tiles' K and V rows once for all G query heads that share the
// kv head (the next tile's loads in flight while the current one is used),
// with an online softmax, and writes an unnormalised partial output with its
// running max and sum.  attn_combine_kernel merges the chunks with a
// log-sum-exp rescale and applies sigmoid(gate).  Chunks past the sequence's
// length exit at once, so one launch shape (sized for the cache capacity)
// serves every position and can be captured in a graph while pos lives in
// device memory.
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

// Barrier for LDS traffic only: waves do not wait for their outstanding
// global loads (the next tile's K / V) here.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kPer = (kCh * kHd / 8) / kThreads;  // 16-byte vectors of a 64-row tile per thread
constexpr int kWord3 = 0x00020000;               // raw buffer resource word 3 (gfx9 family)

// K and V rows of one 64-position tile into registers: vector q = i * 256 + t
// is row q / 32, 16-byte part q % 32.  The buffer resources cover positions
// [0, pos) of this sequence and kv head only, so rows >= pos (the current
// row, whose k / v come from this step, and rows past it) read zeros
// without a memory access and without a branch.
__device__ __forceinline__ void load_kv_tile(u32x4 *kr, u32x4 *vr, __amdgpu_buffer_rsrc_t krs,
                                             __amdgpu_buffer_rsrc_t vrs, int row0, int t) {
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int q = i * kThreads + t;
        const int off = ((row0 + (q >> 5)) * kHd + (q & 31) * 8) * 2;
        kr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, 0));
        vr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, 0));
    }
}

// grid = (chunks, n_kv_heads, batch); a chunk is `tpw` tiles of 64 positions
// (tiles_per_chunk()).  mix: per sequence [q_full | k | v] rows (K-split
// partial slices); q_full is [n_heads][q(256) | gate(256)].  The workgroup
// walks its tiles with the next tile's K / V loads in flight while the
// current one is used, keeping per query head (wave) an online-softmax
// running max, sum and output; it writes one unnormalised partial.
template <int G>
__global__ __launch_bounds__(kThreads) void attn_partial_kernel(
    MixIn mix, const float *__restrict__ q_norm, const float *__restrict__ k_norm,
    const float *__restrict__ inv_freq, const uint32_t *__restrict__ pos_arr, __half *__restrict__ k_cache,
    __half *__restrict__ v_cache, int max_seq, int n_heads, int n_kv, int tpw, float *__restrict__ part_o,
    float *__restrict__ part_ml) {
    __shared__ float qs[G][kHd];
    __shared__ __half tile[kCh * kRowH];
    __shared__ __half knew[kHd], vnew[kHd];
    __shared__ float probs[G][kCh];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int c = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const uint32_t pos = pos_arr[b];
    const int len = (int)pos + 1;
    const int tb = c * tpw, te = min(tb + tpw, (len + kCh - 1) / kCh);  // tiles [tb, te)
    if (tb >= te) return;  // uniform exit: nothing of this sequence here
    const int nch = gridDim.x;
    const size_t cache_base = ((size_t)b * n_kv + kvh) * (size_t)max_seq * kHd;
    const bool has_new = (int)pos < te * kCh;  // this chunk holds the current position
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(k_cache + cache_base, 0, (int)pos * kHd * 2, kWord3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(v_cache + cache_base, 0, (int)pos * kHd * 2, kWord3);

    // the first tile's loads go out before the q / k preparation
    u32x4 ka[kPer], va[kPer], kb[kPer], vb[kPer];
    load_kv_tile(ka, va, krs, vrs, tb * kCh, t);

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
    lds_barrier();

    // tile: 64 rows x 32 vectors of 16 bytes; row pos takes this step's k / v
    auto store_tile = [&](const u32x4 *reg, const __half *fresh, int row0) {
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            const int q = i * kThreads + t;
            const int r = q >> 5, part = q & 31;
            u32x4 v = reg[i];
            if (row0 + r == (int)pos) v = *reinterpret_cast<const u32x4 *>(fresh + part * 8);
            *reinterpret_cast<u32x4 *>(&tile[r * kRowH + part * 8]) = v;
        }
    };
    const float sdiv = sqrtf((float)kHd);
    // per query head (wave < G): running max, sum and output dims 4l..4l+3
    float m_run = -INFINITY, l_run = 0.f, o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
    auto process = [&](const u32x4 *kr, const u32x4 *vr, int ti) {
        const int row0 = ti * kCh;
        store_tile(kr, knew, row0);
        lds_barrier();
        // scores: wave = query head of the group, lane = position in the tile
        if (wave < G) {
            const int p = row0 + lane;
            // 8 independent partial sums (dims d % 8), added pairwise at the end
            float dp[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            const __half *krow = &tile[lane * kRowH];
#pragma unroll 4
            for (int d = 0; d < kHd; d += 8) {
                u32x4 kv8 = *reinterpret_cast<const u32x4 *>(krow + d);
                const float4 qa = *reinterpret_cast<const float4 *>(&qs[wave][d]);
                const float4 qb = *reinterpret_cast<const float4 *>(&qs[wave][d + 4]);
                const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
                const __half2 *h2 = reinterpret_cast<const __half2 *>(&kv8);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float2 kf = __half22float2(h2[e]);
                    dp[2 * e] += qv[2 * e] * kf.x;
                    dp[2 * e + 1] += qv[2 * e + 1] * kf.y;
                }
            }
            const float dot = ((dp[0] + dp[1]) + (dp[2] + dp[3])) + ((dp[4] + dp[5]) + (dp[6] + dp[7]));
            const float sc = p < len ? dot / sdiv : -INFINITY;
            const float mn = fmaxf(m_run, wave_max(sc));  // finite: the tile has a valid row
            const float scale = expf(m_run - mn);         // 0 on the first tile
            const float e = p < len ? expf(sc - mn) : 0.0f;
            l_run = l_run * scale + wave_sum(e);
            o0 *= scale;
            o1 *= scale;
            o2 *= scale;
            o3 *= scale;
            m_run = mn;
            probs[wave][lane] = e;
        }
        lds_barrier();
        store_tile(vr, vnew, row0);
        lds_barrier();
        // PV: wave = query head, lane = 4 consecutive dims
        if (wave < G) {
            // rows past the sequence have zero probability (and zero V), so
            // all 64 rows are summed: two independent chains, even / odd rows
            float e0 = 0.f, e1 = 0.f, e2 = 0.f, e3 = 0.f;
#pragma unroll 8
            for (int p = 0; p < kCh; p += 2) {
                const float2 pr = *reinterpret_cast<const float2 *>(&probs[wave][p]);
                const __half2 *va2 = reinterpret_cast<const __half2 *>(&tile[p * kRowH + 4 * lane]);
                const __half2 *vb2 = reinterpret_cast<const __half2 *>(&tile[(p + 1) * kRowH + 4 * lane]);
                const float2 a = __half22float2(va2[0]), bb = __half22float2(va2[1]);
                const float2 c = __half22float2(vb2[0]), dd = __half22float2(vb2[1]);
                o0 += pr.x * a.x;
                o1 += pr.x * a.y;
                o2 += pr.x * bb.x;
                o3 += pr.x * bb.y;
                e0 += pr.y * c.x;
                e1 += pr.y * c.y;
                e2 += pr.y * dd.x;
                e3 += pr.y * dd.y;
            }
            o0 += e0;
            o1 += e1;
            o2 += e2;
            o3 += e3;
        }
        lds_barrier();  // the tile is rewritten by the next K
    };
    // two register buffers.  Steady state: two tiles per trip with both next
    // loads real and unconditional (every path into a trip carries the same
    // loads, so the vmcnt waits stay exact); then the last one or two tiles.
    int ti = tb;
    while (ti + 2 < te) {
        load_kv_tile(kb, vb, krs, vrs, (ti + 1) * kCh, t);
        process(ka, va, ti);
        load_kv_tile(ka, va, krs, vrs, (ti + 2) * kCh, t);
        process(kb, vb, ti + 1);
        ti += 2;
    }
    if (ti + 1 < te) {
        load_kv_tile(kb, vb, krs, vrs, (ti + 1) * kCh, t);
        process(ka, va, ti);
        process(kb, vb, ti + 1);
    } else {
        process(ka, va, ti);
    }
    if (wave < G) {
        const size_t slot = (((size_t)b * n_kv + kvh) * nch + c) * G + wave;
        *reinterpret_cast<float4 *>(part_o + slot * kHd + 4 * lane) = make_float4(o0, o1, o2, o3);
        if (lane == 0) {
            part_ml[slot * 2] = m_run;
            part_ml[slot * 2 + 1] = l_run;
        }
    }
}

// grid = (n_heads, batch), 256 threads: thread (g = t / 64, l = t % 64) takes
// dims 4l..4l+3 of chunks g, g + 4, g + 8, ...; merges them with a log-sum-exp
// rescale against the maximum over all chunks, adds the 4 groups through
// LDS, normalises and multiplies by sigmoid(gate) (deltanet.rs:667-669).
// out: [batch][n_heads * 256] fp32, or fragment-order fp16 hi/lo planes
// out_hi / out_lo when out_hi is not null.
template <int G>
__global__ __launch_bounds__(kThreads) void attn_combine_kernel(MixIn mix, const uint32_t *__restrict__ pos_arr,
                                                                const float *__restrict__ part_o,
                                                                const float *__restrict__ part_ml, int nch, int tpw,
                                                                int n_heads, int n_kv, float *__restrict__ out,
                                                                _Float16 *__restrict__ out_hi,
                                                                _Float16 *__restrict__ out_lo) {
    __shared__ float red[4];
    __shared__ float4 accs[4][64];
    __shared__ float dens[4][64];
    const int t = threadIdx.x, g = t >> 6, l = t & 63, h = blockIdx.x, b = blockIdx.y;
    const int kvh = h / G, hh = h % G;
    const int len = (int)pos_arr[b] + 1;
    const int nc = ((len + kCh - 1) / kCh + tpw - 1) / tpw;  // active chunks
    const size_t base = ((size_t)b * n_kv + kvh) * nch;
    const float4 gate = mix.at4(b, h * 2 * kHd + kHd + 4 * l);  // independent of the partials
    // maximum over the chunks
    float mx = -INFINITY;
    for (int cc = t; cc < nc; cc += kThreads) mx = fmaxf(mx, part_ml[((base + cc) * G + hh) * 2]);
    mx = wave_max(mx);
    if (l == 0) red[g] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // this group's chunks, 4 per trip with their loads issued together
    float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
    float den = 0.f;
    int cc = g;
    for (; cc + 12 < nc; cc += 16) {
        float4 o4[4];
        float m4[4], l4[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const size_t slot = (base + cc + 4 * i) * G + hh;
            o4[i] = *reinterpret_cast<const float4 *>(part_o + slot * kHd + 4 * l);
            m4[i] = part_ml[slot * 2];
            l4[i] = part_ml[slot * 2 + 1];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float w = expf(m4[i] - M);
            num = make_float4(num.x + w * o4[i].x, num.y + w * o4[i].y, num.z + w * o4[i].z, num.w + w * o4[i].w);
            den += w * l4[i];
        }
    }
    for (; cc < nc; cc += 4) {
        const size_t slot = (base + cc) * G + hh;
        const float4 o = *reinterpret_cast<const float4 *>(part_o + slot * kHd + 4 * l);
        const float w = expf(part_ml[slot * 2] - M);
        num = make_float4(num.x + w * o.x, num.y + w * o.y, num.z + w * o.z, num.w + w * o.w);
        den += w * part_ml[slot * 2 + 1];
    }
    accs[g][l] = num;
    dens[g][l] = den;
    __syncthreads();
    if (g != 0) return;
    float4 s = accs[0][l];
    float dsum = dens[0][l];
#pragma unroll
    for (int k = 1; k < 4; k++) {
        const float4 o = accs[k][l];
        s = make_float4(s.x + o.x, s.y + o.y, s.z + o.z, s.w + o.w);
        dsum += dens[k][l];
    }
    const float gv[4] = {gate.x, gate.y, gate.z, gate.w};
    const float sv[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int d = 4 * l + i;
        const float v = (sv[i] / dsum) * (1.0f / (1.0f + expf(-gv[i])));
        if (out_hi) {
            const size_t o = xf_index(b, h * kHd + d);
            const _Float16 hi = (_Float16)v;
            out_hi[o] = hi;
            out_lo[o] = (_Float16)(v - (float)hi);
        } else {
            out[(size_t)b * n_heads * kHd + (size_t)h * kHd + d] = v;
        }
    }
}

// Tiles of 64 positions per chunk (workgroup): a power of two that keeps at
// most 128 chunks per sequence and kv head at the cache's capacity, so the
// combine merges at most 128 partials per head.
int tiles_per_chunk(int max_seq) {
    const int tiles = (max_seq + kCh - 1) / kCh;
    int tpw = 1;
    while ((tiles + tpw - 1) / tpw > 128) tpw *= 2;
    return tpw;
}

}  // namespace

size_t attn_partial_floats(int batch, int n_kv, int max_seq, int G) {
    const int tpw = tiles_per_chunk(max_seq);
    const size_t nch = (size_t)((max_seq + kCh - 1) / kCh + tpw - 1) / tpw;
    return (size_t)batch * n_kv * nch * G * (kHd + 2);
}

// part: workspace of attn_partial_floats() floats.
int launch_attention(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, int n_kv, int max_seq,
                     const MixIn &mix, const float *q_norm, const float *k_norm, const float *inv_freq,
                     const uint32_t *pos, __half *k_cache, __half *v_cache, float *part, float *out,
                     _Float16 *out_hi, _Float16 *out_lo) {
    const int G = n_heads / n_kv;
    const int tpw = tiles_per_chunk(max_seq);
    const int nch = ((max_seq + kCh - 1) / kCh + tpw - 1) / tpw;
    if ((size_t)max_seq * kHd * 2 >= (size_t)1 << 30)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "attention: max_seq %d too large", max_seq);
    float *part_o = part;
    float *part_ml = part + (size_t)batch * n_kv * nch * G * kHd;
    dim3 g1(nch, n_kv, batch), g2(n_heads, batch);
#define ANEHIP_ATTN_CASE(GG)                                                                                   \
    case GG:                                                                                                   \
        hipLaunchKernelGGL(attn_partial_kernel<GG>, g1, dim3(kThreads), 0, stream, mix, q_norm, k_norm,        \
                           inv_freq, pos, k_cache, v_cache, max_seq, n_heads, n_kv, tpw, part_o, part_ml);    \
        ANEHIP_HIP_TRY(ctx->err, hipGetLastError());                                                           \
        hipLaunchKernelGGL(attn_combine_kernel<GG>, g2, dim3(kThreads), 0, stream, mix, pos, part_o, part_ml,  \
                           nch, tpw, n_heads, n_kv, out, out_hi, out_lo);                                     \
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
