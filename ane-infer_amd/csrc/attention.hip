// attention.hip — GQA decode attention over an fp16 KV cache for gfx950.
//
// Replaces q_gate_split, rmsnorm_gated (q/k norm use), rope_apply, the KV
// append gpu_memcpys, sdpa_causal and sigmoid_gate (crates/engine/metal/
// attention.metal:9-121, deltanet.metal:184-220; dispatched at
// gpu_full_decode.rs:628-903) and the CPU core of full_attn_decode_step
// (crates/engine/src/deltanet.rs:565-669).
//
// Split-K ("flash-decoding"): the positions 0..pos of one sequence are cut
// into tiles of 64, and the live tiles are spread evenly over the launch's
// chunks (chunk_count(): at most 128 per sequence and kv head, about one
// workgroup per CU over the whole batch); one workgroup per (chunk, kv head,
// sequence) streams its tiles' K and V rows once for all G query heads that
// share the kv head (the next tile's loads in flight while the current one is
// used), with an online softmax, and writes an unnormalised partial output
// with its running max and sum.  attn_combine_kernel merges the chunks with a
// log-sum-exp rescale and applies sigmoid(gate).  Each workgroup derives its
// tile range from the device-resident position (chunk_tiles()), so the work
// follows the live length, not the cache's capacity, while one launch shape
// serves every position and can be captured in a graph; with fewer live
// tiles than chunks the chunks past the tile count exit at once.
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

// RMSNorm (eps 1e-6, deltanet.rs:575-598) + RoPE (deltanet.rs:600-623) of one
// 256-dim head by one wave: lane l owns dims 4l..4l+3 = rotary pairs 2l, 2l+1.
// The same arithmetic as the decode kernel's preparation (rsqrt, one sincos
// per pair), so prefill and decode append identical k rows.
__device__ __forceinline__ void norm_rope_head(const MixIn &mix, int b, int base, const float *__restrict__ w,
                                               const float *__restrict__ inv_freq, uint32_t pos, int lane,
                                               float *dst) {
    float4 x = mix.at4(b, base + 4 * lane);
    float ss = wave_sum(x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w);
    const float inv_rms = rsqrtf(ss / (float)kHd + 1e-6f);
    float4 wv = *reinterpret_cast<const float4 *>(w + 4 * lane);
    float a0 = (x.x * inv_rms) * wv.x, a1 = (x.y * inv_rms) * wv.y;
    float a2 = (x.z * inv_rms) * wv.z, a3 = (x.w * inv_rms) * wv.w;
    const float fpos = (float)pos;
    float s0, c0, s1, c1;
    sincosf(fpos * inv_freq[2 * lane], &s0, &c0);
    sincosf(fpos * inv_freq[2 * lane + 1], &s1, &c1);
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
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kWord3 = 0x00020000;  // raw buffer resource word 3 (gfx9 family)
constexpr float kPScale = 16384.0f;  // 2^14: probabilities in the PV MFMA operands
// Cache-policy bit nt of the K / V cache loads, for launches whose caches
// (capacity) reach kNtKvBytes: each cached row is read once per step and the
// caches of a batch exceed the L2s and the MALL.  Measured on MI355X (caches
// rotated past the MALL): batch 32 ctx 1k / 8k / 32k 19.1 / 94-98 / 364-369
// -> 17.1 / 82.3 / 307.3 us, batch 1 ctx 32k 18.6 -> 17.4, batch 1 ctx 1k
// 6.8 -> 7.0; batch-1 decode ctx 1k / 8k / 32k with the bit on every launch
// 1248 / 1241 / 1166 tok/s against 1254 / 1245 / 1130 with it on none.
constexpr int kCpolNt = 2;
constexpr size_t kNtKvBytes = (size_t)32 << 20;

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// grid = (chunks, n_kv_heads, batch); chunk c takes the live tiles
// [tb, te) of 64 positions that chunk_tiles() gives it.  mix: per
// sequence [q_full | k | v] rows (K-split partial slices); q_full is
// [n_heads][q(256) | gate(256)].
//
// Wave w takes positions 16 w .. 16 w + 15 of every tile and keeps its own
// online softmax and output for them; the 4 waves merge once, at the end.
// Per tile and wave, on MFMA (16 x 16 x K f16 forms: operands A[i][k] /
// B[k][j] in lane i (j) + 16 (k / (K / 4)), elements k % (K / 4); D[i][j]
// in lane j + 16 (i / 4), element i % 4):
//  * scores S[pos][head] = K q^T / 16 (K = 32): A = the wave's 16 K rows,
//    loaded straight from the cache (lane l: row l % 16, dims 32 s + 8 (l /
//    16) of k-step s), B = q as fp16 hi + lo fragments (columns = the G
//    query heads, others zero), so K is read once for all G heads;
//  * lane l then holds the scores of head l % 16 at positions 4 (l / 16) ..
//    + 3: the max and sum over the wave's 16 positions are two lane swaps
//    (v_permlane16_swap / v_permlane32_swap), no LDS and no barrier;
//  * O[head][dim] += P V (K = 16): those probabilities (x 2^14, fp16 hi +
//    lo) are already the A operand; B = V rows 4 (l / 16) .. + 3 of the
//    wave, loaded as 8-byte pieces (dims 64 q + 4 (l % 16) .. + 3), and MFMA
//    (q, c) takes element c of each piece, so its output column l % 16 is
//    dim 64 q + 4 (l % 16) + c: 16 MFMA column blocks cover the 256 dims
//    with no transpose of V.
// The next tile's K / V loads are in flight while a tile is processed; the
// buffer resources cover positions [0, pos) only, so rows >= pos read zeros
// without a memory access (row pos takes this step's k / v), which also makes
// the prefetch of a tile past the chunk free.  One unnormalised partial per
// (chunk, query head) with its running max and sum.
//
// With one or two tiles per workgroup (batch 1 at short contexts) the kernel
// is a chain of dependent steps on one wave per SIMD, so the q / k
// preparation issues every input load before the position is known, shares
// one sincos per rotary pair and writes the q fragments straight from the
// wave that normalised the head.
//
// Cache addressing: row b's cache is at cache_off + b * row_stride halves
// (decode: every row its own sequence; prefill: row_stride 0, every row a
// token of one sequence whose K / V rows the prefill append kernel wrote
// before this launch -- then `append` is false and no row is written here).
template <int G, bool NT>
__global__ __launch_bounds__(kThreads) void attn_partial_kernel(
    MixIn mix, const float *__restrict__ q_norm, const float *__restrict__ k_norm,
    const float *__restrict__ inv_freq, const uint32_t *__restrict__ pos_arr, __half *__restrict__ k_cache,
    __half *__restrict__ v_cache, int max_seq, int n_heads, int n_kv, float *__restrict__ part_o,
    float *__restrict__ part_ml, size_t cache_off, size_t row_stride, bool append) {
    __shared__ __align__(16) h8v qf[8][2][64];
    __shared__ __align__(16) __half knew[kHd], vnew[kHd];
    __shared__ int qexp[G];
    __shared__ __align__(16) float ob[4][G][kHd];
    __shared__ float wm[4][G], wl[4][G];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int c = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    // inputs that do not depend on the position first: this wave's q head
    // (wave < G) or k / v rows (wave G % 4, used by the chunk holding pos),
    // the norm weights and the RoPE frequencies
    const bool is_q = wave < G, is_k = wave == G % 4;
    const int hq = kvh * G + (wave < G ? wave : 0);
    const int kin = n_heads * 2 * kHd + kvh * kHd;
    const int vin = n_heads * 2 * kHd + n_kv * kHd + kvh * kHd;
    float4 aq[8], ak[8], av[8];
    {
        const float *r0 = mix.p + (size_t)b * mix.stride + 4 * lane;
#pragma unroll
        for (int q = 0; q < 8; q++)
            if (q < mix.kp) {
                const float *rq = r0 + (size_t)q * mix.split;
                if (is_q) aq[q] = *reinterpret_cast<const float4 *>(rq + hq * 2 * kHd);
                if (is_k) {
                    ak[q] = *reinterpret_cast<const float4 *>(rq + kin);
                    av[q] = *reinterpret_cast<const float4 *>(rq + vin);
                }
            }
    }
    const float4 wq = *reinterpret_cast<const float4 *>(q_norm + 4 * lane);
    const float4 wk = *reinterpret_cast<const float4 *>(k_norm + 4 * lane);
    const float2 fr = *reinterpret_cast<const float2 *>(inv_freq + 2 * lane);
    const uint32_t pos = pos_arr[b];
    const int len = (int)pos + 1;
    const int nch = gridDim.x;
    int tb, te;  // tiles [tb, te)
    if (!chunk_tiles(len, nch, c, &tb, &te)) return;  // uniform exit: nothing of this sequence here
    const size_t cache_base = cache_off + (size_t)b * row_stride + (size_t)kvh * max_seq * kHd;
    const bool has_new = (int)pos < te * kCh;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(k_cache + cache_base, 0, (int)pos * kHd * 2, kWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(v_cache + cache_base, 0, (int)pos * kHd * 2, kWord3);
    const int kFar = max_seq;
    auto load_k = [&](u32x4 *kr, int row0) {
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int off = ((row0 + 16 * wave + li) * kHd + 32 * s + 8 * lg) * 2;
            kr[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, NT ? kCpolNt : 0));
        }
    };
    // V rows row0 + 16 wave + 4 lg + r, dims 64 q + 4 li .. + 3 in vr[4 q + r]
    auto load_v = [&](u32x2 *vr, int row0) {
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int off = ((row0 + 16 * wave + 4 * lg + r) * kHd + 64 * q + 4 * li) * 2;
                vr[4 * q + r] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(vrs, off, 0, NT ? kCpolNt : 0));
            }
    };
    auto row_of = [&](int ti) { return ti < te ? ti * kCh : kFar; };
    u32x4 ka[8], kb[8];
    u32x2 va[16], vb[16];
    load_k(ka, tb * kCh);
    load_v(va, tb * kCh);
    load_k(kb, row_of(tb + 1));
    load_v(vb, row_of(tb + 1));

    // preparation, every input load issued first: wave w < G normalises and
    // rotates q head kvh G + w and writes its MFMA B fragments (scaled by
    // 1/16 and 2^-qe, fp16 hi + lo); in the chunk holding pos, wave G % 4
    // also prepares this step's k (RMSNorm + RoPE) and v, rounded to fp16.
    const bool do_q = is_q, do_k = has_new && is_k;
    // rows of the q fragments that belong to no head are zero
    for (int e = t; e < 8 * 64; e += kThreads) {
        const int fl = e & 63;
        if ((fl & 15) >= G) {
            qf[e >> 6][0][fl] = h8v{};
            qf[e >> 6][1][fl] = h8v{};
        }
    }
    float sn0, cs0, sn1, cs1;
    sincosf((float)pos * fr.x, &sn0, &cs0);
    sincosf((float)pos * fr.y, &sn1, &cs1);
    // slices in ascending order; the GEMMs at batch > 1 split K up to 16
    // ways, slices past the 8 held in registers are loaded here
    auto sum4 = [&](const float4 *a, int off) {
        float4 x = a[0];
#pragma unroll
        for (int q = 1; q < 8; q++)
            if (q < mix.kp) x = make_float4(x.x + a[q].x, x.y + a[q].y, x.z + a[q].z, x.w + a[q].w);
        for (int q = 8; q < mix.kp; q++) {
            const float4 v = *reinterpret_cast<const float4 *>(
                mix.p + (size_t)b * mix.stride + 4 * lane + (size_t)q * mix.split + off);
            x = make_float4(x.x + v.x, x.y + v.y, x.z + v.z, x.w + v.w);
        }
        return x;
    };
    auto norm_rope = [&](float4 x, float4 wv, float *dst) {
        const float ss = wave_sum(x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w);
        const float inv_rms = rsqrtf(ss / (float)kHd + 1e-6f);
        const float a0 = (x.x * inv_rms) * wv.x, a1 = (x.y * inv_rms) * wv.y;
        const float a2 = (x.z * inv_rms) * wv.z, a3 = (x.w * inv_rms) * wv.w;
        dst[0] = a0 * cs0 - a1 * sn0;
        dst[1] = a0 * sn0 + a1 * cs0;
        dst[2] = a2 * cs1 - a3 * sn1;
        dst[3] = a2 * sn1 + a3 * cs1;
    };
    if (do_q) {
        float q4[4];
        norm_rope(sum4(aq, hq * 2 * kHd), wq, q4);
        const float qm = wave_max64(fmaxf(fmaxf(fabsf(q4[0]), fabsf(q4[1])), fmaxf(fabsf(q4[2]), fabsf(q4[3]))));
        const int qe = group_exp(qm * 0.0625f);
        if (lane == 0) qexp[wave] = qe;
        // dims 4 lane .. + 3 = k-step lane / 8, lane group (lane % 8) / 2, half lane % 2
        h4v hi, lo;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float x = ldexpf(q4[i] * 0.0625f, -qe);
            hi[i] = (_Float16)x;
            lo[i] = (_Float16)(x - (float)hi[i]);
        }
        const int fs = lane >> 3, fl = wave + 16 * ((lane & 7) >> 1), half = lane & 1;
        reinterpret_cast<h4v *>(&qf[fs][0][fl])[half] = hi;
        reinterpret_cast<h4v *>(&qf[fs][1][fl])[half] = lo;
    }
    if (do_k) {
        float k4[4];
        norm_rope(sum4(ak, kin), wk, k4);
        const float4 v4 = sum4(av, vin);
        const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            knew[4 * lane + i] = __float2half_rn(k4[i]);
            vnew[4 * lane + i] = __float2half_rn(vv[i]);
        }
        if (append) {
            __half *kd = k_cache + cache_base + (size_t)pos * kHd + 4 * lane;
            __half *vd = v_cache + cache_base + (size_t)pos * kHd + 4 * lane;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kd[i] = knew[4 * lane + i];
                vd[i] = vnew[4 * lane + i];
            }
        }
    }
    lds_barrier();
    const int qe_li = li < G ? qexp[li] : 0;

    float m_run = -INFINITY, l_run = 0.f;
    f32x4 o[16] = {};
    auto process = [&](u32x4 *kr, u32x2 *vr, int ti, bool first) {
        const int row0 = ti * kCh;
        if (row0 + 16 * wave + li == (int)pos) {
#pragma unroll
            for (int s = 0; s < 8; s++) kr[s] = *reinterpret_cast<const u32x4 *>(&knew[32 * s + 8 * lg]);
        }
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (row0 + 16 * wave + 4 * lg + r == (int)pos) {
#pragma unroll
                for (int q = 0; q < 4; q++) vr[4 * q + r] = *reinterpret_cast<const u32x2 *>(&vnew[64 * q + 4 * li]);
            }
        f32x4 s0 = {}, s1 = {};
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const h8v a = __builtin_bit_cast(h8v, kr[s]);
            s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[s][0][lane], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[s][1][lane], s1, 0, 0, 0);
        }
        load_k(kr, row_of(ti + 2));
        const int p0 = row0 + 16 * wave + 4 * lg;
        float sv[4];
#pragma unroll
        for (int e = 0; e < 4; e++) sv[e] = p0 + e < len ? ldexpf(s0[e] + s1[e], qe_li) : -INFINITY;
        const float tm = lanes_max4(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
        const float mn = fmaxf(m_run, tm);
        const float mref = mn == -INFINITY ? 0.0f : mn;
        const float scale = expf(m_run - mref);
        float pe[4], ps = 0.f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            pe[e] = (li < G && p0 + e < len) ? expf(sv[e] - mref) : 0.0f;
            ps += pe[e];
        }
        l_run = l_run * scale + lanes_sum4(ps);
        m_run = mn;
        float rs[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            rs[e] = e < G ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, scale), e)) : 0.0f;
        if (!first) {
#pragma unroll
            for (int k = 0; k < 16; k++)
#pragma unroll
                for (int e = 0; e < 4; e++) o[k][e] *= rs[e];
        }
        h4v ph, pl;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float x = pe[e] * kPScale;
            ph[e] = (_Float16)x;
            pl[e] = (_Float16)(x - (float)ph[e]);
        }
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                const int w = cc >> 1;
                const uint32_t x0 = vr[4 * q][w], x1 = vr[4 * q + 1][w], x2 = vr[4 * q + 2][w], x3 = vr[4 * q + 3][w];
                u32x2 bw;
                if (cc & 1) {
                    bw[0] = (x0 >> 16) | (x1 & 0xffff0000u);
                    bw[1] = (x2 >> 16) | (x3 & 0xffff0000u);
                } else {
                    bw[0] = (x0 & 0xffffu) | (x1 << 16);
                    bw[1] = (x2 & 0xffffu) | (x3 << 16);
                }
                const h4v bv = __builtin_bit_cast(h4v, bw);
                o[4 * q + cc] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, bv, o[4 * q + cc], 0, 0, 0);
                o[4 * q + cc] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, bv, o[4 * q + cc], 0, 0, 0);
            }
        load_v(vr, row_of(ti + 2));
    };
    process(ka, va, tb, true);
    int ti = tb + 1;
    while (ti + 1 < te) {
        process(kb, vb, ti, false);
        process(ka, va, ti + 1, false);
        ti += 2;
    }
    if (ti < te) process(kb, vb, ti, false);
    // merge the 4 waves: lanes 0-15 hold heads e < G, dims 64 q + 4 li + cc
    if (lane < G) {
        wm[wave][lane] = m_run;
        wl[wave][lane] = l_run;
    }
    if (lg == 0) {
#pragma unroll
        for (int e = 0; e < G; e++)
#pragma unroll
            for (int q = 0; q < 4; q++)
                *reinterpret_cast<float4 *>(&ob[wave][e][64 * q + 4 * li]) =
                    make_float4(o[4 * q][e], o[4 * q + 1][e], o[4 * q + 2][e], o[4 * q + 3][e]);
    }
    lds_barrier();
    for (int idx = t; idx < G * 64; idx += kThreads) {
        const int hh = idx >> 6, d4 = idx & 63;
        float M = wm[0][hh];
#pragma unroll
        for (int w = 1; w < 4; w++) M = fmaxf(M, wm[w][hh]);
        float L = 0.f;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float sw = expf(wm[w][hh] - M);
            const float4 v = *reinterpret_cast<const float4 *>(&ob[w][hh][4 * d4]);
            L += sw * wl[w][hh];
            acc = make_float4(acc.x + sw * v.x, acc.y + sw * v.y, acc.z + sw * v.z, acc.w + sw * v.w);
        }
        const size_t slot = (((size_t)b * n_kv + kvh) * nch + c) * G + hh;
        const float inv = 1.0f / kPScale;
        *reinterpret_cast<float4 *>(part_o + slot * kHd + 4 * d4) =
            make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
        if (d4 == 0) {
            part_ml[slot * 2] = M;
            part_ml[slot * 2 + 1] = L;
        }
    }
}

// Prefill: the k / v rows of T consecutive tokens of one sequence (row t at
// position pos_arr[t]) -- RMSNorm + RoPE of k, both rounded to fp16 -- written
// to the cache at cache_off, as the decode kernel appends one row.  grid =
// (n_kv, T), one wave.
__global__ __launch_bounds__(64) void attn_append_kernel(MixIn mix, const float *__restrict__ k_norm,
                                                         const float *__restrict__ inv_freq,
                                                         const uint32_t *__restrict__ pos_arr,
                                                         __half *__restrict__ k_cache, __half *__restrict__ v_cache,
                                                         size_t cache_off, int max_seq, int n_heads, int n_kv) {
    const int lane = threadIdx.x, kvh = blockIdx.x, b = blockIdx.y;
    const uint32_t pos = pos_arr[b];
    const int kin = n_heads * 2 * kHd + kvh * kHd;
    const int vin = n_heads * 2 * kHd + n_kv * kHd + kvh * kHd;
    float k4[4];
    norm_rope_head(mix, b, kin, k_norm, inv_freq, pos, lane, k4);
    const float4 v4 = mix.at4(b, vin + 4 * lane);
    const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
    const size_t o = cache_off + ((size_t)kvh * max_seq + pos) * kHd + 4 * lane;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        k_cache[o + i] = __float2half_rn(k4[i]);
        v_cache[o + i] = __float2half_rn(vv[i]);
    }
}

// grid = (n_heads, batch), 256 threads: thread (g = t / 64, l = t % 64) takes
// dims 4l..4l+3 of chunks g, g + 4, g + 8, ...; merges them with a log-sum-exp
// rescale against the maximum over all chunks, adds the 4 groups through
// LDS, normalises and multiplies by sigmoid(gate) (deltanet.rs:667-669).
// out: [batch][n_heads * 256] fp32, or range-safe fragment-order planes xp
// (Planes) when xp.hi is not null.
template <int G>
__global__ __launch_bounds__(kThreads) void attn_combine_kernel(MixIn mix, const uint32_t *__restrict__ pos_arr,
                                                                const float *__restrict__ part_o,
                                                                const float *__restrict__ part_ml, int nch,
                                                                int n_heads, int n_kv, float *__restrict__ out,
                                                                Planes xp) {
    __shared__ float red[4];
    __shared__ float4 accs[4][64];
    __shared__ float dens[4][64];
    const int t = threadIdx.x, g = t >> 6, l = t & 63, h = blockIdx.x, b = blockIdx.y;
    const int kvh = h / G, hh = h % G;
    const int len = (int)pos_arr[b] + 1;
    const int nc = active_chunks(len, nch);
    const size_t base = ((size_t)b * n_kv + kvh) * nch;
    // the gate's K-split slices (independent of the partials) and this
    // group's first 4 chunks (g, g + 4, g + 8, g + 12; the only ones at batch
    // 32) are loaded together, before the maximum is known
    float4 gq[8];
    {
        const float *g0 = mix.p + (size_t)b * mix.stride + h * 2 * kHd + kHd + 4 * l;
#pragma unroll
        for (int q = 0; q < 8; q++) gq[q] = *reinterpret_cast<const float4 *>(g0 + (size_t)min(q, mix.kp - 1) * mix.split);
    }
    float4 p4[4];
    float pm[4], pl[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const size_t slot = (base + min(g + 4 * i, nc - 1)) * G + hh;
        p4[i] = *reinterpret_cast<const float4 *>(part_o + slot * kHd + 4 * l);
        pm[i] = part_ml[slot * 2];
        pl[i] = part_ml[slot * 2 + 1];
    }
    float4 gate = gq[0];
#pragma unroll
    for (int q = 1; q < 8; q++)
        if (q < mix.kp) gate = make_float4(gate.x + gq[q].x, gate.y + gq[q].y, gate.z + gq[q].z, gate.w + gq[q].w);
    for (int q = 8; q < mix.kp; q++) {
        const float4 v = *reinterpret_cast<const float4 *>(mix.p + (size_t)b * mix.stride + h * 2 * kHd + kHd + 4 * l +
                                                           (size_t)q * mix.split);
        gate = make_float4(gate.x + v.x, gate.y + v.y, gate.z + v.z, gate.w + v.w);
    }
    // maximum over the chunks: each group's (the same in all its lanes), then
    // over the 4 groups
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; i++) mx = g + 4 * i < nc ? fmaxf(mx, pm[i]) : mx;
    for (int c2 = g + 16; c2 < nc; c2 += 4) mx = fmaxf(mx, part_ml[((base + c2) * G + hh) * 2]);
    if (l == 0) red[g] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // this group's chunks in order: the 4 loaded above, then 4 per trip with
    // their loads issued together
    float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
    float den = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (g + 4 * i < nc) {
            const float w = expf(pm[i] - M);
            num = make_float4(num.x + w * p4[i].x, num.y + w * p4[i].y, num.z + w * p4[i].z, num.w + w * p4[i].w);
            den += w * pl[i];
        }
    }
    int cc = g + 16;
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
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = (sv[i] / dsum) * (1.0f / (1.0f + expf(-gv[i])));
    if (xp.hi) {
        // the head is two 128-column groups: lanes 0-31 and 32-63
        const int e = group_exp(half_max32(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])))));
        h4v vh, vl;  // 4 consecutive columns of a fragment-order plane
        split4_scaled(v, e, vh, vl);
        const size_t o = xf_index(b, h * kHd + 4 * l, n_heads * kHd);
        *reinterpret_cast<h4v *>(xp.hi + o) = vh;
        *reinterpret_cast<h4v *>(xp.lo + o) = vl;
        if ((l & 31) == 0) xp.xe[xe_index(b, h * kHd + 4 * l, n_heads * kHd)] = (int8_t)e;
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) out[(size_t)b * n_heads * kHd + (size_t)h * kHd + 4 * l + i] = v[i];
    }
}

// Chunks per (sequence, kv head): at most 128, at most one per 64-position
// tile of the cache, and about one workgroup per CU over the launch
// (kAttnWorkgroups / (batch x kv heads): batch 32 with 2 kv heads 4 chunks,
// batch 1 with 2 kv heads 128, with 4 kv heads 64).  256 chunks at batch 1
// were slower at 32k (the o_proj prologue merges twice the partials:
// 1049 against 1064 tok/s).  Longer chunks at batch > 1 amortise each
// workgroup's q / k preparation and partial write (batch 32, capacity =
// context 1k / 8k / 32k: 20.6k / 15.4k / 8.4k tok/s at ~256 workgroups
// against 20.1–20.3k / 14.7–14.9k / 8.4k at ~2048).
int chunk_count(int max_seq, int batch, int n_kv) {
    const int tiles = (max_seq + kCh - 1) / kCh;
    const int fill = std::max(1, kAttnWorkgroups / std::max(1, batch * n_kv));
    return std::max(1, std::min(std::min(tiles, 128), fill));
}

}  // namespace

int attn_chunks(int max_seq, int batch, int n_kv) { return chunk_count(max_seq, batch, n_kv); }

size_t attn_partial_floats(int batch, int n_kv, int max_seq, int G) {
    return (size_t)batch * n_kv * chunk_count(max_seq, batch, n_kv) * G * (kHd + 2);
}

namespace {

int attention_impl(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, int n_kv, int max_seq,
                   const MixIn &mix, const float *q_norm, const float *k_norm, const float *inv_freq,
                   const uint32_t *pos, __half *k_cache, __half *v_cache, float *part, float *out, const Planes &xp,
                   size_t cache_off, size_t row_stride, bool append) {
    const int G = n_heads / n_kv;
    const int nch = chunk_count(max_seq, batch, n_kv);
    if ((size_t)max_seq * kHd * 2 >= (size_t)1 << 30)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "attention: max_seq %d too large", max_seq);
    float *part_o = part;
    float *part_ml = part + (size_t)batch * n_kv * nch * G * kHd;
    dim3 g1(nch, n_kv, batch), g2(n_heads, batch);
    // the caches this launch can read (prefill rows share one sequence's)
    const bool nt = (size_t)(row_stride ? batch : 1) * n_kv * max_seq * 2 * kHd * sizeof(__half) >= kNtKvBytes;
#define ANEHIP_ATTN_CASE(GG)                                                                                   \
    case GG:                                                                                                   \
        if (nt)                                                                                                \
            hipLaunchKernelGGL((attn_partial_kernel<GG, true>), g1, dim3(kThreads), 0, stream, mix, q_norm,    \
                               k_norm, inv_freq, pos, k_cache, v_cache, max_seq, n_heads, n_kv, part_o,       \
                               part_ml, cache_off, row_stride, append);                                       \
        else                                                                                                   \
            hipLaunchKernelGGL((attn_partial_kernel<GG, false>), g1, dim3(kThreads), 0, stream, mix, q_norm,   \
                               k_norm, inv_freq, pos, k_cache, v_cache, max_seq, n_heads, n_kv, part_o,       \
                               part_ml, cache_off, row_stride, append);                                       \
        ANEHIP_HIP_TRY(ctx->err, hipGetLastError());                                                           \
        if (!out && !xp.hi) return ANEHIP_OK; /* partials only */                                              \
        hipLaunchKernelGGL(attn_combine_kernel<GG>, g2, dim3(kThreads), 0, stream, mix, pos, part_o, part_ml,  \
                           nch, n_heads, n_kv, out, xp);                                                      \
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

}  // namespace

// part: workspace of attn_partial_floats() floats.
int launch_attention(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, int n_kv, int max_seq,
                     const MixIn &mix, const float *q_norm, const float *k_norm, const float *inv_freq,
                     const uint32_t *pos, __half *k_cache, __half *v_cache, float *part, float *out,
                     const Planes &xp) {
    return attention_impl(ctx, stream, batch, n_heads, n_kv, max_seq, mix, q_norm, k_norm, inv_freq, pos, k_cache,
                          v_cache, part, out, xp, 0, (size_t)n_kv * max_seq * kHd, true);
}

int launch_attention_prefill(anehip_ctx *ctx, hipStream_t stream, int rows, int n_heads, int n_kv, int max_seq,
                             const MixIn &mix, const float *q_norm, const float *k_norm, const float *inv_freq,
                             const uint32_t *pos, __half *k_cache, __half *v_cache, size_t cache_off, float *part,
                             const Planes &xp) {
    hipLaunchKernelGGL(attn_append_kernel, dim3(n_kv, rows), dim3(64), 0, stream, mix, k_norm, inv_freq, pos, k_cache,
                       v_cache, cache_off, max_seq, n_heads, n_kv);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return attention_impl(ctx, stream, rows, n_heads, n_kv, max_seq, mix, q_norm, k_norm, inv_freq, pos, k_cache,
                          v_cache, part, nullptr, xp, cache_off, 0, false);
}

}  // namespace anehip
