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
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kWord3 = 0x00020000;  // raw buffer resource word 3 (gfx9 family)
constexpr float kPScale = 16384.0f;  // 2^14: probabilities in the PV MFMA operands

// LDS row of V^T (one head dim, 64 positions = 8 chunks of 8): chunk c of
// row D sits at slot c ^ swz(D), which keeps both the transposing writes (8
// lanes: rows 8p + d, p varying) and the MFMA operand reads (8 lanes: 8
// consecutive rows) free of bank conflicts.
__device__ __forceinline__ int vt_slot(int D, int c) { return c ^ ((D ^ (D >> 3)) & 7); }

// fp32 x 8 -> fp16 hi / lo with hi + lo ~= x (|error| <= 2^-22 |x|)
__device__ __forceinline__ void split8(const float *x, h8v &hi, h8v &lo) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
        hi[e] = (_Float16)x[e];
        lo[e] = (_Float16)(x[e] - (float)hi[e]);
    }
}

// grid = (chunks, n_kv_heads, batch); chunk c takes the live tiles
// chunk_tiles() gives it.  mix: per sequence [q_full | k | v] rows (K-split
// partial slices); q_full is [n_heads][q(256) | gate(256)].
//
// Per tile, on MFMA (v_mfma_f32_16x16x32_f16; operands A[i][k] / B[k][j] in
// lane i (j) + 16 (k / 8), element k % 8; D[i][j] in lane j + 16 (i / 4),
// element i % 4):
//  * scores S[pos][head] = K q^T / 16: wave w takes positions 16w..16w+15;
//    its K fragments are loaded straight from the cache (A: lane l = row
//    16w + l % 16, dims 32s + 8 (l / 16) of k-step s), q as fp16 hi + lo
//    B fragments (columns = the G query heads, others zero), so K is read
//    once for all G heads;
//  * online softmax per head across the 4 waves (LDS);
//  * O[head][dim] += P V: A = P (fp16 hi + lo of the probabilities), B = V
//    from an LDS copy of the tile transposed to [dim][pos] (each thread holds
//    an 8 x 8 block of V -- rows 8 rb .. +7, dims 8p .. +7 -- and transposes
//    it in registers); wave w takes dims 64w..64w+63.
// The next tiles' K / V loads are in flight while a tile is processed; the
// buffer resources cover positions [0, pos) only, so rows >= pos read zeros
// without a memory access (row pos takes this step's k / v), which also makes
// the prefetch of a tile past the chunk free.  One
// unnormalised partial per (chunk, query head) with its running max and sum.
//
// Cache addressing: row b's cache is at cache_off + b * row_stride halves
// (decode: every row its own sequence; prefill: row_stride 0, every row a
// token of one sequence whose K / V rows the prefill append kernel wrote
// before this launch -- then `append` is false and no row is written here).
template <int G>
__global__ __launch_bounds__(kThreads) void attn_partial_kernel(
    MixIn mix, const float *__restrict__ q_norm, const float *__restrict__ k_norm,
    const float *__restrict__ inv_freq, const uint32_t *__restrict__ pos_arr, __half *__restrict__ k_cache,
    __half *__restrict__ v_cache, int max_seq, int n_heads, int n_kv, float *__restrict__ part_o,
    float *__restrict__ part_ml, size_t cache_off, size_t row_stride, bool append) {
    __shared__ __align__(16) _Float16 vt[kHd * kCh];  // V^T of the tile, swizzled chunks
    __shared__ __align__(16) float qs[G][kHd];
    __shared__ __align__(16) h8v qf[8][2][64];         // q B fragments: k-step, hi / lo, lane
    __shared__ __align__(16) float pt[G][kCh];        // probabilities of the tile
    __shared__ __align__(16) __half knew[kHd], vnew[kHd];
    // per-tile maxima and sums of the 16 (wave, lane group) pieces of each
    // head's column, [piece][head]: combined after the barrier, no shuffles
    __shared__ float rmax[16][16], rsum[16][16], rscale[16];
    __shared__ float qmax[G];  // largest |q| / 16 of each query head (range-safe q fragments)

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int li = lane & 15, lg = lane >> 4;  // MFMA operand row / column, k group
    const int vp = t & 31, vrb = t >> 5;       // V block: dims 8 vp .., rows 8 vrb ..
    const int c = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const uint32_t pos = pos_arr[b];
    const int len = (int)pos + 1;
    const int nch = gridDim.x;
    int tb, te;  // tiles [tb, te)
    if (!chunk_tiles(len, nch, c, &tb, &te)) return;  // uniform exit: nothing of this sequence here
    const size_t cache_base = cache_off + (size_t)b * row_stride + (size_t)kvh * max_seq * kHd;
    const bool has_new = (int)pos < te * kCh;  // this chunk holds the current position
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(k_cache + cache_base, 0, (int)pos * kHd * 2, kWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(v_cache + cache_base, 0, (int)pos * kHd * 2, kWord3);
    // K fragments of this wave's 16 rows; V block of this thread.  A tile
    // past the chunk is loaded from row kFar (>= pos: zeros, no memory access),
    // so every step issues the same loads.
    const int kFar = max_seq;
    auto load_k = [&](u32x4 *kr, int row0) {
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int off = ((row0 + 16 * wave + li) * kHd + 32 * s + 8 * lg) * 2;
            kr[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, 0));
        }
    };
    auto load_v = [&](u32x4 *vr, int row0) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int off = ((row0 + 8 * vrb + i) * kHd + 8 * vp) * 2;
            vr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, 0));
        }
    };
    auto row_of = [&](int ti) { return ti < te ? ti * kCh : kFar; };
    // the first tile's loads (and the second's K) go out before the q / k
    // preparation
    u32x4 ka[8], kb[8], vr[8];
    load_k(ka, tb * kCh);
    load_v(vr, tb * kCh);
    load_k(kb, row_of(tb + 1));

    // q heads of this kv group: wave w < G prepares head kvh*G + w
    if (wave < G) {
        const int h = kvh * G + wave;
        float q4[4];
        norm_rope_head(mix, b, h * 2 * kHd, q_norm, inv_freq, pos, lane, q4);
        *reinterpret_cast<float4 *>(&qs[wave][4 * lane]) = make_float4(q4[0], q4[1], q4[2], q4[3]);
        const float qm = wave_max64(fmaxf(fmaxf(fabsf(q4[0]), fabsf(q4[1])), fmaxf(fabsf(q4[2]), fabsf(q4[3]))));
        if (lane == 0) qmax[wave] = qm * 0.0625f;
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
    // q B fragments (lane l: head l % 16, dims 32s + 8 (l / 16) ..), scaled by
    // 1/sqrt(256) = 1/16 (exact) and by 2^-qe per head (qe from the head's
    // largest value, so that fp16 neither overflows nor loses the low bits;
    // the scores are scaled back by 2^qe), as fp16 hi + lo; 4 (k-step, lane)
    // pairs per thread
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int e = t + 256 * j, fs = e >> 6, fl = e & 63, fh = fl & 15, fg = fl >> 4;
        float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (fh < G) {
            const int qe = group_exp(qmax[fh]);
            const float4 a = *reinterpret_cast<const float4 *>(&qs[fh][32 * fs + 8 * fg]);
            const float4 bq = *reinterpret_cast<const float4 *>(&qs[fh][32 * fs + 8 * fg + 4]);
            const float qv[8] = {a.x, a.y, a.z, a.w, bq.x, bq.y, bq.z, bq.w};
#pragma unroll
            for (int i = 0; i < 8; i++) x[i] = ldexpf(qv[i] * 0.0625f, -qe);
        }
        split8(x, qf[fs][0][fl], qf[fs][1][fl]);
    }
    lds_barrier();
    // scores of head li come out scaled by 2^-qe (li < G)
    const int qe_li = li < G ? group_exp(qmax[li]) : 0;

    // per head li (< G): running max / sum; PV accumulators of dim block db:
    // rows = heads 4 lg .. 4 lg + 3, column = dim 64 wave + 16 db + li
    float m_run = -INFINITY, l_run = 0.f;
    f32x4 o[4] = {};
    // tile ti with K in kr and V in vr; refills vr with tile ti + 1's V right
    // after storing it, and kr with tile ti + 2's K right after the scores
    auto process = [&](u32x4 *kr, int ti) {
        const int row0 = ti * kCh;
        // this step's row: K from knew, V from vnew (loaded as zeros)
        if (row0 + 16 * wave + li == (int)pos) {
#pragma unroll
            for (int s = 0; s < 8; s++) kr[s] = *reinterpret_cast<const u32x4 *>(&knew[32 * s + 8 * lg]);
        }
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (row0 + 8 * vrb + i == (int)pos) vr[i] = *reinterpret_cast<const u32x4 *>(&vnew[8 * vp]);
        // V block -> V^T rows 8 vp + d, chunk vrb
#pragma unroll
        for (int d = 0; d < 8; d++) {
            const int w = d >> 1;
            u32x4 col;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t x0 = vr[2 * k][w], x1 = vr[2 * k + 1][w];
                col[k] = (d & 1) ? ((x0 >> 16) | (x1 & 0xffff0000u)) : ((x0 & 0xffffu) | (x1 << 16));
            }
            const int D = 8 * vp + d;
            *reinterpret_cast<u32x4 *>(&vt[D * kCh + 8 * vt_slot(D, vrb)]) = col;
        }
        load_v(vr, row_of(ti + 1));
        // scores of positions 16 wave + 4 lg + e, head li
        f32x4 sc = {};
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const h8v a = __builtin_bit_cast(h8v, kr[s]);
            sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[s][0][lane], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[s][1][lane], sc, 0, 0, 0);
        }
        load_k(kr, row_of(ti + 2));
        const int p0 = row0 + 16 * wave + 4 * lg;
        float sv[4];
#pragma unroll
        for (int e = 0; e < 4; e++) sv[e] = p0 + e < len ? ldexpf(sc[e], qe_li) : -INFINITY;
        rmax[4 * wave + lg][li] = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        lds_barrier();
        float tm = rmax[0][li];
#pragma unroll
        for (int j = 1; j < 16; j++) tm = fmaxf(tm, rmax[j][li]);
        const float mn = fmaxf(m_run, tm);     // finite for li < G: the tile has a valid row
        const float scale = expf(m_run - mn);  // 0 on the first tile
        float pe[4], ps = 0.f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            pe[e] = p0 + e < len ? expf(sv[e] - mn) : 0.0f;
            ps += pe[e];
        }
        rsum[4 * wave + lg][li] = ps;
        if (wave == 0 && lane < 16) rscale[lane] = scale;
        if (li < G) *reinterpret_cast<float4 *>(&pt[li][16 * wave + 4 * lg]) = make_float4(pe[0], pe[1], pe[2], pe[3]);
        lds_barrier();
        float ts[4];
#pragma unroll
        for (int w = 0; w < 4; w++)
            ts[w] = (rsum[4 * w][li] + rsum[4 * w + 1][li]) + (rsum[4 * w + 2][li] + rsum[4 * w + 3][li]);
        l_run = l_run * scale + ((ts[0] + ts[1]) + (ts[2] + ts[3]));
        m_run = mn;
        // PV: rescale the rows (heads 4 lg + e), then P (hi + lo) times V^T
        float rs[4];
#pragma unroll
        for (int e = 0; e < 4; e++) rs[e] = 4 * lg + e < G ? rscale[4 * lg + e] : 0.0f;
#pragma unroll
        for (int db = 0; db < 4; db++)
#pragma unroll
            for (int e = 0; e < 4; e++) o[db][e] *= rs[e];
        // probabilities (<= 1) times 2^14 as fp16 hi + lo: the low bits of
        // small probabilities stay out of fp16's subnormal range; the
        // partial output is scaled back by 2^-14 at the end
        h8v ph[2], pl[2];
#pragma unroll
        for (int s = 0; s < 2; s++) {
            float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (li < G) {
                const float4 a = *reinterpret_cast<const float4 *>(&pt[li][32 * s + 8 * lg]);
                const float4 bq = *reinterpret_cast<const float4 *>(&pt[li][32 * s + 8 * lg + 4]);
                x[0] = a.x * kPScale; x[1] = a.y * kPScale; x[2] = a.z * kPScale; x[3] = a.w * kPScale;
                x[4] = bq.x * kPScale; x[5] = bq.y * kPScale; x[6] = bq.z * kPScale; x[7] = bq.w * kPScale;
            }
            split8(x, ph[s], pl[s]);
        }
#pragma unroll
        for (int db = 0; db < 4; db++) {
            const int D = 64 * wave + 16 * db + li;
#pragma unroll
            for (int s = 0; s < 2; s++) {
                const h8v bv = *reinterpret_cast<const h8v *>(&vt[D * kCh + 8 * vt_slot(D, 4 * s + lg)]);
                o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[s], bv, o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[s], bv, o[db], 0, 0, 0);
            }
        }
        lds_barrier();  // vt / pt / rmax are rewritten by the next tile
    };
    // K in two register buffers (a tile's K is in flight during the tile
    // before it), V in one.  Pairs of tiles, then the last one
    int ti = tb;
    while (ti + 1 < te) {
        process(ka, ti);
        process(kb, ti + 1);
        ti += 2;
    }
    if (ti < te) process(ka, ti);
    // lane (lg, li): heads 4 lg + e, dims 64 wave + 16 db + li
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int hh = 4 * lg + e;
        if (hh < G) {
            const size_t slot = (((size_t)b * n_kv + kvh) * nch + c) * G + hh;
#pragma unroll
            for (int db = 0; db < 4; db++) part_o[slot * kHd + 64 * wave + 16 * db + li] = o[db][e] * (1.0f / kPScale);
        }
    }
    if (wave == 0 && lane < G) {
        const size_t slot = (((size_t)b * n_kv + kvh) * nch + c) * G + lane;
        part_ml[slot * 2] = m_run;
        part_ml[slot * 2 + 1] = l_run;
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
    const float4 gate = mix.at4(b, h * 2 * kHd + kHd + 4 * l);  // independent of the partials
    // maximum over the chunks
    float mx = -INFINITY;
    for (int cc = t; cc < nc; cc += kThreads) mx = fmaxf(mx, part_ml[((base + cc) * G + hh) * 2]);
    mx = wave_max64(mx);
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
#define ANEHIP_ATTN_CASE(GG)                                                                                   \
    case GG:                                                                                                   \
        hipLaunchKernelGGL(attn_partial_kernel<GG>, g1, dim3(kThreads), 0, stream, mix, q_norm, k_norm,        \
                           inv_freq, pos, k_cache, v_cache, max_seq, n_heads, n_kv, part_o, part_ml,          \
                           cache_off, row_stride, append);                                                    \
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
