// deltanet.hip — fused Gated DeltaNet decode step for gfx950.
//
// Replaces conv1d_silu, the q/k gpu_memcpy split, l2_normalize_scale,
// compute_beta_decay and deltanet_recurrence (crates/engine/metal/
// deltanet.metal:16-156, dispatched at gpu_full_decode.rs:350-456) and the CPU
// core of deltanet_decode_step (crates/engine/src/deltanet.rs:444-512), and
// rmsnorm_gated in its DeltaNet use (deltanet.metal:184-220,
// deltanet.rs:517-533).
//
// One workgroup (one wave) per (sequence, head, 8-column slice of the value
// dim).  Every workgroup of a head recomputes the head's conv + SiLU + L2
// norm of q and k (256 channels, cheap) from the old conv window; each slice
// writes back the window of its own 8 v channels.  The q/k windows are read
// by all 16 slices of a head, so they are committed (shift + append) by the
// next kernel, dn_finish_kernel, after every slice has read them.
// The state slice S[h][0:128][c0:c0+8] is read once and written once:
//   S' = decay * S;  sk = S'^T k;  delta = beta (v - sk);
//   S'' = S' + k delta^T;  o = S''^T q
// which is the reference's per-head order (decay, recall, delta, rank-1
// update, query) with the three global passes of the Metal kernel fused into
// one read and one write of the 64 KiB head state.
#include "common.h"

namespace anehip {

namespace {

constexpr int kDk = 128;     // key dim == value dim (ssm_state_size)
constexpr int kCols = 32;    // value columns per workgroup
constexpr int kThreads = 256;
constexpr int kKsize = 4;    // conv width (ssm_conv_kernel)
constexpr int kWave = 64;

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float silu_ref(float x) { return x / (1.0f + expf(-x)); }


// Range-safe plane write (see Planes) of one head's gated-norm output: a
// head is one 128-column group, column c0 + t held by thread t < 128.  The
// group's exponent e comes from the caller, which takes the largest |value|
// along with the norm's sum of squares: |v| = inv_rms * |o * w * SiLU(g)|,
// so max |o * w * SiLU(g)| times inv_rms gives the group's binade (to a few
// ulps, which only moves the scaled maximum within [2^14, 2^15] by as much).
__device__ __forceinline__ void head_to_planes(float v, int b, int c0, int n, int e, const Planes &xp) {
    const int t = threadIdx.x;
    const size_t o = xf_index(b, c0 + t, n);
    split_scaled(v, e, xp.hi[o], xp.lo[o]);
    if (t == 0) xp.xe[xe_index(b, c0, n)] = (int8_t)e;
}

// grid = (dv / 32, n_heads, batch), 256 threads: a workgroup takes 32 value
// columns of one head (64 workgroups of 16 KiB of state for a batch-1 step of
// 16 heads).  Thread t holds rows 4 rg .. +3 (rg = t / 8) of columns
// c0 + 4 cq .. +3 (cq = t % 8) in registers.  mix / mbeta / malpha: the qkv,
// beta and alpha projections of each sequence ([3 chunk], [n_heads],
// [n_heads]), read as K-split partial slices (KP >= their number).
//
// Each lane convolves one q / k channel, row 4 rg + cq % 4 of q (cq < 4) or
// of k (cq >= 4), so a group of 8 lanes makes exactly the rows it holds and
// shares them through LDS within the wave (no barrier).  Column sums over
// the 128 rows: lanes l ^ 8, l ^ 16, l ^ 32 (the wave's 8 row groups) are
// added by lane exchanges, the 4 waves through LDS; the q / k L2 norms are
// applied to those sums (q and k stay raw in registers), and their sums of
// squares go through the same barrier as the recall.  Two barriers a step.
//
// COUNT: the q / k windows are committed by this kernel, with one zeroed
// counter per (sequence, head, thread): the same thread of every workgroup
// of a head reads the same window, counts itself in once its convolution
// has consumed that window, and the last one to count in (all others have
// read it by then) shifts the window, appends the new input and sets the
// counter back to zero.  Without COUNT the windows are left to dn_finish /
// the ssm_out GEMV's prologue.  The v windows (one workgroup each) are
// committed by their own thread.
template <int KP, bool COUNT>
__global__ __launch_bounds__(256) void deltanet_step_kernel(
    MixIn mix, MixIn mbeta, MixIn malpha, const float *__restrict__ conv_w, const float *__restrict__ ssm_a,
    const float *__restrict__ dt_bias, float *__restrict__ conv_state, float *__restrict__ S, float *__restrict__ out,
    int n_heads, uint32_t *__restrict__ count) {
    constexpr int NQ = 8, NT = 32 * NQ, NW = NT / kWave, COLS = 4 * NQ;
    __shared__ __align__(16) float qn[kDk], kn[kDk];
    __shared__ float vv[COLS];
    __shared__ __align__(16) float part[NW][COLS + 4];  // recall sums, then the q / k sums of squares
    __shared__ __align__(16) float part2[NW][COLS];     // query sums

    const int t = threadIdx.x, lane = t & (kWave - 1), wave = t / kWave;
    const int slice = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int chunk = n_heads * kDk;  // = dim
    const int C = 3 * chunk;
    const int c0 = slice * COLS;
    float *cs = conv_state + (size_t)b * C * kKsize;
    const int cq = t % NQ;  // column quad: columns c0 + 4cq .. +3
    const int rg = t / NQ;  // row group: rows 4rg .. 4rg+3
    const int row = 4 * rg + (cq & 3);
    const int ch = (cq < 4 ? 0 : chunk) + h * kDk + row;    // this lane's q / k channel
    const int chv = 2 * chunk + h * kDk + c0 + (t % COLS);  // v channel (t < COLS)

    // Every small input is loaded first and the state slice after it (vector
    // loads complete in order, so the conv and norms wait only for the small
    // loads while the state is in flight).
    f32x4 win = *reinterpret_cast<const f32x4 *>(cs + (size_t)ch * kKsize);
    f32x4 wk = *reinterpret_cast<const f32x4 *>(conv_w + (size_t)ch * kKsize);
    float xa[KP];
    mix.load<KP>(b, ch, xa);
    f32x4 winv = *reinterpret_cast<const f32x4 *>(cs + (size_t)chv * kKsize);
    f32x4 wkv = *reinterpret_cast<const f32x4 *>(conv_w + (size_t)chv * kKsize);
    float xv[KP], xb[KP], xal[KP];
    mix.load<KP>(b, chv, xv);
    mbeta.load<KP>(b, h, xb);
    malpha.load<KP>(b, h, xal);
    const float sa = ssm_a[h], dtb = dt_bias[h];
    asm volatile("" ::: "memory");  // keeps the state loads behind the small ones
    float *Sh = S + (((size_t)b * n_heads + h) * kDk) * kDk + c0 + 4 * cq;
    float4 s[4];
#pragma unroll
    for (int r = 0; r < 4; r++) s[r] = ld_nt4(Sh + (size_t)(4 * rg + r) * kDk);  // streamed: see deltanet_head_kernel
    // the arithmetic on the small inputs starts after the state loads were
    // issued (else it is scheduled above them, with its waits)
    asm volatile("" : "+v"(win), "+v"(wk)::"memory");
    asm volatile("" : "+v"(winv), "+v"(wkv)::"memory");
#pragma unroll
    for (int q = 0; q < KP; q++) asm volatile("" : "+v"(xa[q]), "+v"(xv[q]), "+v"(xb[q]), "+v"(xal[q]));

    // 1. conv + SiLU (conv_shift_and_append + conv_apply, deltanet_cache.rs:
    // 34-54) from the old window
    const auto conv = [](f32x4 w0, f32x4 k, float x) {
        float sum = 0.0f;
        sum += w0.y * k.x;
        sum += w0.z * k.y;
        sum += w0.w * k.z;
        sum += x * k.w;
        return silu_ref(sum);
    };
    const float xin = mix.add<KP>(xa);
    const float y = conv(win, wk, xin);
    (cq < 4 ? qn : kn)[row] = y;
    // this thread has consumed its window: count it in.  The atomic is issued
    // by every lane (no branch), so waits for the state loads issued before
    // it need not wait for it too.
    asm volatile("" ::"v"(y) : "memory");
    uint32_t old = 0;
    uint32_t *cnt = COUNT ? count + ((size_t)b * n_heads + h) * NT + t : nullptr;
    if (COUNT) old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float xvin = mix.add<KP>(xv);
    if (t < COLS) vv[t] = conv(winv, wkv, xvin);
    // deltanet.rs:474-480, by every thread (no shared copy needed)
    const float beta = 1.0f / (1.0f + expf(-mbeta.add<KP>(xb)));
    const float decay = expf(sa * logf(1.0f + expf(malpha.add<KP>(xal) + dtb)));
    // 2. the L2 norms (deltanet.rs:25-31, 461-467): q *= 1/sqrt(sum q^2 +
    // 1e-12) / sqrt(dk), k *= 1/sqrt(sum k^2 + 1e-12), applied to the sums
    // below.  The wave's sums of squares: its 32 q rows (lanes cq < 4, the
    // quad by DPP) and its 32 k rows (cq >= 4).
    float ss = dpp_add<0x4E>(dpp_add<0xB1>(y * y));
    ss = lanes_sum4(dpp_add<0x128>(ss));
    // column sums over the wave's 8 row groups (every lane gets its columns')
    const auto wave_cols = [&](float4 v) {
        return make_float4(lanes_sum4(dpp_add<0x128>(v.x)), lanes_sum4(dpp_add<0x128>(v.y)),
                           lanes_sum4(dpp_add<0x128>(v.z)), lanes_sum4(dpp_add<0x128>(v.w)));
    };
    // rows 4 rg .. +3 were written by this lane's group of 8, in this wave
    // (LDS accesses of one wave are performed in order)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float4 q4 = *reinterpret_cast<const float4 *>(&qn[4 * rg]);
    const float4 k4 = *reinterpret_cast<const float4 *>(&kn[4 * rg]);
    const float kr[4] = {k4.x, k4.y, k4.z, k4.w}, qr[4] = {q4.x, q4.y, q4.z, q4.w};

    // 3. S' = decay S, recall S'^T k over this thread's rows (raw k)
    float4 sk = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const float ki = kr[r];
        s[r].x *= decay; s[r].y *= decay; s[r].z *= decay; s[r].w *= decay;
        sk.x += s[r].x * ki; sk.y += s[r].y * ki; sk.z += s[r].z * ki; sk.w += s[r].w * ki;
    }
    sk = wave_cols(sk);
    if (lane < NQ) *reinterpret_cast<float4 *>(&part[wave][4 * cq]) = sk;
    if (lane == 0) part[wave][COLS] = ss;
    if (lane == 4) part[wave][COLS + 1] = ss;
    __syncthreads();
    // delta_j = beta (v_j - sk_j), every thread for its 4 columns (waves in order)
    float4 delta;
    float invq, invk;
    {
        float a[4] = {0.f, 0.f, 0.f, 0.f}, sq = 0.f, skk = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float4 p = *reinterpret_cast<const float4 *>(&part[w][4 * cq]);
            a[0] += p.x; a[1] += p.y; a[2] += p.z; a[3] += p.w;
            sq += part[w][COLS];
            skk += part[w][COLS + 1];
        }
        invq = (1.0f / sqrtf(sq + 1e-12f)) * (1.0f / sqrtf((float)kDk));
        invk = 1.0f / sqrtf(skk + 1e-12f);
        delta.x = beta * (vv[4 * cq + 0] - a[0] * invk);
        delta.y = beta * (vv[4 * cq + 1] - a[1] * invk);
        delta.z = beta * (vv[4 * cq + 2] - a[2] * invk);
        delta.w = beta * (vv[4 * cq + 3] - a[3] * invk);
    }
    // S'' = S' + k delta^T (written back), query S''^T q over this thread's rows (raw q)
    float4 so = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const float ki = kr[r] * invk, qi = qr[r];
        s[r].x += ki * delta.x; s[r].y += ki * delta.y; s[r].z += ki * delta.z; s[r].w += ki * delta.w;
        st_nt4(Sh + (size_t)(4 * rg + r) * kDk, s[r]);
        so.x += s[r].x * qi; so.y += s[r].y * qi; so.z += s[r].z * qi; so.w += s[r].w * qi;
    }
    so = wave_cols(so);
    if (lane < NQ) *reinterpret_cast<float4 *>(&part2[wave][4 * cq]) = so;
    // the window stores go out before the last barrier (issued at the end
    // they would lengthen the tail by their own latency)
    if (COUNT && old == gridDim.x - 1) {
        // q / k window: shift left, append the new input (deltanet_cache.rs:34-42)
        *reinterpret_cast<float4 *>(cs + (size_t)ch * kKsize) = make_float4(win.y, win.z, win.w, xin);
        __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // v window: shift left, append the new input
    if (t < COLS) *reinterpret_cast<float4 *>(cs + (size_t)chv * kKsize) = make_float4(winv.y, winv.z, winv.w, xvin);
    __syncthreads();
    if (t < COLS) {
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) o += part2[w][t];
        out[(size_t)b * chunk + h * kDk + c0 + t] = o * invq;
    }
}

// Runs after deltanet_step_kernel.  If `conv_state` is not null, commits the
// q/k conv windows of head h (shift left, append the new input:
// deltanet_cache.rs:34-42); if `heads` is not null, applies the per-head
// RMSNorm with ssm_norm and the SiLU(gate) product (deltanet.rs:517-533),
// written as fp32 (out) or as range-safe fragment-order planes (xp, the
// input format of the panel MFMA GEMM).  grid = (n_heads, batch), 128
// threads (one per element of the head).
__global__ __launch_bounds__(kDk) void dn_finish_kernel(MixIn mix, float *__restrict__ conv_state,
                                                        const float *__restrict__ heads, int gate_off,
                                                        const float *__restrict__ norm_w, float *__restrict__ out,
                                                        Planes xp, int n_heads, float eps) {
    __shared__ float red[2], mred[2];
    const int t = threadIdx.x, h = blockIdx.x, b = blockIdx.y;
    const int chunk = n_heads * kDk;
    if (conv_state) {
        float *cs = conv_state + (size_t)b * 3 * chunk * kKsize;
        const int cq = h * kDk + t, ck = chunk + h * kDk + t;
        float4 a = *reinterpret_cast<const float4 *>(cs + (size_t)cq * kKsize);
        float4 c = *reinterpret_cast<const float4 *>(cs + (size_t)ck * kKsize);
        *reinterpret_cast<float4 *>(cs + (size_t)cq * kKsize) = make_float4(a.y, a.z, a.w, mix.at(b, cq));
        *reinterpret_cast<float4 *>(cs + (size_t)ck * kKsize) = make_float4(c.y, c.z, c.w, mix.at(b, ck));
    }
    if (!heads) return;
    const float x = heads[(size_t)b * chunk + h * kDk + t];
    const float g = mix.at(b, gate_off + h * kDk + t);
    const float gs = g / (1.0f + expf(-g));
    float ss = wave_sum(x * x);
    const float wm = xp.hi ? wave_max64(fabsf(x * norm_w[t] * gs)) : 0.0f;
    if ((t & 63) == 0) {
        red[t >> 6] = ss;
        mred[t >> 6] = wm;
    }
    __syncthreads();
    const float ms = (red[0] + red[1]) / (float)kDk;
    const float inv_rms = 1.0f / sqrtf(ms + eps);
    const float v = ((x * inv_rms) * norm_w[t]) * gs;
    if (xp.hi) head_to_planes(v, b, h * kDk, chunk, group_exp(fmaxf(mred[0], mred[1]) * inv_rms), xp);
    else out[(size_t)b * chunk + h * kDk + t] = v;
}

// Batch > 1: one workgroup (256 threads) per (head, sequence) holding the
// whole 128 x 128 head state (thread: columns 4 cq .. +3, rows 16 rg .. +15),
// so the same step as deltanet_step_kernel can also commit all of the head's
// conv windows (no other workgroup reads them) and finish with the gated
// RMSNorm (deltanet.rs:517-533), written as fragment-order fp16 hi/lo planes
// for the panel GEMM; with `out` it writes the raw head outputs (fp32)
// instead.  grid = (n_heads, batch).  KP >= the K splits of the projections.
template <int KP>
__global__ __launch_bounds__(kThreads) void deltanet_head_kernel(
    MixIn mix, MixIn mbeta, MixIn malpha, const float *__restrict__ conv_w, const float *__restrict__ ssm_a,
    const float *__restrict__ dt_bias, float *__restrict__ conv_state, float *__restrict__ S, float *__restrict__ out,
    int gate_off, const float *__restrict__ norm_w, float eps, Planes xp, int n_heads) {
    __shared__ float qn[kDk], kn[kDk], vv[kDk];
    __shared__ __align__(16) float part[8][kDk];
    __shared__ float red[4], mred[2];

    const int t = threadIdx.x;
    const int h = blockIdx.x, b = blockIdx.y;
    const int chunk = n_heads * kDk;
    const int C = 3 * chunk;
    float *cs = conv_state + (size_t)b * C * kKsize;
    const int cq = t & 31, rg = t >> 5;
    float *Sh = S + (((size_t)b * n_heads + h) * kDk) * kDk + 4 * cq;

    // Every small input is loaded first and the state after it: vector loads
    // complete in order, so the conv, norms and gates wait only for the small
    // loads while the 64 KiB state is in flight.  Thread t convolves a q
    // (t < 128) or k channel, and the v channel t % 128 (kept by t < 128).
    const int e = t & (kDk - 1);
    const int ch = t < kDk ? h * kDk + t : chunk + h * kDk + e, chv = 2 * chunk + h * kDk + e;
    f32x4 win = *reinterpret_cast<const f32x4 *>(cs + (size_t)ch * kKsize);
    f32x4 wk = *reinterpret_cast<const f32x4 *>(conv_w + (size_t)ch * kKsize);
    f32x4 winv = *reinterpret_cast<const f32x4 *>(cs + (size_t)chv * kKsize);
    f32x4 wkv = *reinterpret_cast<const f32x4 *>(conv_w + (size_t)chv * kKsize);
    float xa[KP], xv[KP], xg[KP], xb[KP], xal[KP];
    mix.load<KP>(b, ch, xa);
    mix.load<KP>(b, chv, xv);
    mix.load<KP>(b, gate_off + h * kDk + e, xg);
    mbeta.load<KP>(b, h, xb);
    malpha.load<KP>(b, h, xal);
    const float sa = ssm_a[h], dtb = dt_bias[h], nw = out ? 0.0f : norm_w[e];
    asm volatile("" ::: "memory");  // keeps the state loads behind the small ones
    // The state is streamed with non-temporal loads and stores: each head's
    // 64 KiB is read and written once per step and the batch's states do not
    // fit the caches.  Measured on MI355X (states rotated past the MALL): 18.6
    // -> 13.8-14.1 us per step at batch 32, 7.6 -> 6.2 at batch 8 (plain
    // stores with non-temporal loads: 16.1 / 7.1; the reverse: no change).
    float4 s[16];
#pragma unroll
    for (int r = 0; r < 16; r++)
        s[r] = ld_nt4(Sh + (size_t)(16 * rg + r) * kDk);
    // the arithmetic on the small inputs starts here, after the state loads
    // were issued (else it is scheduled above them, with its waits)
    asm volatile("" : "+v"(win), "+v"(wk), "+v"(winv), "+v"(wkv)::"memory");
#pragma unroll
    for (int q = 0; q < KP; q++) asm volatile("" : "+v"(xa[q]), "+v"(xv[q]), "+v"(xb[q]), "+v"(xal[q]));

    // 1. conv + SiLU (conv_shift_and_append + conv_apply, deltanet_cache.rs:
    // 34-54); the windows are committed here
    const auto conv = [&](f32x4 w0, f32x4 k, float x, int c, bool write) {
        const float4 ns = make_float4(w0.y, w0.z, w0.w, x);
        float sum = 0.0f;
        sum += ns.x * k.x;
        sum += ns.y * k.y;
        sum += ns.z * k.z;
        sum += ns.w * k.w;
        if (write) *reinterpret_cast<float4 *>(cs + (size_t)c * kKsize) = ns;
        return silu_ref(sum);
    };
    {
        const float y = conv(win, wk, mix.add<KP>(xa), ch, true);
        const float sq = wave_sum(y * y);
        if ((t & 63) == 0) red[t >> 6] = sq;
        if (t < kDk) qn[t] = y;
        else kn[e] = y;
        if (t < kDk) vv[t] = conv(winv, wkv, mix.add<KP>(xv), chv, true);
    }
    // deltanet.rs:474-480, by every thread (no shared copy needed)
    const float beta = 1.0f / (1.0f + expf(-mbeta.add<KP>(xb)));
    const float decay = expf(sa * logf(1.0f + expf(malpha.add<KP>(xal) + dtb)));
    __syncthreads();
    // 2. L2 normalise (deltanet.rs:25-31, 461-467): x *= 1/sqrt(sum x^2 + 1e-12); q *= 1/sqrt(dk)
    if (t < kDk) {
        const float inv = 1.0f / sqrtf((red[0] + red[1]) + 1e-12f);
        const float scale = 1.0f / sqrtf((float)kDk);
        qn[t] = (qn[t] * inv) * scale;
    } else {
        const float inv = 1.0f / sqrtf((red[2] + red[3]) + 1e-12f);
        kn[e] = kn[e] * inv;
    }
    __syncthreads();

    // 3. S' = decay * S, partial recall sum_i S'_ij k_i over this thread's rows
    float4 sk = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const float ki = kn[16 * rg + r];
        s[r].x *= decay; s[r].y *= decay; s[r].z *= decay; s[r].w *= decay;
        sk.x += s[r].x * ki; sk.y += s[r].y * ki; sk.z += s[r].z * ki; sk.w += s[r].w * ki;
    }
    *reinterpret_cast<float4 *>(&part[rg][4 * cq]) = sk;
    __syncthreads();
    // delta_j = beta (v_j - sk_j), every thread for its 4 columns (fixed order)
    float4 delta;
    {
        float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int g = 0; g < 8; g++) {
            float4 p = *reinterpret_cast<const float4 *>(&part[g][4 * cq]);
            a[0] += p.x; a[1] += p.y; a[2] += p.z; a[3] += p.w;
        }
        delta.x = beta * (vv[4 * cq + 0] - a[0]);
        delta.y = beta * (vv[4 * cq + 1] - a[1]);
        delta.z = beta * (vv[4 * cq + 2] - a[2]);
        delta.w = beta * (vv[4 * cq + 3] - a[3]);
    }
    __syncthreads();  // part[] is reused below
    // S'' = S' + k delta^T (written back), partial query sum_i S''_ij q_i
    float4 so = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const float ki = kn[16 * rg + r], qi = qn[16 * rg + r];
        s[r].x += ki * delta.x; s[r].y += ki * delta.y; s[r].z += ki * delta.z; s[r].w += ki * delta.w;
        st_nt4(Sh + (size_t)(16 * rg + r) * kDk, s[r]);
        so.x += s[r].x * qi; so.y += s[r].y * qi; so.z += s[r].z * qi; so.w += s[r].w * qi;
    }
    *reinterpret_cast<float4 *>(&part[rg][4 * cq]) = so;
    __syncthreads();
    // 4. head output o_j (j = t < 128), then raw or gated-RMSNorm output
    float o = 0.f;
    if (t < kDk) {
#pragma unroll
        for (int g = 0; g < 8; g++) o += part[g][t];
    }
    if (out) {
        if (t < kDk) out[(size_t)b * chunk + h * kDk + t] = o;
        return;
    }
    const float gt = mix.add<KP>(xg);
    const float gs = gt / (1.0f + expf(-gt));
    const float ss = wave_sum(o * o);  // waves 2-3 contribute zeros
    const float wm = wave_max64(fabsf(o * nw * gs));
    __syncthreads();                   // red[] is reused
    if ((t & 63) == 0) {
        red[t >> 6] = ss;
        if (t < kDk) mred[t >> 6] = wm;  // waves 0-1 hold the head's outputs
    }
    __syncthreads();
    if (t >= kDk) return;
    const float inv_rms = 1.0f / sqrtf((red[0] + red[1]) / (float)kDk + eps);
    const float v = ((o * inv_rms) * nw) * gs;
    head_to_planes(v, b, h * kDk, chunk, group_exp(fmaxf(mred[0], mred[1]) * inv_rms), xp);
}

// Prefill: T consecutive tokens of one sequence (mix row t = token t), in
// three kernels.  Only the state is recurrent: the conv over time, the q / k
// L2 norms, v, beta and the decay of every token are independent, so
// dn_prep_kernel forms them for all (token, head) pairs at once; the scan then
// runs the recurrence alone; dn_scan_finish_kernel applies the gated RMSNorm
// and commits the conv windows.

// Token b's conv taps for channel ch: the last kKsize values of (the old
// window, the inputs of tokens 0..b) (conv_shift_and_append + conv_apply,
// deltanet_cache.rs:34-54), then SiLU.
template <int KP>
__device__ __forceinline__ float conv_token(const MixIn &mix, const float *__restrict__ cs,
                                            const float *__restrict__ conv_w, int ch, int b) {
    const f32x4 old = *reinterpret_cast<const f32x4 *>(cs + (size_t)ch * kKsize);
    const f32x4 wk = *reinterpret_cast<const f32x4 *>(conv_w + (size_t)ch * kKsize);
    float xs[kKsize][KP];
#pragma unroll
    for (int i = 0; i < kKsize; i++) mix.load<KP>(max(b - kKsize + 1 + i, 0), ch, xs[i]);
    const float ov[kKsize] = {old.x, old.y, old.z, old.w};
    const float kw[kKsize] = {wk.x, wk.y, wk.z, wk.w};
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kKsize; i++) {
        const int src = b - kKsize + 1 + i;  // < 0: from the old window
        sum += (src >= 0 ? mix.add<KP>(xs[i]) : ov[(kKsize + src) & (kKsize - 1)]) * kw[i];
    }
    return silu_ref(sum);
}

// grid = (n_heads, T), 256 threads: thread t forms channel t % 128 of q (t <
// 128) or k, normalised (deltanet.rs:25-31, 461-467), and threads t < 128 also
// v channel t; thread 0 the token's beta and decay (deltanet.rs:474-480).
// prep[(b * n_heads + h) * 384 + {0, 128, 256} + c] = q, k, v; bd[(b * n_heads
// + h) * 2 + {0, 1}] = beta, decay.
template <int KP>
__global__ __launch_bounds__(kThreads) void dn_prep_kernel(MixIn mix, MixIn mbeta, MixIn malpha,
                                                           const float *__restrict__ conv_w,
                                                           const float *__restrict__ ssm_a,
                                                           const float *__restrict__ dt_bias,
                                                           const float *__restrict__ cs, float *__restrict__ prep,
                                                           float *__restrict__ bd, int n_heads) {
    __shared__ float red[4];
    const int t = threadIdx.x, h = blockIdx.x, b = blockIdx.y;
    const int chunk = n_heads * kDk, e = t & (kDk - 1);
    const float y = conv_token<KP>(mix, cs, conv_w, t < kDk ? h * kDk + t : chunk + h * kDk + e, b);
    const float vy = t < kDk ? conv_token<KP>(mix, cs, conv_w, 2 * chunk + h * kDk + t, b) : 0.0f;
    const float sq = wave_sum(y * y);
    if ((t & 63) == 0) red[t >> 6] = sq;
    __syncthreads();
    float *out = prep + ((size_t)b * n_heads + h) * 3 * kDk;
    if (t < kDk) {
        const float inv = 1.0f / sqrtf((red[0] + red[1]) + 1e-12f);
        out[t] = (y * inv) * (1.0f / sqrtf((float)kDk));
        out[2 * kDk + t] = vy;
    } else {
        out[kDk + e] = y * (1.0f / sqrtf((red[2] + red[3]) + 1e-12f));
    }
    if (t == 0) {
        float xb[KP], xa[KP];
        mbeta.load<KP>(b, h, xb);
        malpha.load<KP>(b, h, xa);
        float *o = bd + ((size_t)b * n_heads + h) * 2;
        o[0] = 1.0f / (1.0f + expf(-mbeta.add<KP>(xb)));
        o[1] = expf(ssm_a[h] * logf(1.0f + expf(malpha.add<KP>(xa) + dt_bias[h])));
    }
}

// The recurrence is independent per value column j (recall sk_j, delta_j,
// column j of the rank-1 update and the query o_j), so a head is split over
// kDk / C single-wave workgroups of C columns each, grid = (kDk / C, n_heads).
// The workgroup copies its head's q and k, its columns' v and the tokens' beta
// and decay into LDS, kScanMaxT tokens at a time; the token loop then has no
// global load.  Lane l holds rows R (l % G) .. + R - 1 of column C g + l / G (G =
// 64 / C lanes per column, R = 128 / G rows per lane) in registers across all
// T steps (state read and written once per chunk); a sum over rows is 4
// interleaved partial sums of R / 4 rows, then a DPP sum over the column's G
// consecutive lanes.  Raw head outputs go to out[t][chunk].
constexpr int kScanCols = 4;
constexpr int kScanMaxT = 32;    // tokens staged in LDS at a time
constexpr int kScanMaxRows = 256;  // tokens per launch
constexpr int kDropOffset = 0x7ffffff0;  // buffer offset past any output: the store is dropped

// sum over each 16-lane row: row_ror 8, 4, 2, 1
__device__ __forceinline__ float sum16(float v) {
    return dpp_add<0x121>(dpp_add<0x122>(dpp_add<0x124>(dpp_add<0x128>(v))));
}

template <int C>
__global__ __launch_bounds__(kWave) void deltanet_scan_kernel(const float *__restrict__ prep,
                                                              const float *__restrict__ bd, float *__restrict__ S,
                                                              float *__restrict__ out, int n_heads, int T) {
    constexpr int G = kWave / C, R = kDk / G;
    static_assert(G == 8 || G == 16, "a column's lanes are summed within one DPP row");
    static_assert(C % 2 == 0 && C + 2 <= kWave, "lanes C, C + 1 carry beta and decay");
    __shared__ __align__(16) float qks[kScanMaxT][2 * kDk];  // q then k of each token
    __shared__ float exs[kScanMaxT][kWave];  // lanes 0..C-1: v of the columns, C, C+1: beta, decay
    const int l = threadIdx.x, h = blockIdx.y;
    const int chunk = n_heads * kDk;
    const int rgp = l % G, jl = l / G, j = blockIdx.x * C + jl;
    float *Sh = S + (size_t)h * kDk * kDk + j;
    float st[R];
#pragma unroll
    for (int r = 0; r < R; r++) st[r] = Sh[(size_t)(R * rgp + r) * kDk];
    const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(out, 0, 4 * T * chunk, 0x00020000);
    const auto colsum = [](float v) { return G == 16 ? sum16(v) : sum8(v); };
    // the tokens in sub-chunks of kScanMaxT, the state in registers throughout
    for (int c0 = 0; c0 < T; c0 += kScanMaxT) {
        if (c0) __syncthreads();  // the previous sub-chunk's reads of qks / exs are done
        // all loads of a half of the sub-chunk in flight at once (clamped to
        // the last token; slots past T are never read): lane l copies float4 l
        // of q | k, lanes 0..C-1 also v of column l, lanes >= C beta (even) /
        // decay (odd)
#pragma unroll
        for (int b0 = 0; b0 < kScanMaxT; b0 += kScanMaxT / 2) {
            float4 qk[kScanMaxT / 2];
            float ex[kScanMaxT / 2];
#pragma unroll
            for (int i = 0; i < kScanMaxT / 2; i++) {
                const int b = min(c0 + b0 + i, T - 1);
                const float *src = prep + ((size_t)b * n_heads + h) * 3 * kDk;
                qk[i] = reinterpret_cast<const float4 *>(src)[l];
                ex[i] = l < C ? src[2 * kDk + blockIdx.x * C + l] : bd[((size_t)b * n_heads + h) * 2 + (l & 1)];
            }
#pragma unroll
            for (int i = 0; i < kScanMaxT / 2; i++) {
                reinterpret_cast<float4 *>(qks[b0 + i])[l] = qk[i];
                exs[b0 + i][l] = ex[i];
            }
        }
        __syncthreads();
        const int te = min(kScanMaxT, T - c0);
        for (int bb = 0; bb < te; bb++) {
            const int b = c0 + bb;
            const float beta = exs[bb][C], decay = exs[bb][C + 1], v = exs[bb][jl];
            float kr[R], qr[R];
#pragma unroll
            for (int r = 0; r < R; r += 4) {
                const float4 k4 = *reinterpret_cast<const float4 *>(&qks[bb][kDk + R * rgp + r]);
                const float4 q4 = *reinterpret_cast<const float4 *>(&qks[bb][R * rgp + r]);
                kr[r] = k4.x, kr[r + 1] = k4.y, kr[r + 2] = k4.z, kr[r + 3] = k4.w;
                qr[r] = q4.x, qr[r + 1] = q4.y, qr[r + 2] = q4.z, qr[r + 3] = q4.w;
            }
            // S' = decay S; sk_j = sum_i S'_ij k_i
            float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int r = 0; r < R; r++) {
                st[r] *= decay;
                p[r & 3] += st[r] * kr[r];
            }
            const float sk = colsum((p[0] + p[1]) + (p[2] + p[3]));
            const float delta = beta * (v - sk);
            // S'' = S' + k delta^T; o_j = sum_i S''_ij q_i
#pragma unroll
            for (int r = 0; r < 4; r++) p[r] = 0.f;
#pragma unroll
            for (int r = 0; r < R; r++) {
                st[r] += kr[r] * delta;
                p[r & 3] += st[r] * qr[r];
            }
            const float o = colsum((p[0] + p[1]) + (p[2] + p[3]));
            // lanes of row group 0 store (the others' offset is past the buffer: dropped)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, o), orsrc,
                                                  rgp == 0 ? 4 * (b * chunk + h * kDk + j) : kDropOffset, 0, 0);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) Sh[(size_t)(R * rgp + r) * kDk] = st[r];
}

// After deltanet_scan_kernel: row b of the gated RMSNorm (deltanet.rs:517-533)
// of the raw head outputs to the planes, and (row 0's workgroups) the conv
// windows of the head's q, k and v channels after the T tokens: the last
// kKsize values of (old window, the T inputs).  grid = (n_heads, T), 128 threads.
template <int KP>
__global__ __launch_bounds__(kDk) void dn_scan_finish_kernel(MixIn mix, float *__restrict__ conv_state,
                                                             const float *__restrict__ heads, int gate_off,
                                                             const float *__restrict__ norm_w, Planes xp,
                                                             int n_heads, float eps, int T) {
    __shared__ float red[2], mred[2];
    const int t = threadIdx.x, h = blockIdx.x, b = blockIdx.y;
    const int chunk = n_heads * kDk;
    // every load first (partial slices clamped to the last one, window
    // sources clamped to row 0; unused values are discarded)
    float xg[KP];
    mix.load<KP>(b, gate_off + h * kDk + t, xg);
    const float x = heads[(size_t)b * chunk + h * kDk + t];
    if (b == 0) {
        f32x4 old[3];
        float xw[3][kKsize][KP];
#pragma unroll
        for (int c = 0; c < 3; c++) {
            old[c] = *reinterpret_cast<const f32x4 *>(conv_state + (size_t)(c * chunk + h * kDk + t) * kKsize);
#pragma unroll
            for (int i = 0; i < kKsize; i++) mix.load<KP>(max(T - kKsize + i, 0), c * chunk + h * kDk + t, xw[c][i]);
        }
#pragma unroll
        for (int c = 0; c < 3; c++) {
            const float ov[kKsize] = {old[c].x, old[c].y, old[c].z, old[c].w};
            float nv[kKsize];
#pragma unroll
            for (int i = 0; i < kKsize; i++) {
                const int src = T - kKsize + i;  // < 0: from the old window
                nv[i] = src >= 0 ? mix.add<KP>(xw[c][i]) : ov[(kKsize + src) & (kKsize - 1)];
            }
            *reinterpret_cast<f32x4 *>(conv_state + (size_t)(c * chunk + h * kDk + t) * kKsize) =
                f32x4{nv[0], nv[1], nv[2], nv[3]};
        }
    }
    const float g = mix.add<KP>(xg);
    const float gs = g / (1.0f + expf(-g));
    const float ss = wave_sum(x * x);
    const float wm = wave_max64(fabsf(x * norm_w[t] * gs));
    if ((t & 63) == 0) {
        red[t >> 6] = ss;
        mred[t >> 6] = wm;
    }
    __syncthreads();
    const float inv_rms = 1.0f / sqrtf((red[0] + red[1]) / (float)kDk + eps);
    const float v = ((x * inv_rms) * norm_w[t]) * gs;
    head_to_planes(v, b, h * kDk, chunk, group_exp(fmaxf(mred[0], mred[1]) * inv_rms), xp);
}

}  // namespace

int launch_deltanet_scan(anehip_ctx *ctx, hipStream_t stream, int rows, int n_heads, const MixIn &mix,
                         const MixIn &beta, const MixIn &alpha, const float *conv_w, const float *ssm_a,
                         const float *dt_bias, float *conv_state, float *S, float *prep, float *heads,
                         int gate_off, const float *norm_w, float eps, const Planes &xp) {
    const int kp = max(mix.kp, max(beta.kp, alpha.kp));
    if (kp > 16 || rows < 1 || rows > kScanMaxRows)
        return set_error(ctx->err, ANEHIP_EINVAL, "deltanet_scan: %d K splits (at most 16), %d rows (1..%d)", kp, rows,
                         kScanMaxRows);
    float *bd = prep + (size_t)rows * n_heads * 3 * kDk;
#define DN_SCAN(KP)                                                                                                  \
    hipLaunchKernelGGL(dn_prep_kernel<KP>, dim3(n_heads, rows), dim3(kThreads), 0, stream, mix, beta, alpha, conv_w, \
                       ssm_a, dt_bias, conv_state, prep, bd, n_heads);                                               \
    hipLaunchKernelGGL(deltanet_scan_kernel<kScanCols>, dim3(kDk / kScanCols, n_heads), dim3(kWave), 0, stream,     \
                       prep, bd, S, heads, n_heads, rows);                                                           \
    hipLaunchKernelGGL(dn_scan_finish_kernel<KP>, dim3(n_heads, rows), dim3(kDk), 0, stream, mix, conv_state, heads, \
                       gate_off, norm_w, xp, n_heads, eps, rows)
    if (kp <= 1) {
        DN_SCAN(1);
    } else if (kp <= 4) {
        DN_SCAN(4);
    } else {
        DN_SCAN(16);
    }
#undef DN_SCAN
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

namespace {

// The batch-1 step's deferred state updates (launch_deltanet_apply): grid =
// (kDk / kCols, n_heads, layers); thread (cq, rg) takes columns c0 + 4 cq ..
// + 3 and rows 4 rg .. + 3 of head h, as deltanet_step_kernel does, and
// applies S' = decay S, S'' = S' + k delta^T in that order; threads < 3 kCols
// commit the conv windows of the q, k and v channels of those columns.
__global__ __launch_bounds__(kThreads) void dn_apply_kernel(DnApplyTab tab, int n_heads, int d) {
    const int t = threadIdx.x, slice = blockIdx.x, h = blockIdx.y, l = blockIdx.z;
    float *S = tab.S[l];
    float *conv = tab.conv[l];
    const float *pend = tab.pend[l];
    const int c0 = slice * kCols;
    const int cq = t & 7, rg = t >> 3;
    const float decay = pend[2 * d + h];
    const float4 delta = *reinterpret_cast<const float4 *>(pend + h * kDk + c0 + 4 * cq);
    const float4 kv = *reinterpret_cast<const float4 *>(pend + d + h * kDk + 4 * rg);
    const float kr[4] = {kv.x, kv.y, kv.z, kv.w};
    float *Sh = S + (size_t)h * kDk * kDk + c0 + 4 * cq;
    float4 s[4];
#pragma unroll
    for (int r = 0; r < 4; r++) s[r] = ld_nt4(Sh + (size_t)(4 * rg + r) * kDk);  // streamed states
#pragma unroll
    for (int r = 0; r < 4; r++) {
        s[r].x *= decay; s[r].y *= decay; s[r].z *= decay; s[r].w *= decay;
        s[r].x += kr[r] * delta.x; s[r].y += kr[r] * delta.y; s[r].z += kr[r] * delta.z; s[r].w += kr[r] * delta.w;
        st_nt4(Sh + (size_t)(4 * rg + r) * kDk, s[r]);
    }
    if (t < 3 * kCols) {
        const int ch = (t / kCols) * d + h * kDk + c0 + t % kCols;
        float4 *w = reinterpret_cast<float4 *>(conv + (size_t)ch * kKsize);
        const float4 o = *w;
        *w = make_float4(o.y, o.z, o.w, pend[2 * d + n_heads + ch]);
    }
}

}  // namespace

int launch_deltanet_apply(anehip_ctx *ctx, hipStream_t stream, const DnApplyTab &tab, int n_heads, int dim) {
    if (tab.n <= 0 || tab.n > kMaxDnApplyLayers || dim != n_heads * kDk)
        return set_error(ctx->err, ANEHIP_EINVAL, "deltanet_apply: %d layers, dim %d, %d heads", tab.n, dim, n_heads);
    hipLaunchKernelGGL(dn_apply_kernel, dim3(kDk / kCols, n_heads, tab.n), dim3(kThreads), 0, stream, tab, n_heads,
                       dim);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_deltanet_head(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, const MixIn &mix,
                         const MixIn &beta, const MixIn &alpha, const float *conv_w, const float *ssm_a,
                         const float *dt_bias, float *conv_state, float *S, float *out, int gate_off,
                         const float *norm_w, float eps, const Planes &xp) {
    if (!out && !xp.hi) return set_error(ctx->err, ANEHIP_EINVAL, "deltanet_head: no output");
    const int kp = max(mix.kp, max(beta.kp, alpha.kp));
    if (kp > 16) return set_error(ctx->err, ANEHIP_EINVAL, "deltanet_head: %d K splits (at most 16)", kp);
    const dim3 grid(n_heads, batch), block(kThreads);
#define DN_HEAD(KP)                                                                                                  \
    hipLaunchKernelGGL(deltanet_head_kernel<KP>, grid, block, 0, stream, mix, beta, alpha, conv_w, ssm_a, dt_bias,   \
                       conv_state, S, out, gate_off, norm_w, eps, xp, n_heads)
    if (kp <= 1)
        DN_HEAD(1);
    else if (kp <= 4)
        DN_HEAD(4);
    else
        DN_HEAD(16);
#undef DN_HEAD
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_deltanet_step(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, const MixIn &mix,
                         const MixIn &beta, const MixIn &alpha, const float *conv_w, const float *ssm_a,
                         const float *dt_bias, float *conv_state, float *S, float *out, uint32_t *count) {
    const int kp = max(mix.kp, max(beta.kp, alpha.kp));
    if (kp > 16) return set_error(ctx->err, ANEHIP_EINVAL, "deltanet_step: %d K splits (at most 16)", kp);
    if (count && (size_t)batch * n_heads * 256 > (size_t)kDnCounters)
        return set_error(ctx->err, ANEHIP_EINVAL, "deltanet_step: %d x %d heads exceed the window counters", batch,
                         n_heads);
    // 32 value columns per 4-wave workgroup (64 workgroups at batch 1)
    const dim3 grid(kDk / 32, n_heads, batch), block(256);
#define DN_STEP(KP, C)                                                                                               \
    hipLaunchKernelGGL((deltanet_step_kernel<KP, C>), grid, block, 0, stream, mix, beta, alpha, conv_w, ssm_a,       \
                       dt_bias, conv_state, S, out, n_heads, count)
#define DN_STEP_KP(C)                                                                                                \
    if (kp <= 1)                                                                                                     \
        DN_STEP(1, C);                                                                                               \
    else if (kp <= 4)                                                                                                \
        DN_STEP(4, C);                                                                                               \
    else                                                                                                             \
        DN_STEP(16, C)
    if (count) {
        DN_STEP_KP(true);
    } else {
        DN_STEP_KP(false);
    }
#undef DN_STEP_KP
#undef DN_STEP
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_dn_finish(anehip_ctx *ctx, hipStream_t stream, int batch, int n_heads, const MixIn &mix,
                     float *conv_state, const float *heads, int gate_off, const float *norm_w, float *out,
                     const Planes &xp, float eps) {
    hipLaunchKernelGGL(dn_finish_kernel, dim3(n_heads, batch), dim3(kDk), 0, stream, mix, conv_state, heads, gate_off,
                       norm_w, out, xp, n_heads, eps);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

}  // namespace anehip
