// gemv.hip — Q8_0 / Q4_0 dequant-GEMV and small-batch GEMM for gfx950.
//
// Replaces the q8_gemv / q4_gemv Metal kernels (crates/engine/metal/
// q8_gemv.metal:15-87, q4_gemv.metal:25-98) and the CPU q8_gemv
// (crates/engine/src/q8_gemv.rs:130-148).  Same result: y[r] = sum over
// blocks b of scale(r,b) * sum_i q(r,b,i) * x[32b+i], fp32 accumulate.
//
// Work decomposition (wave64, bandwidth-bound):
//   * a "super-block" is 8 consecutive quant blocks of one row = 256 columns;
//     for Q8_0 that is 272 bytes (17 x 16 B), for Q4_0 144 bytes (9 x 16 B),
//     so rows of n = 256k columns start 16-byte aligned and a super-block
//     column of a 64-row tile is exactly 17 (or 9) KiB;
//   * a wave loads that tile with coalesced 16-byte-per-lane loads (each load
//     instruction covers contiguous row segments), stages it through LDS and
//     reads back one row per lane.  The activation values a lane needs are
//     then the same for all 64 lanes: they are wave-uniform (scalar) loads,
//     and every lane accumulates its own row with no cross-lane reduction;
//   * 4 waves of a workgroup take interleaved super-blocks of the same 64
//     rows and are reduced through LDS.  When there are too few row tiles to
//     fill the chip, K is split across workgroups, which write partial sums
//     to a workspace; a second pass adds them in fixed order, so results are
//     deterministic and no device-wide fence is needed.
#include "common.h"

namespace anehip {

namespace {

constexpr int kWave = 64;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <uint32_t T> struct QTraits;
template <> struct QTraits<ANEHIP_GGML_Q8_0> {
    static constexpr int kBlockBytes = 34;
    static constexpr int kSbBytes = 272;  // 8 blocks
    static constexpr int kSbVec = 17;     // 16-byte vectors per super-block
};
template <> struct QTraits<ANEHIP_GGML_Q4_0> {
    static constexpr int kBlockBytes = 18;
    static constexpr int kSbBytes = 144;
    static constexpr int kSbVec = 9;
};

__device__ __forceinline__ float half_at(const uint32_t *w, int off) {
    // off is even, so the two bytes never straddle a 32-bit word
    uint32_t bits = (w[off >> 2] >> ((off & 3) * 8)) & 0xffffu;
    return __half2float(__ushort_as_half((unsigned short)bits));
}

// ---------------------------------------------------------------------------
// Batch-1 GEMV input as int8 digits.  Each 32-column block of the input slice
// is held in LDS as x = 2^-sh (d0 + d1 / 128 + d2 / 16384) + e, with int8
// digits d0 = trunc(x 2^sh), d1 = trunc(frac 128), d2 = rint(frac' 128), and
// sh per block from its largest magnitude M (M 2^sh in [64, 128)), so |e| <=
// 2^-21 M.  A block's sum q . x (q8_gemv.rs:234-242: per block, then scaled
// by d) is then three exact int32 dot products over the int8 weights
// (v_dot4_i32_i8, 4 products per instruction) combined in fp32: about half
// the VALU work of one conversion and one FMA per weight, which was a third of
// the busy time of the large batch-1 GEMVs.  The result differs from the
// per-element fp32 sum by rounding only (both are within ~2^-21 of the exact
// sum relative to max|x| |q|).
// LDS per block: kXdWords dwords (digit planes 0, 1, 2; byte i of dword w is
// column 4 w + i) and a uint4 {2^-sh as float bits, 8 sum(d0), 8 sum(d1),
// 8 sum(d2)} (the sums serve Q4_0's -8 offset).  A block holding an inf or NaN
// gets zero digits and a NaN factor, so its rows come out NaN.
// ---------------------------------------------------------------------------
constexpr int kXdWords = 24;

// Digitises 4 consecutive columns v of the slice (float4 index i4); lanes
// 8 k .. 8 k + 7 of the wave must hold one block (i4 & 7 = lane & 7).  Every
// lane of the wave calls it (DPP needs all lanes active); only `store` lanes
// write.
template <int CTRL>
__device__ __forceinline__ int dpp_iadd(int v) {
    return v + __builtin_amdgcn_update_dpp(v, v, CTRL, 0xf, 0xf, false);
}

template <uint32_t T>
__device__ __forceinline__ void put_digits(float4 v, int i4, bool store, uint32_t *xd, uint4 *xq) {
    const float xv[4] = {v.x, v.y, v.z, v.w};
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) mx = fmaxf(mx, __builtin_isnan(xv[i]) ? INFINITY : fabsf(xv[i]));
    // the block's maximum over its 8 lanes on DPP (xor 1, xor 2, half-row mirror)
    mx = dpp_max<0x141>(dpp_max<0x4E>(dpp_max<0xB1>(mx)));
    const bool bad = mx == INFINITY;  // an inf or NaN in the block
    // mx in [2^(e-1), 2^e): mx 2^(7-e) in [64, 128); the smallest subnormals
    // keep sh at 149 so that 2^-sh stays representable
    const int sh = bad || mx == 0.0f ? 0 : min(7 - __builtin_amdgcn_frexp_expf(mx), 149);
    uint32_t p0 = 0, p1 = 0, p2 = 0;
    int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float y = bad ? 0.0f : ldexpf(xv[i], sh);  // |y| < 128
        const float f0 = truncf(y);
        const float r = (y - f0) * 128.0f;  // exact
        const float f1 = truncf(r);
        const float f2 = fminf(fmaxf(rintf((r - f1) * 128.0f), -127.0f), 127.0f);
        const int i0 = (int)f0, i1 = (int)f1, i2 = (int)f2;
        p0 |= ((uint32_t)i0 & 0xffu) << (8 * i);
        p1 |= ((uint32_t)i1 & 0xffu) << (8 * i);
        p2 |= ((uint32_t)i2 & 0xffu) << (8 * i);
        if constexpr (T == ANEHIP_GGML_Q4_0) {
            s0 += i0;
            s1 += i1;
            s2 += i2;
        }
    }
    if constexpr (T == ANEHIP_GGML_Q4_0) {
        s0 = dpp_iadd<0x141>(dpp_iadd<0x4E>(dpp_iadd<0xB1>(s0)));
        s1 = dpp_iadd<0x141>(dpp_iadd<0x4E>(dpp_iadd<0xB1>(s1)));
        s2 = dpp_iadd<0x141>(dpp_iadd<0x4E>(dpp_iadd<0xB1>(s2)));
    }
    if (store) {
        const int blk = i4 >> 3, w = i4 & 7;
        uint32_t *p = xd + blk * kXdWords + w;
        p[0] = p0;
        p[8] = p1;
        p[16] = p2;
        if (w == 0)
            xq[blk] = make_uint4(__float_as_uint(bad ? __builtin_nanf("") : ldexpf(1.0f, -sh)), (uint32_t)(8 * s0),
                                 (uint32_t)(8 * s1), (uint32_t)(8 * s2));
    }
}

// Digitises xs[0, len) (floats in LDS, len a multiple of 32) into xd / xq;
// the caller synchronises before and after.
template <uint32_t T, int NT>
__device__ __forceinline__ void digitize_lds(const float *xs, int len, uint32_t *xd, uint4 *xq) {
    const int n4 = len >> 2;
    for (int b4 = 0; b4 < n4; b4 += NT) {  // uniform trip count
        const int i4 = b4 + (int)threadIdx.x;
        const float4 v = reinterpret_cast<const float4 *>(xs)[min(i4, n4 - 1)];
        put_digits<T>(v, i4, i4 < n4, xd, xq);
    }
}

// The same in place: the digits overwrite xs itself (kXdWords dwords and a
// uint4 per block fit in the block's 32 floats), for kernels whose LDS
// budget has no room for a second copy.  Every value is read before any
// digit is written; the caller synchronises after.
template <uint32_t T, int NT, int MAXLEN>
__device__ __forceinline__ void digitize_lds_inplace(float *xs, int len) {
    constexpr int IT = MAXLEN / 4 / NT;
    const int n4 = len >> 2, t = (int)threadIdx.x;
    float4 v[IT];
#pragma unroll
    for (int i = 0; i < IT; i++) v[i] = reinterpret_cast<const float4 *>(xs)[min(t + i * NT, max(n4 - 1, 0))];
    __syncthreads();
    uint32_t *xd = reinterpret_cast<uint32_t *>(xs);
    uint4 *xq = reinterpret_cast<uint4 *>(xs + MAXLEN / 32 * kXdWords);
#pragma unroll
    for (int i = 0; i < IT; i++)
        if (i * NT < n4) put_digits<T>(v[i], t + i * NT, t + i * NT < n4, xd, xq);  // uniform condition
}

// One block's q . x from its digits, times 2^-sh (q: the block's quant
// vectors, 2 for Q8_0 with columns 0-15 and 16-31, 1 for Q4_0; xdb: the
// block's kXdWords digit dwords; xqv: its uint4).
template <uint32_t T>
__device__ __forceinline__ float block_dot_digits(const u32x4 *q, const uint32_t *xdb, const uint4 xqv) {
    const u32x4 *x4 = reinterpret_cast<const u32x4 *>(xdb);
    const u32x4 a0 = x4[0], b0 = x4[1], a1 = x4[2], b1 = x4[3], a2 = x4[4], b2 = x4[5];
    const uint32_t d0[8] = {a0.x, a0.y, a0.z, a0.w, b0.x, b0.y, b0.z, b0.w};
    const uint32_t d1[8] = {a1.x, a1.y, a1.z, a1.w, b1.x, b1.y, b1.z, b1.w};
    const uint32_t d2[8] = {a2.x, a2.y, a2.z, a2.w, b2.x, b2.y, b2.z, b2.w};
    int s0 = 0, s1 = 0, s2 = 0;
    if constexpr (T == ANEHIP_GGML_Q8_0) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t w4[4] = {q[h].x, q[h].y, q[h].z, q[h].w};
#pragma unroll
            for (int w = 0; w < 4; w++) {
                s0 = __builtin_amdgcn_sdot4((int)w4[w], (int)d0[4 * h + w], s0, false);
                s1 = __builtin_amdgcn_sdot4((int)w4[w], (int)d1[4 * h + w], s1, false);
                s2 = __builtin_amdgcn_sdot4((int)w4[w], (int)d2[4 * h + w], s2, false);
            }
        }
    } else {
        // byte i of the block: element i in the low nibble, i + 16 in the high
        // one (dequant.rs:12-25); nibbles are 0..15, the -8 comes off as 8 sum(d)
        const uint32_t w4[4] = {q[0].x, q[0].y, q[0].z, q[0].w};
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const int lo = (int)(w4[w] & 0x0f0f0f0fu), hi = (int)((w4[w] >> 4) & 0x0f0f0f0fu);
            s0 = __builtin_amdgcn_sdot4(lo, (int)d0[w], s0, false);
            s1 = __builtin_amdgcn_sdot4(lo, (int)d1[w], s1, false);
            s2 = __builtin_amdgcn_sdot4(lo, (int)d2[w], s2, false);
            s0 = __builtin_amdgcn_sdot4(hi, (int)d0[4 + w], s0, false);
            s1 = __builtin_amdgcn_sdot4(hi, (int)d1[4 + w], s1, false);
            s2 = __builtin_amdgcn_sdot4(hi, (int)d2[4 + w], s2, false);
        }
        s0 -= (int)xqv.y;
        s1 -= (int)xqv.z;
        s2 -= (int)xqv.w;
    }
    const float bs = fmaf((float)s2, 1.0f / 16384.0f, fmaf((float)s1, 1.0f / 128.0f, (float)s0));
    return bs * __uint_as_float(xqv.x);
}

// 4 dwords of a GGUF row starting at byte offset `off` (even; blocks are 34
// or 18 bytes, so a block's quants start 2 bytes into a dword for every
// second block): one v_alignbyte per dword when misaligned.
__device__ __forceinline__ u32x4 words_at(const uint32_t *w, int off) {
    u32x4 r;
    const int i = off >> 2;
    if ((off & 3) == 0) {
        r = u32x4{w[i], w[i + 1], w[i + 2], w[i + 3]};
    } else {
        r = u32x4{__builtin_amdgcn_alignbyte(w[i + 1], w[i], 2), __builtin_amdgcn_alignbyte(w[i + 2], w[i + 1], 2),
                  __builtin_amdgcn_alignbyte(w[i + 3], w[i + 2], 2), __builtin_amdgcn_alignbyte(w[i + 4], w[i + 3], 2)};
    }
    return r;
}

// Dot product of one super-block (8 GGUF blocks) of the lane's row, held in
// LDS as words w, with the digits of the super-block's 256 inputs (xd, xq:
// its first block; see put_digits): per block, then scaled by the block's d
// (q8_gemv.rs:234-242).
template <uint32_t T>
__device__ __forceinline__ float sb_dot(const uint32_t *w, const uint32_t *xd, const uint4 *xq, float acc) {
    // pairs of blocks: block 2 p starts at a multiple of 4 bytes, block 2 p + 1
    // two bytes past one, so each pair's alignment is known at compile time
#pragma unroll 1
    for (int k = 0; k < 8; k += 2) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int base = (k + j) * QTraits<T>::kBlockBytes;
            const uint32_t *wb = w + (base >> 2);
            constexpr int Q = QTraits<T>::kBlockBytes;
            const int o = ((j * Q) & 3) + 2;  // the quants' byte offset from wb
            const float d = half_at(wb, (j * Q) & 3);
            u32x4 q[2];
            q[0] = words_at(wb, o);
            if constexpr (T == ANEHIP_GGML_Q8_0) q[1] = words_at(wb, o + 16);
            acc = fmaf(block_dot_digits<T>(q, xd + (k + j) * kXdWords, xq[k + j]), d, acc);
        }
    }
    return acc;
}

// Coalesced load of one super-block column of a 64-row tile: the tile holds
// 64 rows x kSbBytes, i.e. kSbVec * 64 chunks of 16 bytes.  Load j of lane l
// fetches chunk c = 64 j + l = (row c / kSbVec, part c % kSbVec), so each
// load instruction reads whole contiguous row segments.  `off` holds the
// lane's byte offsets of its chunks relative to the tile's first row (32-bit,
// loop-invariant; rows past m are clamped to the last row and never stored),
// so every load is "uniform base + 32-bit lane offset".
template <uint32_t T>
__device__ __forceinline__ void tile_offsets(uint32_t *off, uint32_t row_bytes, int rows_left, int lane) {
    constexpr int V = QTraits<T>::kSbVec;
#pragma unroll
    for (int j = 0; j < V; j++) {
        const int c = j * kWave + lane;
        const int r = min(c / V, rows_left - 1);
        off[j] = (uint32_t)r * row_bytes + (uint32_t)(c % V) * 16u;
    }
}

template <uint32_t T>
__device__ __forceinline__ void load_tile(u32x4 *regs, const uint8_t *tile_base, const uint32_t *off) {
    constexpr int V = QTraits<T>::kSbVec;
#pragma unroll
    for (int j = 0; j < V; j++)
        regs[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(tile_base + off[j]));
}

// Stage the tile through this wave's LDS slice (chunk c at byte 16 c, i.e.
// row-major [64][kSbBytes]); the lane then reads its own row from LDS.  LDS
// operations of one wave complete in issue order, so only compiler ordering
// is needed between the writes and the reads of the same wave.
template <uint32_t T>
__device__ __forceinline__ void stage_tile(const u32x4 *regs, u32x4 *lds, int lane) {
    constexpr int V = QTraits<T>::kSbVec;
#pragma unroll
    for (int j = 0; j < V; j++) lds[j * kWave + lane] = regs[j];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int kWavesPerWg = 4;

// Sum over an NT-thread workgroup (red: NT / 64 floats of LDS); every thread
// gets the total.
template <int NT = 256>
__device__ __forceinline__ float wg_sum(float v, float *red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) s += red[w];
    return s;
}

constexpr int kMaxSplit = 8;     // K splits a batch-1 consumer may have to add
constexpr int kMaxGemmSplit = 16;  // K splits of the x-stationary GEMM (batch > 1)
constexpr int kMaxSliceSb = 8;   // super-blocks of input one workgroup may need
constexpr int kAttnHd = 256;     // attention head dim (GEMV_IN_ATTN_COMBINE slices)

// sum over p < kp of part[p * stride + i], p ascending.  All kMaxSplit loads
// are issued unconditionally (slices past kp re-read slice 0) so they overlap
// instead of costing kp dependent round trips.
__device__ __forceinline__ float sum_parts(const float *__restrict__ part, int kp, size_t stride, size_t i) {
    float v[kMaxSplit];
#pragma unroll
    for (int p = 0; p < kMaxSplit; p++) v[p] = part[(p < kp ? (size_t)p * stride : 0) + i];
    float s = v[0];
#pragma unroll
    for (int p = 1; p < kMaxSplit; p++) s += p < kp ? v[p] : 0.0f;
    return s;
}

// Forms the workgroup's input slice xs[0, len) = input[c0, c0 + len) of length-n
// input vector `in` (see GemvInMode), with NT threads (red: NT / 64 floats of
// LDS).  Every mode issues its global loads in batches of RB elements per
// thread, then computes, so with RB = 8 the prologue costs about one memory
// round trip; smaller RB trades round trips for registers.
//
// `first` is false when a workgroup forms a second slice of the same input in
// one launch: the one-off side effects (the x_out copy, the conv-window
// commit) are then skipped.
template <int KP, int NT, class Issue, class Store>
__device__ __forceinline__ void attn_combine_slice(const GemvInput &in, int c0, Issue &&issue, Store &&store);

template <int MODE, int RB = 8, int NT = 256>
__device__ __forceinline__ void gemv_prologue(const GemvInput &in, int n, int c0, int len, float *xs, float *red,
                                              bool first = true) {
    constexpr int IT = kMaxSliceSb * 256 / NT;  // slice elements per thread
    const int t = threadIdx.x;
    if constexpr (MODE == GEMV_IN_PLAIN) {
        float v[IT];
#pragma unroll
        for (int i = 0; i < IT; i++) v[i] = t + NT * i < len ? in.x[c0 + t + NT * i] : 0.0f;
#pragma unroll
        for (int i = 0; i < IT; i++)
            if (t + NT * i < len) xs[t + NT * i] = v[i];
    } else if constexpr (MODE == GEMV_IN_SILU_MUL) {
        // scratch.rs:181-186: a = (a / (1 + exp(-a))) * b
        constexpr int B = RB < IT ? RB : IT;
        for (int i0 = 0; i0 < IT && NT * i0 < len; i0 += B) {
            float g[B], u[B];
#pragma unroll
            for (int i = 0; i < B; i++) {
                const int j = min(t + NT * (i0 + i), len - 1);
                const int gi = gu_index(c0 + j);  // the products' interleaved [gate; up] order
                g[i] = sum_parts(in.part, in.kp, in.part_stride, (size_t)gi);
                u[i] = sum_parts(in.part, in.kp, in.part_stride, (size_t)gi + 32);
            }
#pragma unroll
            for (int i = 0; i < B; i++)
                if (t + NT * (i0 + i) < len) xs[t + NT * (i0 + i)] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
        }
    } else if constexpr (MODE == GEMV_IN_ATTN_COMBINE) {
        // one head per slice (the launcher checks that each split is one panel)
        attn_combine_slice<kMaxSplit, NT>(in, c0, [] {}, [&](float4 v, int i4, bool ok) {
            if (ok) reinterpret_cast<float4 *>(xs)[i4] = v;
        });
    } else if constexpr (MODE == GEMV_IN_GATED_NORM) {
        // deltanet.rs:517-533, per 128-wide head; a wave handles whole heads
        constexpr int W = NT / 64;                      // waves
        constexpr int HI = kMaxSliceSb * 2 / W;         // heads per wave for a full slice
        constexpr int HB = RB >= 8 ? HI : (RB >= 4 ? (HI < 2 ? HI : 2) : 1);
        const int lane = t & 63, wave = t >> 6;
        const int nh = len / 128;
        for (int i0 = 0; i0 < HI; i0 += HB) {
            float a[HB], b[HB], ga[HB], gb[HB];
#pragma unroll
            for (int i = 0; i < HB; i++) {
                const int hh = min(wave + W * (i0 + i), nh - 1);
                const int k0 = c0 + hh * 128;
                a[i] = in.x[k0 + lane];
                b[i] = in.x[k0 + 64 + lane];
                ga[i] = sum_parts(in.part, in.kp, in.part_stride, (size_t)in.gate_off + k0 + lane);
                gb[i] = sum_parts(in.part, in.kp, in.part_stride, (size_t)in.gate_off + k0 + 64 + lane);
            }
#pragma unroll
            for (int i = 0; i < HB; i++) {
                const int hh = wave + W * (i0 + i);
                const float ss = wave_sum(a[i] * a[i] + b[i] * b[i]);
                if (hh < nh) {
                    const float inv_rms = 1.0f / sqrtf(ss / 128.0f + in.eps);
                    xs[hh * 128 + lane] = ((a[i] * inv_rms) * in.w[lane]) * (ga[i] / (1.0f + expf(-ga[i])));
                    xs[hh * 128 + 64 + lane] =
                        ((b[i] * inv_rms) * in.w[64 + lane]) * (gb[i] / (1.0f + expf(-gb[i])));
                }
            }
        }
        // commit the q/k conv windows, spread over the launch's workgroups
        if (in.conv_state && first) {
            const int nwg = gridDim.x * gridDim.y, wg = blockIdx.y * gridDim.x + blockIdx.x;
            for (int c = wg * NT + t; c < 2 * n; c += nwg * NT) {
                float4 *cs = reinterpret_cast<float4 *>(in.conv_state) + c;
                const float4 o = *cs;
                const float nv = sum_parts(in.part, in.kp, in.part_stride, (size_t)c);
                *cs = make_float4(o.y, o.z, o.w, nv);
            }
        }
    } else {
        // RMSNORM / RESID_RMSNORM / EMBED_RMSNORM: the full row is needed for
        // mean(r^2); the slice is kept in xs and scaled after the reduction
        // (main.rs:1106-1113: out = (r * inv_rms) * w).  Residual: r = x + s
        // with s the partials added in split order.
        const bool writer = first && blockIdx.x == 0 && blockIdx.y == 0;
        const uint32_t tok = MODE == GEMV_IN_EMBED_RMSNORM ? in.token[0] : 0;
        float ss = 0.0f;
        for (int base = 0; base < n; base += NT * RB) {
            float r[RB];
#pragma unroll
            for (int i = 0; i < RB; i++) {
                const int k = min(base + t + NT * i, n - 1);
                if constexpr (MODE == GEMV_IN_EMBED_RMSNORM) {
                    r[i] = tok < in.vocab ? in.emb[(size_t)tok * n + k] : 0.0f;
                } else if constexpr (MODE == GEMV_IN_RESID_RMSNORM) {
                    r[i] = in.x[k] + sum_parts(in.part, in.kp, in.part_stride, (size_t)k);
                } else {
                    r[i] = in.x[k];
                }
            }
#pragma unroll
            for (int i = 0; i < RB; i++) {
                const int k = base + t + NT * i;
                if (k < n) {
                    ss += r[i] * r[i];
                    if (k >= c0 && k < c0 + len) xs[k - c0] = r[i];
                    if (MODE != GEMV_IN_RMSNORM && writer) in.x_out[k] = r[i];
                }
            }
        }
        ss = wg_sum<NT>(ss, red);
        const float inv_rms = 1.0f / sqrtf(ss / (float)n + in.eps);
        for (int j = t; j < len; j += NT) xs[j] = (xs[j] * inv_rms) * in.w[c0 + j];
    }
    __syncthreads();
}

// Batch-1 GEMV: grid = (row tiles of 64, K splits); 4 waves per workgroup.
// Workgroup (tile, ks) covers super-blocks [ks * sb_per_split, ...) of its 64
// rows; wave w takes every 4th of them.  The input slice is formed in LDS by
// the prologue and read with wave-uniform (broadcast) LDS loads.  The 4
// waves are reduced through LDS; the result (or this split's partial sum) goes
// to out[ks * split_stride + row].
template <uint32_t T, int MODE>
__global__ __launch_bounds__(kWave *kWavesPerWg) void gemv_fused(const uint8_t *__restrict__ W, GemvInput in,
                                                                float *__restrict__ out, int m, int n,
                                                                int sb_per_split, size_t split_stride) {
    constexpr int V = QTraits<T>::kSbVec;
    __shared__ u32x4 lds[kWavesPerWg][V * kWave];
    // the input slice, then (in place) its digits: kept at 8 KiB so that two
    // workgroups fit a CU's LDS
    __shared__ __align__(16) float xs[kMaxSliceSb * 256];
    __shared__ float red4[4];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
    const int tile = blockIdx.x;
    const int ks = blockIdx.y;
    const int nsb = n >> 8;
    const size_t row_bytes = (size_t)nsb * QTraits<T>::kSbBytes;
    const int row0 = tile * kWave;
    const int sb_begin = ks * sb_per_split;
    const int sb_end = min(nsb, sb_begin + sb_per_split);

    // issue the first weight tile before the prologue so both overlap
    u32x4 regs[V];
    uint32_t off[V];
    tile_offsets<T>(off, (uint32_t)row_bytes, m - row0, lane);
    const uint8_t *tile_base = W + (size_t)row0 * row_bytes;
    int sb = sb_begin + wave;
    if (sb < sb_end) load_tile<T>(regs, tile_base + (size_t)sb * QTraits<T>::kSbBytes, off);

    gemv_prologue<MODE>(in, n, sb_begin * 256, (sb_end - sb_begin) * 256, xs, red4);
    digitize_lds_inplace<T, kWave * kWavesPerWg, kMaxSliceSb * 256>(xs, (sb_end - sb_begin) * 256);
    __syncthreads();
    const uint32_t *xd = reinterpret_cast<const uint32_t *>(xs);
    const uint4 *xq = reinterpret_cast<const uint4 *>(xs + kMaxSliceSb * 8 * kXdWords);

    float acc = 0.0f;
    const uint32_t *wl = reinterpret_cast<const uint32_t *>(&lds[wave][lane * V]);
    for (; sb < sb_end; sb += kWavesPerWg) {
        stage_tile<T>(regs, lds[wave], lane);
        if (sb + kWavesPerWg < sb_end)
            load_tile<T>(regs, tile_base + (size_t)(sb + kWavesPerWg) * QTraits<T>::kSbBytes, off);
        acc = sb_dot<T>(wl, xd + (sb - sb_begin) * 8 * kXdWords, xq + (sb - sb_begin) * 8, acc);
        wave_sync_lds();  // this tile's reads precede the next tile's writes
    }
    __syncthreads();
    float *red = reinterpret_cast<float *>(&lds[0][0]);
    red[wave * kWave + lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    const int row = row0 + lane;
    if (row >= m) return;
    float sum = red[lane];
#pragma unroll
    for (int v = 1; v < kWavesPerWg; v++) sum += red[v * kWave + lane];
    out[(size_t)ks * split_stride + row] = sum;
}

// x-stationary form of gemv_fused (plain input, matrices of many row tiles,
// K splits of 8 super-blocks): 8 waves per workgroup, wave w takes
// super-block ks * 8 + w of every row tile t = blockIdx.x, + gridDim.x, ...
// (staged through its own LDS slice, the next tile's loads issued at once),
// with the split's x digitised once per workgroup instead of once per tile;
// the 8 waves' row sums meet in LDS (two buffers, one barrier per tile).
// lm_head 151936 x 2048 (GGUF layout): 66.0 us against 72.2-72.7 us
// (graphs of back-to-back launches).
template <uint32_t T>
__global__ __launch_bounds__(512) void gemv_fused_xs(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                     float *__restrict__ out, int m, int n, size_t split_stride) {
    constexpr int V = QTraits<T>::kSbVec;
    constexpr int NT = 512;
    __shared__ u32x4 lds[8][V * kWave];
    __shared__ __align__(16) float xs[kMaxSliceSb * 256];  // the split's x, then (in place) its digits
    __shared__ float red[2][8][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int G = gridDim.x, ks = blockIdx.y;
    const int nsb = n >> 8, tiles = (m + kWave - 1) / kWave;
    const uint32_t row_bytes = (uint32_t)nsb * QTraits<T>::kSbBytes;
    const int sb = ks * 8 + wave;
    int t = blockIdx.x;
    if (t >= tiles) return;  // uniform
    u32x4 regs[V];
    auto issue = [&](int tt) {
        int ln = lane;
        asm volatile("" : "+v"(ln));  // not loop-invariant: the offsets are not kept in registers
        const int rows_left = m - tt * kWave;
        const uint8_t *base = W + (size_t)tt * kWave * row_bytes + (size_t)sb * QTraits<T>::kSbBytes;
#pragma unroll
        for (int j = 0; j < V; j++) {
            const int c = j * kWave + ln;
            const uint32_t o = (uint32_t)min(c / V, rows_left - 1) * row_bytes + (uint32_t)(c % V) * 16u;
            regs[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base + o));
        }
    };
    issue(t);
    {
        constexpr int IT = kMaxSliceSb * 256 / NT;
        float v[IT];
#pragma unroll
        for (int i = 0; i < IT; i++) v[i] = x[(size_t)ks * 2048 + threadIdx.x + NT * i];
#pragma unroll
        for (int i = 0; i < IT; i++) xs[threadIdx.x + NT * i] = v[i];
    }
    __syncthreads();
    digitize_lds_inplace<T, NT, kMaxSliceSb * 256>(xs, kMaxSliceSb * 256);
    __syncthreads();
    const uint32_t *xd = reinterpret_cast<const uint32_t *>(xs) + wave * 8 * kXdWords;
    const uint4 *xq = reinterpret_cast<const uint4 *>(xs + kMaxSliceSb * 8 * kXdWords) + wave * 8;
    const uint32_t *wl = reinterpret_cast<const uint32_t *>(&lds[wave][lane * V]);  // this lane's row
    float *dst = out + (size_t)ks * split_stride;
    for (int p = 0; t < tiles; t += G, p ^= 1) {
        stage_tile<T>(regs, lds[wave], lane);
        if (t + G < tiles) issue(t + G);
        const float acc = sb_dot<T>(wl, xd, xq, 0.0f);
        wave_sync_lds();  // this tile's reads precede the next tile's writes
        red[p][wave][lane] = acc;
        __syncthreads();  // red[p] complete; red[p ^ 1] was read before this barrier
        if (wave == 0) {
            const int row = t * kWave + lane;
            if (row < m) {
                float sum = red[p][0][lane];
#pragma unroll
                for (int w = 1; w < 8; w++) sum += red[p][w][lane];
                dst[row] = sum;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Panel layout.  The decode step keeps its weights in a GPU-native
// permutation of the GGUF blocks (same bytes, same values), built once at
// upload: row tiles of 64 rows, each cut into panels of 256 columns (8
// blocks).  A panel is
//   quants: [chunk][64 rows][16 bytes]  (Q8_0: 16 chunks = 2 per block;
//                                        Q4_0: 8 chunks = 1 per block, the
//                                        block's 16 nibble bytes)
//   scales: [64 rows][8 x fp16]          (the rows' 8 block scales)
// so 17 (Q8_0) or 9 (Q4_0) 1 KiB-contiguous wave loads bring every lane its
// own row's 256 weights and scales, with no LDS transposition.  Panels of a
// tile are consecutive; rows past m are zero.
// ---------------------------------------------------------------------------

template <uint32_t T> struct Panel;
template <> struct Panel<ANEHIP_GGML_Q8_0> {
    static constexpr int kChunks = 16;
    static constexpr int kBytes = 17 * 1024;
};
template <> struct Panel<ANEHIP_GGML_Q4_0> {
    static constexpr int kChunks = 8;
    static constexpr int kBytes = 9 * 1024;
};

// The GGUF row behind panel row `row`: the identity, or (il = F > 0, a
// stacked [gate (F rows); up (F rows)] matrix) gate rows 32 t .. 32 t + 31 in
// the first half of tile t and the same features' up rows in its second
// half, so that one 64-row tile of the panel copy holds the gate and the up
// row of each of its 32 features.
__host__ __device__ __forceinline__ int src_row(int row, int il) {
    if (!il) return row;
    const int t = row >> 6, r = row & 63;
    return (r < 32 ? 0 : il) + 32 * t + (r & 31);
}

// One thread per 16-byte destination vector of the panel buffer.
template <uint32_t T>
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                    int m, int n, size_t nvec, int il) {
    const size_t v = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (v >= nvec) return;
    constexpr int BB = QTraits<T>::kBlockBytes;
    const int nsb = n >> 8;
    const size_t panel = v / (Panel<T>::kBytes / 16);
    const int within = (int)(v % (Panel<T>::kBytes / 16));  // 16-byte vector index inside the panel
    const int tile = (int)(panel / nsb), sb = (int)(panel % nsb);
    const int chunk = within / 64, r = within % 64;  // chunk == kChunks: the scale vector
    const int row = tile * 64 + r;
    uint8_t out[16];
    const size_t row_off = (size_t)src_row(row, il) * (n / 32) * BB;
    for (int i = 0; i < 16; i++) {
        uint8_t b = 0;
        if (row < m) {
            if (chunk < Panel<T>::kChunks) {
                const int blk = T == ANEHIP_GGML_Q8_0 ? chunk / 2 : chunk;
                const int q0 = T == ANEHIP_GGML_Q8_0 ? 2 + 16 * (chunk & 1) : 2;
                b = src[row_off + (size_t)(sb * 8 + blk) * BB + q0 + i];
            } else {
                b = src[row_off + (size_t)(sb * 8 + i / 2) * BB + (i & 1)];
            }
        }
        out[i] = b;
    }
    u32x4 w;
    w.x = out[0] | (out[1] << 8) | (out[2] << 16) | ((uint32_t)out[3] << 24);
    w.y = out[4] | (out[5] << 8) | (out[6] << 16) | ((uint32_t)out[7] << 24);
    w.z = out[8] | (out[9] << 8) | (out[10] << 16) | ((uint32_t)out[11] << 24);
    w.w = out[12] | (out[13] << 8) | (out[14] << 16) | ((uint32_t)out[15] << 24);
    reinterpret_cast<u32x4 *>(dst)[v] = w;
}

// The inverse permutation: one thread per 16-byte vector of the panel
// buffer scatters its bytes back to their GGUF positions (rows < m; the
// padding rows of the last tile hold zeros and have no GGUF position).
template <uint32_t T>
__global__ __launch_bounds__(256) void unpack_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                    int m, int n, size_t nvec, int il) {
    const size_t v = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (v >= nvec) return;
    constexpr int BB = QTraits<T>::kBlockBytes;
    const int nsb = n >> 8;
    const size_t panel = v / (Panel<T>::kBytes / 16);
    const int within = (int)(v % (Panel<T>::kBytes / 16));
    const int tile = (int)(panel / nsb), sb = (int)(panel % nsb);
    const int chunk = within / 64, r = within % 64;
    const int row = tile * 64 + r;
    if (row >= m) return;
    const u32x4 w = reinterpret_cast<const u32x4 *>(src)[v];
    const uint32_t w4[4] = {w.x, w.y, w.z, w.w};
    const size_t row_off = (size_t)src_row(row, il) * (n / 32) * BB;
    for (int i = 0; i < 16; i++) {
        const uint8_t b = (uint8_t)(w4[i >> 2] >> (8 * (i & 3)));
        if (chunk < Panel<T>::kChunks) {
            const int blk = T == ANEHIP_GGML_Q8_0 ? chunk / 2 : chunk;
            const int q0 = T == ANEHIP_GGML_Q8_0 ? 2 + 16 * (chunk & 1) : 2;
            dst[row_off + (size_t)(sb * 8 + blk) * BB + q0 + i] = b;
        } else {
            dst[row_off + (size_t)(sb * 8 + i / 2) * BB + (i & 1)] = b;
        }
    }
}

// A wave's share of a panel: blocks [NB * part, NB * (part + 1)) of the 8,
// i.e. kChunks * NB / 8 quant vectors, plus the panel's scale vector.
template <uint32_t T, int NB>
struct PanelPart {
    static constexpr int kVecs = Panel<T>::kChunks * NB / 8;
};

// Loads one wave's share of a panel.  Idle waves (valid false) load one
// 16-byte vector of the panel base with all lanes instead, so every wave
// issues the same, unconditional load sequence.  The scale vector goes
// first: every block's dot product needs it, and with it first (vmcnt waits
// are in issue order) block j waits only for its own quant vectors, so the
// dot products run while the later blocks are still arriving.
template <uint32_t T, int NB>
__device__ __forceinline__ void load_part(u32x4 *q, u32x4 &sc, const uint8_t *panel, const uint8_t *dummy, int part,
                                          int lane, bool valid) {
    const u32x4 *p4 = reinterpret_cast<const u32x4 *>(valid ? panel : dummy);
    const int l = valid ? lane : 0;
    constexpr int V = PanelPart<T, NB>::kVecs;
    const int c0 = valid ? V * part : 0;
    // the scheduling barriers keep this issue order (and the loads together)
    __builtin_amdgcn_sched_barrier(0);
    sc = __builtin_nontemporal_load(p4 + Panel<T>::kChunks * 64 + l);
#pragma unroll
    for (int c = 0; c < V; c++) {
        __builtin_amdgcn_sched_barrier(0);
        q[c] = __builtin_nontemporal_load(p4 + (c0 + c) * 64 + l);
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Dot product of a wave's panel share held in registers (q, sc: see
// load_part) with the digits of the panel's 256 inputs (xd, xq: the panel's
// first block; wave-uniform, so broadcast LDS reads): per block, then scaled
// by the block's d (q8_gemv.rs:234-242).
template <uint32_t T, int NB>
__device__ __forceinline__ float panel_dot(const u32x4 *q, const u32x4 &sc, const uint32_t *xd, const uint4 *xq,
                                           int part, float acc) {
    const uint32_t scw[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const int b = NB * part + j;  // block within the panel
        uint32_t word;
        if constexpr (NB == 8) {
            word = scw[j >> 1];
        } else {
            // b >> 1 is wave-uniform but not a compile-time index
            const int wi = b >> 1;
            word = wi == 0 ? scw[0] : wi == 1 ? scw[1] : wi == 2 ? scw[2] : scw[3];
        }
        const float d = __half2float(__ushort_as_half((unsigned short)(word >> (16 * (b & 1)))));
        constexpr int VB = T == ANEHIP_GGML_Q8_0 ? 2 : 1;
        acc = fmaf(block_dot_digits<T>(q + VB * j, xd + b * kXdWords, xq[b]), d, acc);
    }
    return acc;
}

// ---------------------------------------------------------------------------
// Overlapped prologue of the panel GEMV.  The slow part of a prologue is its
// global-load round trip, and vmcnt waits are in issue order, so the loads
// of the input (x, residual partial slices, norm weights, gates) are issued
// first, then `issue()` starts the workgroup's weight loads, and only then is
// the input formed -- its wait no longer includes the weights.  Fast paths
// take the shapes of the decode step (norms over n <= 2048, SiLU-mul and
// gated-norm slices <= 1024, 16-byte aligned slices) with float4 loads and KP
// (2 or 8) partial slices per value; anything else falls back to issue() +
// the generic prologue.  Same arithmetic per element as gemv_prologue.
// ---------------------------------------------------------------------------

__device__ __forceinline__ float4 f4_add(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

__device__ __forceinline__ float silu1(float g) { return g / (1.0f + expf(-g)); }

// KP unconditional loads (slices past kp re-read slice kp - 1) and their
// branch-free sum in split order: straight-line code keeps the compiler's
// vmcnt accounting exact, so waiting for these loads does not wait for
// loads issued after them.
template <int KP>
__device__ __forceinline__ void load_parts4(float4 *v, const float *part, int kp, size_t stride, size_t off4) {
    const float4 *p4 = reinterpret_cast<const float4 *>(part);
#pragma unroll
    for (int p = 0; p < KP; p++) v[p] = p4[(size_t)min(p, max(kp - 1, 0)) * (stride / 4) + off4];
}

template <int KP>
__device__ __forceinline__ float4 sum_parts4(const float4 *v, int kp) {
    float4 s = v[0];
#pragma unroll
    for (int p = 1; p < KP; p++) {
        const bool on = p < kp;
        s.x += on ? v[p].x : 0.0f;
        s.y += on ? v[p].y : 0.0f;
        s.z += on ? v[p].z : 0.0f;
        s.w += on ? v[p].w : 0.0f;
    }
    return s;
}

// Whether prologue_overlapped covers this launch (a single slice of len
// floats per workgroup; uniform).
template <int MODE, int NT>
__device__ __forceinline__ bool overlapped_ok(const GemvInput &in, int n, int len) {
    if constexpr (MODE == GEMV_IN_PLAIN) return len <= 4 * NT && ((uintptr_t)in.x & 15) == 0;
    const bool aligned = ((in.part_stride | (size_t)in.gate_off) & 3) == 0;
    if constexpr (MODE == GEMV_IN_RMSNORM || MODE == GEMV_IN_RESID_RMSNORM || MODE == GEMV_IN_EMBED_RMSNORM)
        return n <= 4 * NT && aligned;
    if constexpr (MODE == GEMV_IN_SILU_MUL) return len <= 4 * NT && aligned;
    if constexpr (MODE == GEMV_IN_GATED_NORM)
        return len <= 4 * NT && aligned && (!in.conv_state || 2 * n <= (int)(gridDim.x * gridDim.y) * NT);
    if constexpr (MODE == GEMV_IN_ATTN_COMBINE) return len == kAttnHd && NT >= 4 * kWave && aligned;
    return false;
}

// GEMV_IN_ATTN_COMBINE: head c0 / 256 of batch row 0, the decode attention's
// merge of its chunk partials (attn_combine_kernel's arithmetic and order:
// the maximum over the active chunks, then 4 groups of 64 lanes sum chunks
// g, g + 4, ... with weights exp(m - M), the groups added in order, num / den
// times sigmoid(gate)) into xs[0..256).  The gate and the first 16 chunks are
// loaded before `issue` starts the weight loads; groups 4.. (threads >= 256)
// mirror groups 0..3 for those loads, so every address stays in bounds.
template <int KP, int NT, class Issue, class Store>
__device__ __forceinline__ void attn_combine_slice(const GemvInput &in, int c0, Issue &&issue, Store &&store) {
    static_assert(NT >= 4 * kWave, "attn_combine_slice needs 4 waves");
    __shared__ float cmax[NT / kWave];
    __shared__ float4 accs[4][kWave];
    __shared__ float dens[4][kWave];
    const int t = threadIdx.x, g = t >> 6, gq = g & 3, l = t & (kWave - 1);
    const int h = c0 / kAttnHd, G = in.att_g, kvh = h / G, hh = h % G;
    const int len = (int)in.att_pos[0] + 1;
    const int nc = active_chunks(len, in.att_nch);  // >= 1
    const size_t base = (size_t)kvh * in.att_nch;
    float4 gv[KP];
    load_parts4<KP>(gv, in.part, in.kp, in.part_stride, (size_t)((h * 2 * kAttnHd + kAttnHd) >> 2) + l);
    float4 o4[4];
    float m4[4], l4[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const size_t slot = (base + min(gq + 4 * i, nc - 1)) * G + hh;
        o4[i] = *reinterpret_cast<const float4 *>(in.att_o + slot * kAttnHd + 4 * l);
        m4[i] = in.att_ml[slot * 2];
        l4[i] = in.att_ml[slot * 2 + 1];
    }
    float mx = -INFINITY;
    for (int cc = 16 + t; cc < nc; cc += NT) mx = fmaxf(mx, in.att_ml[((base + cc) * G + hh) * 2]);
    issue();
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (gq + 4 * i < nc) mx = fmaxf(mx, m4[i]);
    mx = wave_max64(mx);
    if (l == 0) cmax[g] = mx;
    __syncthreads();
    float M = cmax[0];
#pragma unroll
    for (int w = 1; w < NT / kWave; w++) M = fmaxf(M, cmax[w]);
    if (g < 4) {
        float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
        float den = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (g + 4 * i < nc) {
                const float w = expf(m4[i] - M);
                num = make_float4(num.x + w * o4[i].x, num.y + w * o4[i].y, num.z + w * o4[i].z,
                                  num.w + w * o4[i].w);
                den += w * l4[i];
            }
        int cc = g + 16;
        for (; cc + 12 < nc; cc += 16) {  // 4 chunks per trip, their loads issued together
            float4 p4[4];
            float pm[4], pl[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const size_t slot = (base + cc + 4 * i) * G + hh;
                p4[i] = *reinterpret_cast<const float4 *>(in.att_o + slot * kAttnHd + 4 * l);
                pm[i] = in.att_ml[slot * 2];
                pl[i] = in.att_ml[slot * 2 + 1];
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float w = expf(pm[i] - M);
                num = make_float4(num.x + w * p4[i].x, num.y + w * p4[i].y, num.z + w * p4[i].z,
                                  num.w + w * p4[i].w);
                den += w * pl[i];
            }
        }
        for (; cc < nc; cc += 4) {
            const size_t slot = (base + cc) * G + hh;
            const float4 o = *reinterpret_cast<const float4 *>(in.att_o + slot * kAttnHd + 4 * l);
            const float w = expf(in.att_ml[slot * 2] - M);
            num = make_float4(num.x + w * o.x, num.y + w * o.y, num.z + w * o.z, num.w + w * o.w);
            den += w * in.att_ml[slot * 2 + 1];
        }
        accs[g][l] = num;
        dens[g][l] = den;
    }
    __syncthreads();
    if (g == 0) {
        float4 sum = accs[0][l];
        float dsum = dens[0][l];
#pragma unroll
        for (int k = 1; k < 4; k++) {
            const float4 o = accs[k][l];
            sum = make_float4(sum.x + o.x, sum.y + o.y, sum.z + o.z, sum.w + o.w);
            dsum += dens[k][l];
        }
        const float4 ga = sum_parts4<KP>(gv, in.kp);
        store(make_float4((sum.x / dsum) * (1.0f / (1.0f + expf(-ga.x))), (sum.y / dsum) * (1.0f / (1.0f + expf(-ga.y))),
                          (sum.z / dsum) * (1.0f / (1.0f + expf(-ga.z))), (sum.w / dsum) * (1.0f / (1.0f + expf(-ga.w)))),
              l, true);
    }
    __syncthreads();
}

template <int MODE, int KP, int NT, class Issue, class Store>
__device__ __forceinline__ void prologue_overlapped(const GemvInput &in, int n, int c0, int len, float *red,
                                                    Issue &&issue, Store &&store) {
    const int t = threadIdx.x;
    if constexpr (MODE == GEMV_IN_PLAIN) {
        const float4 v = reinterpret_cast<const float4 *>(in.x + c0)[min(t, (len >> 2) - 1)];
        issue();
        store(v, t, t < (len >> 2));
        __syncthreads();
    } else if constexpr (MODE == GEMV_IN_RMSNORM || MODE == GEMV_IN_RESID_RMSNORM || MODE == GEMV_IN_EMBED_RMSNORM) {
        // one float4 of the n-vector per thread
        const int n4 = n >> 2, e4 = min(t, n4 - 1);
        const float4 *src;
        bool zero = false;
        if constexpr (MODE == GEMV_IN_EMBED_RMSNORM) {
            const uint32_t tok = in.token[0];
            zero = tok >= in.vocab;
            src = reinterpret_cast<const float4 *>(in.emb + (size_t)(zero ? 0u : tok) * n);
        } else {
            src = reinterpret_cast<const float4 *>(in.x);
        }
        float4 r = src[e4];
        const float4 w = reinterpret_cast<const float4 *>(in.w)[e4];
        float4 pv[KP];
        if constexpr (MODE == GEMV_IN_RESID_RMSNORM) load_parts4<KP>(pv, in.part, in.kp, in.part_stride, e4);
        issue();
        if (zero) r = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (MODE == GEMV_IN_RESID_RMSNORM) r = f4_add(r, sum_parts4<KP>(pv, in.kp));
        float ss = 0.0f;
        if (t < n4) {
            ss = r.x * r.x;
            ss += r.y * r.y;
            ss += r.z * r.z;
            ss += r.w * r.w;
            if (MODE != GEMV_IN_RMSNORM && blockIdx.x == 0 && blockIdx.y == 0)
                reinterpret_cast<float4 *>(in.x_out)[t] = r;
        }
        // the slice is stored as r * w, and the GEMV's sums are scaled by
        // inv_rms = 1 / sqrt(sum(r^2) / n + eps) at the end (post_scale):
        // the reduction no longer sits between the loads and the dot products
        ss = wave_sum(ss);
        if ((t & (kWave - 1)) == 0) red[t / kWave] = ss;
        const int e = 4 * t;
        store(make_float4(r.x * w.x, r.y * w.y, r.z * w.z, r.w * w.w), (e - c0) >> 2, t < n4 && e >= c0 && e < c0 + len);
        __syncthreads();
    } else if constexpr (MODE == GEMV_IN_SILU_MUL) {
        const int e4 = min(t, (len >> 2) - 1);
        // features c0 + 4 e4 .. + 3: one group of 32 in the products'
        // interleaved [gate; up] order, their up sums 32 positions on
        const int gi = gu_index(c0 + 4 * e4);
        float4 g[KP], u[KP];
        load_parts4<KP>(g, in.part, in.kp, in.part_stride, (size_t)(gi >> 2));
        load_parts4<KP>(u, in.part, in.kp, in.part_stride, (size_t)((gi + 32) >> 2));
        issue();
        const float4 gs = sum_parts4<KP>(g, in.kp), us = sum_parts4<KP>(u, in.kp);
        store(make_float4(silu1(gs.x) * us.x, silu1(gs.y) * us.y, silu1(gs.z) * us.z, silu1(gs.w) * us.w), t,
              t < (len >> 2));
        __syncthreads();
    } else if constexpr (MODE == GEMV_IN_ATTN_COMBINE) {
        attn_combine_slice<KP, NT>(in, c0, issue, store);
    } else if constexpr (MODE == GEMV_IN_GATED_NORM) {
        const int wg = blockIdx.y * gridDim.x + blockIdx.x;
        const bool commit = in.conv_state != nullptr;
        // one 128-wide head per 32 threads (deltanet.rs:517-533)
        const int e4 = min(t, (len >> 2) - 1);
        const float4 a = reinterpret_cast<const float4 *>(in.x)[(c0 >> 2) + e4];
        const float4 w = reinterpret_cast<const float4 *>(in.w)[e4 & 31];
        float4 ga[KP];
        load_parts4<KP>(ga, in.part, in.kp, in.part_stride, (size_t)((in.gate_off + c0) >> 2) + e4);
        // the q/k conv-window commit, at most one window per thread of the launch
        const int c = wg * NT + t;
        const bool has = commit && c < 2 * n;
        float4 old = make_float4(0.f, 0.f, 0.f, 0.f);
        float nv[KP];
        {
            // (loads stay in bounds and unconditional; only `has` lanes store)
            const int cc = commit ? min(c, 2 * n - 1) : 0;
            old = reinterpret_cast<const float4 *>(commit ? in.conv_state : in.x)[cc];
#pragma unroll
            for (int p = 0; p < KP; p++) nv[p] = in.part[(size_t)min(p, max(in.kp - 1, 0)) * in.part_stride + cc];
        }
        issue();
        const float ss = half_sum(a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w);
        const float inv_rms = 1.0f / sqrtf(ss / 128.0f + in.eps);
        const float4 g = sum_parts4<KP>(ga, in.kp);
        store(make_float4(((a.x * inv_rms) * w.x) * silu1(g.x), ((a.y * inv_rms) * w.y) * silu1(g.y),
                          ((a.z * inv_rms) * w.z) * silu1(g.z), ((a.w * inv_rms) * w.w) * silu1(g.w)),
              t, t < (len >> 2));
        if (has) {
            float sv = nv[0];
#pragma unroll
            for (int p = 1; p < KP; p++) sv += p < in.kp ? nv[p] : 0.0f;
            reinterpret_cast<float4 *>(in.conv_state)[c] = make_float4(old.y, old.z, old.w, sv);
        }
        __syncthreads();
    }
}

// The factor prologue_overlapped leaves for the GEMV's sums: the norm modes
// store r * w and defer inv_rms (main.rs:1106-1113: out = (r * inv_rms) * w,
// here sum_k q_k (r_k w_k) * inv_rms); red holds the waves' sums of r^2.
template <int MODE, int NT>
__device__ __forceinline__ float post_scale(const GemvInput &in, int n, const float *red) {
    if constexpr (MODE == GEMV_IN_RMSNORM || MODE == GEMV_IN_RESID_RMSNORM || MODE == GEMV_IN_EMBED_RMSNORM) {
        float ss = red[0];
#pragma unroll
        for (int w = 1; w < NT / kWave; w++) ss += red[w];
        return 1.0f / sqrtf(ss / (float)n + in.eps);
    }
    return 1.0f;
}

// Batch-1 GEMV over panels: grid = (row-tile groups, K splits), 8 waves per
// workgroup.  Each panel is shared by S waves (S = 1, 2, 4, 8; wave w takes
// part w % S, 8 / S blocks, of panel w / S), so a round covers 8 / S panels
// and small K slices still keep all 8 waves loading.  A workgroup covers
// `tiles_per_wg` consecutive 64-row tiles with one input slice (the prologue
// runs once).  When the slice fits one round, the input loads are issued
// before the weight loads (prologue_overlapped); otherwise rounds take the
// generic prologue.  Every wave issues its weight loads unconditionally (idle
// waves read one shared vector), which keeps the vmcnt waits exact.  The 8
// waves are reduced through LDS; the result (or this split's partial sum)
// goes to out[ks * split_stride + row].
constexpr int kPackedWaves = 8;

template <uint32_t T, int MODE, int KP, int S>
__global__ __launch_bounds__(kWave *kPackedWaves) void gemv_packed(const uint8_t *__restrict__ Wp, GemvInput in,
                                                                  float *__restrict__ out, int m, int n,
                                                                  int sb_per_split, size_t split_stride,
                                                                  int tiles_per_wg) {
    constexpr int NB = 8 / S, P = kPackedWaves / S, V = PanelPart<T, NB>::kVecs;
    constexpr int NT = kWave * kPackedWaves;
    __shared__ __align__(16) float xs[kMaxSliceSb * 256];  // the generic path's input slice
    __shared__ __align__(16) uint32_t xd[kMaxSliceSb * 8 * kXdWords];
    __shared__ uint4 xq[kMaxSliceSb * 8];
    __shared__ float red[kPackedWaves][kWave];
    __shared__ float redw[kPackedWaves];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int pi = wave / S, part = wave % S;
    const int nsb = n >> 8, tiles = (m + kWave - 1) / kWave;
    const int ks = blockIdx.y;
    const int sb_begin = ks * sb_per_split;
    const int sb_end = min(nsb, sb_begin + sb_per_split);
    const int t0 = blockIdx.x * tiles_per_wg, t1 = min(tiles, t0 + tiles_per_wg);
    const size_t tile_bytes = (size_t)nsb * Panel<T>::kBytes;
    const bool fast = sb_end - sb_begin <= P && overlapped_ok<MODE, NT>(in, n, (sb_end - sb_begin) * 256);
    auto digits = [&](float4 v, int i4, bool ok) { put_digits<T>(v, i4, ok, xd, xq); };

    u32x4 q[V], sc;
    // the 8 waves' sums of a tile through LDS; the result (times the input's
    // deferred factor) goes out
    auto finish = [&](int tile, float acc, float scale) {
        red[wave][lane] = acc;
        __syncthreads();
        if (wave == 0) {
            const int row = tile * kWave + lane;
            if (row < m) {
                float sum = red[0][lane];
#pragma unroll
                for (int v = 1; v < kPackedWaves; v++) sum += red[v][lane];
                out[(size_t)ks * split_stride + row] = sum * scale;
            }
        }
        __syncthreads();  // red (and, in the generic path, xs and xd) are reused by the next tile
    };
    if (fast) {
        // a loop of its own: joined with the generic path's code, the dot
        // products would wait for every load either path may have pending
        const int sb = sb_begin + pi;
        const bool valid = sb < sb_end;
        float scale = 1.0f;
        for (int tile = t0; tile < t1; tile++) {
            const uint8_t *pp = Wp + (size_t)tile * tile_bytes + (size_t)sb * Panel<T>::kBytes;
            if (tile == t0) {
                // the slice's digits are formed once and kept for later tiles
                auto issue = [&]() { load_part<T, NB>(q, sc, pp, Wp, part, lane, valid); };
                prologue_overlapped<MODE, KP, NT>(in, n, sb_begin * 256, (sb_end - sb_begin) * 256, redw, issue,
                                                  digits);
                scale = post_scale<MODE, NT>(in, n, redw);
            } else {
                load_part<T, NB>(q, sc, pp, Wp, part, lane, valid);
            }
            float acc = 0.0f;
            if (valid) acc = panel_dot<T, NB>(q, sc, xd + pi * 8 * kXdWords, xq + pi * 8, part, acc);
            finish(tile, acc, scale);
        }
        return;
    }
    for (int tile = t0; tile < t1; tile++) {
        const uint8_t *tb = Wp + (size_t)tile * tile_bytes;
        float acc = 0.0f;
        for (int r0 = sb_begin; r0 < sb_end; r0 += P) {
            const int r1 = min(sb_end, r0 + P);
            const int sb = r0 + pi;
            const bool valid = sb < r1;
            load_part<T, NB>(q, sc, tb + (size_t)sb * Panel<T>::kBytes, Wp, part, lane, valid);
            if (r0 != sb_begin) __syncthreads();  // the previous round's reads of xd are done
            gemv_prologue<MODE, 2, NT>(in, n, r0 * 256, (r1 - r0) * 256, xs, redw, tile == t0 && r0 == sb_begin);
            digitize_lds<T, NT>(xs, (r1 - r0) * 256, xd, xq);
            __syncthreads();
            if (valid) acc = panel_dot<T, NB>(q, sc, xd + (sb - r0) * 8 * kXdWords, xq + (sb - r0) * 8, part, acc);
        }
        finish(tile, acc, 1.0f);
    }
}

// Batch-1 DeltaNet step fused into the ssm_out GEMV (one launch per DeltaNet
// layer instead of two).  The ssm_out GEMV takes one K split per panel, i.e.
// per two 128-wide heads; workgroup (split ks, row tile) runs the step of
// heads 2 ks and 2 ks + 1 itself (the 32 row tiles of a split each recompute
// it), forms their gated-RMSNorm outputs as the GEMV's input slice and
// multiplies its tile.  The recurrent state and the conv windows are read,
// not written: the head output is o = S'^T q + delta (k . q) with S' = decay
// S and delta = beta (v - S'^T k) (the same value as S''^T q with S'' = S' +
// k delta^T, deltanet.rs:485-512), and the split's row-tile-0 workgroup
// leaves delta, k, decay and the new conv inputs in `pend` for
// launch_deltanet_apply.  Thread t: head hh = t / 256; within the head the
// layout of deltanet_head_kernel (a q or k channel, the v channel t % 128;
// columns 4 cq .. + 3 and rows 16 rg .. + 15 of the state).  The linear
// workgroup index puts a split's workgroups on one XCD (blockIdx % 8).
constexpr int kDnDk = 128;
constexpr int kDnK = 4;  // conv width

struct DnSsmArgs {
    MixIn mix, beta, alpha;  // [q | k | v][gate], [n_heads], [n_heads]
    const float *conv_w = nullptr, *conv_state = nullptr, *ssm_a = nullptr, *dt_bias = nullptr, *S = nullptr;
    const float *norm_w = nullptr;
    float *pend = nullptr;
    int n_heads = 0, d = 0;
    float eps = 0.0f;
};

__device__ __forceinline__ float silu_dn(float x) { return x / (1.0f + expf(-x)); }

template <uint32_t T, int KP>
__global__ __launch_bounds__(kWave *kPackedWaves) void dn_ssm_kernel(const uint8_t *__restrict__ Wp, DnSsmArgs a,
                                                                    float *__restrict__ out, int m, int nsplit) {
    constexpr int V = PanelPart<T, 1>::kVecs;
    __shared__ float qn[2][kDnDk], kn[2][kDnDk], vv[2][kDnDk];
    __shared__ __align__(16) float4 pk[2][8][32], pq[2][8][32];  // [head][row group][column quad]
    __shared__ float red[kPackedWaves], red2[kPackedWaves];
    __shared__ __align__(16) uint32_t xd[8 * kXdWords];
    __shared__ uint4 xq[8];
    __shared__ float gred[kPackedWaves][kWave];
    const int t = threadIdx.x, lane = t & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int ks = blockIdx.x % nsplit, tile = blockIdx.x / nsplit;
    const int hh = t >> 8, tt = t & 255, e = tt & (kDnDk - 1);
    const int d = a.d, h = 2 * ks + hh, C = 3 * d;
    const bool writer = tile == 0;
    const int nsb = d >> 8;

    // small inputs first, then the weights, then the state (in-order waits)
    const int ch = tt < kDnDk ? h * kDnDk + tt : d + h * kDnDk + e, chv = 2 * d + h * kDnDk + e;
    const float4 win = *reinterpret_cast<const float4 *>(a.conv_state + (size_t)ch * kDnK);
    const float4 wk = *reinterpret_cast<const float4 *>(a.conv_w + (size_t)ch * kDnK);
    const float4 winv = *reinterpret_cast<const float4 *>(a.conv_state + (size_t)chv * kDnK);
    const float4 wkv = *reinterpret_cast<const float4 *>(a.conv_w + (size_t)chv * kDnK);
    float xa[KP], xv[KP], xb[KP], xl[KP];
    a.mix.load<KP>(0, ch, xa);
    a.mix.load<KP>(0, chv, xv);
    a.beta.load<KP>(0, h, xb);
    a.alpha.load<KP>(0, h, xl);
    // gate, columns 4 (lane % 32) .. + 3 of the head (used by lanes < 32 of waves 0 and 4)
    float4 gz[KP];
    {
        const float *g0 = a.mix.p + C + h * kDnDk + 4 * (lane & 31);
#pragma unroll
        for (int q = 0; q < KP; q++)
            gz[q] = *reinterpret_cast<const float4 *>(g0 + (size_t)min(q, a.mix.kp - 1) * a.mix.split);
    }
    const float sa = a.ssm_a[h], dtb = a.dt_bias[h];
    const float4 nw = reinterpret_cast<const float4 *>(a.norm_w)[lane & 31];
    u32x4 q[V], sc;
    load_part<T, 1>(q, sc, Wp + ((size_t)tile * nsb + ks) * Panel<T>::kBytes, Wp, wave, lane, true);
    asm volatile("" ::: "memory");
    const int cq = tt & 31, rg = tt >> 5;
    const float *Sh = a.S + ((size_t)h * kDnDk) * kDnDk + 4 * cq;
    float4 s[16];
#pragma unroll
    for (int r = 0; r < 16; r++) s[r] = *reinterpret_cast<const float4 *>(Sh + (size_t)(16 * rg + r) * kDnDk);

    // 1. conv + SiLU (deltanet_cache.rs:34-54) from the old windows; beta and
    // decay (deltanet.rs:474-480)
    const auto conv = [](float4 w0, float4 k, float x) {
        float sum = 0.0f;
        sum += w0.y * k.x;
        sum += w0.z * k.y;
        sum += w0.w * k.z;
        sum += x * k.w;
        return silu_dn(sum);
    };
    const float xin = a.mix.add<KP>(xa), xvin = a.mix.add<KP>(xv);
    const float y = conv(win, wk, xin);
    const float sq = wave_sum(y * y);  // waves 4 hh + 0 / 1: q, 4 hh + 2 / 3: k
    if (lane == 0) red[wave] = sq;
    if (tt < kDnDk) qn[hh][tt] = y;
    else kn[hh][e] = y;
    if (tt < kDnDk) vv[hh][tt] = conv(winv, wkv, xvin);
    const float beta = 1.0f / (1.0f + expf(-a.beta.add<KP>(xb)));
    const float decay = expf(sa * logf(1.0f + expf(a.alpha.add<KP>(xl) + dtb)));
    if (writer) {
        float *px = a.pend + 2 * d + a.n_heads;  // new conv inputs [3 d]
        px[ch] = xin;
        if (tt < kDnDk) px[chv] = xvin;
        if (tt == 0) a.pend[2 * d + h] = decay;
    }
    __syncthreads();
    // 2. L2 normalise (deltanet.rs:25-31, 461-467)
    if (tt < kDnDk) {
        const float inv = 1.0f / sqrtf((red[4 * hh] + red[4 * hh + 1]) + 1e-12f);
        qn[hh][tt] = (qn[hh][tt] * inv) * (1.0f / sqrtf((float)kDnDk));
    } else {
        const float inv = 1.0f / sqrtf((red[4 * hh + 2] + red[4 * hh + 3]) + 1e-12f);
        kn[hh][e] = kn[hh][e] * inv;
    }
    __syncthreads();
    // 3. S' = decay S, partial sums of S'^T k and S'^T q over this thread's
    // rows; k . q by the head's first two waves
    float4 sk = make_float4(0.f, 0.f, 0.f, 0.f), sqv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const float ki = kn[hh][16 * rg + r], qi = qn[hh][16 * rg + r];
        s[r].x *= decay; s[r].y *= decay; s[r].z *= decay; s[r].w *= decay;
        sk.x += s[r].x * ki; sk.y += s[r].y * ki; sk.z += s[r].z * ki; sk.w += s[r].w * ki;
        sqv.x += s[r].x * qi; sqv.y += s[r].y * qi; sqv.z += s[r].z * qi; sqv.w += s[r].w * qi;
    }
    pk[hh][rg][cq] = sk;
    pq[hh][rg][cq] = sqv;
    {
        const float kq = wave_sum(tt < kDnDk ? kn[hh][tt] * qn[hh][tt] : 0.0f);
        if (lane == 0) red2[wave] = kq;
    }
    if (writer && tt < kDnDk) a.pend[d + h * kDnDk + tt] = kn[hh][tt];
    __syncthreads();
    // 4. o = S'^T q + delta (k . q), delta = beta (v - S'^T k); gated RMSNorm
    // (deltanet.rs:517-533) into the digits of the GEMV input: lanes < 32 of
    // waves 0 and 4 hold 4 columns each of heads 2 ks and 2 ks + 1
    if ((wave & 3) == 0) {
        const int c4 = lane & 31;
        float4 a4 = pk[hh][0][c4], b4 = pq[hh][0][c4];
#pragma unroll
        for (int g = 1; g < 8; g++) {
            const float4 x = pk[hh][g][c4], z = pq[hh][g][c4];
            a4 = make_float4(a4.x + x.x, a4.y + x.y, a4.z + x.z, a4.w + x.w);
            b4 = make_float4(b4.x + z.x, b4.y + z.y, b4.z + z.z, b4.w + z.w);
        }
        const float kq = red2[4 * hh] + red2[4 * hh + 1];
        const float4 v4 = *reinterpret_cast<const float4 *>(&vv[hh][4 * c4]);
        const float4 dl = make_float4(beta * (v4.x - a4.x), beta * (v4.y - a4.y), beta * (v4.z - a4.z),
                                      beta * (v4.w - a4.w));
        const float4 o = make_float4(b4.x + dl.x * kq, b4.y + dl.y * kq, b4.z + dl.z * kq, b4.w + dl.w * kq);
        if (writer && lane < 32) *reinterpret_cast<float4 *>(a.pend + h * kDnDk + 4 * c4) = dl;
        float4 g = gz[0];
#pragma unroll
        for (int p = 1; p < KP; p++) {
            const bool on = p < a.mix.kp;
            g.x += on ? gz[p].x : 0.0f;
            g.y += on ? gz[p].y : 0.0f;
            g.z += on ? gz[p].z : 0.0f;
            g.w += on ? gz[p].w : 0.0f;
        }
        const float ss = half_sum(o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w);
        const float inv_rms = 1.0f / sqrtf(ss / (float)kDnDk + a.eps);
        const float4 u = make_float4(((o.x * inv_rms) * nw.x) * silu_dn(g.x), ((o.y * inv_rms) * nw.y) * silu_dn(g.y),
                                     ((o.z * inv_rms) * nw.z) * silu_dn(g.z), ((o.w * inv_rms) * nw.w) * silu_dn(g.w));
        put_digits<T>(u, 32 * hh + lane, lane < 32, xd, xq);
    }
    __syncthreads();
    // 5. the tile's rows over the split's panel: wave w takes block w (two
    // row tiles per workgroup, halving the state re-reads, measured slower:
    // 1189 against 1210 tok/s at batch 1)
    const float acc = panel_dot<T, 1>(q, sc, xd, xq, wave, 0.0f);
    gred[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        const int row = tile * kWave + lane;
        if (row < m) {
            float sum = gred[0][lane];
#pragma unroll
            for (int w = 1; w < kPackedWaves; w++) sum += gred[w][lane];
            out[(size_t)ks * m + row] = sum;
        }
    }
}

// Batch-1 GEMV of a matrix with few row tiles, in one launch: a workgroup of
// NW waves takes R = 64 / H rows of one tile over the whole K range, so the
// grid has tiles * H workgroups and no K split (no partial sums, no second
// launch).  Lane l serves row l % R of the workgroup's rows and slot
// wave * H + l / R; slot s takes the row's Q8_0 / Q4_0 blocks s, s + NW H,
// ... (J of them: 8 n / 256 = NW H J), whole blocks with their scales, every
// load issued before any is used.  x is staged in LDS (its loads issued
// before the weights', so waiting for them does not wait for the weights) as
// int8 digits (put_digits).  Per lane: block sums in block order, each scaled
// (q8_gemv.rs:234-242); then the H slots of a row held by one wave are added
// by lane exchanges and the NW waves' sums through LDS in wave order.
// Two forms: 16 waves with H = 4 (or 2), and 8 waves with H = 8 for
// matrices whose tiles x 4 would leave CUs idle.  Measured on MI355X (graphs
// of back-to-back launches, weights rotated, two boxes): 6144 x 2048 5.07 us
// (16 waves, H 4, 384 workgroups) against 5.43 (8 waves, H 8); 2048 x 6144
// 5.81-5.96 (8 waves, H 8, 256 workgroups) against 6.31-7.01 (16 waves, H 4,
// 128); 2048 x 2048 3.51 against 3.66-3.70; 4 waves of 4 rows (H 16)
// 8.4-9.0 us.
constexpr int kRowsWaves = 16;
constexpr int rows_waves(int H) { return H == 8 ? 8 : kRowsWaves; }
// blocks per lane slot of gemv_rows for n = 256 nsb columns and row split H
// (0 if they do not divide evenly)
inline int rows_blocks_per_slot(int nsb, int H) {
    const int slots = rows_waves(H) * H;
    return (8 * nsb) % slots ? 0 : 8 * nsb / slots;
}
constexpr int kRowsMaxN = 8192;

template <uint32_t T, int H, int J>
__global__ __launch_bounds__(kWave *rows_waves(H)) void gemv_rows(const uint8_t *__restrict__ Wp,
                                                                 const float *__restrict__ x, float *__restrict__ y,
                                                                 int m, int n) {
    constexpr int NW = rows_waves(H), R = kWave / H, SLOTS = NW * H, NT = kWave * NW;
    constexpr int VB = T == ANEHIP_GGML_Q8_0 ? 2 : 1;  // 16-byte quant vectors per block
    constexpr int XV = kRowsMaxN / 4 / NT;              // float4 of x per thread, at most
    __shared__ __align__(16) uint32_t xd[kRowsMaxN / 32 * kXdWords];
    __shared__ uint4 xq[kRowsMaxN / 32];
    __shared__ float red[NW][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int tile = blockIdx.x / H, h = blockIdx.x % H;
    const int r = lane % R, slot = wave * H + lane / R;
    const int rr = h * R + r;  // row within the tile
    const int nsb = n >> 8;

    float4 xv[XV];
    const int n4 = n >> 2;
#pragma unroll
    for (int i = 0; i < XV; i++) {
        const int e = min((int)threadIdx.x + i * NT, n4 - 1);
        xv[i] = reinterpret_cast<const float4 *>(x)[e];
    }
    const uint8_t *tb = Wp + (size_t)tile * nsb * Panel<T>::kBytes;
    u32x4 q[J][VB];
    uint32_t scw[J];
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int b = slot + j * SLOTS, bi = b & 7;
        const u32x4 *pp = reinterpret_cast<const u32x4 *>(tb + (size_t)(b >> 3) * Panel<T>::kBytes);
#pragma unroll
        for (int v = 0; v < VB; v++) q[j][v] = __builtin_nontemporal_load(pp + (VB * bi + v) * kWave + rr);
        scw[j] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(pp + Panel<T>::kChunks * kWave + rr) +
                                            (bi >> 1));
    }
#pragma unroll
    for (int i = 0; i < XV; i++) {
        const int e = (int)threadIdx.x + i * NT;
        if (i * NT < n4) put_digits<T>(xv[i], e, e < n4, xd, xq);  // uniform condition
    }
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int b = slot + j * SLOTS;
        const float d = __half2float(__ushort_as_half((unsigned short)(scw[j] >> (16 * (b & 1)))));
        acc = fmaf(block_dot_digits<T>(q[j], xd + b * kXdWords, xq[b]), d, acc);
    }
    // the H slots of a row within the wave (lanes r, r + R, ...) first, by
    // lane exchanges, then the 16 waves' sums through LDS
#pragma unroll
    for (int k = R; k < kWave; k <<= 1) acc += __shfl_xor(acc, k);
    if (lane < R) red[wave][lane] = acc;
    __syncthreads();
    if (threadIdx.x < R) {
        const int row = tile * kWave + h * R + (int)threadIdx.x;
        float sum = red[0][threadIdx.x];
#pragma unroll
        for (int w = 1; w < NW; w++) sum += red[w][threadIdx.x];
        if (row < m) y[row] = sum;
    }
}

// ---------------------------------------------------------------------------
// Small-batch GEMM over panels on MFMA (batch 2..32).
//
// v_mfma_f32_32x32x16_f16 with A = activations (32 batch rows x 16 columns,
// lane l: row l % 32, columns 8 (l / 32) .. +7) and B = weights (16 columns x
// 32 weight rows, lane l: weight row l % 32, columns 8 (l / 32) .. +7), so a
// lane's 16 outputs D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32] share one weight
// row and therefore one block scale.  A panel chunk gives lane l the 16
// columns of tile row l; one v_permlane32_swap per dword pair exchanges the
// upper lanes' first 8 columns with the lower lanes' last 8, which turns the
// chunk into the B operands of rows 0-31 and rows 32-63 with no LDS round
// trip.  int8 / nibble values become fp16 exactly (0x6400 | (u8) is 1024 + u8,
// minus 1152 or 1032).  Activations arrive as fp16 hi and lo planes (hi =
// fp16(x), lo = fp16(x - hi), |x - hi - lo| <= 2^-22 |x|), written by the
// producer of x, and read by each wave straight from global memory (a few
// hundred KiB, cache-resident): the two products summed in fp32 reproduce the
// fp32 GEMV within its tolerance.
// Per block: C = sum over its 2 column steps and the 2 planes, then
// acc += C * d (q8_gemv.rs:234-242 order within a block up to fp32 summation).
// ---------------------------------------------------------------------------

typedef _Float16 h8v __attribute__((ext_vector_type(8)));

// Range-safe planes on the GEMM side (see Planes): the largest exponent of
// groups [g0, g0 + ng) of batch row b.
// The row's exponents are read as dwords (a row starts 16-byte aligned, its
// length padded to 16 bytes), four at a time with every load issued before
// any is used, so the groups of a 2048-column row take one round trip.
__device__ __forceinline__ int xe_max(const int8_t *__restrict__ xe, int b, int g0, int ng, int n) {
    int E = kXeEmpty;
    const uint32_t *row = reinterpret_cast<const uint32_t *>(xe + (size_t)b * xe_stride(n));
    const int w0 = g0 >> 2, w1 = (g0 + ng + 3) >> 2, wl = xe_stride(n) / 4 - 1;
    for (int w = w0; w < w1; w += 4) {
        uint32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = row[min(w + k, wl)];
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int g = 4 * w + k;
            const int e = (int)(int8_t)(v[k >> 2] >> (8 * (k & 3)));
            E = g >= g0 && g < g0 + ng ? max(E, e) : E;
        }
    }
    return E;
}

// fp32 sums of x * 2^-E back to x's scale.
__device__ __forceinline__ float4 ldexp4(float4 v, int E) {
    return make_float4(ldexpf(v.x, E), ldexpf(v.y, E), ldexpf(v.z, E), ldexpf(v.w, E));
}
// The same as one multiply by 2^E: exact for every exponent group_exp gives
// (2^E is an fp32 value for E >= -149).
__device__ __forceinline__ float xe_scale(int E) { return ldexpf(1.0f, E); }
__device__ __forceinline__ float4 mul4(float4 v, float f) { return make_float4(v.x * f, v.y * f, v.z * f, v.w * f); }
// The exponent of batch row first + (threadIdx / 16) % 4, read from lanes
// first .. first + 3 (which hold rows first .. first + 3; first uniform):
// readlane, no LDS -- an LDS permute here measured slower.
__device__ __forceinline__ int row_exp4(int E, int first) {
    const int e0 = __builtin_amdgcn_readlane(E, first), e1 = __builtin_amdgcn_readlane(E, first + 1);
    const int e2 = __builtin_amdgcn_readlane(E, first + 2), e3 = __builtin_amdgcn_readlane(E, first + 3);
    const int k = (threadIdx.x >> 4) & 3;
    return k == 0 ? e0 : k == 1 ? e1 : k == 2 ? e2 : e3;
}

// The fp32-rows path of the x-stationary kernels: 8 consecutive columns of a
// row, and their hi / lo fragments for x * 2^-E.
__device__ __forceinline__ void load8(const float *p, float (&v)[8]) {
    const float4 a = *reinterpret_cast<const float4 *>(p), b = *reinterpret_cast<const float4 *>(p + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}
__device__ __forceinline__ float amax8(const float *p, float m) {
    float v[8];
    load8(p, v);
#pragma unroll
    for (int i = 0; i < 8; i++) m = fmaxf(m, fabsf(v[i]));
    return m;
}
__device__ __forceinline__ void split8_scaled(const float (&v)[8], int E, h8v &hi, h8v &lo) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        _Float16 h, l;
        split_scaled(v[i], E, h, l);
        hi[i] = h;
        lo[i] = l;
    }
}

typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemmWaves = 4;
constexpr int kGemmRing = 2;  // panel GEMM: units in flight per wave
// word 3 of a raw buffer resource on gfx9-family parts (data format 32 bit)
constexpr int kBufferWord3 = 0x00020000;

// Four signed int8 (one dword) -> four fp16, exact.
__device__ __forceinline__ void i8x4_to_h(uint32_t d, _Float16 *o) {
    const uint32_t u = d ^ 0x80808080u;  // q + 128 as unsigned bytes
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // (1024 + u0, 1024 + u1)
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // (1024 + u2, 1024 + u3)
    const h2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const h2v a = __builtin_bit_cast(h2v, p0) - bias, b = __builtin_bit_cast(h2v, p1) - bias;
    o[0] = a[0];
    o[1] = a[1];
    o[2] = b[0];
    o[3] = b[1];
}

// Four nibbles in bytes (values 0..15, one dword) -> four fp16 of (v - 8), exact.
__device__ __forceinline__ void u4x4_to_h(uint32_t nib, _Float16 *o) {
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, nib, 0x04010400u);
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, nib, 0x04030402u);
    const h2v bias = {(_Float16)1032.0f, (_Float16)1032.0f};
    const h2v a = __builtin_bit_cast(h2v, p0) - bias, b = __builtin_bit_cast(h2v, p1) - bias;
    o[0] = a[0];
    o[1] = a[1];
    o[2] = b[0];
    o[3] = b[1];
}

__device__ __forceinline__ h8v dwords_to_h8_i8(uint32_t d0, uint32_t d1) {
    _Float16 t[8];
    i8x4_to_h(d0, t);
    i8x4_to_h(d1, t + 4);
    return h8v{t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7]};
}

__device__ __forceinline__ h8v dwords_to_h8_u4(uint32_t d0, uint32_t d1) {
    _Float16 t[8];
    u4x4_to_h(d0, t);
    u4x4_to_h(d1, t + 4);
    return h8v{t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7]};
}

// Swaps the upper lanes' (a0, a1) with the lower lanes' (b0, b1): afterwards
// (a0, a1) hold the columns of rows 0-31 and (b0, b1) those of rows 32-63.
__device__ __forceinline__ void swap_halves(uint32_t &a0, uint32_t &a1, uint32_t &b0, uint32_t &b1) {
    const auto s0 = __builtin_amdgcn_permlane32_swap(a0, b0, false, false);
    const auto s1 = __builtin_amdgcn_permlane32_swap(a1, b1, false, false);
    a0 = s0[0];
    b0 = s0[1];
    a1 = s1[0];
    b1 = s1[1];
}

// Barrier for LDS traffic only: the fences order LDS accesses, so waves do
// not wait for their outstanding global loads (the prefetched units) here.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One wave's operands for one panel of its TV tiles: per tile the quant
// vectors of its column quarter q (blocks 2q, 2q + 1: Q8_0 chunks 4q..4q+3,
// Q4_0 chunks 2q, 2q+1) and the lane row's 16-byte scale vector; and the A
// fragments of x for the quarter's 4 column steps (hi and lo planes, fragment
// order), shared by the TV tiles.
template <uint32_t T, int TV> struct GemmUnit {
    static constexpr int kQ = T == ANEHIP_GGML_Q8_0 ? 4 : 2;
    u32x4 q[TV][kQ];
    u32x4 sc[TV];
    h8v ah[4], al[4];
    int xe;  // exponent of the fragments' column group (range-safe planes)
};

// Loads one unit: every lane issues the same, fully contiguous 1 KiB loads
// (no lane masking, so the compiler's vmcnt waits stay exact).  `panel` is the
// first tile's panel, the others follow at `tile_bytes`.  `xo` is the lane's
// element offset of its first A fragment in the fragment-order planes (rows
// past the batch are redirected to row batch - 1: those lanes only feed MFMA
// output rows that are never stored, and their loads hit the cache).
template <uint32_t T, int TV>
__device__ __forceinline__ void gemm_load(GemmUnit<T, TV> &u, const uint8_t *panel, size_t tile_bytes,
                                          const _Float16 *__restrict__ xh, const _Float16 *__restrict__ xl, size_t xo,
                                          const int8_t *__restrict__ xe, int quarter, int lane) {
    constexpr int Q = GemmUnit<T, TV>::kQ;
#pragma unroll
    for (int t = 0; t < TV; t++) {
        const u32x4 *p4 = reinterpret_cast<const u32x4 *>(panel + t * tile_bytes);
#pragma unroll
        for (int c = 0; c < Q; c++) u.q[t][c] = __builtin_nontemporal_load(p4 + (Q * quarter + c) * kWave + lane);
        u.sc[t] = __builtin_nontemporal_load(p4 + Panel<T>::kChunks * kWave + lane);
    }
#pragma unroll
    for (int s = 0; s < 4; s++) {
        u.ah[s] = *reinterpret_cast<const h8v *>(xh + xo + 512 * s);
        u.al[s] = *reinterpret_cast<const h8v *>(xl + xo + 512 * s);
    }
    u.xe = *xe;
}

// acc{0,1} += one tile's two blocks of a quarter: q = its quant vectors, sc
// the lane row's scale vector, ah / al the x fragments of the quarter's 4
// column steps.  Per block C = sum over its 2 column steps and the 2 planes
// (4 MFMAs per 32 weight rows), then acc += C * d (q8_gemv.rs:234-242 order
// within a block up to fp32 summation).
template <uint32_t T>
__device__ __forceinline__ uint32_t quarter_scales(const u32x4 &sv, int quarter) {
    return quarter == 0 ? sv.x : quarter == 1 ? sv.y : quarter == 2 ? sv.z : sv.w;
}

// sw: dword `quarter` of the lane's scale vector (blocks 2q, 2q + 1)
template <uint32_t T>
__device__ __forceinline__ void mma_tile(const u32x4 *q, uint32_t sw, const h8v *ah, const h8v *al, f32x16 &acc0,
                                         f32x16 &acc1) {
    // after the swap s0 / s1 are the scales of weight rows l % 32 and 32 + l % 32
    const auto sp = __builtin_amdgcn_permlane32_swap(sw, sw, false, false);
    const uint32_t s0 = sp[0], s1 = sp[1];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        f32x16 c0 = {}, c1 = {};
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int s = 2 * j + h;  // column step: columns 16 s .. 16 s + 15 of the quarter
            h8v b0, b1;
            if constexpr (T == ANEHIP_GGML_Q8_0) {
                const u32x4 v = q[s];
                uint32_t a0 = v.x, a1 = v.y, c0w = v.z, c1w = v.w;
                swap_halves(a0, a1, c0w, c1w);
                b0 = dwords_to_h8_i8(a0, a1);
                b1 = dwords_to_h8_i8(c0w, c1w);
            } else {
                const u32x4 v = q[j];
                uint32_t a0 = v.x, a1 = v.y, c0w = v.z, c1w = v.w;
                swap_halves(a0, a1, c0w, c1w);
                const uint32_t sh = 4 * h;  // step 0: low nibbles, step 1: high nibbles
                b0 = dwords_to_h8_u4((a0 >> sh) & 0x0F0F0F0Fu, (a1 >> sh) & 0x0F0F0F0Fu);
                b1 = dwords_to_h8_u4((c0w >> sh) & 0x0F0F0F0Fu, (c1w >> sh) & 0x0F0F0F0Fu);
            }
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[s], b0, c0, 0, 0, 0);
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[s], b0, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[s], b1, c1, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[s], b1, c1, 0, 0, 0);
        }
        const float d0 = __half2float(__ushort_as_half((unsigned short)(s0 >> (16 * j))));
        const float d1 = __half2float(__ushort_as_half((unsigned short)(s1 >> (16 * j))));
#pragma unroll
        for (int r = 0; r < 16; r++) {
            acc0[r] = fmaf(c0[r], d0, acc0[r]);
            acc1[r] = fmaf(c1[r], d1, acc1[r]);
        }
    }
}

template <uint32_t T, int TV>
__device__ __forceinline__ void gemm_mma(const GemmUnit<T, TV> &u, int quarter, f32x16 (&acc)[TV][2]) {
#pragma unroll
    for (int t = 0; t < TV; t++)
        mma_tile<T>(u.q[t], quarter_scales<T>(u.sc[t], quarter), u.ah, u.al, acc[t][0], acc[t][1]);
}

// End of a tile's item: every wave parks its 32 sums per lane (accumulator
// element r of lane l: batch row 8 (r / 4 % 4) + 4 (l / 32) + r % 4, tile row
// l % 32 + 32 (r / 16)); then each of the 256 threads adds the 4 quarters of
// two 4-row vectors of one batch row and stores them with 16-byte buffer
// stores (rows outside the batch or the matrix, or store == false, take an
// offset past the buffer and are dropped).  red: [4][32][64] floats.  CPOL:
// the stores' cache-policy bits.
constexpr int kBadOffset = 0x7ffffff0;  // buffer offset past any output: the store is dropped
// Cache-policy bit sc1 (device scope): the store is written through to the
// point of coherence of all XCDs.  For the K-split partials, which a later
// kernel reads once, this measured 2 % faster over a batch-32 decode step
// (non-temporal stores: 2 % slower).
constexpr int kCpolDevice = 16;
// Cache-policy bit nt for streamed weight loads through buffer resources (the
// other kernels use __builtin_nontemporal_load): prefill of 2048 tokens
// 48.6 -> 47.9-48.1 ms.
constexpr int kCpolNtLoad = 2;

template <int CPOL = 0>
__device__ __forceinline__ void gemm_tile_epilogue(float (*red)[32][kWave], const float (&fEb)[2], const f32x16 &acc0,
                                                   const f32x16 &acc1, int quarter, int lane, int tile, int ks,
                                                   int batch, int m, size_t split_stride,
                                                   __amdgpu_buffer_rsrc_t orsrc, bool store) {
#pragma unroll
    for (int r = 0; r < 16; r++) {
        red[quarter][r][lane] = acc0[r];
        red[quarter][16 + r][lane] = acc1[r];
    }
    lds_barrier();
    const int th = threadIdx.x & (kWave * kGemmWaves - 1);
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int v = th + 256 * i;  // 512 vectors: batch row b, rows 4 j .. 4 j + 3
        const int b = v >> 4, j = v & 15;
        const int r = 4 * (b >> 3) + (b & 3) + (j >= 8 ? 16 : 0);
        const int l = ((4 * j) & 31) + 32 * ((b >> 2) & 1);
        float4 sum = *reinterpret_cast<const float4 *>(&red[0][r][l]);
#pragma unroll
        for (int w = 1; w < kGemmWaves; w++) {
            const float4 o = *reinterpret_cast<const float4 *>(&red[w][r][l]);
            sum = make_float4(sum.x + o.x, sum.y + o.y, sum.z + o.z, sum.w + o.w);
        }
        sum = mul4(sum, fEb[i]);  // the fragments' exponent of batch row b
        const int row = tile * kWave + 4 * j;
        const int off = store && b < batch && row < m ? 4 * (ks * (int)split_stride + b * m + row) : kBadOffset;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sum), orsrc, off, 0, CPOL);
    }
    lds_barrier();  // red is free again
}

// Persistent panel GEMM.  A workgroup has 4 waves, one per column quarter q
// (blocks 2q, 2q + 1 of every panel), and covers TV consecutive 64-row tiles:
// each wave multiplies the x fragments it loads with all TV tiles' weights
// (TV = 2 halves the x loads per weight byte, at one wave per SIMD for the
// registers).  Work items are (tile group, K split), item = group * ksplit +
// split; workgroup g takes items g, g + G, g + 2G, ...  A tile's 4 quarter
// sums are added through LDS.  The waves walk their (item, panel) units with
// D units in flight in registers -- the loads of unit u + D are issued right
// after unit u is multiplied, across item boundaries too -- so the main loop
// has no barrier and no wait for the prefetched loads.  Output as
// quant_gemm_tiled: out[split * split_stride + b * m + row], stored as
// 16-byte row vectors (m % 4 == 0).
template <uint32_t T, int TV, int D, int WPE = (TV == 1 ? 2 : 1)>
__global__ __launch_bounds__(kWave *kGemmWaves) __attribute__((amdgpu_waves_per_eu(WPE))) void gemm_packed(
    const uint8_t *__restrict__ Wp, Planes xp, float *__restrict__ out, int m, int n, int batch, int ksplit, int per,
    size_t split_stride) {
    __shared__ __align__(16) float red[kGemmWaves][TV * 32][kWave];
    __shared__ int xeE[32];
    const _Float16 *__restrict__ xh = xp.hi;
    const _Float16 *__restrict__ xl = xp.lo;
    const int nsb = n >> 8, tiles = (m + kWave - 1) / kWave, groups = (tiles + TV - 1) / TV;
    const int items = groups * ksplit, G = gridDim.x;
    if ((int)blockIdx.x >= items) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int quarter = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int brow = min(lane & 31, batch - 1);
    const size_t xbase = (size_t)(4 * quarter * kWave + brow + 32 * (lane >> 5)) * 8;
    // range-safe planes: every unit's fragments are brought to one exponent
    // per batch row over the whole row (units are loaded across items)
    const int E = xe_max(xp.xe, brow, 0, 2 * nsb, n);
    if (quarter == 0 && lane < 32) xeE[lane] = E;  // read after the first epilogue barrier
    const int8_t *xe_lane = xp.xe + (size_t)brow * xe_stride(n) + (quarter >> 1);  // + 2 per panel
    const size_t tile_bytes = (size_t)nsb * Panel<T>::kBytes;
    const __amdgpu_buffer_rsrc_t orsrc =
        __builtin_amdgcn_make_buffer_rsrc(out, 0, (int)(4 * ksplit * split_stride), kBufferWord3);
    // first tile of an item's group (clamped so that all TV tiles' loads stay
    // inside the matrix; outputs of tiles past the last are dropped)
    auto first_tile = [&](int item) { return min((item / ksplit) * TV, tiles - TV); };

    // compute cursor (ci, cp, ce) and load cursor (li, lp, le): item, panel, end panel
    int ci = blockIdx.x, cp = (ci % ksplit) * per, ce = min(nsb, cp + per);
    int li = ci, lp = cp, le = ce;
    const uint8_t *lpanel = Wp + (size_t)first_tile(li) * tile_bytes + (size_t)lp * Panel<T>::kBytes;
    size_t lxo = xbase + 16 * 512 * (size_t)lp;
    // the load cursor steps to the next unit; every step issues its loads
    auto load_next = [&](GemmUnit<T, TV> &u) {
        gemm_load<T, TV>(u, lpanel, tile_bytes, xh, xl, lxo, xe_lane + 2 * lp, quarter, lane);
        // branch-free cursor step (selects keep the loop body one basic block)
        const bool wrap = ++lp == le;
        const int ni = li + G;
        const int np = (ni % ksplit) * per;
        li = wrap ? ni : li;
        lp = wrap ? np : lp;
        le = wrap ? min(nsb, np + per) : le;
        // past the last item the unit is a valid panel of the last group (lp
        // always lies in a non-empty split), loaded and never used
        lpanel = Wp + (size_t)first_tile(min(li, items - 1)) * tile_bytes + (size_t)lp * Panel<T>::kBytes;
        lxo = xbase + 16 * 512 * (size_t)lp;
    };
    f32x16 acc[TV][2];
#pragma unroll
    for (int t = 0; t < TV; t++) acc[t][0] = acc[t][1] = f32x16{};
    // multiplies unit u, refills it with the unit D ahead; at the end of an
    // item reduces and stores it.  Past the workgroup's last item (ci >=
    // items) a step is harmless: its loads are valid and its stores fall
    // outside the output range and are dropped.
    auto step = [&](GemmUnit<T, TV> &u) {
        const _Float16 f = xe_factor(u.xe, E);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            u.ah[s] = u.ah[s] * f;
            u.al[s] = u.al[s] * f;
        }
        gemm_mma<T, TV>(u, quarter, acc);
        // the refill reuses u's registers only if it is issued after u's last
        // use (the scale FMAs); otherwise the loop carries register copies
        // that wait for the prefetched loads.  The empty asm pins the
        // accumulation here.
#pragma unroll
        for (int t = 0; t < TV; t++) asm volatile("" : "+v"(acc[t][0]), "+v"(acc[t][1])::"memory");
        load_next(u);
        if (++cp < ce) return;
        // item done: every wave parks its 32 sums per lane and tile
        // (accumulator element r of lane l: batch row 8 (r / 4 % 4) +
        // 4 (l / 32) + r % 4, tile row l % 32 + 32 (r / 16)); then each thread
        // adds the 4 quarters of 4-row vectors of one batch row and stores them
#pragma unroll
        for (int t = 0; t < TV; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                red[quarter][32 * t + r][lane] = acc[t][0][r];
                red[quarter][32 * t + 16 + r][lane] = acc[t][1][r];
            }
        lds_barrier();
        {
            const int ks = ci % ksplit, tile0 = (ci / ksplit) * TV, ft = first_tile(ci);
            const int th = threadIdx.x;
#pragma unroll
            for (int i = 0; i < 2 * TV; i++) {
                const int v = th + 256 * i;  // 512 vectors per tile: batch row b, rows 4 j .. 4 j + 3
                const int t = v >> 9, b = (v >> 4) & 31, j = v & 15;
                const int r = 32 * t + 4 * (b >> 3) + (b & 3) + (j >= 8 ? 16 : 0);
                const int l = ((4 * j) & 31) + 32 * ((b >> 2) & 1);
                float4 sum = *reinterpret_cast<const float4 *>(&red[0][r][l]);
#pragma unroll
                for (int w = 1; w < kGemmWaves; w++) {
                    const float4 o = *reinterpret_cast<const float4 *>(&red[w][r][l]);
                    sum = make_float4(sum.x + o.x, sum.y + o.y, sum.z + o.z, sum.w + o.w);
                }
                sum = ldexp4(sum, xeE[b]);
                // the group's tile t is tile ft + t of the loads; it is stored
                // only if it is the item's own tile (not a clamped re-read)
                const int tile = ft + t, row = tile * kWave + 4 * j;
                const int off = b < batch && tile >= tile0 && row < m && ci < items
                                    ? 4 * (ks * (int)split_stride + b * m + row)
                                    : kBadOffset;
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sum), orsrc, off, 0, 0);
            }
        }
        lds_barrier();  // red is free again
#pragma unroll
        for (int t = 0; t < TV; t++) acc[t][0] = acc[t][1] = f32x16{};
        ci += G;
        cp = (ci % ksplit) * per;
        ce = min(nsb, cp + per);
    };
    // a ring of D units in registers (constant indices after unrolling)
    GemmUnit<T, TV> ring[D];
#pragma unroll
    for (int k = 0; k < D; k++) load_next(ring[k]);
    // one exit, after the last step of the ring: an exit between steps would
    // give the back edge a path that skips a refill (the compiler merges exit
    // tests into the latch) and make the load waits conservative
    do {
#pragma unroll
        for (int k = 0; k < D; k++) step(ring[k]);
    } while (ci < items);
}

// ---- batch <= 16: v_mfma_f32_16x16x32_f16 ----
// A 16 x 16 x 32 MFMA covers one 32-column block: lane l holds A row l % 16
// (a batch row) and B column l % 16 (a weight row), each with columns
// 8 (l / 16) .. 8 (l / 16) + 7, and gets C rows 4 (l / 16) .. + 3 of column
// l % 16.  Against the 32 x 32 x 16 form at batch <= 16 it halves the MFMA
// work, the block-scale FMAs and the x fragments a unit loads.

// 4 x 4 transpose over the 16-lane groups of a wave: afterwards r[g] of the
// lane at position i of group G holds what r[G] held at position i of group
// g.  (v_permlane32_swap exchanges the upper half of its first operand with
// the lower half of its second; v_permlane16_swap the odd 16-lane groups of
// its first operand with the even groups of its second.)
__device__ __forceinline__ void transpose_groups(uint32_t (&r)[4]) {
    const auto s02 = __builtin_amdgcn_permlane32_swap(r[0], r[2], false, false);
    const auto s13 = __builtin_amdgcn_permlane32_swap(r[1], r[3], false, false);
    const auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
    const auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
    r[0] = s01[0];
    r[1] = s01[1];
    r[2] = s23[0];
    r[3] = s23[1];
}

// One wave's operands for one quarter of one panel: the quant vectors as in
// GemmUnit, the quarter's dword of the lane row's scale vector, and the A
// fragments of the quarter's two blocks (hi and lo planes).
template <uint32_t T> struct GemmUnit16 {
    static constexpr int kQ = GemmUnit<T, 1>::kQ;
    u32x4 q[kQ];
    uint32_t sc;
    h8v ah[2], al[2];
};

// acc[g] += the quarter's two blocks for weight rows 16 g .. 16 g + 15 of the
// tile.  The panel gives lane l weight row l; the B fragment of row group g
// needs, at lane l of group G, row 16 g + l % 16 and the block's columns
// 8 G .. 8 G + 7, so the quant dwords (and the row scales) go through
// transpose_groups first.  Per block and row group: C = A_hi B + A_lo B, then
// acc += C * d (q8_gemv.rs:234-242 order within a block up to fp32 summation).
template <uint32_t T>
__device__ __forceinline__ void mma_tile16(const u32x4 *q, uint32_t sw, const h8v *ah, const h8v *al,
                                           f32x4 (&acc)[4], int grp) {
    uint32_t s[4] = {sw, sw, sw, sw};
    transpose_groups(s);  // s[g]: scales of blocks 2q, 2q + 1 of weight row 16 g + lane % 16
#pragma unroll
    for (int j = 0; j < 2; j++) {
        // piece G' of a row = the dwords of its block columns 8 G' .. 8 G' + 7
        uint32_t lo[4], hi[4];
        if constexpr (T == ANEHIP_GGML_Q8_0) {
            const u32x4 a = q[2 * j], b = q[2 * j + 1];
            lo[0] = a.x, hi[0] = a.y, lo[1] = a.z, hi[1] = a.w;
            lo[2] = b.x, hi[2] = b.y, lo[3] = b.z, hi[3] = b.w;
        } else {
            // columns 0-15 are the low nibbles of the block's 16 bytes, 16-31
            // the high ones: pieces 2, 3 repeat the bytes of pieces 0, 1
            const u32x4 v = q[j];
            lo[0] = lo[2] = v.x, hi[0] = hi[2] = v.y;
            lo[1] = lo[3] = v.z, hi[1] = hi[3] = v.w;
        }
        transpose_groups(lo);
        transpose_groups(hi);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            h8v b;
            if constexpr (T == ANEHIP_GGML_Q8_0) {
                b = dwords_to_h8_i8(lo[g], hi[g]);
            } else {
                const uint32_t sh = 4 * (grp >> 1);  // groups 2, 3: high nibbles
                b = dwords_to_h8_u4((lo[g] >> sh) & 0x0F0F0F0Fu, (hi[g] >> sh) & 0x0F0F0F0Fu);
            }
            f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[j], b, f32x4{}, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[j], b, c, 0, 0, 0);
            const float d = __half2float(__ushort_as_half((unsigned short)(s[g] >> (16 * j))));
#pragma unroll
            for (int r = 0; r < 4; r++) acc[g][r] = fmaf(c[r], d, acc[g][r]);
        }
    }
}

// x-stationary GEMM for batch <= 16 on the 16 x 16 x 32 MFMA.  Workgroup g
// works on split ks = g % ksplit (P consecutive panels) and the tiles
// g / ksplit + i * (gridDim.x / ksplit); each of its 4 waves holds its column
// quarter's A fragments of the split's P panels (16 P VGPRs) and streams
// units of one panel quarter of one tile (4 quant vectors and one scale
// dword, 17 VGPRs), D of them in flight in a register ring.  The loop body
// covers U = max(P, D) units so that ring slots and panels are compile-time
// indices; a tile's sums are added over the quarters through LDS.  Loads
// past the last tile are clamped to it and their results stored nowhere.
// Output: out[ks * split_stride + b * m + row] (device-scope stores).
template <uint32_t T, int P, int D, int WPE, bool XROWS = false>
__global__ __launch_bounds__(kWave *kGemmWaves) __attribute__((amdgpu_waves_per_eu(WPE))) void gemm_xs16(
    const uint8_t *__restrict__ Wp, Planes xp, const float *__restrict__ xrows, float *__restrict__ out, int m, int n,
    int batch, int ksplit, size_t split_stride) {
    constexpr int Q = GemmUnit16<T>::kQ;
    constexpr int U = P > D ? P : D;
    static_assert(U % P == 0 && U % D == 0, "ring and panel counts must divide the loop body");
    __shared__ __align__(16) float red[kGemmWaves][16][kWave];
    __shared__ int emax[kGemmWaves][16];
    __shared__ int ew[kGemmWaves][16];  // [wave][batch row]: the exponent of the wave's fragments
    const int nsb = n >> 8, tiles = (m + kWave - 1) / kWave;
    const int gs = gridDim.x / ksplit;  // workgroups per split
    const int ks = blockIdx.x % ksplit, g0 = blockIdx.x / ksplit;
    if (g0 >= gs || g0 >= tiles) return;
    const int lane = threadIdx.x & (kWave - 1), grp = lane >> 4;
    // the weight base in SGPRs now: the weight ring's first loads must not
    // wait for a kernel-argument load issued after the x loads
    asm volatile("" ::"s"(Wp));
    const int quarter = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const size_t tile_bytes = (size_t)nsb * Panel<T>::kBytes;
    const __amdgpu_buffer_rsrc_t orsrc =
        __builtin_amdgcn_make_buffer_rsrc(out, 0, (int)(4 * ksplit * split_stride), kBufferWord3);
    // A fragments: batch row lane % 16 (clamped to the batch), columns
    // 64 quarter + 32 j + 8 (lane / 16) of each panel of the split, brought
    // to x * 2^-E: from the planes one exponent E per batch row for the whole
    // split, from fp32 rows one per batch row and wave (over the wave's
    // columns); each wave's sums are scaled by its 2^E when the quarters are
    // added.  The x loads go out first, then the weight ring's, and the
    // fragments are formed after both were issued: that waits for the x
    // loads only.
    h8v xa[P][2], xb[P][2];
    float xv[XROWS ? P : 1][2][8];  // fp32 rows: the split's values of this lane
    const int brow = min(lane & 15, batch - 1);
    const float *xr = XROWS ? xrows + (size_t)brow * n : nullptr;
    auto xcol = [&](int p, int j) { return 256 * (ks * P + p) + 64 * quarter + 32 * j + 8 * grp; };
    int xe_own[P];  // exponents of this quarter's group of each panel
    // small splits load every group's exponent (no exchange between waves)
    constexpr int NG = 2 * P;
    constexpr bool kDirect = NG <= 8;
    int xe_all[kDirect ? NG : 1];
    int E = 0;
    if constexpr (!XROWS) {
        const size_t xbase = (size_t)((4 * quarter + (grp >> 1)) * kWave + brow + 32 * (grp & 1)) * 8 +
                             16 * 512 * (size_t)(ks * P);
        if constexpr (kDirect) {
#pragma unroll
            for (int g = 0; g < NG; g++) xe_all[g] = xp.xe[(size_t)brow * xe_stride(n) + 2 * ks * P + g];
        }
#pragma unroll
        for (int p = 0; p < P; p++) {
            if constexpr (kDirect) xe_own[p] = (quarter >> 1) ? xe_all[2 * p + 1] : xe_all[2 * p];
            else xe_own[p] = xp.xe[(size_t)brow * xe_stride(n) + 2 * (ks * P + p) + (quarter >> 1)];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                xa[p][j] = *reinterpret_cast<const h8v *>(xp.hi + xbase + 16 * 512 * p + 1024 * j);
                xb[p][j] = *reinterpret_cast<const h8v *>(xp.lo + xbase + 16 * 512 * p + 1024 * j);
            }
        }
    } else {
#pragma unroll
        for (int p = 0; p < P; p++)
#pragma unroll
            for (int j = 0; j < 2; j++) load8(xr + xcol(p, j), xv[p][j]);
    }
    const uint8_t *wsplit = Wp + (size_t)(ks * P) * Panel<T>::kBytes;
    int lt = g0, lp = 0;  // load cursor: tile, panel within the split
    auto load_next = [&](GemmUnit16<T> &u) {
        const u32x4 *p4 = reinterpret_cast<const u32x4 *>(wsplit + (size_t)min(lt, tiles - 1) * tile_bytes +
                                                          (size_t)lp * Panel<T>::kBytes);
#pragma unroll
        for (int c = 0; c < Q; c++) u.q[c] = __builtin_nontemporal_load(p4 + (Q * quarter + c) * kWave + lane);
        u.sc = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p4 + Panel<T>::kChunks * kWave + lane) +
                                          quarter);
        const bool wrap = ++lp == P;
        lp = wrap ? 0 : lp;
        lt = wrap ? lt + gs : lt;
    };
    // the empty asm statements keep the ring in order (as in gemm_xs)
    GemmUnit16<T> ring[D];
#pragma unroll
    for (int k = 0; k < D; k++) {
        load_next(ring[k]);
        asm volatile("" ::: "memory");
    }
    if constexpr (!XROWS) {
        // planes: E over the split -- from all of its exponents, or each
        // wave's groups and then the 4 waves through LDS (quarters 0, 1 hold
        // a panel's first group, 2, 3 its second); the scaling waits for the
        // x loads only
        if constexpr (kDirect) {
            E = kXeEmpty;
#pragma unroll
            for (int g = 0; g < NG; g++) E = max(E, xe_all[g]);
        } else {
            int e = kXeEmpty;
#pragma unroll
            for (int p = 0; p < P; p++) e = max(e, xe_own[p]);
            if (lane < 16) emax[quarter][lane] = e;
            lds_barrier();
            E = max(max(emax[0][lane & 15], emax[1][lane & 15]), max(emax[2][lane & 15], emax[3][lane & 15]));
        }
#pragma unroll
        for (int p = 0; p < P; p++) {
            const _Float16 f = xe_factor(xe_own[p], E);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                xa[p][j] = xa[p][j] * f;
                xb[p][j] = xb[p][j] * f;
            }
        }
    } else {
        // fp32 rows (API path, splits of at most 2 panels): E from the row's
        // largest |x| over this wave's columns -- lanes l, l ^ 16, l ^ 32,
        // l ^ 48 hold the row
        float amax = 0.0f;
#pragma unroll
        for (int p = 0; p < P; p++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(xv[p][j][i]));
        E = group_exp(lanes_max4(amax));
#pragma unroll
        for (int p = 0; p < P; p++)
#pragma unroll
            for (int j = 0; j < 2; j++) split8_scaled(xv[p][j], E, xa[p][j], xb[p][j]);
    }
    if (lane < 16) ew[quarter][lane] = E;  // lane l holds batch row l (read after the tile's barrier)
    int ct = g0;  // tile being multiplied
    f32x4 acc[4];
#pragma unroll
    for (int g = 0; g < 4; g++) acc[g] = f32x4{};
    do {
#pragma unroll
        for (int k = 0; k < U; k++) {
            GemmUnit16<T> &u = ring[k % D];
#pragma unroll
            for (int c = 0; c < Q; c++) asm volatile("" : "+v"(u.q[c])::"memory");
            asm volatile("" : "+v"(u.sc)::"memory");
            mma_tile16<T>(u.q, u.sc, xa[k % P], xb[k % P], acc, grp);
#pragma unroll
            for (int g = 0; g < 4; g++) asm volatile("" : "+v"(acc[g])::"memory");
            load_next(u);
            if (k % P == P - 1) {
                // tile done: park the 16 sums per lane (acc[g][r] of lane l:
                // batch row 4 (l / 16) + r, tile row 16 g + l % 16), then each
                // thread adds the 4 quarters of one 4-row vector of one batch row
#pragma unroll
                for (int g = 0; g < 4; g++)
#pragma unroll
                    for (int r = 0; r < 4; r++) red[quarter][4 * g + r][lane] = acc[g][r];
                lds_barrier();
                {
                    const int th = threadIdx.x, b = th >> 4, j = th & 15;
                    const int reg = 4 * (j >> 2) + (b & 3), l = 16 * (b >> 2) + 4 * (j & 3);
                    // each quarter's sums times its 2^E (exact), added in quarter order
                    float4 sum = mul4(*reinterpret_cast<const float4 *>(&red[0][reg][l]), xe_scale(ew[0][b]));
#pragma unroll
                    for (int w = 1; w < kGemmWaves; w++) {
                        const float4 o = mul4(*reinterpret_cast<const float4 *>(&red[w][reg][l]), xe_scale(ew[w][b]));
                        sum = make_float4(sum.x + o.x, sum.y + o.y, sum.z + o.z, sum.w + o.w);
                    }
                    const int row = ct * kWave + 4 * j;
                    const int off = b < batch && row < m && ct < tiles ? 4 * (ks * (int)split_stride + b * m + row)
                                                                       : kBadOffset;
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sum), orsrc, off, 0,
                                                           kCpolDevice);
                }
                lds_barrier();  // red is free again
#pragma unroll
                for (int g = 0; g < 4; g++) acc[g] = f32x4{};
                ct += gs;
            }
        }
    } while (ct < tiles);
}

// x-stationary panel GEMM for K-split shapes.  Workgroup g works on split
// ks = g % ksplit only (its P panels); each wave loads the x fragments of its
// column quarter in those panels once (32 P VGPRs) and then streams the
// weights of its tiles t = g / ksplit, g / ksplit + G / ksplit, ...: a unit
// (one panel of one tile) is 5 loads -- 4 quant vectors and the quarter's
// dword of the scale vector -- instead of 13.  R tiles (R * P units) are in flight in a register ring;
// as in gemm_packed the loop's single exit and branch-free cursors keep the
// vmcnt waits exact, and tiles past the workgroup's last are loaded clamped
// and stored nowhere.  Same arithmetic and output as gemm_packed.
template <uint32_t T> struct WUnit {
    u32x4 q[GemmUnit<T, 1>::kQ];
    uint32_t sc;  // the quarter's dword of the lane's scale vector
};

template <uint32_t T, int P, int R, bool XROWS = false>
__global__ __launch_bounds__(kWave *kGemmWaves) __attribute__((amdgpu_waves_per_eu(2))) void gemm_xs(
    const uint8_t *__restrict__ Wp, Planes xp, const float *__restrict__ xrows, float *__restrict__ out, int m, int n,
    int batch, int ksplit, size_t split_stride) {
    constexpr int Q = GemmUnit<T, 1>::kQ;
    __shared__ __align__(16) float red[kGemmWaves][32][kWave];
    __shared__ float wmax[2 * kGemmWaves][32];  // [wave, lane half][row]
    __shared__ int emax[kGemmWaves][32];
    const int nsb = n >> 8, tiles = (m + kWave - 1) / kWave;
    const int gs = gridDim.x / ksplit;  // workgroups per split
    const int ks = blockIdx.x % ksplit, g0 = blockIdx.x / ksplit;
    if (g0 >= gs || g0 >= tiles) return;
    const int lane = threadIdx.x & (kWave - 1);
    // the weight base in SGPRs now: the weight ring's first loads must not
    // wait for a kernel-argument load issued after the x loads
    asm volatile("" ::"s"(Wp));
    const int quarter = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const size_t tile_bytes = (size_t)nsb * Panel<T>::kBytes;
    const __amdgpu_buffer_rsrc_t orsrc =
        __builtin_amdgcn_make_buffer_rsrc(out, 0, (int)(4 * ksplit * split_stride), kBufferWord3);
    // this quarter's x fragments of the split's panels: lane l holds batch row
    // l % 32 (rows past the batch repeat the last), 8 consecutive columns;
    // from the fragment-order planes, or (XROWS) split from fp32 rows x[b][n];
    // brought to x * 2^-E with one exponent E per batch row for the whole
    // split; from the planes after the weight ring's loads were issued (as in
    // gemm_xs16)
    h8v xa[P][4], xb[P][4];
    const int brow = min(lane & 31, batch - 1);
    const float *xr = XROWS ? xrows + (size_t)brow * n : nullptr;
    auto xcol = [&](int p, int st) { return 16 * (16 * (ks * P + p) + 4 * quarter + st) + 8 * (lane >> 5); };
    int xe_own[P];
    constexpr int NG = 2 * P;
    constexpr bool kDirect = NG <= 8;  // as in gemm_xs16
    int xe_all[kDirect ? NG : 1];
    int E = 0;
    if constexpr (!XROWS) {
        const size_t xbase = (size_t)(4 * quarter * kWave + brow + 32 * (lane >> 5)) * 8 + 16 * 512 * (size_t)(ks * P);
        if constexpr (kDirect) {
#pragma unroll
            for (int g = 0; g < NG; g++) xe_all[g] = xp.xe[(size_t)brow * xe_stride(n) + 2 * ks * P + g];
        }
#pragma unroll
        for (int p = 0; p < P; p++) {
            if constexpr (kDirect) xe_own[p] = (quarter >> 1) ? xe_all[2 * p + 1] : xe_all[2 * p];
            else xe_own[p] = xp.xe[(size_t)brow * xe_stride(n) + 2 * (ks * P + p) + (quarter >> 1)];
#pragma unroll
            for (int st = 0; st < 4; st++) {
                xa[p][st] = *reinterpret_cast<const h8v *>(xp.hi + xbase + 16 * 512 * p + 512 * st);
                xb[p][st] = *reinterpret_cast<const h8v *>(xp.lo + xbase + 16 * 512 * p + 512 * st);
            }
        }
    } else {
        // fp32 rows, split before the ring: lanes l, l + 32 and the 4 waves
        // hold a row's columns
        float amax = 0.0f;
#pragma unroll
        for (int p = 0; p < P; p++)
#pragma unroll
            for (int st = 0; st < 4; st++) amax = amax8(xr + xcol(p, st), amax);
        wmax[2 * quarter + (lane >> 5)][lane & 31] = amax;
        lds_barrier();
        float rmax = wmax[0][lane & 31];
#pragma unroll
        for (int w = 1; w < 2 * kGemmWaves; w++) rmax = fmaxf(rmax, wmax[w][lane & 31]);
        E = group_exp(rmax);
#pragma unroll
        for (int p = 0; p < P; p++)
#pragma unroll
            for (int st = 0; st < 4; st++) {
                float v[8];
                load8(xr + xcol(p, st), v);
                split8_scaled(v, E, xa[p][st], xb[p][st]);
            }
    }
    const uint8_t *wsplit = Wp + (size_t)(ks * P) * Panel<T>::kBytes;
    int lt = g0;  // next tile to load
    auto load_tile = [&](WUnit<T> (&u)[P]) {
        const u32x4 *p4 = reinterpret_cast<const u32x4 *>(wsplit + (size_t)min(lt, tiles - 1) * tile_bytes);
#pragma unroll
        for (int p = 0; p < P; p++) {
            const u32x4 *pp = p4 + p * (Panel<T>::kBytes / 16);
#pragma unroll
            for (int c = 0; c < Q; c++) u[p].q[c] = __builtin_nontemporal_load(pp + (Q * quarter + c) * kWave + lane);
            u[p].sc = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(pp + Panel<T>::kChunks * kWave + lane) + quarter);
        }
        lt += gs;
    };
    // The empty asm statements order the ring: the prologue's loads stay in
    // ring order (else the loop-header wait merges in the prologue's order),
    // and a step waits for its own unit at its start, after the previous
    // step's refill was issued (else the next unit's dequantisation is
    // hoisted above that refill, with a wait for all loads in flight).
    WUnit<T> ring[R][P];
#pragma unroll
    for (int r = 0; r < R; r++) {
        load_tile(ring[r]);
        asm volatile("" ::: "memory");
    }
    if constexpr (!XROWS) {
        if constexpr (kDirect) {
            E = kXeEmpty;
#pragma unroll
            for (int g = 0; g < NG; g++) E = max(E, xe_all[g]);
        } else {
            int e = kXeEmpty;
#pragma unroll
            for (int p = 0; p < P; p++) e = max(e, xe_own[p]);
            if (lane < 32) emax[quarter][lane] = e;
            lds_barrier();
            E = max(max(emax[0][lane & 31], emax[1][lane & 31]), max(emax[2][lane & 31], emax[3][lane & 31]));
        }
#pragma unroll
        for (int p = 0; p < P; p++) {
            const _Float16 f = xe_factor(xe_own[p], E);
#pragma unroll
            for (int st = 0; st < 4; st++) {
                xa[p][st] = xa[p][st] * f;
                xb[p][st] = xb[p][st] * f;
            }
        }
    }
    // the epilogue's batch rows (threadIdx / 16, + 16) take their exponent
    // from the lanes holding those rows
    const float fEb[2] = {xe_scale(row_exp4(E, 4 * quarter)), xe_scale(row_exp4(E, 16 + 4 * quarter))};
    int ct = g0;  // tile being multiplied
    auto step = [&](WUnit<T> (&u)[P]) {
#pragma unroll
        for (int p = 0; p < P; p++) {
#pragma unroll
            for (int c = 0; c < Q; c++) asm volatile("" : "+v"(u[p].q[c])::"memory");
            asm volatile("" : "+v"(u[p].sc)::"memory");
        }
        f32x16 acc0 = {}, acc1 = {};
#pragma unroll
        for (int p = 0; p < P; p++) mma_tile<T>(u[p].q, u[p].sc, xa[p], xb[p], acc0, acc1);
        asm volatile("" : "+v"(acc0), "+v"(acc1)::"memory");
        load_tile(u);
        gemm_tile_epilogue<kCpolDevice>(red, fEb, acc0, acc1, quarter, lane, ct, ks, batch, m, split_stride, orsrc,
                                        ct < tiles);
        ct += gs;
    };
    do {
#pragma unroll
        for (int r = 0; r < R; r++) step(ring[r]);
    } while (ct < tiles);
}

// x-stationary 32-wide GEMM with the split's panels shared by H groups of 4
// waves: wave w takes column quarter w % 4 of panels ks * H * PW + (w / 4) * PW
// .. + PW - 1, holds their A fragments (32 PW VGPRs) and streams its units
// (4 quant vectors + 1 scale dword) D deep; a tile's sums are added over the
// 4 H waves through LDS.  With H = 2 the split's x fragments (up to 8 panels)
// fit in registers at two waves per SIMD, so lm_head needs no K split and no
// x loads in its main loop.  Output as gemm_xs; with SILU (one K split, the
// interleaved [gate; up] panel matrix, m = 2 F) the tile's 32 gate sums meet
// their 32 up sums in the epilogue, which writes h[b][f] = SiLU(gate) * up
// (scratch.rs:181-186) as fp32 rows [batch][F] instead of the sums.
template <uint32_t T, int PW, int D, int H, bool XROWS = false, bool SILU = false, bool RS = false>
__global__ __launch_bounds__(kWave *kGemmWaves *H) __attribute__((amdgpu_waves_per_eu(2))) void gemm_xsh(
    const uint8_t *__restrict__ Wp, Planes xp, const float *__restrict__ xrows, float *__restrict__ out, int m, int n,
    int batch, int ksplit, size_t split_stride) {
    constexpr int Q = GemmUnit<T, 1>::kQ;
    constexpr int U = PW > D ? PW : D;
    constexpr int NW = kGemmWaves * H;
    static_assert(U % PW == 0 && U % D == 0, "ring and panel counts must divide the loop body");
    __shared__ __align__(16) float red[NW][32][kWave];
    __shared__ int emax[NW][32];
    __shared__ int ew[NW][32];  // [wave][batch row]: the exponent of the wave's fragments
    const int nsb = n >> 8, tiles = (m + kWave - 1) / kWave;
    const int gs = gridDim.x / ksplit;  // workgroups per split
    const int ks = blockIdx.x % ksplit, g0 = blockIdx.x / ksplit;
    if (g0 >= gs || g0 >= tiles) return;
    const int lane = threadIdx.x & (kWave - 1);
    // the weight base in SGPRs now: the weight ring's first loads must not
    // wait for a kernel-argument load issued after the x loads
    asm volatile("" ::"s"(Wp));
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int quarter = wave & 3, panel0 = (ks * H + (wave >> 2)) * PW;
    const size_t tile_bytes = (size_t)nsb * Panel<T>::kBytes;
    const __amdgpu_buffer_rsrc_t orsrc =
        __builtin_amdgcn_make_buffer_rsrc(out, 0, (int)(4 * ksplit * split_stride), kBufferWord3);
    // fragments brought to x * 2^-E: from the planes one exponent E per
    // batch row for the split (all H * PW panels of the workgroup), from fp32
    // rows one per batch row and wave; formed after the weight ring's loads
    // were issued, each wave's sums scaled by its 2^E (as in gemm_xs16)
    h8v xa[PW][4], xb[PW][4];
    float xv[XROWS ? PW : 1][4][8];  // fp32 rows: the wave's values of this lane
    const int brow = min(lane & 31, batch - 1);
    const float *xr = XROWS ? xrows + (size_t)brow * n : nullptr;
    auto xcol = [&](int p, int st) { return 16 * (16 * (panel0 + p) + 4 * quarter + st) + 8 * (lane >> 5); };
    int xe_own[PW];
    constexpr int NG = 2 * H * PW;  // groups of the split
    constexpr bool kDirect = NG <= 8;  // as in gemm_xs16
    int xe_all[kDirect ? NG : 1];
    int E = 0;
    if constexpr (!XROWS) {
        const size_t xbase = (size_t)(4 * quarter * kWave + brow + 32 * (lane >> 5)) * 8 + 16 * 512 * (size_t)panel0;
        if constexpr (kDirect) {
#pragma unroll
            for (int g = 0; g < NG; g++) xe_all[g] = xp.xe[(size_t)brow * xe_stride(n) + 2 * ks * H * PW + g];
        }
#pragma unroll
        for (int p = 0; p < PW; p++) {
            xe_own[p] = xp.xe[(size_t)brow * xe_stride(n) + 2 * (panel0 + p) + (quarter >> 1)];
#pragma unroll
            for (int st = 0; st < 4; st++) {
                xa[p][st] = *reinterpret_cast<const h8v *>(xp.hi + xbase + 16 * 512 * p + 512 * st);
                xb[p][st] = *reinterpret_cast<const h8v *>(xp.lo + xbase + 16 * 512 * p + 512 * st);
            }
        }
    } else {
#pragma unroll
        for (int p = 0; p < PW; p++)
#pragma unroll
            for (int st = 0; st < 4; st++) load8(xr + xcol(p, st), xv[p][st]);
    }
    // RS: the norm sums of this thread's epilogue batch row, loaded with x
    // (ahead of the weight ring) and turned into its scale once E is known
    static_assert(!RS || !XROWS, "the deferred norm scale comes with planes");
    float rsv[RS ? kMaxRsParts : 1];
    if constexpr (RS) rs_load(xp, min((int)(threadIdx.x >> 4), batch - 1), rsv);
    const uint8_t *wpart = Wp + (size_t)panel0 * Panel<T>::kBytes;
    int lt = g0, lp = 0;  // load cursor: tile, panel of the wave's part
    auto load_next = [&](WUnit<T> &u) {
        const u32x4 *p4 = reinterpret_cast<const u32x4 *>(wpart + (size_t)min(lt, tiles - 1) * tile_bytes +
                                                          (size_t)lp * Panel<T>::kBytes);
#pragma unroll
        for (int c = 0; c < Q; c++) u.q[c] = __builtin_nontemporal_load(p4 + (Q * quarter + c) * kWave + lane);
        u.sc = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p4 + Panel<T>::kChunks * kWave + lane) +
                                          quarter);
        const bool wrap = ++lp == PW;
        lp = wrap ? 0 : lp;
        lt = wrap ? lt + gs : lt;
    };
    WUnit<T> ring[D];
#pragma unroll
    for (int k = 0; k < D; k++) {
        load_next(ring[k]);
        asm volatile("" ::: "memory");
    }
    if constexpr (!XROWS) {
        if constexpr (kDirect) {
            E = kXeEmpty;
#pragma unroll
            for (int g = 0; g < NG; g++) E = max(E, xe_all[g]);
        } else {
            int e = kXeEmpty;
#pragma unroll
            for (int p = 0; p < PW; p++) e = max(e, xe_own[p]);
            if (lane < 32) emax[wave][lane] = e;
            lds_barrier();
            E = emax[0][lane & 31];
#pragma unroll
            for (int w = 1; w < NW; w++) E = max(E, emax[w][lane & 31]);
        }
#pragma unroll
        for (int p = 0; p < PW; p++) {
            const _Float16 f = xe_factor(xe_own[p], E);
#pragma unroll
            for (int st = 0; st < 4; st++) {
                xa[p][st] = xa[p][st] * f;
                xb[p][st] = xb[p][st] * f;
            }
        }
    } else {
        // fp32 rows (API path, splits of 2 panels): E from the row's largest
        // |x| over this wave's columns -- lanes l and l ^ 32 hold the row
        float amax = 0.0f;
#pragma unroll
        for (int p = 0; p < PW; p++)
#pragma unroll
            for (int st = 0; st < 4; st++)
#pragma unroll
                for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(xv[p][st][i]));
        E = group_exp(lanes_max2(amax));
#pragma unroll
        for (int p = 0; p < PW; p++)
#pragma unroll
            for (int st = 0; st < 4; st++) split8_scaled(xv[p][st], E, xa[p][st], xb[p][st]);
    }
    if (lane < 32) ew[wave][lane] = E;  // lane l holds batch row l (read after the tile's barrier)
    float rsc = 1.0f;
    if constexpr (RS) {
#pragma unroll
        for (int k = 0; k < kMaxRsParts; k++) asm volatile("" : "+v"(rsv[k]));
        rsc = rs_finish(xp, rsv, n);
    }
    static_assert(512 / (kWave * NW) == 1, "one output vector per thread");
    int ct = g0;  // tile being multiplied
    f32x16 acc0 = {}, acc1 = {};
    do {
#pragma unroll
        for (int k = 0; k < U; k++) {
            WUnit<T> &u = ring[k % D];
#pragma unroll
            for (int c = 0; c < Q; c++) asm volatile("" : "+v"(u.q[c])::"memory");
            asm volatile("" : "+v"(u.sc)::"memory");
            mma_tile<T>(u.q, u.sc, xa[k % PW], xb[k % PW], acc0, acc1);
            asm volatile("" : "+v"(acc0), "+v"(acc1)::"memory");
            load_next(u);
            if (k % PW == PW - 1) {
                // tile done: park the 32 sums per lane (element r of lane l:
                // batch row 8 (r / 4 % 4) + 4 (l / 32) + r % 4, tile row
                // l % 32 + 32 (r / 16)); each thread then adds the NW waves'
                // sums of 4-row vectors of one batch row and stores them
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    red[wave][r][lane] = acc0[r];
                    red[wave][16 + r][lane] = acc1[r];
                }
                lds_barrier();
#pragma unroll
                for (int i = 0; i < 512 / (kWave * NW); i++) {
                    const int v = threadIdx.x + kWave * NW * i;  // 512 vectors: batch row b, rows 4 j .. 4 j + 3
                    const int b = v >> 4, j = v & 15;
                    const int r = 4 * (b >> 3) + (b & 3) + (j >= 8 ? 16 : 0);
                    const int l = ((4 * j) & 31) + 32 * ((b >> 2) & 1);
                    // each wave's sums times its 2^E (exact), added in wave order
                    float4 sum = mul4(*reinterpret_cast<const float4 *>(&red[0][r][l]), xe_scale(ew[0][b]));
#pragma unroll
                    for (int w = 1; w < NW; w++) {
                        const float4 o = mul4(*reinterpret_cast<const float4 *>(&red[w][r][l]), xe_scale(ew[w][b]));
                        sum = make_float4(sum.x + o.x, sum.y + o.y, sum.z + o.z, sum.w + o.w);
                    }
                    if constexpr (RS) sum = mul4(sum, rsc);
                    if constexpr (SILU) {
                        // rows 4 j .. + 3 (j < 8): the gate sums of features
                        // 32 ct + 4 j .. + 3; their up sums are rows 32 + 4 j
                        // .., held by lane + 8 (same batch row)
                        const float4 up = make_float4(__shfl_down(sum.x, 8), __shfl_down(sum.y, 8),
                                                      __shfl_down(sum.z, 8), __shfl_down(sum.w, 8));
                        const float4 h4 = make_float4((sum.x / (1.0f + expf(-sum.x))) * up.x,
                                                      (sum.y / (1.0f + expf(-sum.y))) * up.y,
                                                      (sum.z / (1.0f + expf(-sum.z))) * up.z,
                                                      (sum.w / (1.0f + expf(-sum.w))) * up.w);
                        const int f = 32 * ct + 4 * j;
                        const int off = j < 8 && b < batch && ct < tiles ? 4 * (b * (m >> 1) + f) : kBadOffset;
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, h4), orsrc, off, 0,
                                                               kCpolDevice);
                    } else {
                        const int row = ct * kWave + 4 * j;
                        const int off = b < batch && row < m && ct < tiles
                                            ? 4 * (ks * (int)split_stride + b * m + row)
                                            : kBadOffset;
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sum), orsrc, off, 0,
                                                               kCpolDevice);
                    }
                }
                lds_barrier();  // red is free again
                acc0 = f32x16{};
                acc1 = f32x16{};
                ct += gs;
            }
        }
    } while (ct < tiles);
}

// Prefill GEMM: up to 256 rows of x (compute wave w takes rows 32 w .. 32 w +
// 31, that group's 32-row planes) against 64-row weight tiles.  Items are
// (tile, K split); one workgroup per CU walks the panels ("units") of items
// g, g + G, ... as one pipeline.  Per unit:
//  * a ninth wave (the loader) loaded the panel's bytes into registers a unit
//    ahead and turned them into MFMA B fragments of the quantised values q as
//    fp16 (exact: |q| <= 127) in LDS, with each weight row's fp16 block
//    scales d beside them (the compute waves then wait on nothing but their
//    own x loads, which come from L2: a load waits for every load its wave
//    issued before it, so panel loads of their own would hold up the next x
//    wait for an HBM round trip);
//  * each wave multiplies its rows' x fragments (hi + lo at x 2^-E, E the
//    row's largest group exponent) with them on v_mfma_f32_32x32x16_f16,
//    one 32-column block at a time: c = x_hi q + x_lo q over the block's two
//    16-column steps, then sums += c d, the block's (sum q x) d of
//    q8_gemv.rs:234-242 (x_lo q is exact in the MFMA's fp32 products; x_hi +
//    x_lo holds x to 2^-22);
//  * an item's sums go out, times 2^E, after its last unit.
// out[ks * split_stride + row * m + r] (rows past `rows` or m: not stored).
constexpr int kTallWaves = 8;
constexpr int kTallMaxRows = 32 * kTallWaves;

// 8 signed bytes q (Q8_0) as fp16 q, exactly: q + 128 placed in the
// mantissa of 1024 (fp16 0x64xx is 1024 + xx), minus 1152
__device__ __forceinline__ h8v q8_fragment(uint32_t w0, uint32_t w1) {
    const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
    const u32x4 p = {__builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u),
                     __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u),
                     __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u),
                     __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)};
    const h8v k = {1152, 1152, 1152, 1152, 1152, 1152, 1152, 1152};
    return __builtin_bit_cast(h8v, p) - k;
}
// 8 nibbles (Q4_0: the low, shift 0, or high, shift 4, nibbles of 8 bytes)
// as fp16 nibble - 8, exactly (1024 + nibble, minus 1032)
__device__ __forceinline__ h8v q4_fragment(uint32_t w0, uint32_t w1, int shift) {
    const uint32_t n0 = (w0 >> shift) & 0x0f0f0f0fu, n1 = (w1 >> shift) & 0x0f0f0f0fu;
    const u32x4 p = {__builtin_amdgcn_perm(0x64646464u, n0, 0x04010400u),
                     __builtin_amdgcn_perm(0x64646464u, n0, 0x04030402u),
                     __builtin_amdgcn_perm(0x64646464u, n1, 0x04010400u),
                     __builtin_amdgcn_perm(0x64646464u, n1, 0x04030402u)};
    const h8v k = {1032, 1032, 1032, 1032, 1032, 1032, 1032, 1032};
    return __builtin_bit_cast(h8v, p) - k;
}

template <uint32_t T>
__global__ __launch_bounds__(kWave *(kTallWaves + 1)) __attribute__((amdgpu_waves_per_eu(3, 3))) void gemm_tall(
    const uint8_t *__restrict__ Wp, Planes xp, float *__restrict__ out, int m, int n, int rows, int ksplit, int per,
    size_t split_stride) {
    constexpr int CH = Panel<T>::kChunks;  // quant chunks of a tile's panel
    __shared__ h8v wf[2][16][2][kWave];    // B fragments [unit parity][16-column step][weight block][lane]
    __shared__ u32x4 dsc[2][kWave];        // 8 fp16 block scales of each weight row [unit parity][row]
    __shared__ uint16_t xes[2][kTallMaxRows];  // the panel's two group exponents of each x row [unit parity][row]
    __shared__ int erow[kTallWaves][32];
    const int nsb = n >> 8, ptiles = (m + kWave - 1) / kWave;
    const int items = ptiles * ksplit, G = (int)gridDim.x;
    // this workgroup's units: the panels of items g, g + G, ... in order
    const int units = ((items - (int)blockIdx.x + G - 1) / G) * per;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    auto item_of = [&](int u) { return (int)blockIdx.x + G * (u / per); };
    auto panel_of = [&](int u) { return (item_of(u) % ksplit) * per + u % per; };
    if (units == 0) return;

    if (wave == kTallWaves) {
        // The loader wave: unit u's panel bytes (lane l: chunk c of weight row
        // l for every c, row l's scale vector, and the two group exponents of
        // x rows l, l + 64, l + 128, l + 192 (the last row past the rows); a
        // tile past the matrix reads the last one again: its rows are never
        // stored) into registers, then into the B fragments of q as fp16 of
        // the unit's parity.  Its loads are the only ones it waits on, so
        // each has a whole unit to arrive.  Buffer loads: the offset within a
        // panel per lane, the panel's offset wave-uniform.
        const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(Wp), 0, (int)((size_t)ptiles * nsb * Panel<T>::kBytes), kBufferWord3);
        const __amdgpu_buffer_rsrc_t xersrc =
            __builtin_amdgcn_make_buffer_rsrc(xp.xe, 0, rows * xe_stride(n), kBufferWord3);
        u32x4 rq[CH], rs;
        uint32_t rxe[kTallMaxRows / kWave];
        auto load_raw = [&](int u) {
            const int tile = min(item_of(u) / ksplit, ptiles - 1), p = panel_of(u);
            const int base = (tile * nsb + p) * Panel<T>::kBytes;
#pragma unroll
            for (int c = 0; c < CH; c++)
                rq[c] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, 16 * (c * kWave + lane), base, kCpolNtLoad));
            rs = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, 16 * (CH * kWave + lane), base, kCpolNtLoad));
#pragma unroll
            for (int i = 0; i < kTallMaxRows / kWave; i++)
                rxe[i] = __builtin_amdgcn_raw_buffer_load_b16(xersrc, min(lane + kWave * i, rows - 1) * xe_stride(n),
                                                              2 * p, 0);
        };
        // Q8_0 chunk c holds a row's columns 16 c .. + 15 (step c); Q4_0
        // chunk c its block c, byte i the columns 32 c + i (low nibble, step
        // 2 c) and 32 c + 16 + i (high, step 2 c + 1).  Lane l of a step's
        // fragment: weight row l % 32 of the block, columns 8 (l / 32) .. + 7
        // of the step.
        auto convert = [&](int b) {
            const int cb = lane / 32, l = lane % 32;
#pragma unroll
            for (int c = 0; c < CH; c++) {
                const u32x4 q = rq[c];
                if constexpr (T == ANEHIP_GGML_Q8_0) {
                    wf[b][c][cb][l] = q8_fragment(q.x, q.y);
                    wf[b][c][cb][l + 32] = q8_fragment(q.z, q.w);
                } else {
                    wf[b][2 * c][cb][l] = q4_fragment(q.x, q.y, 0);
                    wf[b][2 * c][cb][l + 32] = q4_fragment(q.z, q.w, 0);
                    wf[b][2 * c + 1][cb][l] = q4_fragment(q.x, q.y, 4);
                    wf[b][2 * c + 1][cb][l + 32] = q4_fragment(q.z, q.w, 4);
                }
                __builtin_amdgcn_sched_barrier(0);  // one chunk's fragments at a time
            }
            dsc[b][lane] = rs;
#pragma unroll
            for (int i = 0; i < kTallMaxRows / kWave; i++) xes[b][lane + kWave * i] = (uint16_t)rxe[i];
        };
        load_raw(0);
        convert(0);
        load_raw(1);
        __syncthreads();  // unit 0's fragments ready
        for (int u = 0; u < units; u++) {
            // unit u + 1 into the parity unit u - 1 read (past the last unit:
            // not read), then the loads of unit u + 2
            convert((u + 1) & 1);
            load_raw(u + 2);
            __syncthreads();  // end of unit u
        }
        return;
    }

    // The compute waves: wave w takes x rows 32 w .. + 31
    const int grows = rows - 32 * wave;  // rows of this wave's group (<= 0: products not stored)
    const bool active = grows > 0;
    const Planes gp = xp.group(active ? wave : 0, n);
    const int brow = min(lane & 31, (active ? min(grows, 32) : 1) - 1);  // rows past the group repeat its last
    const int8_t *xe_row = gp.xe + (size_t)brow * xe_stride(n);
    // block j of panel p (steps 16 p + 2 j, + 1): hi and lo fragments
    // (buffer loads: the lane's offset in a step's 1 KiB, the step's offset
    // wave-uniform)
    const int plane_bytes = (int)(2 * xf_plane_len((size_t)n));
    const __amdgpu_buffer_rsrc_t hrsrc = __builtin_amdgcn_make_buffer_rsrc(gp.hi, 0, plane_bytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t lrsrc = __builtin_amdgcn_make_buffer_rsrc(gp.lo, 0, plane_bytes, kBufferWord3);
    const int xoff = 16 * (brow + 32 * (lane >> 5));
    auto load_x = [&](int p, int j, h8v (&a)[4]) {
        const int so = (16 * p + 2 * j) * 1024;
        a[0] = __builtin_bit_cast(h8v, __builtin_amdgcn_raw_buffer_load_b128(hrsrc, xoff, so, 0));
        a[1] = __builtin_bit_cast(h8v, __builtin_amdgcn_raw_buffer_load_b128(lrsrc, xoff, so, 0));
        a[2] = __builtin_bit_cast(h8v, __builtin_amdgcn_raw_buffer_load_b128(hrsrc, xoff, so + 1024, 0));
        a[3] = __builtin_bit_cast(h8v, __builtin_amdgcn_raw_buffer_load_b128(lrsrc, xoff, so + 1024, 0));
    };
    f32x16 acc[2] = {f32x16{}, f32x16{}};
    // an item's sums: element r of lane l is row 8 (r / 4) + 4 (l / 32) +
    // r % 4 of the group, weight row 32 cb + l % 32 of the tile
    auto store_item = [&](int item) {
        const int tile = item / ksplit, ks = item % ksplit;
        // opaque copies: the row addresses and scales are rebuilt here, not
        // kept live across the unit loop
        float *ob = out;
        int w = wave, ln = lane;
        asm volatile("" : "+s"(ob), "+s"(w), "+v"(ln));
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int gr = 8 * (r >> 2) + 4 * (ln >> 5) + (r & 3);
            if (gr < grows) {
                const float sc = xe_scale(erow[w][gr]);
                float *orow = ob + (size_t)ks * split_stride + (size_t)(32 * w + gr) * m;
#pragma unroll
                for (int cb = 0; cb < 2; cb++) {
                    const int wr = tile * kWave + 32 * cb + (ln & 31);
                    if (wr < m) orow[wr] = acc[cb][r] * sc;
                }
            }
        }
        acc[0] = f32x16{};
        acc[1] = f32x16{};
    };
    // E over the whole row (one exponent for every K split of it), from
    // 16-byte loads of the row's exponents (a row's are padded to 16 bytes),
    // all issued before the first is used
    int E = kXeEmpty;
    {
        const int ng = 2 * nsb;
        u32x4 ev[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (16 * i < ng) ev[i] = *reinterpret_cast<const u32x4 *>(xe_row + 16 * i);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int k = 0; k < 16; k++)
                if (16 * i + k < ng) E = max(E, (int)(int8_t)(ev[i][k >> 2] >> (8 * (k & 3))));
        for (int g = 64; g < ng; g++) E = max(E, (int)xe_row[g]);  // n > 8192
    }
    if (lane < 32) erow[wave][lane] = E;
    __syncthreads();  // unit 0's fragments ready, erow written
    // x of the next two blocks is always in flight: xa[i % 4] for block i
    // of the workgroup's sequence of units x 8 blocks.  Every wave issues
    // the same loads and products on every unit (waves without rows take
    // group 0's x and store nothing; past the last unit, a valid panel), so
    // that the loop has one path and the loads in flight are the same on it.
    h8v xa[4][4];
    load_x(panel_of(0), 0, xa[0]);
    load_x(panel_of(0), 1, xa[1]);
    for (int u0 = 0; u0 < units; u0 += per) {
    for (int u = u0; u < u0 + per; u++) {
        const int b = u & 1, p = panel_of(u);
        const uint32_t xe2 = xes[b][32 * wave + brow];
        const _Float16 fg[2] = {xe_factor((int)(int8_t)(xe2 & 0xffu), E), xe_factor((int)(int8_t)(xe2 >> 8), E)};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const _Float16 f = fg[j >> 2];
            h8v(&a)[4] = xa[j % 4];
#pragma unroll
            for (int i = 0; i < 4; i++) a[i] *= f;
            // then x of the block two ahead (the next unit's first two)
            __builtin_amdgcn_sched_barrier(0);
            if (j < 6) load_x(p, j + 2, xa[(j + 2) % 4]);
            else load_x(panel_of(u + 1), j - 6, xa[(j + 2) % 4]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int cb = 0; cb < 2; cb++) {
                const h8v b0 = wf[b][2 * j][cb][lane], b1 = wf[b][2 * j + 1][cb][lane];
                f32x16 c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[0], b0, f32x16{}, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[1], b0, c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[2], b1, c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[3], b1, c, 0, 0, 0);
                const uint32_t dw = reinterpret_cast<const uint32_t *>(&dsc[b][32 * cb + (lane & 31)])[j >> 1];
                const float d = __half2float(__ushort_as_half((unsigned short)(dw >> (16 * (j & 1)))));
#pragma unroll
                for (int r = 0; r < 16; r++) acc[cb][r] = fmaf(c[r], d, acc[cb][r]);
                // the sums are added here, not deferred (which would keep
                // every block's products live)
                asm volatile("" : "+v"(acc[cb]));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();  // end of unit u: unit u + 1's fragments ready; every wave is done with parity b
    }
    if (active) store_item(item_of(u0));
    }
}

// fp32 x[batch][n] -> range-safe fragment-order fp16 planes (hi + lo = x *
// 2^-e per 128-column group, the exponents to xe), one thread per 8
// consecutive columns of a row (one 16-byte fragment): a group is 16
// consecutive threads of one wave (n % 128 == 0).
__global__ __launch_bounds__(256) void split_x_frag_kernel(const float *__restrict__ x, Planes xp, int batch, int n) {
    const int g = blockIdx.x * 256 + threadIdx.x, per_row = n >> 3;
    if (g >= batch * per_row) return;  // whole 16-thread groups leave together
    const int b = g / per_row, c = 8 * (g % per_row);
    const float4 *src = reinterpret_cast<const float4 *>(x + (size_t)b * n + c);
    const float4 v0 = src[0], v1 = src[1];
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
    const int ex = group_exp(row_max16(amax));  // a group is a 16-lane row
    h8v h, l;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        _Float16 hh, ll;
        split_scaled(v[e], ex, hh, ll);
        h[e] = hh;
        l[e] = ll;
    }
    *reinterpret_cast<h8v *>(xp.hi + xf_index(b, c, n)) = h;
    *reinterpret_cast<h8v *>(xp.lo + xf_index(b, c, n)) = l;
    if ((g & 15) == 0) xp.xe[xe_index(b, c, n)] = (int8_t)ex;
}

// ---------------------------------------------------------------------------
// Small-batch GEMM on MFMA (batch 2..32).  Weights are exact in fp16 (int8 or
// nibble - 8); each fp32 activation is split into fp16 hi + lo = x to ~2^-22
// relative, so two v_mfma_f32_16x16x32_f16 per (16 rows x 32 columns x 16
// batch) tile give fp32-accurate block sums, which are scaled by the block's
// fp16 scale in fp32 and accumulated: the same per-block order as
// compute_row (q8_gemv.rs:234-242).  One K=32 MFMA step is exactly one quant
// block.
//
// Lane layout of v_mfma_f32_16x16x32_f16 (checked on gfx950): A[i][k] in lane
// i + 16*(k/8), element k%8; B[k][j] in lane j + 16*(k/8), element k%8;
// D[i][j] in lane j + 16*(i/4), element i%4.
// ---------------------------------------------------------------------------

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// fp32 x[batch][n] -> range-safe fp16 planes hi[batch][n], lo[batch][n]
// (row-major; hi + lo = x * 2^-e per 128-column group, exponents to xe), one
// thread per 8 consecutive columns, 16 threads per group (n % 128 == 0).
__global__ __launch_bounds__(256) void split_x_kernel(const float *__restrict__ x, Planes xp, int batch, int n) {
    const int g = blockIdx.x * 256 + threadIdx.x, per_row = n >> 3;
    if (g >= batch * per_row) return;  // whole 16-thread groups leave together
    const int b = g / per_row, c = 8 * (g % per_row);
    const size_t o = (size_t)b * n + c;
    const float4 v0 = *reinterpret_cast<const float4 *>(x + o), v1 = *reinterpret_cast<const float4 *>(x + o + 4);
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
    const int ex = group_exp(row_max16(amax));  // a group is a 16-lane row
    f16x8 h, l;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        _Float16 hh, ll;
        split_scaled(v[e], ex, hh, ll);
        h[e] = hh;
        l[e] = ll;
    }
    *reinterpret_cast<f16x8 *>(xp.hi + o) = h;
    *reinterpret_cast<f16x8 *>(xp.lo + o) = l;
    if ((g & 15) == 0) xp.xe[xe_index(b, c, n)] = (int8_t)ex;
}

// 8 weights of one row of one block, as fp16, from the LDS tile row `wl`
// (u32 words of the row's super-block segment): quant bytes 8g..8g+7 of block
// `blk` (Q8_0: int8; Q4_0: element k < 16 is the low nibble of byte k, k >= 16
// the high nibble of byte k - 16, so group g reads bytes 8(g%2).. and nibble
// g/2).  ODD = blk % 2, which fixes the byte alignment of the quants: blocks
// are 34 / 18 bytes, so odd blocks' quants start on a 4-byte boundary and even
// blocks' 2 bytes past one.
template <uint32_t T, int ODD>
__device__ __forceinline__ f16x8 w_frag(const uint32_t *wl, int blk, int g) {
    constexpr int kBB = QTraits<T>::kBlockBytes;
    const int off = blk * kBB + 2 + (T == ANEHIP_GGML_Q8_0 ? 8 * g : 8 * (g & 1));
    const int w0 = off >> 2;
    uint32_t d0, d1;
    if constexpr (ODD) {
        d0 = wl[w0];
        d1 = wl[w0 + 1];
    } else {
        const uint32_t x0 = wl[w0], x1 = wl[w0 + 1], x2 = wl[w0 + 2];
        d0 = __builtin_amdgcn_alignbyte(x1, x0, 2);
        d1 = __builtin_amdgcn_alignbyte(x2, x1, 2);
    }
    // exact int8 (or nibble - 8) -> fp16 by placing the byte in the mantissa
    // of 1024 (dwords_to_h8_i8 / _u4)
    if constexpr (T == ANEHIP_GGML_Q8_0) {
        return __builtin_bit_cast(f16x8, dwords_to_h8_i8(d0, d1));
    } else {
        const int sh = (g >> 1) * 4;
        return __builtin_bit_cast(f16x8, dwords_to_h8_u4((d0 >> sh) & 0x0F0F0F0Fu, (d1 >> sh) & 0x0F0F0F0Fu));
    }
}

template <uint32_t T>
__device__ __forceinline__ float blk_scale(const uint32_t *wl, int blk) {
    return half_at(wl, blk * QTraits<T>::kBlockBytes);
}

// grid = (row tiles of 64, K splits); 4 waves per workgroup, as the GEMV.
// NT = 16-wide batch tiles (1: batch <= 16, 2: batch <= 32).  xh / xl: fp16
// planes [batch][n].  Output as quant_gemm_tiled.
//
// Operands: A = activations (16 batch rows x 32 columns), B = weights (32
// columns x 16 weight rows), so D[b][r] = sum_k x[b][k] W[r][k]; a lane's four
// D values share one weight row and therefore one block scale.
template <uint32_t T, int NT>
__global__ __launch_bounds__(kWave *kWavesPerWg) void quant_gemm_mfma(const uint8_t *__restrict__ W, Planes xp,
                                                                     float *__restrict__ out, int m, int n,
                                                                     int batch, int sb_per_split,
                                                                     size_t split_stride) {
    constexpr int V = QTraits<T>::kSbVec;
    __shared__ u32x4 lds[kWavesPerWg][V * kWave];
    __shared__ int xeE[32];
    const _Float16 *__restrict__ xh = xp.hi;
    const _Float16 *__restrict__ xl = xp.lo;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int tile = blockIdx.x;
    const int ks = blockIdx.y;
    const int nsb = n >> 8;
    const size_t row_bytes = (size_t)nsb * QTraits<T>::kSbBytes;
    const int row0 = tile * kWave;
    const int sb_begin = ks * sb_per_split;
    const int sb_end = min(nsb, sb_begin + sb_per_split);
    const int li = lane & 15;  // A row (batch) / B column (weight row) within a 16 tile
    const int g = lane >> 4;   // k group (8 columns) / D row group

    f32x4 acc[4][NT];
#pragma unroll
    for (int rs = 0; rs < 4; rs++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[rs][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 regs[V];
    uint32_t off[V];
    tile_offsets<T>(off, (uint32_t)row_bytes, m - row0, lane);
    const uint8_t *tile_base = W + (size_t)row0 * row_bytes;
    const uint32_t *lds_words = reinterpret_cast<const uint32_t *>(lds[wave]);
    constexpr int kSegWords = QTraits<T>::kSbBytes / 4;

    // the two group exponents of super-block s for batch row li + 16 nt,
    // loaded with that super-block's weights (one super-block ahead), so the
    // block loop multiplies by a factor already in registers
    auto xe_pair = [&](int s, int nt) {
        const int8_t *e = xp.xe + (size_t)min(li + 16 * nt, batch - 1) * xe_stride(n) + 2 * s;
        return make_int2(e[0], e[1]);
    };
    int2 xen[NT];
    int sb = sb_begin + wave;
    if (sb < sb_end) {
        load_tile<T>(regs, tile_base + (size_t)sb * QTraits<T>::kSbBytes, off);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) xen[nt] = xe_pair(sb, nt);
    }
    // range-safe planes: the split's groups (2 per super-block) of batch row
    // li + 16 nt brought to one exponent En[nt] (read after the first weight
    // loads were issued)
    int En[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int b = min(li + 16 * nt, batch - 1);
        En[nt] = xe_max(xp.xe, b, 2 * sb_begin, 2 * (sb_end - sb_begin), n);
        if (wave == 0 && g == 0) xeE[li + 16 * nt] = En[nt];  // read after the reduction barrier
    }
    for (; sb < sb_end; sb += kWavesPerWg) {
        _Float16 fgrp[NT][2];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            fgrp[nt][0] = xe_factor(xen[nt].x, En[nt]);
            fgrp[nt][1] = xe_factor(xen[nt].y, En[nt]);
        }
        // A fragments of block blk: x[b = li + 16 nt][sb*256 + 32 blk + 8 g +
        // e]; rows past the batch read row batch - 1 (branch-free; those MFMA
        // output rows are never stored)
        auto load_x = [&](int blk, f16x8 (&ah)[NT], f16x8 (&al)[NT]) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const int b = min(li + 16 * nt, batch - 1);
                const size_t xo = (size_t)b * n + (size_t)sb * 256 + 32 * blk + 8 * g;
                ah[nt] = *reinterpret_cast<const f16x8 *>(xh + xo);
                al[nt] = *reinterpret_cast<const f16x8 *>(xl + xo);
            }
        };
        f16x8 nh[2][NT], nl[2][NT];  // the next block pair's fragments
        load_x(0, nh[0], nl[0]);
        load_x(1, nh[1], nl[1]);
        stage_tile<T>(regs, lds[wave], lane);
        // blocks in pairs (even, odd): a runtime loop bounds the live
        // registers; each pair's x is loaded one pair ahead (unconditionally:
        // the last pair re-reads its own, which keeps the loop body
        // straight-line and the waits exact).  The next super-block's weights
        // are loaded after the loop: loads complete in issue order, so an x
        // load issued after them would wait for their HBM round trip.
#pragma unroll 1
        for (int bp = 0; bp < 4; bp++) {
            f16x8 ch[2][NT], cl[2][NT];
#pragma unroll
            for (int odd = 0; odd < 2; odd++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    ch[odd][nt] = nh[odd][nt];
                    cl[odd][nt] = nl[odd][nt];
                }
            const int np = min(bp + 1, 3);
            load_x(2 * np, nh[0], nl[0]);
            load_x(2 * np + 1, nh[1], nl[1]);
#pragma unroll
            for (int odd = 0; odd < 2; odd++) {
                const int blk = 2 * bp + odd;
                f16x8 ah[NT], al[NT];
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    const _Float16 f = bp < 2 ? fgrp[nt][0] : fgrp[nt][1];
                    ah[nt] = ch[odd][nt] * f;
                    al[nt] = cl[odd][nt] * f;
                }
#pragma unroll
                for (int rs = 0; rs < 4; rs++) {
                    const uint32_t *wl = lds_words + (rs * 16 + li) * kSegWords;
                    const f16x8 bw = odd ? w_frag<T, 1>(wl, blk, g) : w_frag<T, 0>(wl, blk, g);
                    const float d = blk_scale<T>(wl, blk);
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        f32x4 c =
                            __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[nt], bw, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[nt], bw, c, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[rs][nt][r] = fmaf(c[r], d, acc[rs][nt][r]);
                    }
                }
            }
        }
        if (sb + kWavesPerWg < sb_end) {
            load_tile<T>(regs, tile_base + (size_t)(sb + kWavesPerWg) * QTraits<T>::kSbBytes, off);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) xen[nt] = xe_pair(sb + kWavesPerWg, nt);
        }
        wave_sync_lds();
    }
    // reduce the 4 waves through LDS (the staging buffer is free now)
    __syncthreads();
    float *red = reinterpret_cast<float *>(&lds[0][0]);  // [4 waves][4 rs][NT][4][64]
    constexpr int per = 4 * NT * 4;
#pragma unroll
    for (int rs = 0; rs < 4; rs++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[((wave * per) + (rs * NT + nt) * 4 + r) * kWave + lane] = acc[rs][nt][r];
    __syncthreads();
    if (wave != 0) return;
    float *dst = out + (size_t)ks * split_stride;
#pragma unroll
    for (int rs = 0; rs < 4; rs++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int idx = (rs * NT + nt) * 4 + r;
                float sum = red[idx * kWave + lane];
#pragma unroll
                for (int v = 1; v < kWavesPerWg; v++) sum += red[(v * per + idx) * kWave + lane];
                const int row = row0 + rs * 16 + li;
                const int b = 16 * nt + 4 * g + r;
                if (row < m && b < batch) dst[(size_t)b * m + row] = ldexpf(sum, xeE[b]);
            }
}

// x-stationary form of quant_gemm_mfma for matrices of many row tiles at
// batch 2..16 (lm_head): 8 waves per workgroup, wave w holds the x fragments
// (hi + lo, brought to one exponent per batch row over the split's 16
// groups, as quant_gemm_mfma) of super-block ks * 8 + w in registers, and
// the workgroup walks the row tiles t = blockIdx.x, + gridDim.x, ...  Per
// tile each wave stages its 64 rows x 1 super-block of GGUF blocks through
// its own LDS slice and issues the next tile's loads at once (in flight
// while this tile is multiplied), then the 8 waves' sums are added through
// LDS (the staging area, after a barrier).  The x fragments are loaded once
// per workgroup instead of once per tile (lm_head at batch 16: 2374 tiles x
// 128 KiB of x from L2 otherwise).  grid = (workgroups per split, K splits
// of 8 super-blocks); output as quant_gemm_mfma.
template <uint32_t T>
__global__ __launch_bounds__(512) void quant_gemm_xs(const uint8_t *__restrict__ W, Planes xp, float *__restrict__ out,
                                                     int m, int n, int batch, size_t split_stride) {
    constexpr int V = QTraits<T>::kSbVec;
    constexpr int NW = 8;
    constexpr int kSegWords = QTraits<T>::kSbBytes / 4;
    constexpr int RED = 16;  // sums per lane: [row group rs][element r]
    static_assert(NW * RED * kWave * 4 <= NW * V * kWave * 16, "the reduction fits the staging area");
    __shared__ u32x4 lds[NW][V * kWave];
    __shared__ int xeE[16];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int G = gridDim.x, ks = blockIdx.y;
    const int nsb = n >> 8, tiles = (m + kWave - 1) / kWave;
    const uint32_t row_bytes = (uint32_t)nsb * QTraits<T>::kSbBytes;
    const int sb = ks * NW + wave;
    const int li = lane & 15, g = lane >> 4;
    int t = blockIdx.x;
    if (t >= tiles) return;  // uniform
    // chunk c = 64 j + lane of a tile's super-block column: (row c / V, part
    // c % V), rows past m clamped to the last row (never stored)
    u32x4 regs[V];
    auto issue = [&](int tt) {
        const int rows_left = m - tt * kWave;
        const uint8_t *base = W + (size_t)tt * kWave * row_bytes + (size_t)sb * QTraits<T>::kSbBytes;
#pragma unroll
        for (int j = 0; j < V; j++) {
            const int c = j * kWave + lane;
            const uint32_t o = (uint32_t)min(c / V, rows_left - 1) * row_bytes + (uint32_t)(c % V) * 16u;
            regs[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base + o));
        }
    };
    issue(t);
    // A fragments x[b = li][sb * 256 + 32 blk + 8 g + e] (rows past the batch
    // read row batch - 1; their outputs are never stored), loaded after the
    // first tile's weights were issued
    h8v ah[8], al[8];
    {
        const int b = min(li, batch - 1);
        const int En = xe_max(xp.xe, b, 2 * ks * NW, 2 * NW, n);
        if (wave == 0 && g == 0) xeE[li] = En;
        const int8_t *e = xp.xe + (size_t)b * xe_stride(n) + 2 * sb;
        const _Float16 f0 = xe_factor(e[0], En), f1 = xe_factor(e[1], En);
#pragma unroll
        for (int blk = 0; blk < 8; blk++) {
            const size_t xo = (size_t)b * n + (size_t)sb * 256 + 32 * blk + 8 * g;
            const _Float16 f = blk < 4 ? f0 : f1;
            ah[blk] = *reinterpret_cast<const h8v *>(xp.hi + xo) * f;
            al[blk] = *reinterpret_cast<const h8v *>(xp.lo + xo) * f;
        }
    }
    const uint32_t *lw = reinterpret_cast<const uint32_t *>(lds[wave]);
    float *red = reinterpret_cast<float *>(&lds[0][0]);  // [wave][RED][lane], after the tile's barrier
    float *dst = out + (size_t)ks * split_stride;
    for (; t < tiles; t += G) {
        stage_tile<T>(regs, lds[wave], lane);
        if (t + G < tiles) issue(t + G);
        f32x4 acc[4];
#pragma unroll
        for (int rs = 0; rs < 4; rs++) acc[rs] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int blk = 0; blk < 8; blk++) {
#pragma unroll
            for (int rs = 0; rs < 4; rs++) {
                const uint32_t *wl = lw + (rs * 16 + li) * kSegWords;
                const h8v bw = (blk & 1) ? w_frag<T, 1>(wl, blk, g) : w_frag<T, 0>(wl, blk, g);
                const float d = blk_scale<T>(wl, blk);
                f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[blk], bw, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[blk], bw, c, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) acc[rs][r] = fmaf(c[r], d, acc[rs][r]);
            }
            __builtin_amdgcn_sched_barrier(0);  // one block's weight fragments live at a time
        }
        __syncthreads();  // every wave is done with its slice
#pragma unroll
        for (int rs = 0; rs < 4; rs++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[(wave * RED + rs * 4 + r) * kWave + lane] = acc[rs][r];
        __syncthreads();
        // outputs (tile row rs * 16 + l % 16, batch row 4 (l / 16) + r), the
        // 8 waves added in wave order
#pragma unroll
        for (int k = 0; k < RED * kWave / 512; k++) {
            const int o = (int)threadIdx.x + 512 * k;
            const int idx = o >> 6, l = o & 63;
            float s = red[idx * kWave + l];
#pragma unroll
            for (int w = 1; w < NW; w++) s += red[(w * RED + idx) * kWave + l];
            const int row = t * kWave + (idx >> 2) * 16 + (l & 15), b = 4 * (l >> 4) + (idx & 3);
            if (row < m && b < batch) dst[(size_t)b * m + row] = ldexpf(s, xeE[b]);
        }
        __syncthreads();  // the staging area is free again
    }
}

// The same for batch 17..32: wave w = 4 h + q holds the x fragments of batch
// rows 16 h .. + 15 for the two super-blocks ks * 8 + 2 q, + 1 (128
// registers: 32 rows of one super-block would not fit beside the weights in
// flight at two waves per SIMD) and loads segment 2 q + h of each tile; the
// pair's two segments are shared through LDS by waves q and q + 4, and each
// batch half's 4 waves are added per tile.  The lane's load offsets are
// recomputed per tile (held across the loop they cost 34 registers and the
// kernel spilled).  lm_head 151936 x 2048 at batch 17 / 32: 126.8-128.0 /
// 133.4-133.6 us against 134.3-141.8 / 160.3-166.1 us on quant_gemm_mfma<T,
// 2> (graphs of back-to-back launches).
template <uint32_t T>
__global__ __launch_bounds__(512) void quant_gemm_xs32(const uint8_t *__restrict__ W, Planes xp,
                                                       float *__restrict__ out, int m, int n, int batch,
                                                       size_t split_stride) {
    constexpr int V = QTraits<T>::kSbVec;
    constexpr int kSegWords = QTraits<T>::kSbBytes / 4;
    constexpr int RED = 16;  // sums per lane: [row group rs][element r]
    static_assert(8 * RED * kWave * 4 <= 8 * V * kWave * 16, "the reduction fits the staging area");
    __shared__ u32x4 lds[4][2][V * kWave];
    __shared__ int xeE[32];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int hh = wave >> 2, q = wave & 3;
    const int G = gridDim.x, ks = blockIdx.y;
    const int nsb = n >> 8, tiles = (m + kWave - 1) / kWave;
    const uint32_t row_bytes = (uint32_t)nsb * QTraits<T>::kSbBytes;
    const int sb0 = ks * 8 + 2 * q;
    const int li = lane & 15, g = lane >> 4;
    int t = blockIdx.x;
    if (t >= tiles) return;  // uniform
    u32x4 regs[V];
    auto issue = [&](int tt) {
        int ln = lane;
        asm volatile("" : "+v"(ln));  // not loop-invariant: the offsets are not kept in registers
        const int rows_left = m - tt * kWave;
        const uint8_t *base = W + (size_t)tt * kWave * row_bytes + (size_t)(sb0 + hh) * QTraits<T>::kSbBytes;
#pragma unroll
        for (int j = 0; j < V; j++) {
            const int c = j * kWave + ln;
            const uint32_t o = (uint32_t)min(c / V, rows_left - 1) * row_bytes + (uint32_t)(c % V) * 16u;
            regs[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base + o));
        }
    };
    issue(t);
    h8v ah[2][8], al[2][8];
    {
        const int b = min(li + 16 * hh, batch - 1);
        const int En = xe_max(xp.xe, b, 2 * ks * 8, 16, n);
        if (q == 0 && g == 0) xeE[li + 16 * hh] = En;
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int8_t *e = xp.xe + (size_t)b * xe_stride(n) + 2 * (sb0 + s);
            const _Float16 f0 = xe_factor(e[0], En), f1 = xe_factor(e[1], En);
#pragma unroll
            for (int blk = 0; blk < 8; blk++) {
                const size_t xo = (size_t)b * n + (size_t)(sb0 + s) * 256 + 32 * blk + 8 * g;
                const _Float16 f = blk < 4 ? f0 : f1;
                ah[s][blk] = *reinterpret_cast<const h8v *>(xp.hi + xo) * f;
                al[s][blk] = *reinterpret_cast<const h8v *>(xp.lo + xo) * f;
            }
        }
    }
    float *red = reinterpret_cast<float *>(&lds[0][0][0]);  // [wave][RED][lane], after the tile's barrier
    float *dst = out + (size_t)ks * split_stride;
    for (; t < tiles; t += G) {
#pragma unroll
        for (int j = 0; j < V; j++) lds[q][hh][j * kWave + lane] = regs[j];
        __syncthreads();  // both segments of every pair staged
        if (t + G < tiles) issue(t + G);
        f32x4 acc[4];
#pragma unroll
        for (int rs = 0; rs < 4; rs++) acc[rs] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const uint32_t *lw = reinterpret_cast<const uint32_t *>(lds[q][s]);
#pragma unroll
            for (int blk = 0; blk < 8; blk++) {
#pragma unroll
                for (int rs = 0; rs < 4; rs++) {
                    const uint32_t *wl = lw + (rs * 16 + li) * kSegWords;
                    const h8v bw = (blk & 1) ? w_frag<T, 1>(wl, blk, g) : w_frag<T, 0>(wl, blk, g);
                    const float d = blk_scale<T>(wl, blk);
                    f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[s][blk], bw, f32x4{0.f, 0.f, 0.f, 0.f}, 0,
                                                                     0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[s][blk], bw, c, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[rs][r] = fmaf(c[r], d, acc[rs][r]);
                    __builtin_amdgcn_sched_barrier(0);  // one weight fragment live at a time
                }
            }
        }
        __syncthreads();  // every wave is done with the staged segments
#pragma unroll
        for (int rs = 0; rs < 4; rs++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[(wave * RED + rs * 4 + r) * kWave + lane] = acc[rs][r];
        __syncthreads();
        // output o: batch half h = o / 1024, then (rs, r, lane); the half's 4
        // waves added in wave order
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int o = (int)threadIdx.x + 512 * k;
            const int h = o >> 10, idx = (o >> 6) & 15, l = o & 63;
            float sum = red[((4 * h) * RED + idx) * kWave + l];
#pragma unroll
            for (int w = 1; w < 4; w++) sum += red[((4 * h + w) * RED + idx) * kWave + l];
            const int row = t * kWave + (idx >> 2) * 16 + (l & 15), b = 16 * h + 4 * (l >> 4) + (idx & 3);
            if (row < m && b < batch) dst[(size_t)b * m + row] = ldexpf(sum, xeE[b]);
        }
        __syncthreads();  // the staging area is free again
    }
}

// y[i] = sum over k of part[k][i], k ascending (deterministic).
__global__ __launch_bounds__(256) void sum_partials(const float *__restrict__ part, float *__restrict__ y,
                                                   size_t count, int ksplit) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= count) return;
    float s = part[i];
    for (int k = 1; k < ksplit; k++) s += part[(size_t)k * count + i];
    y[i] = s;
}
// The same, 4 consecutive values per thread (count % 4 == 0) with every slice
// loaded before the first add (slices past ksplit re-read the last one and are
// not added), so a thread waits for one round trip instead of ksplit.
template <int KP>
__global__ __launch_bounds__(256) void sum_partials4(const float4 *__restrict__ part, float4 *__restrict__ y,
                                                     size_t count4, int ksplit) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= count4) return;
    float4 v[KP];
#pragma unroll
    for (int k = 0; k < KP; k++) v[k] = part[(size_t)min(k, ksplit - 1) * count4 + i];
    float4 s = v[0];
#pragma unroll
    for (int k = 1; k < KP; k++) {
        const bool on = k < ksplit;
        s.x = on ? s.x + v[k].x : s.x;
        s.y = on ? s.y + v[k].y : s.y;
        s.z = on ? s.z + v[k].z : s.z;
        s.w = on ? s.w + v[k].w : s.w;
    }
    y[i] = s;
}

// K splits: the smallest divisor k of the super-block count with at most 8
// super-blocks per workgroup, and at most one per wave (4) unless the row
// tiles alone already fill the chip (tiles * k >= 2 workgroups per CU).
int choose_ksplit(int tiles, int nsb, int cus, int max_k) {
    int best = 0;
    for (int k = 1; k <= nsb && k <= max_k; k++) {
        const int per = (nsb + k - 1) / k;
        if ((k - 1) * per >= nsb) continue;  // would leave a split empty
        if (per > kMaxSliceSb) continue;
        if (!best) best = k;
        if (per <= kWavesPerWg || tiles * k >= 2 * cus) return k;
    }
    return best ? best : min(nsb, max_k);
}

template <uint32_t T, int MODE>
int launch_fused(anehip_ctx *ctx, hipStream_t stream, const void *w, uint32_t m, uint32_t n, const GemvInput &in,
                 float *out, size_t split_stride, int ksplit) {
    const int tiles = (int)((m + kWave - 1) / kWave);
    const int per = split_len((int)(n / 256), ksplit);
    if (per > kMaxSliceSb)
        return set_error(ctx->err, ANEHIP_EINVAL, "gemv: %d super-blocks per split (max %d)", per, kMaxSliceSb);
    hipLaunchKernelGGL((gemv_fused<T, MODE>), dim3(tiles, ksplit), dim3(kWave * kWavesPerWg), 0, stream,
                       static_cast<const uint8_t *>(w), in, out, (int)m, (int)n, per, split_stride);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

template <uint32_t T>
int dispatch_fused(anehip_ctx *ctx, hipStream_t stream, const void *w, uint32_t m, uint32_t n, const GemvInput &in,
                   float *out, int ksplit) {
    const size_t ss = m;
    switch (in.mode) {
        case GEMV_IN_PLAIN: return launch_fused<T, GEMV_IN_PLAIN>(ctx, stream, w, m, n, in, out, ss, ksplit);
        case GEMV_IN_RMSNORM: return launch_fused<T, GEMV_IN_RMSNORM>(ctx, stream, w, m, n, in, out, ss, ksplit);
        case GEMV_IN_RESID_RMSNORM:
            return launch_fused<T, GEMV_IN_RESID_RMSNORM>(ctx, stream, w, m, n, in, out, ss, ksplit);
        case GEMV_IN_EMBED_RMSNORM:
            return launch_fused<T, GEMV_IN_EMBED_RMSNORM>(ctx, stream, w, m, n, in, out, ss, ksplit);
        case GEMV_IN_GATED_NORM: return launch_fused<T, GEMV_IN_GATED_NORM>(ctx, stream, w, m, n, in, out, ss, ksplit);
        case GEMV_IN_SILU_MUL: return launch_fused<T, GEMV_IN_SILU_MUL>(ctx, stream, w, m, n, in, out, ss, ksplit);
        default: return set_error(ctx->err, ANEHIP_EINVAL, "gemv: input mode %d", in.mode);
    }
}

template <uint32_t T, int NT>
int launch_mfma(anehip_ctx *ctx, hipStream_t stream, const void *w, uint32_t m, uint32_t n, const Planes &xp,
                uint32_t batch, float *out, size_t split_stride, int ksplit) {
    const int tiles = (int)((m + kWave - 1) / kWave);
    const int per = split_len((int)(n / 256), ksplit);
    hipLaunchKernelGGL((quant_gemm_mfma<T, NT>), dim3(tiles, ksplit), dim3(kWave * kWavesPerWg), 0, stream,
                       static_cast<const uint8_t *>(w), xp, out, (int)m, (int)n, (int)batch, per, split_stride);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

template <uint32_t T>
int dispatch_raw(anehip_ctx *ctx, hipStream_t stream, const void *w, uint32_t m, uint32_t n, const float *x,
                 uint32_t batch, float *out, int ksplit, _Float16 *xsplit) {
    const size_t split_stride = (size_t)batch * m;
    const int tiles = (int)((m + kWave - 1) / kWave), cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    // many row tiles (at least 4 per CU) with K splits of 8 super-blocks: the
    // x-stationary kernels, one workgroup per CU walking the row tiles with
    // the split's x staged once (batch 1: as digits in LDS; batch 2..32: as
    // MFMA fragments in registers)
    const bool xs = (int)(n / 256) == 8 * ksplit && tiles >= 4 * cus;
    if (batch == 1) {
        if (xs) {
            hipLaunchKernelGGL((gemv_fused_xs<T>), dim3(min(tiles, cus), ksplit), dim3(512), 0, stream,
                               static_cast<const uint8_t *>(w), x, out, (int)m, (int)n, split_stride);
            ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
            return ANEHIP_OK;
        }
        GemvInput in;
        in.x = x;
        return dispatch_fused<T>(ctx, stream, w, m, n, in, out, ksplit);
    }
    // batch 2..32: split x into range-safe fp16 hi/lo planes (row-major),
    // then the MFMA kernel
    const size_t count = (size_t)batch * n;
    Planes xp;
    xp.hi = xsplit;
    xp.lo = xsplit + count;
    xp.xe = reinterpret_cast<int8_t *>(xsplit + 2 * count);
    const size_t vecs = count / 8;
    hipLaunchKernelGGL(split_x_kernel, dim3((unsigned)((vecs + 255) / 256)), dim3(256), 0, stream, x, xp, (int)batch,
                       (int)n);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    // (lm_head 151936 x 2048 at batch 4 / 16 / 32: 75.6-77.2 / 80.1-82.9 /
    // 133.4-133.6 us against 95.8-102.8 / 104.7-113.5 / 160.3-166.1 us on
    // quant_gemm_mfma, graphs of back-to-back launches)
    if (xs) {
        const dim3 grid(min(tiles, cus), ksplit);
        const uint8_t *wb = static_cast<const uint8_t *>(w);
        if (batch <= 16)
            hipLaunchKernelGGL((quant_gemm_xs<T>), grid, dim3(512), 0, stream, wb, xp, out, (int)m, (int)n,
                               (int)batch, split_stride);
        else
            hipLaunchKernelGGL((quant_gemm_xs32<T>), grid, dim3(512), 0, stream, wb, xp, out, (int)m, (int)n,
                               (int)batch, split_stride);
        ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
        return ANEHIP_OK;
    }
    if (batch <= 16) return launch_mfma<T, 1>(ctx, stream, w, m, n, xp, batch, out, split_stride, ksplit);
    // 17..32 rows: a matrix that stays in the 256 MiB MALL takes two 16-row
    // passes (the second reads the weights from the MALL), a larger one the
    // 32-row kernel.  Measured on MI355X (graphs of back-to-back launches):
    // 6144 x 2048 at 32 rows 24.7 us in one 32-row pass against 9.3 us for
    // one 16-row pass.
    if ((double)m * (n / 32) * QTraits<T>::kBlockBytes <= 128.0 * (1 << 20)) {
        int rc = launch_mfma<T, 1>(ctx, stream, w, m, n, xp, 16, out, split_stride, ksplit);
        if (rc) return rc;
        Planes x2;
        x2.hi = xp.hi + (size_t)16 * n;
        x2.lo = xp.lo + (size_t)16 * n;
        x2.xe = xp.xe + (size_t)16 * xe_stride((int)n);
        return launch_mfma<T, 1>(ctx, stream, w, m, n, x2, batch - 16, out + (size_t)16 * m, split_stride, ksplit);
    }
    return launch_mfma<T, 2>(ctx, stream, w, m, n, xp, batch, out, split_stride, ksplit);
}

}  // namespace

// K splits of the batch-1 panel GEMV: the fewest that give `want` workgroups
// (at most kMaxSplit, whole panels, no empty split).
static int packed_ksplit(int tiles, int nsb, int want) {
    int best = 1;
    for (int k = 1; k <= nsb && k <= kMaxSplit; k++) {
        const int per = (nsb + k - 1) / k;
        if ((k - 1) * per >= nsb) continue;
        best = k;
        if (tiles * k >= want && per <= kMaxSliceSb) return k;
    }
    return best;
}

int gemm_ksplit(const anehip_ctx *ctx, uint32_t m, uint32_t n, int max_k) {
    const int tiles = (int)((m + kWave - 1) / kWave);
    return choose_ksplit(tiles, (int)(n / 256), ctx->cu_count > 0 ? ctx->cu_count : 256, max_k);
}

int gemv_packed_ksplit(const anehip_ctx *ctx, uint32_t m, uint32_t n, int mode) {
    const int tiles = (int)((m + kWave - 1) / kWave);
    const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    // a norm prologue re-reads the whole input vector (and its partial slices)
    // in every workgroup, so such GEMVs stop splitting at half the CUs; a
    // SiLU-mul prologue reads 2 partial slices per element of its split, and
    // stops at 3/4 (ffn_down 2048 x 6144 at batch 1: 5.3 us at 6 splits
    // against 5.7 at 8, measured in a graph of back-to-back launches)
    const bool norm = mode == GEMV_IN_RMSNORM || mode == GEMV_IN_RESID_RMSNORM || mode == GEMV_IN_EMBED_RMSNORM;
    return packed_ksplit(tiles, (int)(n / 256), norm ? cus / 2 : mode == GEMV_IN_SILU_MUL ? 3 * cus / 4 : cus);
}

// K splits of the panel MFMA GEMM.  Matrices of fewer row tiles than CUs
// take an x-stationary kernel with P = 2 panels per split (P = 1 when that
// grid would not reach two workgroups per CU, or for an odd panel count):
// measured on MI355X at batch 4 and 32 it beats the persistent kernel on
// every decode shape (12288 x 2048, batch 32: 10.4 us at k = 4 against
// 11.9 us; 2048 x 2048: 3.9 us at k = 8 against 5.4 us), and P = 2 halves
// the partial sums the consumer reads against P = 1 where the times tie.
// Matrices of at least 4 tiles per CU: no split at batch <= 16 (the 16-wide
// kernel holds 8 panels of x); above, splits of 8 panels (gemm_xsh with 4
// panels per wave: lm_head at batch 32 74 us in one pass, against 71 us at
// k = 2 plus 11 us for the consumer's pass over the two partial sums), else of 4.
// Otherwise, among the even splits of at most kMaxSplit, the one that
// minimises the panels of the busiest CU, ceil(items / CUs) x panels per
// split, with single-panel splits counted double and ties going to fewer
// splits.
int gemm_packed_ksplit(const anehip_ctx *ctx, uint32_t m, uint32_t n, uint32_t batch) {
    const int tiles = (int)((m + kWave - 1) / kWave);
    const int nsb = (int)(n / 256), cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    if (tiles < cus && nsb >= 2) {
        const int P = nsb % 2 == 0 && tiles * nsb > 2 * cus ? 2 : 1;
        if (nsb / P <= kMaxGemmSplit) return nsb / P;
    }
    if (tiles >= 4 * cus) {
        if (batch <= 16) return 1;
        if (nsb % 8 == 0 && nsb / 8 <= kMaxGemmSplit) return nsb / 8;
        return nsb % 4 == 0 && nsb / 4 <= kMaxGemmSplit ? nsb / 4 : 1;
    }
    int best = 1;
    double best_cost = 1e30;
    for (int k = 1; k <= nsb && k <= kMaxSplit; k++) {
        if (nsb % k) continue;
        const int per = nsb / k;
        const double cost = (double)((tiles * k + cus - 1) / cus) * per * (per == 1 ? 2.0 : 1.0);
        if (cost < best_cost) {
            best_cost = cost;
            best = k;
        }
    }
    return best;
}

// Persistent grid of 1-tile workgroups, two per CU.  (Two tiles per wave, at
// one wave per SIMD, halves the x loads but measured no faster: 84 vs 90 us
// on lm_head at batch 32, slower at batch 4 and 16 and on the small shapes.)
template <uint32_t T>
int launch_gemm_packed_t(anehip_ctx *ctx, hipStream_t stream, const uint8_t *w, uint32_t m, uint32_t n,
                         const Planes &xp, uint32_t batch, float *out, int ksplit, int per, size_t ss) {
    const int tiles = (int)((m + kWave - 1) / kWave), cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const int items = tiles * ksplit;
    hipLaunchKernelGGL((gemm_packed<T, 1, kGemmRing>), dim3(min(items, 2 * cus)), dim3(kWave * kGemmWaves), 0, stream,
                       w, xp, out, (int)m, (int)n, (int)batch, ksplit, per, ss);
    return ANEHIP_OK;
}

// Which kernel runs an even or uneven K split of nsb panels at a batch size.
// Batch <= 16: the 16-wide x-stationary kernel on splits of 1, 2, 4 or 8
// panels.  Batch 17-32: gemm_xsh (8 waves, the split's panels shared by two
// groups of 4) on splits of 2 or 4 panels, gemm_xs on single-panel splits.
// Measured on MI355X against the 4-wave x-stationary kernel at P = 2, batch
// 17 / 32: 12288 x 2048 8.7 / 8.8 us against 9.2 / 9.6, 6144 x 2048 6.4 / 6.7
// against 6.8 / 7.1, 2048 x 6144 6.4 / 6.7 against 6.7 / 7.2.  Everything
// else (uneven splits) on the persistent kernel.
enum class GemmKernel { Persistent, Xs16, Xs32, Xsh };
static GemmKernel gemm_kernel(uint32_t batch, int nsb, int ksplit) {
    const int per = nsb / ksplit;
    if (per * ksplit != nsb) return GemmKernel::Persistent;
    if (batch <= 16) return per == 1 || per == 2 || per == 4 || per == 8 ? GemmKernel::Xs16 : GemmKernel::Persistent;
    if (per == 2 || per == 4 || per == 8) return GemmKernel::Xsh;
    if (per == 1 && ksplit >= 2) return GemmKernel::Xs32;
    return GemmKernel::Persistent;
}

// Grids (measured on MI355X at batch 4 to 32): gemm_xs16 four workgroups per
// CU at P = 1 (one unit in flight, a small register file), two at P >= 2
// (two in flight); gemm_xs three per CU; gemm_xsh one 8-wave workgroup per CU
// with one unit in flight at 1 panel per wave, two at 2.  A whole number of
// workgroups per split in every case.
template <uint32_t T>
void launch_gemm_xs_any(anehip_ctx *ctx, hipStream_t stream, GemmKernel kind, const uint8_t *w, uint32_t m,
                        uint32_t n, const Planes &xp, const float *xrows, uint32_t batch, float *out, int ksplit,
                        size_t ss) {
    const int tiles = (int)((m + kWave - 1) / kWave), cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const int per = (int)(n / 256) / ksplit;
    const int wgs = kind == GemmKernel::Xs16 ? (per == 1 ? 4 : 2) : kind == GemmKernel::Xs32 ? 3 : 1;
    const int gs = max(1, min(tiles, wgs * cus / ksplit));
    const dim3 grid(gs * ksplit);
#define ANEHIP_XS(KERNEL, NT)                                                                                       \
    hipLaunchKernelGGL(KERNEL, grid, dim3(NT), 0, stream, w, xp, xrows, out, (int)m, (int)n, (int)batch, ksplit, ss)
#define ANEHIP_XS2(KERNEL, NT, ...)                                                                                \
    do {                                                                                                           \
        if (xrows) ANEHIP_XS((KERNEL<__VA_ARGS__, true>), NT);                                                     \
        else ANEHIP_XS((KERNEL<__VA_ARGS__, false>), NT);                                                          \
    } while (0)
#define ANEHIP_XSH(PW, D)                                                                                          \
    do {                                                                                                           \
        if (xrows) ANEHIP_XS((gemm_xsh<T, PW, D, 2, true>), 512);                                                  \
        else if (xp.rs) ANEHIP_XS((gemm_xsh<T, PW, D, 2, false, false, true>), 512);                               \
        else ANEHIP_XS((gemm_xsh<T, PW, D, 2, false>), 512);                                                       \
    } while (0)
    if (kind == GemmKernel::Xs16) {
        if (per == 1)
            ANEHIP_XS2(gemm_xs16, 256, T, 1, 1, 4);
        else if (per == 2)
            ANEHIP_XS2(gemm_xs16, 256, T, 2, 2, 2);
        else if (per == 4)
            ANEHIP_XS2(gemm_xs16, 256, T, 4, 2, 2);
        else
            ANEHIP_XS2(gemm_xs16, 256, T, 8, 2, 2);
    } else if (kind == GemmKernel::Xsh) {
        if (per == 2)
            ANEHIP_XSH(1, 1);
        else if (per == 4)
            ANEHIP_XSH(2, 2);
        else
            ANEHIP_XSH(4, 2);
    } else {
        ANEHIP_XS2(gemm_xs, 256, T, 1, 1);
    }
#undef ANEHIP_XSH
#undef ANEHIP_XS2
#undef ANEHIP_XS
}

bool gemm_is_xs(const anehip_ctx *ctx, uint32_t m, uint32_t n, uint32_t batch) {
    return gemm_kernel(batch, (int)(n / 256), gemm_packed_ksplit(ctx, m, n, batch)) != GemmKernel::Persistent;
}

bool gemm_takes_norm_scale(const anehip_ctx *ctx, uint32_t m, uint32_t n, uint32_t batch) {
    return n % 256 == 0 && n / 256 <= kMaxRsParts &&
           gemm_kernel(batch, (int)(n / 256), gemm_packed_ksplit(ctx, m, n, batch)) == GemmKernel::Xsh;
}

static int check_gemm_args(anehip_ctx *ctx, uint32_t m, uint32_t n, uint32_t batch, int ksplit, size_t ss) {
    const int nsb = (int)(n / 256), per = split_len(nsb, ksplit);
    if (ksplit < 1 || (ksplit - 1) * per >= nsb || batch < 1 || batch > 32 || m % 4 || ss < (size_t)batch * m)
        return set_error(ctx->err, ANEHIP_EINVAL,
                         "gemm: K split %d of %d super-blocks, batch %u, m %u (multiple of 4) or split stride %zu "
                         "unsupported",
                         ksplit, nsb, batch, m, ss);
    if (4.0 * ksplit * (double)ss > 1073741824.0)  // output byte offsets stay below kBadOffset
        return set_error(ctx->err, ANEHIP_ESHAPE, "gemm: output of %d x %zu floats too large", ksplit, ss);
    return ANEHIP_OK;
}

int launch_gemm_xs_rows(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *wp, uint32_t m,
                        uint32_t n, const float *x, uint32_t batch, float *out) {
    const int ksplit = gemm_packed_ksplit(ctx, m, n, batch);
    if (int rc = check_gemm_args(ctx, m, n, batch, ksplit, (size_t)batch * m)) return rc;
    const GemmKernel kind = gemm_kernel(batch, (int)(n / 256), ksplit);
    if (kind == GemmKernel::Persistent)
        return set_error(ctx->err, ANEHIP_EINVAL, "gemm: %u x %u at batch %u is not an x-stationary shape", m, n,
                         batch);
    const uint8_t *w = static_cast<const uint8_t *>(wp);
    if (ggml_type == ANEHIP_GGML_Q8_0)
        launch_gemm_xs_any<ANEHIP_GGML_Q8_0>(ctx, stream, kind, w, m, n, Planes{}, x, batch, out, ksplit,
                                             (size_t)batch * m);
    else
        launch_gemm_xs_any<ANEHIP_GGML_Q4_0>(ctx, stream, kind, w, m, n, Planes{}, x, batch, out, ksplit,
                                             (size_t)batch * m);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

bool gemm_gate_up_silu_ok(const anehip_ctx *ctx, uint32_t m, uint32_t n, uint32_t batch) {
    (void)ctx;
    const int nsb = (int)(n / 256);
    return batch > 16 && batch <= 32 && n % 256 == 0 && m % 64 == 0 && (nsb == 2 || nsb == 4 || nsb == 8) &&
           gemm_kernel(batch, nsb, 1) == GemmKernel::Xsh;
}

// The FFN's gate / up product in one K split with the SiLU-mul in its
// epilogue (gemm_xsh<..., SILU>): h[b][f] for the interleaved [gate; up]
// panel matrix of m = 2 F rows, fp32 rows [batch][F].  Measured on MI355X at
// batch 32, 12288 x 2048: the unsplit product 11.8 us against 9.7 us in 4
// splits plus 4.8 us for the SiLU-mul launch that read them.
int launch_gemm_gate_up_silu(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *wp, uint32_t m,
                             uint32_t n, const Planes &xp, uint32_t batch, float *h) {
    if (!gemm_gate_up_silu_ok(ctx, m, n, batch))
        return set_error(ctx->err, ANEHIP_EINVAL, "gemm_gate_up_silu: %u x %u at batch %u not covered", m, n, batch);
    if (xp.rs && (xp.rs_parts < 1 || xp.rs_parts > kMaxRsParts))
        return set_error(ctx->err, ANEHIP_EINVAL, "gemm_gate_up_silu: %d norm parts", xp.rs_parts);
    const int tiles = (int)(m / kWave), cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const dim3 grid(max(1, min(tiles, cus)));
    const uint8_t *w = static_cast<const uint8_t *>(wp);
    const size_t ss = (size_t)batch * (m / 2);
#define ANEHIP_GUS(TT, PW, D)                                                                                     \
    do {                                                                                                          \
        if (xp.rs)                                                                                                \
            hipLaunchKernelGGL((gemm_xsh<TT, PW, D, 2, false, true, true>), grid, dim3(512), 0, stream, w, xp,    \
                               nullptr, h, (int)m, (int)n, (int)batch, 1, ss);                                    \
        else                                                                                                      \
            hipLaunchKernelGGL((gemm_xsh<TT, PW, D, 2, false, true>), grid, dim3(512), 0, stream, w, xp, nullptr, \
                               h, (int)m, (int)n, (int)batch, 1, ss);                                             \
    } while (0)
    const int nsb = (int)(n / 256);
    if (ggml_type == ANEHIP_GGML_Q8_0) {
        if (nsb == 2) ANEHIP_GUS(ANEHIP_GGML_Q8_0, 1, 1);
        else if (nsb == 4) ANEHIP_GUS(ANEHIP_GGML_Q8_0, 2, 2);
        else ANEHIP_GUS(ANEHIP_GGML_Q8_0, 4, 2);
    } else {
        if (nsb == 2) ANEHIP_GUS(ANEHIP_GGML_Q4_0, 1, 1);
        else if (nsb == 4) ANEHIP_GUS(ANEHIP_GGML_Q4_0, 2, 2);
        else ANEHIP_GUS(ANEHIP_GGML_Q4_0, 4, 2);
    }
#undef ANEHIP_GUS
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_gemm_packed(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *wp, uint32_t m,
                       uint32_t n, const Planes &xp, uint32_t batch, float *out, int ksplit, size_t split_stride) {
    const size_t ss = split_stride ? split_stride : (size_t)batch * m;
    if (int rc = check_gemm_args(ctx, m, n, batch, ksplit, ss)) return rc;
    if (!xp.hi || !xp.lo || !xp.xe) return set_error(ctx->err, ANEHIP_EINVAL, "gemm: input planes incomplete");
    const int per = split_len((int)(n / 256), ksplit);
    const uint8_t *w = static_cast<const uint8_t *>(wp);
    const GemmKernel kind = gemm_kernel(batch, (int)(n / 256), ksplit);
    if (xp.rs && (kind != GemmKernel::Xsh || xp.rs_parts < 1 || xp.rs_parts > kMaxRsParts))
        return set_error(ctx->err, ANEHIP_EINVAL,
                         "gemm: a deferred norm scale (%d parts) needs the 17..32-row x-stationary kernel", xp.rs_parts);
    const bool q8 = ggml_type == ANEHIP_GGML_Q8_0;
    if (kind != GemmKernel::Persistent && q8)
        launch_gemm_xs_any<ANEHIP_GGML_Q8_0>(ctx, stream, kind, w, m, n, xp, nullptr, batch, out, ksplit, ss);
    else if (kind != GemmKernel::Persistent)
        launch_gemm_xs_any<ANEHIP_GGML_Q4_0>(ctx, stream, kind, w, m, n, xp, nullptr, batch, out, ksplit, ss);
    else if (q8)
        launch_gemm_packed_t<ANEHIP_GGML_Q8_0>(ctx, stream, w, m, n, xp, batch, out, ksplit, per, ss);
    else
        launch_gemm_packed_t<ANEHIP_GGML_Q4_0>(ctx, stream, w, m, n, xp, batch, out, ksplit, per, ss);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

// K split of gemm_tall (one tile per item: two tiles per item measured 9.6 us
// per unit against 4.6 us for one, no gain per row): a divisor of the panel count (at most 16, the partial slices
// a consumer sums) minimising an estimate of the busiest CU's time,
// ceil(items / CUs) x panels per split x the measured time of one unit at 256
// rows (4.6 us on MI355X), plus the traffic of the extra partial slices
// (written here, read by the consumer: 2 x 4 bytes per row and output, at
// 256 rows ~2 KiB per output, at ~5 TB/s).
static int gemm_tall_ksplit(const anehip_ctx *ctx, uint32_t m, uint32_t n) {
    const int ptiles = (int)((m + kWave - 1) / kWave);
    const int nsb = (int)(n / 256), cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const double unit_us = 4.6, part_us_per_row = 2048.0 / 5.0e6;
    int best = 1;
    double best_cost = -1.0;
    for (int k = 1; k <= nsb && k <= 16; k++) {
        if (nsb % k) continue;
        const double cost =
            (double)((ptiles * k + cus - 1) / cus) * (nsb / k) * unit_us + (k - 1) * (double)m * part_us_per_row;
        if (best_cost < 0.0 || cost < best_cost) {
            best_cost = cost;
            best = k;
        }
    }
    return best;
}

int gemm_rows_ksplit(const anehip_ctx *ctx, uint32_t m, uint32_t n, uint32_t rows) {
    return rows <= 32 ? gemm_packed_ksplit(ctx, m, n, rows) : gemm_tall_ksplit(ctx, m, n);
}

int launch_gemm_rows(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *wp, uint32_t m, uint32_t n,
                     const Planes &xp, uint32_t rows, float *out, int ksplit) {
    if (rows <= 32) return launch_gemm_packed(ctx, stream, ggml_type, wp, m, n, xp, rows, out, ksplit);
    const int nsb = (int)(n / 256), ptiles = (int)((m + kWave - 1) / kWave);
    if (rows > kTallMaxRows || ksplit < 1 || nsb % ksplit || m % 4 || !xp.hi || !xp.lo || !xp.xe)
        return set_error(ctx->err, ANEHIP_EINVAL, "gemm_rows: %u rows (at most %d), K split %d of %d panels, m %u",
                         rows, kTallMaxRows, ksplit, nsb, m);
    if (4.0 * ksplit * rows * m > 1073741824.0)
        return set_error(ctx->err, ANEHIP_ESHAPE, "gemm_rows: output of %d x %u x %u floats too large", ksplit, rows, m);
    // gemm_tall addresses the weights with 32-bit buffer offsets
    if ((double)ptiles * nsb * Panel<ANEHIP_GGML_Q8_0>::kBytes > 2147483647.0)
        return set_error(ctx->err, ANEHIP_ESHAPE, "gemm_rows: %u x %u weights too large (2 GiB of panels at most)", m, n);
    const int items = ptiles * ksplit;
    // one workgroup per CU, each walking its items' panels in one pipeline
    const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const dim3 grid((unsigned)std::min(items, cus)), block(kWave * (kTallWaves + 1));
    const uint8_t *w = static_cast<const uint8_t *>(wp);
    const int per = nsb / ksplit;
    const size_t ss = (size_t)rows * m;
    if (ggml_type == ANEHIP_GGML_Q8_0)
        hipLaunchKernelGGL(gemm_tall<ANEHIP_GGML_Q8_0>, grid, block, 0, stream, w, xp, out, (int)m, (int)n,
                           (int)rows, ksplit, per, ss);
    else
        hipLaunchKernelGGL(gemm_tall<ANEHIP_GGML_Q4_0>, grid, block, 0, stream, w, xp, out, (int)m, (int)n,
                           (int)rows, ksplit, per, ss);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_unpack(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *src, uint32_t m, uint32_t n,
                  void *dst, uint32_t il) {
    if (il && (m != 2 * il || il % 32))
        return set_error(ctx->err, ANEHIP_EINVAL, "unpack: %u rows cannot interleave halves of %u", m, il);
    const size_t nvec = packed_bytes(ggml_type, m, n) / 16;
    const unsigned grid = (unsigned)((nvec + 255) / 256);
    if (ggml_type == ANEHIP_GGML_Q8_0)
        hipLaunchKernelGGL(unpack_kernel<ANEHIP_GGML_Q8_0>, dim3(grid), dim3(256), 0, stream,
                           static_cast<const uint8_t *>(src), static_cast<uint8_t *>(dst), (int)m, (int)n, nvec,
                           (int)il);
    else
        hipLaunchKernelGGL(unpack_kernel<ANEHIP_GGML_Q4_0>, dim3(grid), dim3(256), 0, stream,
                           static_cast<const uint8_t *>(src), static_cast<uint8_t *>(dst), (int)m, (int)n, nvec,
                           (int)il);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

size_t packed_bytes(uint32_t ggml_type, uint32_t m, uint32_t n) {
    const size_t tiles = (m + 63) / 64, nsb = n / 256;
    return tiles * nsb * (ggml_type == ANEHIP_GGML_Q8_0 ? Panel<ANEHIP_GGML_Q8_0>::kBytes : Panel<ANEHIP_GGML_Q4_0>::kBytes);
}

int launch_repack(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *src, uint32_t m, uint32_t n,
                  void *dst, uint32_t il) {
    if (il && (m != 2 * il || il % 32))
        return set_error(ctx->err, ANEHIP_EINVAL, "repack: %u rows cannot interleave halves of %u", m, il);
    const size_t nvec = packed_bytes(ggml_type, m, n) / 16;
    const unsigned grid = (unsigned)((nvec + 255) / 256);
    if (ggml_type == ANEHIP_GGML_Q8_0)
        hipLaunchKernelGGL(repack_kernel<ANEHIP_GGML_Q8_0>, dim3(grid), dim3(256), 0, stream,
                           static_cast<const uint8_t *>(src), static_cast<uint8_t *>(dst), (int)m, (int)n, nvec,
                           (int)il);
    else
        hipLaunchKernelGGL(repack_kernel<ANEHIP_GGML_Q4_0>, dim3(grid), dim3(256), 0, stream,
                           static_cast<const uint8_t *>(src), static_cast<uint8_t *>(dst), (int)m, (int)n, nvec,
                           (int)il);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}


template <uint32_t T, int MODE, int KP, int S>
void launch_packed_s(hipStream_t stream, const uint8_t *w, uint32_t m, uint32_t n, const GemvInput &in, float *out,
                     int ksplit, int per, int tpw) {
    const int tiles = (int)((m + kWave - 1) / kWave);
    const dim3 grid((tiles + tpw - 1) / tpw, ksplit), block(kWave * kPackedWaves);
    hipLaunchKernelGGL((gemv_packed<T, MODE, KP, S>), grid, block, 0, stream, w, in, out, (int)m, (int)n, per,
                       (size_t)m, tpw);
}

template <uint32_t T, int MODE, int KP>
void launch_packed_k(hipStream_t stream, const uint8_t *w, uint32_t m, uint32_t n, const GemvInput &in, float *out,
                     int ksplit, int per, int tpw) {
    // waves per panel: as many as keep one round covering the slice
    if (per <= 1) launch_packed_s<T, MODE, KP, 8>(stream, w, m, n, in, out, ksplit, per, tpw);
    else if (per <= 2) launch_packed_s<T, MODE, KP, 4>(stream, w, m, n, in, out, ksplit, per, tpw);
    else if (per <= 4) launch_packed_s<T, MODE, KP, 2>(stream, w, m, n, in, out, ksplit, per, tpw);
    else launch_packed_s<T, MODE, KP, 1>(stream, w, m, n, in, out, ksplit, per, tpw);
}

template <uint32_t T, int MODE>
int launch_packed_t(anehip_ctx *ctx, hipStream_t stream, const void *w, uint32_t m, uint32_t n, const GemvInput &in,
                    float *out, int ksplit) {
    const int tiles = (int)((m + kWave - 1) / kWave);
    const int per = split_len((int)(n / 256), ksplit);
    const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    // a workgroup takes several row tiles when there are many: the prologue's
    // re-reads of the input vector are then shared
    const int tpw = MODE != GEMV_IN_PLAIN && tiles * ksplit >= 8 * cus ? 2 : 1;
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    constexpr bool has_parts =
        MODE == GEMV_IN_RESID_RMSNORM || MODE == GEMV_IN_SILU_MUL || MODE == GEMV_IN_GATED_NORM ||
        MODE == GEMV_IN_ATTN_COMBINE;
    if constexpr (MODE == GEMV_IN_ATTN_COMBINE) {
        if (per != 1 || n % 256 != 0 || !in.att_o || !in.att_ml || !in.att_pos || in.att_g <= 0 || in.att_nch <= 0)
            return set_error(ctx->err, ANEHIP_EINVAL, "gemv: attention combine needs one head (256 columns) per split");
    }
    if constexpr (has_parts) {
        if (in.kp > 2) launch_packed_k<T, MODE, kMaxSplit>(stream, wb, m, n, in, out, ksplit, per, tpw);
        else launch_packed_k<T, MODE, 2>(stream, wb, m, n, in, out, ksplit, per, tpw);
    } else {
        launch_packed_k<T, MODE, 2>(stream, wb, m, n, in, out, ksplit, per, tpw);
    }
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

template <uint32_t T>
int dispatch_packed(anehip_ctx *ctx, hipStream_t s, const void *w, uint32_t m, uint32_t n, const GemvInput &in,
                    float *out, int ksplit) {
    switch (in.mode) {
        case GEMV_IN_PLAIN: return launch_packed_t<T, GEMV_IN_PLAIN>(ctx, s, w, m, n, in, out, ksplit);
        case GEMV_IN_RMSNORM: return launch_packed_t<T, GEMV_IN_RMSNORM>(ctx, s, w, m, n, in, out, ksplit);
        case GEMV_IN_RESID_RMSNORM:
            return launch_packed_t<T, GEMV_IN_RESID_RMSNORM>(ctx, s, w, m, n, in, out, ksplit);
        case GEMV_IN_EMBED_RMSNORM:
            return launch_packed_t<T, GEMV_IN_EMBED_RMSNORM>(ctx, s, w, m, n, in, out, ksplit);
        case GEMV_IN_GATED_NORM:
            return launch_packed_t<T, GEMV_IN_GATED_NORM>(ctx, s, w, m, n, in, out, ksplit);
        case GEMV_IN_SILU_MUL: return launch_packed_t<T, GEMV_IN_SILU_MUL>(ctx, s, w, m, n, in, out, ksplit);
        case GEMV_IN_ATTN_COMBINE:
            return launch_packed_t<T, GEMV_IN_ATTN_COMBINE>(ctx, s, w, m, n, in, out, ksplit);
        default: return set_error(ctx->err, ANEHIP_EINVAL, "gemv: input mode %d", in.mode);
    }
}

// The row split of gemv_rows for an m x n matrix: H row groups per tile
// (J = 8 n / 256 / (waves x H) blocks per slot, 1 <= J <= 4): 4 on 16 waves
// when that fills the CUs, else 8 on 8 waves, else 4 or 2 on 16 waves, when
// the grid gets at least half as many workgroups as CUs; 0 when gemv_rows
// does not apply (matrices the split GEMV covers with row tiles alone keep
// it).  Measured on MI355X at batch 1, in graphs of back-to-back launches,
// against the K split plus its summing launch: 6144 x 2048 5.1 us (H 4) /
// 5.2 (H 2) against 7.0; 2048 x 2048 3.8 (4) / 4.5 (2) against 6.0; 2048 x
// 6144 7.5 (4) against 7.9.
int gemv_rows_split(const anehip_ctx *ctx, uint32_t m, uint32_t n) {
    if (n % 256 || n > (uint32_t)kRowsMaxN) return 0;
    const int nsb = (int)(n / 256), tiles = (int)((m + kWave - 1) / kWave);
    const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    if (gemv_packed_ksplit(ctx, m, n) == 1) return 0;
    for (int H : {4, 8}) {
        const int J = rows_blocks_per_slot(nsb, H);
        if (J >= 1 && J <= 4 && tiles * H >= cus) return H;
    }
    for (int H : {4, 2}) {
        const int J = rows_blocks_per_slot(nsb, H);
        if (J < 1 || J > 4) continue;
        if (tiles * H >= cus / 2) return H;
    }
    return 0;
}

template <uint32_t T>
int launch_rows_t(anehip_ctx *ctx, hipStream_t stream, const void *w, uint32_t m, uint32_t n, const float *x,
                  float *y, int H) {
    const int tiles = (int)((m + kWave - 1) / kWave), J = rows_blocks_per_slot((int)(n / 256), H);
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    const dim3 grid(tiles * H), block(kWave * rows_waves(H));
#define ANEHIP_ROWS(HH, JJ) hipLaunchKernelGGL((gemv_rows<T, HH, JJ>), grid, block, 0, stream, wb, x, y, (int)m, (int)n)
    if (H == 2) {
        switch (J) {
            case 1: ANEHIP_ROWS(2, 1); break;
            case 2: ANEHIP_ROWS(2, 2); break;
            case 3: ANEHIP_ROWS(2, 3); break;
            case 4: ANEHIP_ROWS(2, 4); break;
            default: return set_error(ctx->err, ANEHIP_EINVAL, "gemv_rows: %d blocks per slot", J);
        }
    } else if (H == 4) {
        switch (J) {
            case 1: ANEHIP_ROWS(4, 1); break;
            case 2: ANEHIP_ROWS(4, 2); break;
            case 3: ANEHIP_ROWS(4, 3); break;
            case 4: ANEHIP_ROWS(4, 4); break;
            default: return set_error(ctx->err, ANEHIP_EINVAL, "gemv_rows: %d blocks per slot", J);
        }
    } else if (H == 8) {
        switch (J) {
            case 1: ANEHIP_ROWS(8, 1); break;
            case 2: ANEHIP_ROWS(8, 2); break;
            case 3: ANEHIP_ROWS(8, 3); break;
            case 4: ANEHIP_ROWS(8, 4); break;
            default: return set_error(ctx->err, ANEHIP_EINVAL, "gemv_rows: %d blocks per slot", J);
        }
    } else {
        return set_error(ctx->err, ANEHIP_EINVAL, "gemv_rows: row split %d", H);
    }
#undef ANEHIP_ROWS
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_gemv_rows(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w, uint32_t m, uint32_t n,
                     const float *x, float *y, int H) {
    if (n % 256 || n > (uint32_t)kRowsMaxN || !rows_blocks_per_slot((int)(n / 256), H))
        return set_error(ctx->err, ANEHIP_EINVAL, "gemv_rows: n=%u with row split %d", n, H);
    if (ggml_type == ANEHIP_GGML_Q8_0) return launch_rows_t<ANEHIP_GGML_Q8_0>(ctx, stream, w, m, n, x, y, H);
    return launch_rows_t<ANEHIP_GGML_Q4_0>(ctx, stream, w, m, n, x, y, H);
}

int launch_gemv_packed(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w, uint32_t m, uint32_t n,
                       const GemvInput &in, float *out, int ksplit) {
    if (ggml_type == ANEHIP_GGML_Q8_0)
        return dispatch_packed<ANEHIP_GGML_Q8_0>(ctx, stream, w, m, n, in, out, ksplit);
    return dispatch_packed<ANEHIP_GGML_Q4_0>(ctx, stream, w, m, n, in, out, ksplit);
}

bool dn_ssm_fusable(const anehip_ctx *ctx, uint32_t dim, uint32_t n_heads) {
    return dim == n_heads * (uint32_t)kDnDk && n_heads % 2 == 0 &&
           gemv_packed_ksplit(ctx, dim, dim, GEMV_IN_GATED_NORM) == (int)(dim / 256);
}

int launch_dn_ssm(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w, uint32_t dim,
                  uint32_t n_heads, const MixIn &mix, const float *conv_w, const float *conv_state, const float *ssm_a,
                  const float *dt_bias, const float *S, const float *norm_w, float eps, float *pend, float *out) {
    if (!dn_ssm_fusable(ctx, dim, n_heads) || mix.kp < 1 || mix.kp > kMaxSplit)
        return set_error(ctx->err, ANEHIP_EINVAL, "dn_ssm: dim %u, %u heads, %d K splits not covered", dim, n_heads,
                         mix.kp);
    DnSsmArgs a;
    a.mix = mix;
    a.beta = mix.shifted((int)(4 * dim));
    a.alpha = mix.shifted((int)(4 * dim + n_heads));
    a.conv_w = conv_w;
    a.conv_state = conv_state;
    a.ssm_a = ssm_a;
    a.dt_bias = dt_bias;
    a.S = S;
    a.norm_w = norm_w;
    a.pend = pend;
    a.n_heads = (int)n_heads;
    a.d = (int)dim;
    a.eps = eps;
    const int nsplit = (int)(dim / 256), tiles = (int)((dim + kWave - 1) / kWave);
    const dim3 grid(tiles * nsplit), block(kWave * kPackedWaves);
    const uint8_t *wb = static_cast<const uint8_t *>(w);
#define ANEHIP_DN(TT, KK) \
    hipLaunchKernelGGL((dn_ssm_kernel<TT, KK>), grid, block, 0, stream, wb, a, out, (int)dim, nsplit)
    const bool q8 = ggml_type == ANEHIP_GGML_Q8_0;
    if (mix.kp == 1) {
        if (q8) ANEHIP_DN(ANEHIP_GGML_Q8_0, 1);
        else ANEHIP_DN(ANEHIP_GGML_Q4_0, 1);
    } else {
        if (q8) ANEHIP_DN(ANEHIP_GGML_Q8_0, kMaxSplit);
        else ANEHIP_DN(ANEHIP_GGML_Q4_0, kMaxSplit);
    }
#undef ANEHIP_DN
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_split_x(anehip_ctx *ctx, hipStream_t stream, const float *x, uint32_t batch, uint32_t n, const Planes &xp) {
    if (n % kXeGroup) return set_error(ctx->err, ANEHIP_EINVAL, "split_x: n=%u not a multiple of %d", n, kXeGroup);
    const size_t vecs = (size_t)batch * (n / 8);
    hipLaunchKernelGGL(split_x_frag_kernel, dim3((unsigned)((vecs + 255) / 256)), dim3(256), 0, stream, x, xp,
                       (int)batch, (int)n);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_gemv_fused(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w, uint32_t m,
                      uint32_t n, const GemvInput &in, float *out, int ksplit) {
    if (ggml_type == ANEHIP_GGML_Q8_0) return dispatch_fused<ANEHIP_GGML_Q8_0>(ctx, stream, w, m, n, in, out, ksplit);
    return dispatch_fused<ANEHIP_GGML_Q4_0>(ctx, stream, w, m, n, in, out, ksplit);
}

int launch_gemm_raw(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w, uint32_t m, uint32_t n,
                    const float *x, uint32_t batch, float *out, int ksplit, void *xsplit) {
    _Float16 *xs = static_cast<_Float16 *>(xsplit);
    if (batch > 1 && !xs) return set_error(ctx->err, ANEHIP_EINVAL, "gemm: batch > 1 needs an x split buffer");
    if (ggml_type == ANEHIP_GGML_Q8_0)
        return dispatch_raw<ANEHIP_GGML_Q8_0>(ctx, stream, w, m, n, x, batch, out, ksplit, xs);
    return dispatch_raw<ANEHIP_GGML_Q4_0>(ctx, stream, w, m, n, x, batch, out, ksplit, xs);
}

int launch_sum_partials(anehip_ctx *ctx, hipStream_t stream, const float *part, float *y, size_t count, int ksplit) {
    const bool v4 = count % 4 == 0 && ksplit >= 1 && ksplit <= 16 && reinterpret_cast<uintptr_t>(part) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(y) % 16 == 0;
    if (v4) {
        const size_t c4 = count / 4;
        const dim3 grid((unsigned)((c4 + 255) / 256));
        const float4 *p4 = reinterpret_cast<const float4 *>(part);
        float4 *y4 = reinterpret_cast<float4 *>(y);
        if (ksplit <= 2) hipLaunchKernelGGL(sum_partials4<2>, grid, dim3(256), 0, stream, p4, y4, c4, ksplit);
        else if (ksplit <= 4) hipLaunchKernelGGL(sum_partials4<4>, grid, dim3(256), 0, stream, p4, y4, c4, ksplit);
        else if (ksplit <= 8) hipLaunchKernelGGL(sum_partials4<8>, grid, dim3(256), 0, stream, p4, y4, c4, ksplit);
        else hipLaunchKernelGGL(sum_partials4<16>, grid, dim3(256), 0, stream, p4, y4, c4, ksplit);
        ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
        return ANEHIP_OK;
    }
    hipLaunchKernelGGL(sum_partials, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, stream, part, y, count,
                       ksplit);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int launch_quant_gemm(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w, uint32_t m,
                      uint32_t n, const float *x, uint32_t batch, float *y) {
    // the sum_partials consumer takes any number of splits, so the batch-1
    // kernel never needs more than kMaxSliceSb super-blocks per split
    const int ksplit = gemm_ksplit(ctx, m, n, batch == 1 ? 1 << 20 : kMaxSplit);
    const size_t count = (size_t)batch * m;
    // workspace: [ksplit partials][x hi/lo planes (2 * batch * n halves)][group exponents]
    const size_t part = ksplit > 1 ? (size_t)ksplit * count : 0;
    const size_t xs_floats = batch > 1 ? (size_t)batch * n + (xe_bytes(n) + 3) / 4 : 0;
    int rc = ensure_workspace(ctx, part + xs_floats);
    if (rc) return rc;
    void *xs = batch > 1 ? static_cast<void *>(ctx->ws.partial + part) : nullptr;
    if (ksplit == 1) return launch_gemm_raw(ctx, stream, ggml_type, w, m, n, x, batch, y, 1, xs);
    rc = launch_gemm_raw(ctx, stream, ggml_type, w, m, n, x, batch, ctx->ws.partial, ksplit, xs);
    if (rc) return rc;
    return launch_sum_partials(ctx, stream, ctx->ws.partial, y, count, ksplit);
}

}  // namespace anehip
