/*
 * ane_oracle.c — CPU restatement of ane-infer's decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the CPU
 * baseline.  See ane_oracle.h for the pinning of each function.
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off, no fast-math).
 */
#include "ane_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "../include/anehip.h"

/* ------------------------------------------------------------------------ */
/* fp16                                                                      */
/* ------------------------------------------------------------------------ */

float ao_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: man * 2^-24 is exact in f32 */
            float v = ldexpf((float)man, -24);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t ao_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) /* NaN: keep it quiet and non-zero */
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x47800000u) /* >= 65536 (and inf) */
        return (uint16_t)(sign | 0x7c00u);
    uint32_t e32 = ax >> 23;
    if (e32 < 113) {
        /* f16 subnormal range (< 2^-14) */
        if (e32 < 102) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        uint32_t mi = (ax & 0x7fffffu) | 0x800000u;
        uint32_t s = 126u - e32; /* 14..24 */
        uint32_t r = mi >> s;
        uint32_t rem = mi & ((1u << s) - 1u);
        uint32_t half = 1u << (s - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((e32 - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++; /* carry may reach inf */
    return (uint16_t)(sign | r);
}

void ao_f32_to_f16_array(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = ao_f32_to_f16(src[i]);
}

void ao_f16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = ao_f16_to_f32(src[i]);
}

/* ------------------------------------------------------------------------ */
/* generator                                                                 */
/* ------------------------------------------------------------------------ */

uint64_t ao_splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return ao_splitmix64(ao_splitmix64(seed) ^ (stream * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull));
}

static inline double unit_open(uint64_t key, uint64_t ctr) {
    /* 53 random bits mapped to (0, 1) */
    return ((double)(ao_splitmix64(key + ctr) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

static void fill_normal_range(uint64_t key, double mean, double sd, float *out, size_t start,
                              size_t n) {
    size_t i = start, end = start + n;
    while (i < end) {
        uint64_t j = i >> 1;
        double u1 = unit_open(key, 2 * j), u2 = unit_open(key, 2 * j + 1);
        double r = sqrt(-2.0 * log(u1));
        double t = 6.283185307179586 * u2;
        if ((i & 1) == 0) {
            out[i - start] = (float)(mean + sd * r * cos(t));
            i++;
            if (i < end) {
                out[i - start] = (float)(mean + sd * r * sin(t));
                i++;
            }
        } else {
            out[i - start] = (float)(mean + sd * r * sin(t));
            i++;
        }
    }
}

#define FILL_CHUNK ((size_t)1 << 16)

void ao_fill_normal(uint64_t seed, uint64_t stream, float mean, float stddev, float *out,
                    size_t n) {
    uint64_t key = stream_key(seed, stream);
    long nchunks = (long)((n + FILL_CHUNK - 1) / FILL_CHUNK);
#pragma omp parallel for schedule(static)
    for (long c = 0; c < nchunks; c++) {
        size_t s = (size_t)c * FILL_CHUNK;
        size_t len = n - s < FILL_CHUNK ? n - s : FILL_CHUNK;
        fill_normal_range(key, mean, stddev, out + s, s, len);
    }
}

void ao_fill_uniform(uint64_t seed, uint64_t stream, float lo, float hi, float *out, size_t n) {
    uint64_t key = stream_key(seed, stream);
#pragma omp parallel for schedule(static)
    for (long i = 0; i < (long)n; i++)
        out[i] = (float)((double)lo + ((double)hi - (double)lo) * unit_open(key, (uint64_t)i));
}

void ao_fill_u32(uint64_t seed, uint64_t stream, uint32_t bound, uint32_t *out, size_t n) {
    uint64_t key = stream_key(seed, stream);
    for (size_t i = 0; i < n; i++)
        out[i] = (uint32_t)(((ao_splitmix64(key + i) >> 32) * (uint64_t)bound) >> 32);
}

/* ------------------------------------------------------------------------ */
/* quantisation                                                              */
/* ------------------------------------------------------------------------ */

size_t ao_quant_bytes(uint32_t t, size_t m, size_t n) {
    size_t per = t == ANEHIP_GGML_Q8_0 ? 34 : t == ANEHIP_GGML_Q4_0 ? 18 : 0;
    return m * (n / 32) * per;
}

static void quant_row_q8_0(const float *w, size_t n, uint8_t *out) {
    for (size_t b = 0; b < n / 32; b++) {
        const float *xb = w + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            float a = fabsf(xb[i]);
            if (a > amax) amax = a;
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t dh = ao_f32_to_f16(d);
        uint8_t *blk = out + b * 34;
        blk[0] = (uint8_t)(dh & 0xff);
        blk[1] = (uint8_t)(dh >> 8);
        for (int i = 0; i < 32; i++) {
            float q = roundf(xb[i] * id);
            if (q > 127.0f) q = 127.0f;
            if (q < -127.0f) q = -127.0f;
            blk[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}

static void quant_row_q4_0(const float *w, size_t n, uint8_t *out) {
    for (size_t b = 0; b < n / 32; b++) {
        const float *xb = w + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            float a = fabsf(xb[i]);
            if (a > amax) amax = a;
        }
        float d = amax / 7.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t dh = ao_f32_to_f16(d);
        uint8_t *blk = out + b * 18;
        blk[0] = (uint8_t)(dh & 0xff);
        blk[1] = (uint8_t)(dh >> 8);
        uint8_t q[32];
        for (int i = 0; i < 32; i++) {
            float v = roundf(xb[i] * id) + 8.0f;
            if (v < 0.0f) v = 0.0f;
            if (v > 15.0f) v = 15.0f;
            q[i] = (uint8_t)v;
        }
        for (int i = 0; i < 16; i++) blk[2 + i] = (uint8_t)(q[i] | (q[i + 16] << 4));
    }
}

void ao_quantize_q8_0(const float *w, size_t m, size_t n, uint8_t *out) {
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)m; r++) quant_row_q8_0(w + (size_t)r * n, n, out + (size_t)r * (n / 32) * 34);
}

void ao_quantize_q4_0(const float *w, size_t m, size_t n, uint8_t *out) {
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)m; r++) quant_row_q4_0(w + (size_t)r * n, n, out + (size_t)r * (n / 32) * 18);
}

void ao_gen_quant(uint32_t t, uint64_t seed, uint64_t stream, float stddev, size_t m, size_t n,
                  uint8_t *out) {
    uint64_t key = stream_key(seed, stream);
    size_t rb = ao_quant_bytes(t, 1, n);
#pragma omp parallel
    {
        float *row = (float *)malloc(n * sizeof(float));
#pragma omp for schedule(static)
        for (long r = 0; r < (long)m; r++) {
            fill_normal_range(key, 0.0, stddev, row, (size_t)r * n, n);
            if (t == ANEHIP_GGML_Q8_0)
                quant_row_q8_0(row, n, out + (size_t)r * rb);
            else
                quant_row_q4_0(row, n, out + (size_t)r * rb);
        }
        free(row);
    }
}

/* dequant.rs:12-25 */
void ao_dequant_q4_0_block(const uint8_t *block, float *out) {
    float scale = ao_f16_to_f32((uint16_t)(block[0] | (block[1] << 8)));
    for (int i = 0; i < 16; i++) {
        uint8_t byte = block[2 + i];
        out[i] = (float)((int)(byte & 0x0f) - 8) * scale;
        out[i + 16] = (float)((int)((byte >> 4) & 0x0f) - 8) * scale;
    }
}

/* dequant.rs:29-38 */
void ao_dequant_q8_0_block(const uint8_t *block, float *out) {
    float scale = ao_f16_to_f32((uint16_t)(block[0] | (block[1] << 8)));
    for (int i = 0; i < 32; i++) out[i] = (float)(int8_t)block[2 + i] * scale;
}

/* ------------------------------------------------------------------------ */
/* GEMV                                                                      */
/* ------------------------------------------------------------------------ */

/* q8_gemv.rs:230-244 */
static float row_q8(const uint8_t *data, const float *x, size_t row, size_t bpr) {
    size_t row_off = row * bpr * 34;
    float sum = 0.0f;
    for (size_t b = 0; b < bpr; b++) {
        size_t off = row_off + b * 34;
        float scale = ao_f16_to_f32((uint16_t)(data[off] | (data[off + 1] << 8)));
        float block_sum = 0.0f;
        for (int i = 0; i < 32; i++) block_sum += (float)(int8_t)data[off + 2 + i] * x[b * 32 + i];
        sum += block_sum * scale;
    }
    return sum;
}

/* q8_gemv.rs:60-64 + 80-98: element i and i+16 interleaved per byte */
static float row_q4(const uint8_t *data, const float *x, size_t row, size_t bpr) {
    size_t row_off = row * bpr * 18;
    float sum = 0.0f;
    for (size_t b = 0; b < bpr; b++) {
        size_t off = row_off + b * 18;
        float scale = ao_f16_to_f32((uint16_t)(data[off] | (data[off + 1] << 8)));
        float block_sum = 0.0f;
        for (int i = 0; i < 16; i++) {
            uint8_t packed = data[off + 2 + i];
            float v0 = (float)((int)(packed & 0x0f) - 8);
            float v1 = (float)((int)((packed >> 4) & 0x0f) - 8);
            block_sum += v0 * x[b * 32 + i] + v1 * x[b * 32 + 16 + i];
        }
        sum += block_sum * scale;
    }
    return sum;
}

void ao_quant_gemv(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x, float *y) {
    size_t bpr = n / 32;
    for (size_t r = 0; r < m; r++)
        y[r] = t == ANEHIP_GGML_Q8_0 ? row_q8(w, x, r, bpr) : row_q4(w, x, r, bpr);
}

int ao_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void ao_quant_gemv_mt(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x, float *y,
                      int nthreads) {
    size_t bpr = n / 32;
    if (nthreads <= 0) nthreads = ao_max_threads();
    if (t == ANEHIP_GGML_Q8_0) {
#pragma omp parallel for schedule(static) num_threads(nthreads)
        for (long r = 0; r < (long)m; r++) y[r] = row_q8(w, x, (size_t)r, bpr);
    } else {
#pragma omp parallel for schedule(static) num_threads(nthreads)
        for (long r = 0; r < (long)m; r++) y[r] = row_q4(w, x, (size_t)r, bpr);
    }
}

void ao_quant_gemm(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x, size_t batch,
                   float *y, int nthreads) {
    for (size_t b = 0; b < batch; b++) ao_quant_gemv_mt(t, w, m, n, x + b * n, y + b * m, nthreads);
}

/* ------------------------------------------------------------------------ */
/* elementwise                                                               */
/* ------------------------------------------------------------------------ */

/* deltanet.rs:43-51 == main.rs:1106-1113 */
void ao_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    ss = ss / (float)n;
    float inv_rms = 1.0f / sqrtf(ss + eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] * inv_rms * w[i];
}

/* scratch.rs:181-186 */
void ao_silu_mul_inplace(float *a, const float *b, size_t n) {
    for (size_t i = 0; i < n; i++) a[i] = (a[i] / (1.0f + expf(-a[i]))) * b[i];
}

/* main.rs:983-985 */
void ao_residual_add(float *x, const float *y, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] += y[i];
}

/* deltanet.rs:10-31 */
static inline float softplus(float x) { return logf(1.0f + expf(x)); }
static inline float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
static inline float siluf_(float x) { return x / (1.0f + expf(-x)); }

static void l2_normalize(float *v, size_t n) {
    float norm_sq = 0.0f;
    for (size_t i = 0; i < n; i++) norm_sq += v[i] * v[i];
    float inv_norm = 1.0f / sqrtf(norm_sq + 1e-12f);
    for (size_t i = 0; i < n; i++) v[i] *= inv_norm;
}

/* ------------------------------------------------------------------------ */
/* DeltaNet core: deltanet.rs:444-512                                        */
/* ------------------------------------------------------------------------ */

void ao_deltanet_core(size_t chunk, size_t n_heads, size_t dk, size_t ksize, const float *qkv,
                      const float *beta_raw, const float *alpha_raw, const float *conv_w,
                      const float *ssm_a, const float *dt_bias, float *conv_state, float *S,
                      float *out_heads) {
    size_t inner = 3 * chunk;
    /* deltanet_cache.rs:34-42 conv_shift_and_append */
    for (size_t ch = 0; ch < inner; ch++) {
        size_t base = ch * ksize;
        for (size_t k = 0; k + 1 < ksize; k++) conv_state[base + k] = conv_state[base + k + 1];
        conv_state[base + ksize - 1] = qkv[ch];
    }
    /* deltanet_cache.rs:44-54 conv_apply, then SiLU (deltanet.rs:448-450) */
    float *conv_out = (float *)malloc(inner * sizeof(float));
    for (size_t ch = 0; ch < inner; ch++) {
        float sum = 0.0f;
        size_t base = ch * ksize;
        for (size_t k = 0; k < ksize; k++) sum += conv_state[base + k] * conv_w[base + k];
        conv_out[ch] = sum;
    }
    for (size_t ch = 0; ch < inner; ch++) conv_out[ch] = siluf_(conv_out[ch]);

    size_t hdk = chunk / n_heads;
    float *q = (float *)malloc(chunk * sizeof(float));
    float *k = (float *)malloc(chunk * sizeof(float));
    const float *v = conv_out + 2 * chunk;
    memcpy(q, conv_out, chunk * sizeof(float));
    memcpy(k, conv_out + chunk, chunk * sizeof(float));
    /* deltanet.rs:461-467 */
    float scale = 1.0f / sqrtf((float)dk);
    for (size_t h = 0; h < n_heads; h++) {
        size_t off = h * hdk;
        l2_normalize(q + off, hdk);
        l2_normalize(k + off, hdk);
        for (size_t i = 0; i < hdk; i++) q[off + i] *= scale;
    }
    /* deltanet.rs:474-480 */
    float *beta = (float *)malloc(n_heads * sizeof(float));
    float *decay = (float *)malloc(n_heads * sizeof(float));
    for (size_t h = 0; h < n_heads; h++) {
        beta[h] = sigmoidf_(beta_raw[h]);
        float g = ssm_a[h] * softplus(alpha_raw[h] + dt_bias[h]);
        decay[h] = expf(g);
    }
    /* deltanet.rs:485-512 (x86 mat_vec_transpose :110-120, outer_product_add :154-169) */
    size_t dv = dk, kd = dk < hdk ? dk : hdk, vd = dv < hdk ? dv : hdk;
    float *sk = (float *)malloc(vd * sizeof(float));
    float *delta = (float *)malloc(vd * sizeof(float));
    for (size_t h = 0; h < n_heads; h++) {
        const float *k_h = k + h * hdk, *v_h = v + h * hdk, *q_h = q + h * hdk;
        float *s = S + h * dk * dv;
        for (size_t i = 0; i < kd * vd; i++) s[i] *= decay[h];
        for (size_t col = 0; col < vd; col++) {
            float dot = 0.0f;
            for (size_t row = 0; row < kd; row++) dot += s[row * dv + col] * k_h[row];
            sk[col] = dot;
        }
        for (size_t vi = 0; vi < vd; vi++) delta[vi] = beta[h] * (v_h[vi] - sk[vi]);
        for (size_t row = 0; row < kd; row++)
            for (size_t col = 0; col < vd; col++) s[row * dv + col] += k_h[row] * delta[col];
        for (size_t col = 0; col < vd; col++) {
            float dot = 0.0f;
            for (size_t row = 0; row < kd; row++) dot += s[row * dv + col] * q_h[row];
            sk[col] = dot;
        }
        for (size_t vi = 0; vi < vd; vi++) out_heads[h * hdk + vi] = sk[vi];
    }
    free(sk);
    free(delta);
    free(beta);
    free(decay);
    free(q);
    free(k);
    free(conv_out);
}

/* deltanet.rs:517-533 */
void ao_gated_rmsnorm(float *normed, const float *heads, const float *gate, const float *norm_w,
                      size_t n_heads, size_t head_dim, float eps) {
    for (size_t h = 0; h < n_heads; h++)
        ao_rmsnorm(normed + h * head_dim, heads + h * head_dim, norm_w, head_dim, eps);
    size_t n = n_heads * head_dim;
    for (size_t i = 0; i < n; i++) normed[i] *= gate[i] / (1.0f + expf(-gate[i]));
}

/* ------------------------------------------------------------------------ */
/* attention core: deltanet.rs:565-669                                       */
/* ------------------------------------------------------------------------ */

static inline float kv_read(const void *cache, int f16, size_t idx) {
    return f16 ? ao_f16_to_f32(((const uint16_t *)cache)[idx]) : ((const float *)cache)[idx];
}

static void rope_inplace(float *x, size_t nh, size_t hd, size_t pos, float base) {
    for (size_t h = 0; h < nh; h++) {
        for (size_t i = 0; i < hd; i += 2) {
            float freq = 1.0f / powf(base, (float)i / (float)hd);
            float val = (float)pos * freq;
            float sin_v = sinf(val), cos_v = cosf(val);
            size_t off = h * hd + i;
            float a0 = x[off], a1 = x[off + 1];
            x[off] = a0 * cos_v - a1 * sin_v;
            x[off + 1] = a0 * sin_v + a1 * cos_v;
        }
    }
}

void ao_attention_core(size_t n_heads, size_t n_kv_heads, size_t hd, size_t max_seq, size_t pos,
                       float rope_base, const float *q_full, const float *k_in, const float *v_in,
                       const float *q_norm, const float *k_norm, int kv_f16, void *k_cache,
                       void *v_cache, float *attn_out) {
    size_t qd = n_heads * hd, kvd = n_kv_heads * hd;
    float *q = (float *)malloc(qd * sizeof(float));
    float *gate = (float *)malloc(qd * sizeof(float));
    float *k = (float *)malloc(kvd * sizeof(float));
    float *normed = (float *)malloc(hd * sizeof(float));
    memcpy(k, k_in, kvd * sizeof(float));
    /* deltanet.rs:567-573 */
    for (size_t h = 0; h < n_heads; h++) {
        memcpy(q + h * hd, q_full + h * hd * 2, hd * sizeof(float));
        memcpy(gate + h * hd, q_full + h * hd * 2 + hd, hd * sizeof(float));
    }
    /* deltanet.rs:575-598, eps hard-coded 1e-6 */
    for (size_t h = 0; h < n_heads; h++) {
        ao_rmsnorm(normed, q + h * hd, q_norm, hd, 1e-6f);
        memcpy(q + h * hd, normed, hd * sizeof(float));
    }
    for (size_t h = 0; h < n_kv_heads; h++) {
        ao_rmsnorm(normed, k + h * hd, k_norm, hd, 1e-6f);
        memcpy(k + h * hd, normed, hd * sizeof(float));
    }
    /* deltanet.rs:600-623 */
    rope_inplace(q, n_heads, hd, pos, rope_base);
    rope_inplace(k, n_kv_heads, hd, pos, rope_base);
    /* kv_cache.rs:31-41 write_pos */
    for (size_t h = 0; h < n_kv_heads; h++) {
        size_t co = h * max_seq * hd + pos * hd;
        for (size_t i = 0; i < hd; i++) {
            if (kv_f16) {
                ((uint16_t *)k_cache)[co + i] = ao_f32_to_f16(k[h * hd + i]);
                ((uint16_t *)v_cache)[co + i] = ao_f32_to_f16(v_in[h * hd + i]);
            } else {
                ((float *)k_cache)[co + i] = k[h * hd + i];
                ((float *)v_cache)[co + i] = v_in[h * hd + i];
            }
        }
    }
    /* deltanet.rs:627-665 */
    size_t hpk = n_heads / n_kv_heads, seq = pos + 1;
    float *scores = (float *)malloc(seq * sizeof(float));
    float sd = sqrtf((float)hd);
    for (size_t h = 0; h < n_heads; h++) {
        size_t kvh = h / hpk, cbase = kvh * max_seq * hd;
        float max_score = -INFINITY;
        for (size_t s = 0; s < seq; s++) {
            float dot = 0.0f;
            for (size_t i = 0; i < hd; i++) dot += q[h * hd + i] * kv_read(k_cache, kv_f16, cbase + s * hd + i);
            scores[s] = dot / sd;
            if (scores[s] > max_score) max_score = scores[s];
        }
        float sm = 0.0f;
        for (size_t s = 0; s < seq; s++) {
            scores[s] = expf(scores[s] - max_score);
            sm += scores[s];
        }
        for (size_t s = 0; s < seq; s++) scores[s] /= sm;
        for (size_t i = 0; i < hd; i++) {
            float val = 0.0f;
            for (size_t s = 0; s < seq; s++) val += scores[s] * kv_read(v_cache, kv_f16, cbase + s * hd + i);
            attn_out[h * hd + i] = val;
        }
    }
    /* deltanet.rs:667-669 */
    for (size_t i = 0; i < qd; i++) attn_out[i] *= sigmoidf_(gate[i]);
    free(scores);
    free(normed);
    free(k);
    free(gate);
    free(q);
}

/* ------------------------------------------------------------------------ */
/* model                                                                     */
/* ------------------------------------------------------------------------ */

typedef struct {
    const uint8_t *data;
    uint32_t rows, cols, type;
} qt;

typedef struct {
    const float *f[ANEHIP_T_COUNT];
    size_t fn[ANEHIP_T_COUNT];
    qt q[ANEHIP_T_COUNT];
} layer_t;

struct ao_model {
    uint32_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, vocab;
    uint32_t dk, ksize, H;
    float rope_base, eps;
    uint8_t *types;
    layer_t *layers;
    layer_t glob;
};

struct ao_seq {
    const ao_model *m;
    uint32_t max_seq, pos;
    int kv_f16;
    float **conv, **rec;
    void **kc, **vc;
};

ao_model *ao_model_create(uint32_t dim, uint32_t hidden_dim, uint32_t n_layers, uint32_t n_heads,
                          uint32_t n_kv_heads, uint32_t head_dim, uint32_t vocab_size,
                          uint32_t ssm_state_size, uint32_t ssm_conv_kernel,
                          uint32_t ssm_group_count, float rope_freq_base, float rms_norm_eps,
                          const uint8_t *layer_types) {
    ao_model *m = (ao_model *)calloc(1, sizeof(ao_model));
    m->dim = dim;
    m->hidden_dim = hidden_dim;
    m->n_layers = n_layers;
    m->n_heads = n_heads;
    m->n_kv_heads = n_kv_heads;
    m->head_dim = head_dim;
    m->vocab = vocab_size;
    m->dk = ssm_state_size;
    m->ksize = ssm_conv_kernel;
    m->H = ssm_group_count;
    m->rope_base = rope_freq_base;
    m->eps = rms_norm_eps;
    m->types = (uint8_t *)malloc(n_layers);
    memcpy(m->types, layer_types, n_layers);
    m->layers = (layer_t *)calloc(n_layers, sizeof(layer_t));
    return m;
}

void ao_model_destroy(ao_model *m) {
    if (!m) return;
    free(m->types);
    free(m->layers);
    free(m);
}

static layer_t *layer_of(ao_model *m, int layer) {
    if (layer < 0) return &m->glob;
    if ((uint32_t)layer >= m->n_layers) return NULL;
    return &m->layers[layer];
}

int ao_model_set_quant(ao_model *m, int layer, int kind, const uint8_t *data, uint32_t rows,
                       uint32_t cols, uint32_t t) {
    layer_t *L = layer_of(m, layer);
    if (!L || kind < 0 || kind >= ANEHIP_T_COUNT) return -1;
    L->q[kind].data = data;
    L->q[kind].rows = rows;
    L->q[kind].cols = cols;
    L->q[kind].type = t;
    return 0;
}

int ao_model_set_f32(ao_model *m, int layer, int kind, const float *data, size_t n) {
    layer_t *L = layer_of(m, layer);
    if (!L || kind < 0 || kind >= ANEHIP_T_COUNT) return -1;
    L->f[kind] = data;
    L->fn[kind] = n;
    return 0;
}

ao_seq *ao_seq_create(const ao_model *m, uint32_t max_seq, int kv_f16) {
    ao_seq *s = (ao_seq *)calloc(1, sizeof(ao_seq));
    s->m = m;
    s->max_seq = max_seq;
    s->kv_f16 = kv_f16;
    s->conv = (float **)calloc(m->n_layers, sizeof(float *));
    s->rec = (float **)calloc(m->n_layers, sizeof(float *));
    s->kc = (void **)calloc(m->n_layers, sizeof(void *));
    s->vc = (void **)calloc(m->n_layers, sizeof(void *));
    size_t esz = kv_f16 ? 2 : 4;
    for (uint32_t l = 0; l < m->n_layers; l++) {
        if (m->types[l] == ANEHIP_LAYER_DELTANET) {
            s->conv[l] = (float *)calloc((size_t)3 * m->dim * m->ksize, sizeof(float));
            s->rec[l] = (float *)calloc((size_t)m->H * m->dk * m->dk, sizeof(float));
        } else {
            size_t n = (size_t)m->n_kv_heads * max_seq * m->head_dim;
            s->kc[l] = calloc(n, esz);
            s->vc[l] = calloc(n, esz);
        }
    }
    return s;
}

void ao_seq_destroy(ao_seq *s) {
    if (!s) return;
    for (uint32_t l = 0; l < s->m->n_layers; l++) {
        free(s->conv[l]);
        free(s->rec[l]);
        free(s->kc[l]);
        free(s->vc[l]);
    }
    free(s->conv);
    free(s->rec);
    free(s->kc);
    free(s->vc);
    free(s);
}

void ao_seq_set_pos(ao_seq *s, uint32_t pos) { s->pos = pos; }
uint32_t ao_seq_get_pos(const ao_seq *s) { return s->pos; }
float *ao_seq_conv_state(ao_seq *s, uint32_t l) { return l < s->m->n_layers ? s->conv[l] : NULL; }
float *ao_seq_recurrent_state(ao_seq *s, uint32_t l) { return l < s->m->n_layers ? s->rec[l] : NULL; }
void *ao_seq_k_cache(ao_seq *s, uint32_t l) { return l < s->m->n_layers ? s->kc[l] : NULL; }
void *ao_seq_v_cache(ao_seq *s, uint32_t l) { return l < s->m->n_layers ? s->vc[l] : NULL; }

static int gemv(const qt *w, const float *x, float *y, int nt) {
    if (!w->data) return -1;
    ao_quant_gemv_mt(w->type, w->data, w->rows, w->cols, x, y, nt);
    return 0;
}

/* main.rs:1115-1135 */
static int ffn_forward(const layer_t *L, const float *x, float *out, uint32_t F, int nt) {
    float *h1 = (float *)malloc(F * sizeof(float));
    float *h3 = (float *)malloc(F * sizeof(float));
    int rc = gemv(&L->q[ANEHIP_T_FFN_GATE], x, h1, nt);
    rc |= gemv(&L->q[ANEHIP_T_FFN_UP], x, h3, nt);
    if (!rc) {
        ao_silu_mul_inplace(h1, h3, F);
        rc |= gemv(&L->q[ANEHIP_T_FFN_DOWN], h1, out, nt);
    }
    free(h1);
    free(h3);
    return rc;
}

/* main.rs:953-1023 */
int ao_forward_token(const ao_model *m, ao_seq *s, uint32_t token, float *logits, int nt) {
    uint32_t d = m->dim;
    if (s->pos >= s->max_seq) return -1;
    float *x = (float *)calloc(d, sizeof(float));
    float *xn = (float *)malloc(d * sizeof(float));
    float *mix = (float *)malloc(d * sizeof(float));
    float *ffo = (float *)malloc(d * sizeof(float));
    size_t C = (size_t)3 * d, chunk = d;
    float *qkv = (float *)malloc(C * sizeof(float));
    float *heads = (float *)malloc(chunk * sizeof(float));
    float *normed = (float *)malloc(chunk * sizeof(float));
    float *gate = (float *)malloc(d * sizeof(float));
    float *br = (float *)malloc(m->H * sizeof(float));
    float *ar = (float *)malloc(m->H * sizeof(float));
    size_t qd = (size_t)m->n_heads * m->head_dim, kvd = (size_t)m->n_kv_heads * m->head_dim;
    float *qf = (float *)malloc(2 * qd * sizeof(float));
    float *kk = (float *)malloc(kvd * sizeof(float));
    float *vv = (float *)malloc(kvd * sizeof(float));
    float *ao = (float *)malloc(qd * sizeof(float));
    int rc = 0;
    if (token < m->vocab) {
        if (!m->glob.f[ANEHIP_T_EMBEDDING]) rc = -1;
        else memcpy(x, m->glob.f[ANEHIP_T_EMBEDDING] + (size_t)token * d, d * sizeof(float));
    }
    for (uint32_t l = 0; l < m->n_layers && !rc; l++) {
        const layer_t *L = &m->layers[l];
        if (!L->f[ANEHIP_T_ATTN_NORM] || !L->f[ANEHIP_T_POST_ATTN_NORM]) { rc = -1; break; }
        ao_rmsnorm(xn, x, L->f[ANEHIP_T_ATTN_NORM], d, m->eps);
        if (m->types[l] == ANEHIP_LAYER_DELTANET) {
            /* deltanet.rs:429-539 */
            if (!L->f[ANEHIP_T_SSM_CONV1D] || !L->f[ANEHIP_T_SSM_A] || !L->f[ANEHIP_T_SSM_DT_BIAS] ||
                !L->f[ANEHIP_T_SSM_NORM]) { rc = -1; break; }
            rc |= gemv(&L->q[ANEHIP_T_QKV], xn, qkv, nt);
            rc |= gemv(&L->q[ANEHIP_T_SSM_BETA], xn, br, nt);
            rc |= gemv(&L->q[ANEHIP_T_SSM_ALPHA], xn, ar, nt);
            if (rc) break;
            ao_deltanet_core(chunk, m->H, m->dk, m->ksize, qkv, br, ar, L->f[ANEHIP_T_SSM_CONV1D],
                             L->f[ANEHIP_T_SSM_A], L->f[ANEHIP_T_SSM_DT_BIAS], s->conv[l], s->rec[l],
                             heads);
            rc |= gemv(&L->q[ANEHIP_T_ATTN_GATE], xn, gate, nt);
            if (rc) break;
            ao_gated_rmsnorm(normed, heads, gate, L->f[ANEHIP_T_SSM_NORM], m->H, chunk / m->H, m->eps);
            rc |= gemv(&L->q[ANEHIP_T_SSM_OUT], normed, mix, nt);
        } else {
            /* deltanet.rs:541-675 */
            if (!L->f[ANEHIP_T_Q_NORM] || !L->f[ANEHIP_T_K_NORM]) { rc = -1; break; }
            rc |= gemv(&L->q[ANEHIP_T_WQ], xn, qf, nt);
            rc |= gemv(&L->q[ANEHIP_T_WK], xn, kk, nt);
            rc |= gemv(&L->q[ANEHIP_T_WV], xn, vv, nt);
            if (rc) break;
            ao_attention_core(m->n_heads, m->n_kv_heads, m->head_dim, s->max_seq, s->pos, m->rope_base,
                              qf, kk, vv, L->f[ANEHIP_T_Q_NORM], L->f[ANEHIP_T_K_NORM], s->kv_f16,
                              s->kc[l], s->vc[l], ao);
            rc |= gemv(&L->q[ANEHIP_T_WO], ao, mix, nt);
        }
        if (rc) break;
        ao_residual_add(x, mix, d);
        ao_rmsnorm(xn, x, L->f[ANEHIP_T_POST_ATTN_NORM], d, m->eps);
        rc |= ffn_forward(L, xn, ffo, m->hidden_dim, nt);
        if (rc) break;
        ao_residual_add(x, ffo, d);
    }
    if (!rc) {
        if (!m->glob.f[ANEHIP_T_FINAL_NORM]) rc = -1;
        else {
            ao_rmsnorm(xn, x, m->glob.f[ANEHIP_T_FINAL_NORM], d, m->eps);
            rc |= gemv(&m->glob.q[ANEHIP_T_LM_HEAD], xn, logits, nt);
        }
    }
    if (!rc) s->pos += 1;
    free(x); free(xn); free(mix); free(ffo); free(qkv); free(heads); free(normed); free(gate);
    free(br); free(ar); free(qf); free(kk); free(vv); free(ao);
    return rc ? -1 : 0;
}

/* main.rs:1767-1775: max_by(total_cmp) keeps the last of equal maxima */
uint32_t ao_argmax(const float *logits, size_t n) {
    uint32_t best = 0;
    int32_t bestkey = 0;
    for (size_t i = 0; i < n; i++) {
        int32_t b;
        memcpy(&b, &logits[i], 4);
        b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
        if (i == 0 || b >= bestkey) {
            bestkey = b;
            best = (uint32_t)i;
        }
    }
    return best;
}
