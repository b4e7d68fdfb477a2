/*
 * ane_oracle.h — CPU restatement of ane-infer's decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP decode
 * path and the CPU baseline timed beside it.  Only tests/, the smoke() entry
 * of __graft_entry__.py and the cpu_baseline leg of bench.py may load it; the
 * product library (libanehip.so) never links, loads or calls it.
 *
 * Every function restates a reference function in the same operation order
 * (the x86-64 scalar paths, which are what the reference runs on this host
 * class), cited as path:line under /root/reference.  Compile without
 * fast-math and with -ffp-contract=off: the reference's Rust code does not
 * contract a*b+c into fused multiply-adds.
 *
 * Parity pinning (what checks each function, see tests/test_oracle.py):
 *   f16 conversions     exhaustive vs numpy float16 (both directions)
 *   dequant / GEMV      the reference's own known-answer tests
 *                       (dequant.rs:235-270, q8_gemv.rs:257-314) + float64
 *                       brute force on random shapes
 *   quantisers          round-trip bound |w - deq(q(w))| <= d/2, KAT blocks
 *   DeltaNet core       exact-recall and zero-decay closed forms, conv
 *                       identity, numpy float64 restatement of the recurrence
 *   attention core      seq_len 1 => v, equal keys => mean(v), RoPE pos 0 =
 *                       identity and pair-norm preservation, numpy float64
 *   full forward        composition vs numpy float64 forward on a tiny model,
 *                       batch = independent sequences
 * Transcendental calls (expf, logf, powf, sinf, cosf) go to the host libm as
 * the reference's f32 methods do on x86-64 Linux; their exact bits versus the
 * reference binary are not pinned by any reference test.
 */
#ifndef ANE_ORACLE_H
#define ANE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 (the `half` crate 2.7.1: exact widening, RNE narrowing) ------ */
float ao_f16_to_f32(uint16_t h);
uint16_t ao_f32_to_f16(float f);
void ao_f32_to_f16_array(const float *src, uint16_t *dst, size_t n);
void ao_f16_to_f32_array(const uint16_t *src, float *dst, size_t n);

/* ---- seeded generator ---------------------------------------------------
 * Counter-based: value i of stream (seed, stream) is a pure function of
 * (seed, stream, i), so fills are identical for any thread count.
 * u = SplitMix64(key + i) >> 11, scaled to (0,1); normals by Box-Muller on
 * the pair (2j, 2j+1) in double precision. */
uint64_t ao_splitmix64(uint64_t x);
void ao_fill_normal(uint64_t seed, uint64_t stream, float mean, float stddev, float *out,
                    size_t n);
void ao_fill_uniform(uint64_t seed, uint64_t stream, float lo, float hi, float *out, size_t n);
void ao_fill_u32(uint64_t seed, uint64_t stream, uint32_t bound, uint32_t *out, size_t n);

/* ---- quantisation (build-owned recipes of the benchmark configs) -------
 * Q8_0: d = absmax/127, q = clamp(round(w/d), -127, 127), store fp16(d).
 * Q4_0: d = absmax/7,   q = clamp(round(w/d) + 8, 0, 15), nibble layout of
 *       dequant.rs:12-25.  round() is round-half-away-from-zero. */
void ao_quantize_q8_0(const float *w, size_t m, size_t n, uint8_t *out);
void ao_quantize_q4_0(const float *w, size_t m, size_t n, uint8_t *out);
/* generate N(0, std) weights row by row and quantise (parallel, no [m x n]
 * fp32 temporary) */
void ao_gen_quant(uint32_t ggml_type, uint64_t seed, uint64_t stream, float stddev, size_t m,
                  size_t n, uint8_t *out);
size_t ao_quant_bytes(uint32_t ggml_type, size_t m, size_t n);

/* dequant.rs:12-25, dequant.rs:29-38 */
void ao_dequant_q4_0_block(const uint8_t *block, float *out32);
void ao_dequant_q8_0_block(const uint8_t *block, float *out32);

/* ---- GEMV ----------------------------------------------------------------
 * q8_gemv.rs:230-244 (compute_row, x86 scalar) and q8_gemv.rs:80-98
 * (compute_row_q4).  Single-threaded; rows are independent so the
 * multithreaded variant returns identical bits. */
void ao_quant_gemv(uint32_t ggml_type, const uint8_t *w, size_t m, size_t n, const float *x,
                   float *y);
/* Row-parallel over nthreads (OpenMP), the rayon par_iter_mut of
 * q8_gemv.rs:145-147.  nthreads <= 0 means all available. */
void ao_quant_gemv_mt(uint32_t ggml_type, const uint8_t *w, size_t m, size_t n, const float *x,
                      float *y, int nthreads);
/* batch independent GEMVs: y[b] = W x[b] */
void ao_quant_gemm(uint32_t ggml_type, const uint8_t *w, size_t m, size_t n, const float *x,
                   size_t batch, float *y, int nthreads);

/* ---- elementwise (scratch.rs:152-186, deltanet.rs:10-51, main.rs:1106) -- */
void ao_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps);
void ao_silu_mul_inplace(float *a, const float *b, size_t n);
void ao_residual_add(float *x, const float *y, size_t n);

/* ---- DeltaNet mixer core ---------------------------------------------------
 * deltanet.rs:444-512: conv shift/append/apply (deltanet_cache.rs:34-54),
 * SiLU, q/k split, per-head L2 norm (+ q * 1/sqrt(key_dim)), beta/decay,
 * per-head decay -> recall -> delta -> rank-1 update -> query.
 *   qkv       [3*chunk]              GEMV output of the qkv projection
 *   beta_raw, alpha_raw [n_heads]    GEMV outputs of ssm_beta / ssm_alpha
 *   conv_w    [3*chunk][ksize]       ssm_conv1d
 *   conv_state[3*chunk][ksize]       updated in place
 *   S         [n_heads][dk][dv]      updated in place
 *   out_heads [chunk]                recurrence output (pre-norm)
 * chunk = n_heads * dk and dk == dv (the reference's configuration). */
void ao_deltanet_core(size_t chunk, size_t n_heads, size_t dk, size_t ksize, const float *qkv,
                      const float *beta_raw, const float *alpha_raw, const float *conv_w,
                      const float *ssm_a, const float *dt_bias, float *conv_state, float *S,
                      float *out_heads);
/* deltanet.rs:517-533: per-head RMSNorm with ssm_norm, then * SiLU(gate) */
void ao_gated_rmsnorm(float *normed, const float *heads, const float *gate, const float *norm_w,
                      size_t n_heads, size_t head_dim, float eps);

/* ---- full-attention mixer core ---------------------------------------------
 * deltanet.rs:565-669: q/gate de-interleave, q/k RMSNorm (eps 1e-6), RoPE
 * with freq = 1/base^(i/hd), KV write at pos (kv_cache.rs:31-41), 3-pass
 * softmax over positions 0..pos, weighted V, * sigmoid(gate).
 *   q_full [n_heads][2*hd], k_in, v_in [n_kv_heads][hd]  (GEMV outputs)
 *   cache layout [n_kv_heads][max_seq][hd] (kv_cache.rs:7-27); if kv_f16 the
 *   cache holds fp16 bits (RNE on write) and values are widened on read.
 *   attn_out [n_heads*hd] (input of wo). */
void ao_attention_core(size_t n_heads, size_t n_kv_heads, size_t hd, size_t max_seq, size_t pos,
                       float rope_base, const float *q_full, const float *k_in, const float *v_in,
                       const float *q_norm, const float *k_norm, int kv_f16, void *k_cache,
                       void *v_cache, float *attn_out);

/* ---- model --------------------------------------------------------------
 * qwen35_forward_token (crates/cli/src/main.rs:953-1023) over a model whose
 * tensors are borrowed host pointers registered by kind (the same kinds and
 * shapes as anehip.h).  State per sequence: conv/recurrent state per
 * DeltaNet layer, KV cache per attention layer, pos. */
typedef struct ao_model ao_model;
typedef struct ao_seq ao_seq;

ao_model *ao_model_create(uint32_t dim, uint32_t hidden_dim, uint32_t n_layers, uint32_t n_heads,
                          uint32_t n_kv_heads, uint32_t head_dim, uint32_t vocab_size,
                          uint32_t ssm_state_size, uint32_t ssm_conv_kernel,
                          uint32_t ssm_group_count, float rope_freq_base, float rms_norm_eps,
                          const uint8_t *layer_types);
void ao_model_destroy(ao_model *m);
/* returns 0, or -1 on an unknown kind / bad layer */
int ao_model_set_quant(ao_model *m, int layer, int kind, const uint8_t *data, uint32_t rows,
                       uint32_t cols, uint32_t ggml_type);
int ao_model_set_f32(ao_model *m, int layer, int kind, const float *data, size_t n);

ao_seq *ao_seq_create(const ao_model *m, uint32_t max_seq, int kv_f16);
void ao_seq_destroy(ao_seq *s);
void ao_seq_set_pos(ao_seq *s, uint32_t pos);
uint32_t ao_seq_get_pos(const ao_seq *s);
/* direct views of the state (for seeding and comparison) */
float *ao_seq_conv_state(ao_seq *s, uint32_t layer);      /* [3d][ksize]        */
float *ao_seq_recurrent_state(ao_seq *s, uint32_t layer); /* [H][dk][dv]        */
void *ao_seq_k_cache(ao_seq *s, uint32_t layer);          /* [kvh][max_seq][hd] */
void *ao_seq_v_cache(ao_seq *s, uint32_t layer);

/* One token: logits[vocab]; advances pos by 1.  nthreads as ao_quant_gemv_mt.
 * Returns 0, or -1 if a tensor is missing or pos >= max_seq. */
int ao_forward_token(const ao_model *m, ao_seq *s, uint32_t token, float *logits, int nthreads);

/* greedy_sample at temperature < 0.01 (main.rs:1767-1775): index of the
 * maximum under f32::total_cmp, the last one among equal maxima. */
uint32_t ao_argmax(const float *logits, size_t n);

/* OpenMP thread count actually available */
int ao_max_threads(void);

#ifdef __cplusplus
}
#endif

#endif
