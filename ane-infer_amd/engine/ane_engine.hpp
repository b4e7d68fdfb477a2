// ane_engine.hpp — C++ host API of the decode path, over libanehip's C ABI.
//
// Mirrors the Rust engine API the reference's callers use for this path, with
// the same names, argument meaning and error behaviour, so code and tests
// written against the reference read the same:
//
//   QuantType, Q8Tensor::from_raw           crates/engine/src/q8_gemv.rs:10-57
//   GpuBuffer, GemvOp, SiluMulOp            crates/engine/src/metal_graph.rs:7-30
//   GpuContext (new, upload_quant_weights,  metal_graph.rs:79-265
//     upload_q8_weights, scratch_*,
//     ensure_scratch_capacity)
//   GpuGraph (add_gemv, add_gemv_raw,       metal_graph.rs:268-409
//     add_silu_mul, clear, execute)
//   ModelConfig, Qwen35Config, LayerType,   crates/engine/src/model.rs:7-157
//     FfnWeights, DeltaNetLayerWeights,
//     FullAttnLayerWeights,
//     HybridLayerWeights,
//     Qwen35ModelWeights
//   upload_model_weights, GpuModelWeights   crates/engine/src/gpu_decode.rs:84-283
//   GpuLayerScratch, GpuConstantPool,       crates/engine/src/gpu_full_decode.rs:18-1044
//     encode_full_token_gpu
//
// Rust `anyhow::Result` failures and `assert!` panics both surface as a thrown
// ane::Error carrying the library's status code and message.
//
// Differences a caller sees: the scratch buffers are device memory, written
// and read with write_scratch_input / read_scratch_output (the reference maps
// unified memory); GpuGraph::execute records its ops into a hipGraph on the
// first call and replays it afterwards.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <variant>
#include <vector>

#include "anehip.h"

namespace ane {

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string &msg) : std::runtime_error(msg), code(c) {}
};

// GGML type codes (q8_gemv.rs:10-14).  Q6K is not supported by these kernels.
enum class QuantType : uint32_t { Q4_0 = 2, Q8_0 = 8 };

// A quantised [m x n] matrix in GGUF block layout (q8_gemv.rs:16-21).
struct Q8Tensor {
    std::vector<uint8_t> data;
    size_t m = 0, n = 0;
    QuantType quant_type = QuantType::Q8_0;
    // ne0 = n (input dim), ne1 = m (output dim); checks n % 32 and the byte
    // count as the reference's asserts do (q8_gemv.rs:33-57).
    static Q8Tensor from_raw(std::vector<uint8_t> data, size_t ne0, size_t ne1,
                             QuantType quant_type = QuantType::Q8_0);
};

// Weights resident on the device (metal_graph.rs:7-13).
struct GpuBuffer {
    std::shared_ptr<void> buffer;  // device memory, freed with the last copy
    size_t m = 0, n = 0;
    uint32_t n_blocks = 0;
    QuantType quant_type = QuantType::Q8_0;
};

// y[output_offset..+output_len] = W x[input_offset..+input_len] over the
// context's scratch input / output (f32-element offsets).
struct GemvOp {
    GpuBuffer weight_buffer;
    size_t input_offset = 0, output_offset = 0, input_len = 0, output_len = 0;
};

// scratch_output[gate_offset + i] = SiLU(gate) * scratch_output[up_offset + i], i < n.
struct SiluMulOp {
    size_t gate_offset = 0, up_offset = 0, n = 0;
};

class GpuContext {
  public:
    // GpuContext::new (metal_graph.rs:79): device probe, stream, scratch.
    static GpuContext create(int device = 0);
    GpuContext(GpuContext &&) noexcept = default;
    GpuContext &operator=(GpuContext &&) noexcept = default;
    GpuContext(const GpuContext &) = delete;

    GpuBuffer upload_quant_weights(const Q8Tensor &q) const;
    GpuBuffer upload_q8_weights(const Q8Tensor &q8) const { return upload_quant_weights(q8); }

    float *scratch_input_ptr() const { return scratch_input_; }          // device pointer
    const float *scratch_output_ptr() const { return scratch_output_; }  // device pointer
    size_t scratch_input_size() const { return scratch_input_size_; }    // bytes
    size_t scratch_output_size() const { return scratch_output_size_; }  // bytes
    void ensure_scratch_capacity(size_t input_bytes, size_t output_bytes);
    void write_scratch_input(const float *src, size_t count, size_t offset = 0) const;
    void read_scratch_output(float *dst, size_t count, size_t offset = 0) const;

    anehip_ctx *raw() const { return ctx_; }
    int device() const { return device_; }

  private:
    GpuContext() = default;
    std::shared_ptr<anehip_ctx> hold_;  // shared with every buffer made from this context
    std::shared_ptr<void> in_, out_;
    anehip_ctx *ctx_ = nullptr;
    int device_ = 0;
    float *scratch_input_ = nullptr, *scratch_output_ = nullptr;
    size_t scratch_input_size_ = 0, scratch_output_size_ = 0;
    friend class GpuGraph;
};

// Ops recorded once and run together (metal_graph.rs:268-409): one hipGraph
// replay per execute() instead of one command buffer per call.
class GpuGraph {
  public:
    explicit GpuGraph(GpuContext &ctx);
    ~GpuGraph();
    GpuGraph(const GpuGraph &) = delete;
    void add_gemv(GemvOp op);
    void add_gemv_raw(GpuBuffer weight_buffer, size_t input_offset, size_t output_offset, size_t input_len,
                      size_t output_len);
    void add_silu_mul(SiluMulOp op);
    void clear();
    void execute();  // blocks until done, like commit + wait

  private:
    struct Op {
        bool gemv;
        GemvOp g;
        SiluMulOp s;
    };
    void enqueue() const;
    GpuContext *ctx_;
    std::vector<Op> ops_;
    anehip_graph *graph_ = nullptr;
    const float *graph_in_ = nullptr, *graph_out_ = nullptr;  // scratch the graph was recorded with
};

// ---- model (model.rs) -------------------------------------------------------

enum class LayerType : uint8_t { DeltaNet = 0, FullAttention = 1 };

struct ModelConfig {
    size_t dim = 0, hidden_dim = 0, n_layers = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, vocab_size = 0,
           max_seq_len = 0;
    float rope_freq_base = 10000.0f, rms_norm_eps = 1e-6f;
};

struct Qwen35Config {
    ModelConfig base;
    size_t full_attention_interval = 4, ssm_state_size = 128, ssm_conv_kernel = 4, ssm_group_count = 16,
           ssm_inner_size = 0;
    std::vector<LayerType> layer_types;
};

struct FfnWeights {
    Q8Tensor gate, up, down;
};

struct DeltaNetLayerWeights {
    std::vector<float> attn_norm, post_attn_norm;
    Q8Tensor qkv, attn_gate;
    std::vector<float> ssm_a;
    Q8Tensor ssm_alpha, ssm_beta;
    std::vector<float> ssm_conv1d, ssm_dt_bias, ssm_norm;  // conv1d: [channel][conv_kernel]
    Q8Tensor ssm_out;
    FfnWeights ffn;
};

struct FullAttnLayerWeights {
    std::vector<float> attn_norm, post_attn_norm;
    Q8Tensor wq, wk, wv, wo;
    std::vector<float> q_norm, k_norm;
    FfnWeights ffn;
};

using HybridLayerWeights = std::variant<DeltaNetLayerWeights, FullAttnLayerWeights>;

struct Qwen35ModelWeights {
    Qwen35Config config;
    std::vector<float> embedding;  // [vocab][dim]
    std::vector<HybridLayerWeights> layers;
    std::vector<float> final_norm;
    Q8Tensor lm_head;
};

// Device weights + per-sequence state (gpu_decode.rs:84-150): one model
// context of libanehip, state for one sequence of config.base.max_seq_len.
class GpuModelWeights {
  public:
    GpuModelWeights(GpuModelWeights &&) noexcept;
    GpuModelWeights(const GpuModelWeights &) = delete;
    ~GpuModelWeights();
    anehip_ctx *raw() const { return ctx_; }
    size_t vocab_size() const { return vocab_; }

  private:
    GpuModelWeights() = default;
    anehip_ctx *ctx_ = nullptr;
    size_t vocab_ = 0;
    std::vector<uint8_t> types_;
    friend GpuModelWeights upload_model_weights(const GpuContext &, const Qwen35ModelWeights &);
};

// upload_model_weights (gpu_decode.rs:152-283).
GpuModelWeights upload_model_weights(const GpuContext &ctx, const Qwen35ModelWeights &w);

// GpuLayerScratch (gpu_full_decode.rs:18-44,175-217): holds the position of
// the sequence; the step's scratch lives on the device in GpuModelWeights.
struct GpuLayerScratch {
    size_t pos = 0;
    GpuLayerScratch(size_t dim, size_t hidden_dim, size_t inner_size, size_t n_heads) {
        (void)dim, (void)hidden_dim, (void)inner_size, (void)n_heads;
    }
};

// GpuConstantPool (gpu_full_decode.rs:48-172): the shape constants; kept for
// signature parity (they are baked into the captured step).
struct GpuConstantPool {
    GpuConstantPool(size_t dim, size_t hidden_dim, size_t inner_size, size_t n_heads, size_t key_dim,
                    size_t kernel_size, float eps, size_t n_heads_attn, size_t n_kv_heads, size_t head_dim,
                    float rope_freq_base) {
        (void)dim, (void)hidden_dim, (void)inner_size, (void)n_heads, (void)key_dim, (void)kernel_size, (void)eps,
            (void)n_heads_attn, (void)n_kv_heads, (void)head_dim, (void)rope_freq_base;
    }
};

// encode_full_token_gpu (gpu_full_decode.rs:221-1044): one decode step of
// token_id at scratch.pos; returns the logits [vocab]; scratch.pos advances.
std::vector<float> encode_full_token_gpu(const GpuContext &ctx, const Qwen35ModelWeights &weights,
                                         GpuModelWeights &gpu_weights, GpuLayerScratch &scratch,
                                         const GpuConstantPool &pool, uint32_t token_id);

// greedy_sample (main.rs:1767-1785): index of the maximum logit under
// f32::total_cmp, the last one on ties.
uint32_t greedy_sample(const std::vector<float> &logits);

}  // namespace ane
