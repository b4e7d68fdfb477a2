// ane_engine.cpp — C++ host API of the decode path over libanehip (see
// ane_engine.hpp for the reference functions each piece mirrors).
#include "ane_engine.hpp"

#include <cstring>

namespace ane {

namespace {

constexpr size_t kQ8Block = 34, kQ4Block = 18;

std::string last_error(const anehip_ctx *ctx) {
    const char *m = anehip_last_error(ctx);
    return m ? std::string(m) : std::string("unknown error");
}

void check(const anehip_ctx *ctx, int rc) {
    if (rc != ANEHIP_OK) throw Error(rc, last_error(ctx));
}

size_t block_bytes(QuantType t) { return t == QuantType::Q8_0 ? kQ8Block : kQ4Block; }

std::shared_ptr<void> device_alloc(const std::shared_ptr<anehip_ctx> &ctx, size_t bytes) {
    void *p = nullptr;
    check(ctx.get(), anehip_dev_alloc(ctx.get(), bytes, &p));
    // the deleter keeps the context alive as long as the buffer
    return std::shared_ptr<void>(p, [ctx](void *q) { anehip_dev_free(ctx.get(), q); });
}

}  // namespace

// ---- Q8Tensor -----------------------------------------------------------------

Q8Tensor Q8Tensor::from_raw(std::vector<uint8_t> data, size_t ne0, size_t ne1, QuantType quant_type) {
    const size_t m = ne1, n = ne0;
    if (quant_type != QuantType::Q8_0 && quant_type != QuantType::Q4_0)
        throw Error(ANEHIP_EUNSUPPORTED, "quant type " + std::to_string((uint32_t)quant_type) + " not supported");
    if (n % 32 != 0) throw Error(ANEHIP_ESHAPE, "n must be divisible by 32");
    const size_t expected = m * (n / 32) * block_bytes(quant_type);
    if (data.size() != expected)
        throw Error(ANEHIP_ESHAPE, "Quant size mismatch: got " + std::to_string(data.size()) + ", expected " +
                                       std::to_string(expected) + " (m=" + std::to_string(m) +
                                       ", n=" + std::to_string(n) + ")");
    Q8Tensor t;
    t.data = std::move(data);
    t.m = m;
    t.n = n;
    t.quant_type = quant_type;
    return t;
}

// ---- GpuContext ---------------------------------------------------------------

GpuContext GpuContext::create(int device) {
    check(nullptr, anehip_init());
    anehip_ctx *c = nullptr;
    check(nullptr, anehip_ctx_create(device, nullptr, &c));
    GpuContext g;
    g.hold_ = std::shared_ptr<anehip_ctx>(c, [](anehip_ctx *p) { anehip_ctx_destroy(p); });
    g.ctx_ = c;
    g.device_ = device;
    // the reference's initial scratch: 128 KiB of input, 4 MiB of output
    g.ensure_scratch_capacity(128 << 10, 4 << 20);
    return g;
}

void GpuContext::ensure_scratch_capacity(size_t input_bytes, size_t output_bytes) {
    if (input_bytes > scratch_input_size_) {
        in_ = device_alloc(hold_, input_bytes);
        scratch_input_ = static_cast<float *>(in_.get());
        scratch_input_size_ = input_bytes;
        check(ctx_, anehip_dev_memset(ctx_, scratch_input_, 0, input_bytes));
    }
    if (output_bytes > scratch_output_size_) {
        out_ = device_alloc(hold_, output_bytes);
        scratch_output_ = static_cast<float *>(out_.get());
        scratch_output_size_ = output_bytes;
        check(ctx_, anehip_dev_memset(ctx_, scratch_output_, 0, output_bytes));
    }
}

void GpuContext::write_scratch_input(const float *src, size_t count, size_t offset) const {
    if ((offset + count) * sizeof(float) > scratch_input_size_)
        throw Error(ANEHIP_ESHAPE, "write_scratch_input past the scratch input");
    check(ctx_, anehip_h2d(ctx_, scratch_input_ + offset, src, count * sizeof(float)));
}

void GpuContext::read_scratch_output(float *dst, size_t count, size_t offset) const {
    if ((offset + count) * sizeof(float) > scratch_output_size_)
        throw Error(ANEHIP_ESHAPE, "read_scratch_output past the scratch output");
    check(ctx_, anehip_d2h(ctx_, dst, scratch_output_ + offset, count * sizeof(float)));
}

GpuBuffer GpuContext::upload_quant_weights(const Q8Tensor &q) const {
    const uint32_t type = (uint32_t)q.quant_type;
    // the panel copy needs whole 256-column panels: pad rows with zero blocks
    const size_t bb = block_bytes(q.quant_type), nb = q.n / 32, n_pad = (q.n + 255) / 256 * 256,
                 nb_pad = n_pad / 32;
    std::vector<uint8_t> padded;
    const uint8_t *src = q.data.data();
    if (n_pad != q.n) {
        padded.assign(q.m * nb_pad * bb, 0);
        for (size_t r = 0; r < q.m; r++) std::memcpy(&padded[r * nb_pad * bb], &q.data[r * nb * bb], nb * bb);
        src = padded.data();
    }
    const size_t gguf_bytes = q.m * nb_pad * bb;
    std::shared_ptr<void> gguf = device_alloc(hold_, gguf_bytes);
    check(ctx_, anehip_h2d(ctx_, gguf.get(), src, gguf_bytes));
    const size_t pbytes = anehip_quant_packed_bytes(type, (uint32_t)q.m, (uint32_t)n_pad);
    if (!pbytes) throw Error(ANEHIP_ESHAPE, "upload_quant_weights: unsupported shape");
    GpuBuffer b;
    b.buffer = device_alloc(hold_, pbytes);
    check(ctx_, anehip_quant_pack(ctx_, type, gguf.get(), (uint32_t)q.m, (uint32_t)n_pad, b.buffer.get()));
    check(ctx_, anehip_sync(ctx_));
    b.m = q.m;
    b.n = q.n;
    b.n_blocks = (uint32_t)nb;
    b.quant_type = q.quant_type;
    return b;
}

// ---- GpuGraph -------------------------------------------------------------------

GpuGraph::GpuGraph(GpuContext &ctx) : ctx_(&ctx) {}

GpuGraph::~GpuGraph() { anehip_graph_destroy(graph_); }

void GpuGraph::add_gemv(GemvOp op) {
    if (op.input_len != op.weight_buffer.n || op.output_len != op.weight_buffer.m)
        throw Error(ANEHIP_ESHAPE, "add_gemv: input_len / output_len disagree with the weight shape");
    anehip_graph_destroy(graph_);
    graph_ = nullptr;
    ops_.push_back(Op{true, std::move(op), SiluMulOp{}});
}

void GpuGraph::add_gemv_raw(GpuBuffer weight_buffer, size_t input_offset, size_t output_offset, size_t input_len,
                            size_t output_len) {
    GemvOp op;
    op.weight_buffer = std::move(weight_buffer);
    op.input_offset = input_offset;
    op.output_offset = output_offset;
    op.input_len = input_len;
    op.output_len = output_len;
    add_gemv(std::move(op));
}

void GpuGraph::add_silu_mul(SiluMulOp op) {
    anehip_graph_destroy(graph_);
    graph_ = nullptr;
    ops_.push_back(Op{false, GemvOp{}, op});
}

void GpuGraph::clear() {
    anehip_graph_destroy(graph_);
    graph_ = nullptr;
    ops_.clear();
}

void GpuGraph::enqueue() const {
    anehip_ctx *c = ctx_->ctx_;
    for (const Op &op : ops_) {
        if (op.gemv) {
            const GemvOp &g = op.g;
            const size_t n_pad = (g.weight_buffer.n + 255) / 256 * 256;
            if ((g.input_offset + n_pad) * sizeof(float) > ctx_->scratch_input_size_ ||
                (g.output_offset + g.output_len) * sizeof(float) > ctx_->scratch_output_size_)
                throw Error(ANEHIP_ESHAPE, "gemv: offsets past the scratch buffers (ensure_scratch_capacity)");
            // columns past n read the zero-initialised scratch and meet zero weights
            check(c, anehip_quant_gemv_packed(c, (uint32_t)g.weight_buffer.quant_type, g.weight_buffer.buffer.get(),
                                              (uint32_t)g.weight_buffer.m, (uint32_t)n_pad,
                                              ctx_->scratch_input_ + g.input_offset,
                                              ctx_->scratch_output_ + g.output_offset));
        } else {
            const SiluMulOp &s = op.s;
            check(c, anehip_silu_mul(c, ctx_->scratch_output_ + s.gate_offset, ctx_->scratch_output_ + s.up_offset,
                                     s.n));
        }
    }
}

void GpuGraph::execute() {
    if (ops_.empty()) return;
    anehip_ctx *c = ctx_->ctx_;
    if (graph_ && (graph_in_ != ctx_->scratch_input_ || graph_out_ != ctx_->scratch_output_)) {
        anehip_graph_destroy(graph_);  // the scratch moved since the graph was recorded
        graph_ = nullptr;
    }
    if (!graph_) {
        enqueue();  // eager once: sizes the workspace, and this call's result
        check(c, anehip_sync(c));
        check(c, anehip_capture_begin(c));
        try {
            enqueue();
        } catch (...) {
            anehip_graph *g = nullptr;
            anehip_capture_end(c, &g);
            anehip_graph_destroy(g);
            throw;
        }
        check(c, anehip_capture_end(c, &graph_));
        graph_in_ = ctx_->scratch_input_;
        graph_out_ = ctx_->scratch_output_;
        return;
    }
    check(c, anehip_graph_launch(c, graph_));
    check(c, anehip_sync(c));
}

// ---- model ------------------------------------------------------------------------

GpuModelWeights::GpuModelWeights(GpuModelWeights &&o) noexcept {
    std::swap(ctx_, o.ctx_);
    std::swap(vocab_, o.vocab_);
    std::swap(types_, o.types_);
}

GpuModelWeights::~GpuModelWeights() { anehip_ctx_destroy(ctx_); }

GpuModelWeights upload_model_weights(const GpuContext &ctx, const Qwen35ModelWeights &w) {
    const Qwen35Config &cfg = w.config;
    const ModelConfig &b = cfg.base;
    if (cfg.layer_types.size() != b.n_layers || w.layers.size() != b.n_layers)
        throw Error(ANEHIP_ESHAPE, "upload_model_weights: layer count disagrees with the config");
    GpuModelWeights g;
    g.types_.resize(b.n_layers);
    for (size_t l = 0; l < b.n_layers; l++) g.types_[l] = (uint8_t)cfg.layer_types[l];
    anehip_model_desc d{};
    d.dim = (uint32_t)b.dim;
    d.hidden_dim = (uint32_t)b.hidden_dim;
    d.n_layers = (uint32_t)b.n_layers;
    d.n_heads = (uint32_t)b.n_heads;
    d.n_kv_heads = (uint32_t)b.n_kv_heads;
    d.head_dim = (uint32_t)b.head_dim;
    d.vocab_size = (uint32_t)b.vocab_size;
    d.ssm_state_size = (uint32_t)cfg.ssm_state_size;
    d.ssm_conv_kernel = (uint32_t)cfg.ssm_conv_kernel;
    d.ssm_group_count = (uint32_t)cfg.ssm_group_count;
    d.rope_freq_base = b.rope_freq_base;
    d.rms_norm_eps = b.rms_norm_eps;
    d.layer_types = g.types_.data();
    check(nullptr, anehip_ctx_create(ctx.device(), &d, &g.ctx_));
    g.vocab_ = b.vocab_size;
    anehip_ctx *c = g.ctx_;
    auto q = [c](int layer, uint32_t kind, const Q8Tensor &t) {
        check(c, anehip_upload_quant(c, layer, kind, t.data.data(), t.data.size(), (uint32_t)t.m, (uint32_t)t.n,
                                     (uint32_t)t.quant_type));
    };
    auto f = [c](int layer, uint32_t kind, const std::vector<float> &v) {
        check(c, anehip_upload_f32(c, layer, kind, v.data(), v.size()));
    };
    f(-1, ANEHIP_T_EMBEDDING, w.embedding);
    f(-1, ANEHIP_T_FINAL_NORM, w.final_norm);
    q(-1, ANEHIP_T_LM_HEAD, w.lm_head);
    for (size_t l = 0; l < b.n_layers; l++) {
        const int L = (int)l;
        if (const auto *dn = std::get_if<DeltaNetLayerWeights>(&w.layers[l])) {
            f(L, ANEHIP_T_ATTN_NORM, dn->attn_norm);
            f(L, ANEHIP_T_POST_ATTN_NORM, dn->post_attn_norm);
            q(L, ANEHIP_T_QKV, dn->qkv);
            q(L, ANEHIP_T_ATTN_GATE, dn->attn_gate);
            f(L, ANEHIP_T_SSM_A, dn->ssm_a);
            q(L, ANEHIP_T_SSM_ALPHA, dn->ssm_alpha);
            q(L, ANEHIP_T_SSM_BETA, dn->ssm_beta);
            f(L, ANEHIP_T_SSM_CONV1D, dn->ssm_conv1d);
            f(L, ANEHIP_T_SSM_DT_BIAS, dn->ssm_dt_bias);
            f(L, ANEHIP_T_SSM_NORM, dn->ssm_norm);
            q(L, ANEHIP_T_SSM_OUT, dn->ssm_out);
            q(L, ANEHIP_T_FFN_GATE, dn->ffn.gate);
            q(L, ANEHIP_T_FFN_UP, dn->ffn.up);
            q(L, ANEHIP_T_FFN_DOWN, dn->ffn.down);
        } else {
            const auto &a = std::get<FullAttnLayerWeights>(w.layers[l]);
            f(L, ANEHIP_T_ATTN_NORM, a.attn_norm);
            f(L, ANEHIP_T_POST_ATTN_NORM, a.post_attn_norm);
            q(L, ANEHIP_T_WQ, a.wq);
            q(L, ANEHIP_T_WK, a.wk);
            q(L, ANEHIP_T_WV, a.wv);
            q(L, ANEHIP_T_WO, a.wo);
            f(L, ANEHIP_T_Q_NORM, a.q_norm);
            f(L, ANEHIP_T_K_NORM, a.k_norm);
            q(L, ANEHIP_T_FFN_GATE, a.ffn.gate);
            q(L, ANEHIP_T_FFN_UP, a.ffn.up);
            q(L, ANEHIP_T_FFN_DOWN, a.ffn.down);
        }
    }
    check(c, anehip_alloc_state(c, 1, (uint32_t)(b.max_seq_len ? b.max_seq_len : 4096)));
    return g;
}

std::vector<float> encode_full_token_gpu(const GpuContext &ctx, const Qwen35ModelWeights &weights,
                                         GpuModelWeights &gpu_weights, GpuLayerScratch &scratch,
                                         const GpuConstantPool &pool, uint32_t token_id) {
    (void)ctx, (void)weights, (void)pool;
    anehip_ctx *c = gpu_weights.raw();
    uint32_t pos = 0;
    check(c, anehip_get_pos(c, 0, &pos));
    if (pos != scratch.pos) check(c, anehip_set_pos(c, 0, (uint32_t)scratch.pos));
    std::vector<float> logits(gpu_weights.vocab_size());
    check(c, anehip_decode_step(c, &token_id, 1, logits.data()));
    scratch.pos += 1;
    return logits;
}

uint32_t greedy_sample(const std::vector<float> &logits) {
    // f32::total_cmp: order the bit patterns, negatives reversed
    auto key = [](float f) {
        int32_t b;
        std::memcpy(&b, &f, 4);
        return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
    };
    uint32_t best = 0;
    for (uint32_t i = 1; i < logits.size(); i++)
        if (key(logits[i]) >= key(logits[best])) best = i;
    return best;
}

}  // namespace ane
