// Tests of the C++ engine API (ane-infer_amd/engine), named and shaped after
// the reference's own tests of the API it mirrors:
//   test_gpu_context_creation / test_upload_weights / test_graph_single_gemv
//     crates/engine/src/metal_graph.rs:543-594
//   test_q8_gemv_identity / test_q8_gemv_parallel   crates/engine/src/q8_gemv.rs:257-314
// plus the SiLU-mul graph op, graph replays over new inputs, the from_raw
// shape checks, and encode_full_token_gpu on a tiny seeded hybrid model
// against the CPU oracle (test infrastructure, oracle/ane_oracle.h).
// The GGUF reader (engine/gguf.hpp, mirroring crates/gguf) is checked on
// files written here by a small GGUF writer: metadata of every value type,
// tensor offsets and alignment, the reference's dequant known answers
// (dequant.rs:235-270), malformed files, and the tiny model loaded from its
// GGUF file (load_qwen35_q8) decoding bit-identically to the same weights
// uploaded directly.
// Prints one line per test; exit status 0 iff all pass.
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "ane_engine.hpp"
#include "ane_oracle.h"
#include "gguf.hpp"

using namespace ane;

static int failures = 0;
#define EXPECT(cond, ...)                                      \
    do {                                                       \
        if (!(cond)) {                                         \
            std::printf("    expectation failed: " #cond " "); \
            std::printf(__VA_ARGS__);                          \
            std::printf("\n");                                 \
            throw std::runtime_error("failed");                \
        }                                                      \
    } while (0)

static void run(const char *name, const std::function<void()> &fn) {
    try {
        fn();
        std::printf("PASS %s\n", name);
    } catch (const std::exception &e) {
        std::printf("FAIL %s: %s\n", name, e.what());
        failures++;
    }
    std::fflush(stdout);
}

// m rows of one Q8_0 block each: row r has quant 1 at column r, scale 1.0
// (q8_gemv.rs:257-281 / metal_graph.rs:530-541).
static Q8Tensor make_q8_identity(size_t m, size_t n) {
    std::vector<uint8_t> data(m * (n / 32) * 34, 0);
    for (size_t r = 0; r < m; r++) {
        uint8_t *blk = &data[(r * (n / 32) + r / 32) * 34];
        blk[0] = 0x00;
        blk[1] = 0x3c;  // fp16 1.0
        blk[2 + r % 32] = 1;
    }
    return Q8Tensor::from_raw(std::move(data), n, m);
}

// The reference's patterned matrix (q8_gemv.rs:283-299): every block has
// scale 0.5 and quant i = ((row + i) % 256) as i8.  With integer inputs every
// partial sum is an integer below 2^24, so fp32 results are exact.
static int8_t pattern_q(size_t row, size_t i) { return (int8_t)(uint8_t)((row + i) % 256); }

static Q8Tensor make_patterned(size_t m, size_t n) {
    std::vector<uint8_t> data(m * (n / 32) * 34, 0);
    for (size_t r = 0; r < m; r++)
        for (size_t b = 0; b < n / 32; b++) {
            uint8_t *blk = &data[(r * (n / 32) + b) * 34];
            blk[0] = 0x00;
            blk[1] = 0x38;  // fp16 0.5
            for (size_t i = 0; i < 32; i++) blk[2 + i] = (uint8_t)pattern_q(r, i);
        }
    return Q8Tensor::from_raw(std::move(data), n, m);
}

// ---- a tiny seeded hybrid model, shared by the GPU engine and the oracle ------

struct Tiny {
    Qwen35ModelWeights w;
    ao_model *om = nullptr;
};

static std::vector<float> normal(uint64_t stream, size_t n, float mean, float sd) {
    std::vector<float> v(n);
    ao_fill_normal(77, stream, mean, sd, v.data(), n);
    return v;
}

static std::vector<float> uniform(uint64_t stream, size_t n, float lo, float hi) {
    std::vector<float> v(n);
    ao_fill_uniform(77, stream, lo, hi, v.data(), n);
    return v;
}

static Q8Tensor quant(uint64_t stream, size_t rows, size_t cols) {
    std::vector<uint8_t> d(ao_quant_bytes(8, rows, cols));
    ao_gen_quant(8, 77, stream, 0.02f, rows, cols, d.data());
    return Q8Tensor::from_raw(std::move(d), cols, rows);
}

static Tiny make_tiny() {
    Tiny t;
    Qwen35Config &c = t.w.config;
    c.base.dim = 256;
    c.base.hidden_dim = 512;
    c.base.n_layers = 4;
    c.base.n_heads = 4;
    c.base.n_kv_heads = 1;
    c.base.head_dim = 256;
    c.base.vocab_size = 1000;
    c.base.max_seq_len = 64;
    c.ssm_group_count = 2;
    c.ssm_inner_size = 3 * 256;
    for (size_t l = 0; l < 4; l++) c.layer_types.push_back(l % 4 == 3 ? LayerType::FullAttention : LayerType::DeltaNet);
    const size_t d = 256, F = 512, H = 2, C = 3 * d, hd = 256;
    uint64_t s = 1;
    t.w.embedding = normal(s++, 1000 * d, 0.f, 0.02f);
    t.w.final_norm = normal(s++, d, 1.f, 0.1f);
    t.w.lm_head = quant(s++, 1000, d);
    for (size_t l = 0; l < 4; l++) {
        FfnWeights ffn{quant(s++, F, d), quant(s++, F, d), quant(s++, d, F)};
        if (c.layer_types[l] == LayerType::DeltaNet) {
            DeltaNetLayerWeights x;
            x.attn_norm = normal(s++, d, 1.f, 0.1f);
            x.post_attn_norm = normal(s++, d, 1.f, 0.1f);
            x.qkv = quant(s++, C, d);
            x.attn_gate = quant(s++, d, d);
            x.ssm_a = uniform(s++, H, -1.f, 0.f);
            x.ssm_alpha = quant(s++, H, d);
            x.ssm_beta = quant(s++, H, d);
            x.ssm_conv1d = normal(s++, C * 4, 0.f, 0.3f);
            x.ssm_dt_bias = normal(s++, H, 0.f, 1.f);
            x.ssm_norm = normal(s++, 128, 1.f, 0.1f);
            x.ssm_out = quant(s++, d, d);
            x.ffn = std::move(ffn);
            t.w.layers.emplace_back(std::move(x));
        } else {
            FullAttnLayerWeights x;
            x.attn_norm = normal(s++, d, 1.f, 0.1f);
            x.post_attn_norm = normal(s++, d, 1.f, 0.1f);
            x.wq = quant(s++, 2 * 4 * hd, d);
            x.wk = quant(s++, hd, d);
            x.wv = quant(s++, hd, d);
            x.wo = quant(s++, d, 4 * hd);
            x.q_norm = normal(s++, hd, 1.f, 0.1f);
            x.k_norm = normal(s++, hd, 1.f, 0.1f);
            x.ffn = std::move(ffn);
            t.w.layers.emplace_back(std::move(x));
        }
    }
    // the same tensors in the oracle
    std::vector<uint8_t> types;
    for (auto lt : c.layer_types) types.push_back((uint8_t)lt);
    t.om = ao_model_create(256, 512, 4, 4, 1, 256, 1000, 128, 4, 2, 10000.f, 1e-6f, types.data());
    auto q = [&](int layer, int kind, const Q8Tensor &x) {
        ao_model_set_quant(t.om, layer, kind, x.data.data(), (uint32_t)x.m, (uint32_t)x.n, 8);
    };
    auto f = [&](int layer, int kind, const std::vector<float> &v) {
        ao_model_set_f32(t.om, layer, kind, v.data(), v.size());
    };
    f(-1, ANEHIP_T_EMBEDDING, t.w.embedding);
    f(-1, ANEHIP_T_FINAL_NORM, t.w.final_norm);
    q(-1, ANEHIP_T_LM_HEAD, t.w.lm_head);
    for (int l = 0; l < 4; l++) {
        if (const auto *x = std::get_if<DeltaNetLayerWeights>(&t.w.layers[l])) {
            f(l, ANEHIP_T_ATTN_NORM, x->attn_norm);
            f(l, ANEHIP_T_POST_ATTN_NORM, x->post_attn_norm);
            q(l, ANEHIP_T_QKV, x->qkv);
            q(l, ANEHIP_T_ATTN_GATE, x->attn_gate);
            f(l, ANEHIP_T_SSM_A, x->ssm_a);
            q(l, ANEHIP_T_SSM_ALPHA, x->ssm_alpha);
            q(l, ANEHIP_T_SSM_BETA, x->ssm_beta);
            f(l, ANEHIP_T_SSM_CONV1D, x->ssm_conv1d);
            f(l, ANEHIP_T_SSM_DT_BIAS, x->ssm_dt_bias);
            f(l, ANEHIP_T_SSM_NORM, x->ssm_norm);
            q(l, ANEHIP_T_SSM_OUT, x->ssm_out);
            q(l, ANEHIP_T_FFN_GATE, x->ffn.gate);
            q(l, ANEHIP_T_FFN_UP, x->ffn.up);
            q(l, ANEHIP_T_FFN_DOWN, x->ffn.down);
        } else {
            const auto &a = std::get<FullAttnLayerWeights>(t.w.layers[l]);
            f(l, ANEHIP_T_ATTN_NORM, a.attn_norm);
            f(l, ANEHIP_T_POST_ATTN_NORM, a.post_attn_norm);
            q(l, ANEHIP_T_WQ, a.wq);
            q(l, ANEHIP_T_WK, a.wk);
            q(l, ANEHIP_T_WV, a.wv);
            q(l, ANEHIP_T_WO, a.wo);
            f(l, ANEHIP_T_Q_NORM, a.q_norm);
            f(l, ANEHIP_T_K_NORM, a.k_norm);
            q(l, ANEHIP_T_FFN_GATE, a.ffn.gate);
            q(l, ANEHIP_T_FFN_UP, a.ffn.up);
            q(l, ANEHIP_T_FFN_DOWN, a.ffn.down);
        }
    }
    return t;
}

// ---- a GGUF v3 writer (test infrastructure) ------------------------------------

struct GgufWriter {
    std::vector<uint8_t> kv;
    uint64_t n_kv = 0;
    struct T {
        std::string name;
        std::vector<uint64_t> dims;
        uint32_t type;
        std::vector<uint8_t> data;
    };
    std::vector<T> tensors;
    template <typename V> static void put(std::vector<uint8_t> &b, V v) {
        const uint8_t *p = reinterpret_cast<const uint8_t *>(&v);
        b.insert(b.end(), p, p + sizeof(V));
    }
    static void put_str(std::vector<uint8_t> &b, const std::string &x) {
        put<uint64_t>(b, x.size());
        b.insert(b.end(), x.begin(), x.end());
    }
    void key(const std::string &k, uint32_t type) {
        put_str(kv, k);
        put<uint32_t>(kv, type);
        n_kv++;
    }
    void u32(const std::string &k, uint32_t v) { key(k, 4), put(kv, v); }
    void f32(const std::string &k, float v) { key(k, 6), put(kv, v); }
    void str(const std::string &k, const std::string &v) { key(k, 8), put_str(kv, v); }
    void str_array(const std::string &k, const std::vector<std::string> &v) {
        key(k, 9);
        put<uint32_t>(kv, 8);
        put<uint64_t>(kv, v.size());
        for (const auto &x : v) put_str(kv, x);
    }
    void tensor(const std::string &name, std::vector<uint64_t> dims, uint32_t type, std::vector<uint8_t> data) {
        tensors.push_back(T{name, std::move(dims), type, std::move(data)});
    }
    void f32_tensor(const std::string &name, std::vector<uint64_t> dims, const std::vector<float> &v) {
        std::vector<uint8_t> b(v.size() * 4);
        std::memcpy(b.data(), v.data(), b.size());
        tensor(name, std::move(dims), 0, std::move(b));
    }
    void quant_tensor(const std::string &name, const Q8Tensor &q) {
        tensor(name, {q.n, q.m}, (uint32_t)q.quant_type, q.data);
    }
    std::vector<uint8_t> bytes(uint64_t align = 32) const {
        std::vector<uint8_t> b;
        put<uint32_t>(b, 0x46554747u);
        put<uint32_t>(b, 3);
        put<uint64_t>(b, tensors.size());
        put<uint64_t>(b, n_kv);
        b.insert(b.end(), kv.begin(), kv.end());
        uint64_t off = 0;
        std::vector<uint64_t> offs;
        for (const T &t : tensors) {
            put_str(b, t.name);
            put<uint32_t>(b, (uint32_t)t.dims.size());
            for (uint64_t d : t.dims) put<uint64_t>(b, d);
            put<uint32_t>(b, t.type);
            put<uint64_t>(b, off);
            offs.push_back(off);
            off = (off + t.data.size() + align - 1) / align * align;
        }
        b.resize((b.size() + align - 1) / align * align, 0);
        const size_t base = b.size();
        b.resize(base + off, 0);
        for (size_t i = 0; i < tensors.size(); i++)
            std::memcpy(&b[base + offs[i]], tensors[i].data.data(), tensors[i].data.size());
        return b;
    }
};

// The tiny model's tensors under the checkpoint names load_qwen35_q8 reads
// (crates/gguf/src/to_ane.rs:129-163, crates/cli/src/main.rs:1894-1994).
static std::vector<uint8_t> tiny_gguf(const Tiny &t, bool tied_lm_head) {
    GgufWriter w;
    const ModelConfig &b = t.w.config.base;
    w.str("general.architecture", "qwen35");
    w.u32("general.alignment", 64);
    w.u32("qwen35.embedding_length", (uint32_t)b.dim);
    w.u32("qwen35.attention.head_count", (uint32_t)b.n_heads);
    w.u32("qwen35.attention.head_count_kv", (uint32_t)b.n_kv_heads);
    w.u32("qwen35.block_count", (uint32_t)b.n_layers);
    w.u32("qwen35.feed_forward_length", (uint32_t)b.hidden_dim);
    w.u32("qwen35.context_length", (uint32_t)b.max_seq_len);
    w.u32("qwen35.attention.key_length", (uint32_t)b.head_dim);
    w.f32("qwen35.rope.freq_base", b.rope_freq_base);
    w.f32("qwen35.attention.layer_norm_rms_epsilon", b.rms_norm_eps);
    w.u32("qwen35.full_attention_interval", 4);
    w.u32("qwen35.ssm.state_size", (uint32_t)t.w.config.ssm_state_size);
    w.u32("qwen35.ssm.conv_kernel", (uint32_t)t.w.config.ssm_conv_kernel);
    w.u32("qwen35.ssm.group_count", (uint32_t)t.w.config.ssm_group_count);
    w.u32("qwen35.ssm.inner_size", (uint32_t)t.w.config.ssm_inner_size);
    std::vector<std::string> vocab(b.vocab_size);
    for (size_t i = 0; i < vocab.size(); i++) vocab[i] = "tok" + std::to_string(i);
    w.str_array("tokenizer.ggml.tokens", vocab);
    const uint64_t d = b.dim;
    if (tied_lm_head)  // the embedding stored quantised and read back as fp32 (dequantised)
        w.quant_tensor("token_embd.weight", t.w.lm_head);
    else
        w.f32_tensor("token_embd.weight", {d, b.vocab_size}, t.w.embedding);
    w.f32_tensor("output_norm.weight", {d}, t.w.final_norm);
    if (!tied_lm_head) w.quant_tensor("output.weight", t.w.lm_head);
    for (size_t l = 0; l < b.n_layers; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        auto ffn = [&](const FfnWeights &f) {
            w.quant_tensor(p + "ffn_gate.weight", f.gate);
            w.quant_tensor(p + "ffn_up.weight", f.up);
            w.quant_tensor(p + "ffn_down.weight", f.down);
        };
        if (const auto *x = std::get_if<DeltaNetLayerWeights>(&t.w.layers[l])) {
            w.f32_tensor(p + "attn_norm.weight", {d}, x->attn_norm);
            w.f32_tensor(p + "post_attention_norm.weight", {d}, x->post_attn_norm);
            w.quant_tensor(p + "attn_qkv.weight", x->qkv);
            w.quant_tensor(p + "attn_gate.weight", x->attn_gate);
            w.f32_tensor(p + "ssm_a", {x->ssm_a.size()}, x->ssm_a);
            w.quant_tensor(p + "ssm_alpha.weight", x->ssm_alpha);
            w.quant_tensor(p + "ssm_beta.weight", x->ssm_beta);
            w.f32_tensor(p + "ssm_conv1d.weight", {4, x->ssm_conv1d.size() / 4}, x->ssm_conv1d);
            w.f32_tensor(p + "ssm_dt.bias", {x->ssm_dt_bias.size()}, x->ssm_dt_bias);
            w.f32_tensor(p + "ssm_norm.weight", {x->ssm_norm.size()}, x->ssm_norm);
            w.quant_tensor(p + "ssm_out.weight", x->ssm_out);
            ffn(x->ffn);
        } else {
            const auto &a = std::get<FullAttnLayerWeights>(t.w.layers[l]);
            w.f32_tensor(p + "attn_norm.weight", {d}, a.attn_norm);
            w.f32_tensor(p + "post_attention_norm.weight", {d}, a.post_attn_norm);
            w.quant_tensor(p + "attn_q.weight", a.wq);
            w.quant_tensor(p + "attn_k.weight", a.wk);
            w.quant_tensor(p + "attn_v.weight", a.wv);
            w.quant_tensor(p + "attn_output.weight", a.wo);
            w.f32_tensor(p + "attn_q_norm.weight", {a.q_norm.size()}, a.q_norm);
            w.f32_tensor(p + "attn_k_norm.weight", {a.k_norm.size()}, a.k_norm);
            ffn(a.ffn);
        }
    }
    return w.bytes(64);
}

static bool throws_code(const std::function<void()> &fn, int code) {
    try {
        fn();
    } catch (const Error &e) {
        return e.code == code;
    }
    return false;
}

int main(int argc, char **argv) {
    const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu-only") == 0;
    run("test_from_raw_checks_sizes", [] {
        bool threw = false;
        try {
            Q8Tensor::from_raw(std::vector<uint8_t>(33), 32, 1);
        } catch (const Error &e) {
            threw = e.code == ANEHIP_ESHAPE;
        }
        EXPECT(threw, "size mismatch must be rejected");
        threw = false;
        try {
            Q8Tensor::from_raw(std::vector<uint8_t>(34), 31, 1);
        } catch (const Error &e) {
            threw = e.code == ANEHIP_ESHAPE;
        }
        EXPECT(threw, "n %% 32 != 0 must be rejected");
    });

    run("test_greedy_sample_matches_total_cmp", [] {
        // ties (the last maximum wins), negatives, -0 vs +0, and a NaN ranked
        // by f32::total_cmp (positive NaN above +inf)
        const std::vector<std::vector<float>> cases = {
            {1.f, 3.f, 3.f, 2.f}, {-5.f, -1.f, -3.f}, {-0.f, 0.f, -0.f}, {1.f, INFINITY, NAN, 2.f}};
        for (const auto &c : cases)
            EXPECT(greedy_sample(c) == ao_argmax(c.data(), c.size()), "case of %zu", c.size());
        std::vector<float> r = normal(5, 1000, 0.f, 1.f);
        EXPECT(greedy_sample(r) == ao_argmax(r.data(), r.size()), "random logits");
    });
    run("test_gguf_metadata_and_tensors", [] {
        GgufWriter w;
        w.str("general.architecture", "qwen35");
        w.u32("qwen35.block_count", 7);
        w.f32("qwen35.rope.freq_base", 1e6f);
        w.str_array("tokenizer.ggml.tokens", {"a", "bb", "ccc"});
        // other value types: u8, i16, i64, f64, bool, an array of u32
        w.key("x.u8", 0), GgufWriter::put<uint8_t>(w.kv, 200);
        w.key("x.i16", 3), GgufWriter::put<int16_t>(w.kv, -300);
        w.key("x.i64", 11), GgufWriter::put<int64_t>(w.kv, -5);
        w.key("x.f64", 12), GgufWriter::put<double>(w.kv, 0.25);
        w.key("x.bool", 7), GgufWriter::put<uint8_t>(w.kv, 1);
        w.key("x.arr", 9), GgufWriter::put<uint32_t>(w.kv, 4), GgufWriter::put<uint64_t>(w.kv, 2),
            GgufWriter::put<uint32_t>(w.kv, 10), GgufWriter::put<uint32_t>(w.kv, 20);
        const std::vector<float> a = {1.f, -2.f, 3.5f};
        w.f32_tensor("a", {3}, a);
        w.tensor("h", {4}, 1, {0x00, 0x3c, 0x00, 0xc0, 0x01, 0x00, 0x00, 0x7c});  // 1, -2, 2^-24, +inf
        const std::vector<uint8_t> f = w.bytes(32);
        gguf::GgufFile g = gguf::GgufFile::parse(f.data(), f.size());
        EXPECT(g.version == 3 && g.tensors.size() == 2 && g.metadata.size() == 10, "header");
        EXPECT(g.architecture() && *g.architecture() == "qwen35", "architecture");
        uint32_t v = 0;
        float x = 0;
        EXPECT(g.arch_u32("block_count", v) && v == 7, "block_count %u", v);
        EXPECT(g.arch_f32("rope.freq_base", x) && x == 1e6f, "freq_base");
        EXPECT(!g.arch_u32("rope.freq_base", v), "an f32 key is not a u32 (as_u32 matches the type only)");
        EXPECT(g.vocab_size(v) && v == 3, "vocab %u", v);
        EXPECT(std::get<uint64_t>(g.metadata["x.u8"].v) == 200 && std::get<int64_t>(g.metadata["x.i16"].v) == -300 &&
                   std::get<int64_t>(g.metadata["x.i64"].v) == -5 && std::get<double>(g.metadata["x.f64"].v) == 0.25 &&
                   std::get<bool>(g.metadata["x.bool"].v) && g.metadata["x.arr"].as_array()->size() == 2,
               "value types");
        EXPECT((g.tensor_data_offset & 31) == 0 && g.get_tensor("h")->offset == 32, "alignment / offsets");
        EXPECT(gguf::extract_tensor_f32(g, f.data(), f.size(), "a") == a, "f32 tensor");
        const std::vector<float> h = gguf::extract_tensor_f32(g, f.data(), f.size(), "h");
        EXPECT(h[0] == 1.f && h[1] == -2.f && h[2] == std::ldexp(1.f, -24) && std::isinf(h[3]), "f16 tensor");
        EXPECT(!g.get_tensor("missing") &&
                   throws_code([&] { gguf::extract_tensor_f32(g, f.data(), f.size(), "missing"); }, ANEHIP_EINVAL),
               "a missing tensor is an error");
    });

    // dequant.rs:235-270 (the reference's only dequant known answers), and the
    // Q4_0 nibble order: byte 0x1F -> element i = (15 - 8) d, element i + 16 = (1 - 8) d
    run("test_gguf_dequant_known_answers", [] {
        std::vector<uint8_t> q8(34, 2);
        q8[0] = 0x00, q8[1] = 0x38;  // 0.5
        for (float v : gguf::dequantize_tensor(q8.data(), q8.size(), gguf::GgmlType::Q8_0, 32))
            EXPECT(v == 1.0f, "q8 %f", v);
        std::vector<uint8_t> q4(18, 0x88);
        q4[0] = 0x00, q4[1] = 0x3c;  // 1.0
        for (float v : gguf::dequantize_tensor(q4.data(), q4.size(), gguf::GgmlType::Q4_0, 32))
            EXPECT(v == 0.0f, "q4 %f", v);
        q4[2] = 0x1f;
        const std::vector<float> o = gguf::dequantize_tensor(q4.data(), q4.size(), gguf::GgmlType::Q4_0, 32);
        EXPECT(o[0] == 7.0f && o[16] == -7.0f, "nibble order %f %f", o[0], o[16]);
        // matches the oracle's block dequant on random blocks
        std::vector<uint8_t> r(ao_quant_bytes(8, 4, 64));
        ao_gen_quant(8, 3, 1, 0.02f, 4, 64, r.data());
        const std::vector<float> got = gguf::dequantize_tensor(r.data(), r.size(), gguf::GgmlType::Q8_0, 256);
        for (size_t b = 0; b < 8; b++) {
            float ref[32];
            ao_dequant_q8_0_block(&r[b * 34], ref);
            for (int i = 0; i < 32; i++) EXPECT(got[b * 32 + i] == ref[i], "block %zu elem %d", b, i);
        }
        EXPECT(throws_code([&] { gguf::dequantize_tensor(r.data(), r.size(), gguf::GgmlType::Q6K, 256); },
                           ANEHIP_EUNSUPPORTED) &&
                   throws_code([&] { gguf::dequantize_tensor(r.data(), 10, gguf::GgmlType::Q8_0, 256); }, ANEHIP_EINVAL),
               "unsupported type / short data");
    });

    run("test_gguf_rejects_malformed_files", [] {
        GgufWriter w;
        w.u32("general.alignment", 32);
        w.f32_tensor("a", {3}, {1.f, 2.f, 3.f});
        const std::vector<uint8_t> good = w.bytes();
        auto parse = [](std::vector<uint8_t> b) { gguf::GgufFile::parse(b.data(), b.size()); };
        std::vector<uint8_t> b = good;
        b[0] = 'X';
        EXPECT(throws_code([&] { parse(b); }, ANEHIP_EINVAL), "bad magic");
        b = good;
        b[4] = 1;
        EXPECT(throws_code([&] { parse(b); }, ANEHIP_EINVAL), "version 1");
        EXPECT(throws_code([&] { parse(std::vector<uint8_t>(good.begin(), good.begin() + 40)); }, ANEHIP_EINVAL),
               "truncated");
        GgufWriter u;
        u.key("k", 13);  // unknown value type
        EXPECT(throws_code([&] { parse(u.bytes()); }, ANEHIP_EINVAL), "unknown metadata type");
        GgufWriter t;
        t.tensor("q", {32}, 20, std::vector<uint8_t>(34));  // IQ4_NL: not a type the parser maps
        EXPECT(throws_code([&] { parse(t.bytes()); }, ANEHIP_EUNSUPPORTED), "unsupported tensor type");
        // a tensor whose data lies past the end of the file
        std::vector<uint8_t> cut = good;
        cut.resize(gguf::GgufFile::parse(good.data(), good.size()).tensor_data_offset + 4);
        gguf::GgufFile g = gguf::GgufFile::parse(cut.data(), cut.size());
        EXPECT(throws_code([&] { gguf::extract_tensor_f32(g, cut.data(), cut.size(), "a"); }, ANEHIP_EINVAL),
               "tensor past the end");
    });

    run("test_gguf_config_and_weights_of_the_tiny_model", [] {
        Tiny t = make_tiny();
        for (bool tied : {false, true}) {
            const std::vector<uint8_t> f = tiny_gguf(t, tied);
            // through a mapped file, as a checkpoint is read
            char path[] = "/tmp/ane_gguf_XXXXXX";
            const int fd = mkstemp(path);
            EXPECT(fd >= 0, "mkstemp");
            EXPECT(write(fd, f.data(), f.size()) == (ssize_t)f.size(), "write");
            close(fd);
            gguf::MappedFile mf(path);
            unlink(path);
            gguf::GgufFile g = gguf::GgufFile::parse(mf.data(), mf.size());
            Qwen35Config c = qwen35_config_from_gguf(g);
            const ModelConfig &b = c.base, &r = t.w.config.base;
            EXPECT(b.dim == r.dim && b.hidden_dim == r.hidden_dim && b.n_layers == r.n_layers &&
                       b.n_heads == r.n_heads && b.n_kv_heads == r.n_kv_heads && b.head_dim == r.head_dim &&
                       b.vocab_size == r.vocab_size && b.max_seq_len == r.max_seq_len,
                   "shape");
            EXPECT(c.layer_types == t.w.config.layer_types && c.ssm_group_count == t.w.config.ssm_group_count,
                   "layer types");
            Qwen35ModelWeights w = load_qwen35_q8(g, mf.data(), mf.size(), c);
            EXPECT(w.lm_head.data == t.w.lm_head.data && w.final_norm == t.w.final_norm, "model tensors");
            if (!tied) EXPECT(w.embedding == t.w.embedding, "embedding");
            const auto &d0 = std::get<DeltaNetLayerWeights>(w.layers[0]);
            const auto &r0 = std::get<DeltaNetLayerWeights>(t.w.layers[0]);
            EXPECT(d0.qkv.data == r0.qkv.data && d0.qkv.m == r0.qkv.m && d0.qkv.n == r0.qkv.n &&
                       d0.ssm_conv1d == r0.ssm_conv1d && d0.ssm_a == r0.ssm_a && d0.ffn.down.data == r0.ffn.down.data,
                   "DeltaNet layer");
            const auto &a3 = std::get<FullAttnLayerWeights>(w.layers[3]);
            const auto &r3 = std::get<FullAttnLayerWeights>(t.w.layers[3]);
            EXPECT(a3.wq.data == r3.wq.data && a3.wo.n == r3.wo.n && a3.k_norm == r3.k_norm, "attention layer");
        }
        ao_model_destroy(t.om);
    });

    if (cpu_only) {
        std::printf("%s (%d failed)\n", failures ? "FAILED" : "OK", failures);
        return failures ? 1 : 0;
    }

    GpuContext ctx = GpuContext::create();
    run("test_gpu_context_creation", [&] { EXPECT(ctx.raw() != nullptr, "no context"); });

    run("test_upload_weights", [&] {
        Q8Tensor t = make_q8_identity(4, 32);
        GpuBuffer b = ctx.upload_q8_weights(t);
        EXPECT(b.m == 4 && b.n == 32 && b.n_blocks == 1, "m=%zu n=%zu n_blocks=%u", b.m, b.n, b.n_blocks);
    });

    run("test_graph_single_gemv", [&] {
        GpuBuffer b = ctx.upload_q8_weights(make_q8_identity(4, 32));
        std::vector<float> x(32);
        for (int i = 0; i < 32; i++) x[i] = (float)i;
        ctx.write_scratch_input(x.data(), 32);
        GpuGraph graph(ctx);
        graph.add_gemv(GemvOp{b, 0, 0, 32, 4});
        graph.execute();
        float y[4];
        ctx.read_scratch_output(y, 4);
        for (int i = 0; i < 4; i++) EXPECT(std::fabs(y[i] - (float)i) < 0.01f, "y[%d] = %f", i, y[i]);
    });

    // test_q8_gemv_parallel (q8_gemv.rs:283-314) on the GPU graph, replayed
    // over new inputs (the first execute records, later ones replay)
    run("test_q8_gemv_parallel_graph_replays", [&] {
        const size_t m = 256, n = 1024;
        GpuBuffer b = ctx.upload_q8_weights(make_patterned(m, n));
        GpuGraph graph(ctx);
        graph.add_gemv_raw(b, 0, 0, n, m);
        for (int rep = 0; rep < 4; rep++) {
            std::vector<float> x(n);
            for (size_t i = 0; i < n; i++) x[i] = (float)((i + 13 * rep) % 100);
            ctx.write_scratch_input(x.data(), n);
            graph.execute();
            std::vector<float> y(m);
            ctx.read_scratch_output(y.data(), m);
            for (size_t r = 0; r < m; r++) {
                double ref = 0;
                for (size_t k = 0; k < n; k++) ref += 0.5 * (double)pattern_q(r, k % 32) * x[k];
                EXPECT(std::fabs(y[r] - ref) < 1e-3, "rep %d row %zu: %f vs %f", rep, r, y[r], ref);
            }
        }
    });

    run("test_graph_gemv_then_silu_mul", [&] {
        const size_t m = 512, n = 256;
        GpuBuffer b = ctx.upload_q8_weights(quant(900, m, n));
        std::vector<float> x = normal(901, n, 0.f, 1.f);
        ctx.write_scratch_input(x.data(), n);
        GpuGraph graph(ctx);
        graph.add_gemv(GemvOp{b, 0, 0, n, m});
        graph.add_silu_mul(SiluMulOp{0, m / 2, m / 2});
        graph.execute();
        std::vector<float> y(m / 2), gu(m);
        ctx.read_scratch_output(y.data(), m / 2);
        Q8Tensor t = quant(900, m, n);
        ao_quant_gemv(8, t.data.data(), m, n, x.data(), gu.data());
        ao_silu_mul_inplace(gu.data(), gu.data() + m / 2, m / 2);
        double num = 0, den = 0;
        for (size_t i = 0; i < m / 2; i++) num += (y[i] - gu[i]) * (y[i] - gu[i]), den += gu[i] * gu[i];
        EXPECT(std::sqrt(num / den) < 1e-4, "rel l2 %g", std::sqrt(num / den));
    });

    run("test_encode_full_token_gpu_matches_oracle", [&] {
        Tiny t = make_tiny();
        GpuModelWeights g = upload_model_weights(ctx, t.w);
        GpuLayerScratch scratch(256, 512, 768, 2);
        GpuConstantPool pool(256, 512, 768, 2, 128, 4, 1e-6f, 4, 1, 256, 10000.f);
        ao_seq *seq = ao_seq_create(t.om, 64, 1);
        std::vector<float> ref(1000);
        uint32_t tok = 17;
        for (int step = 0; step < 6; step++) {
            std::vector<float> logits = encode_full_token_gpu(ctx, t.w, g, scratch, pool, tok);
            ao_forward_token(t.om, seq, tok, ref.data(), 0);
            double num = 0, den = 0;
            for (size_t i = 0; i < 1000; i++) num += (logits[i] - ref[i]) * (logits[i] - ref[i]), den += ref[i] * ref[i];
            const double rel = std::sqrt(num / den);
            std::printf("    step %d token %u rel_l2 %.2e\n", step, tok, rel);
            EXPECT(rel < 1e-3, "step %d", step);
            EXPECT(scratch.pos == (size_t)step + 1, "pos %zu", scratch.pos);
            tok = greedy_sample(logits);
            EXPECT(tok == ao_argmax(ref.data(), 1000), "greedy choice differs from the oracle's");
        }
        ao_seq_destroy(seq);
        ao_model_destroy(t.om);
    });

    // load_qwen35_q8 from a GGUF file, uploaded and stepped: the same logits
    // bits as the weights uploaded directly, and the oracle's within 1e-3
    run("test_gguf_model_decodes_like_the_direct_upload", [&] {
        Tiny t = make_tiny();
        const std::vector<uint8_t> f = tiny_gguf(t, false);
        gguf::GgufFile g = gguf::GgufFile::parse(f.data(), f.size());
        Qwen35ModelWeights w = load_qwen35_q8(g, f.data(), f.size(), qwen35_config_from_gguf(g));
        GpuModelWeights gd = upload_model_weights(ctx, t.w), gg = upload_model_weights(ctx, w);
        GpuLayerScratch sd(256, 512, 768, 2), sg(256, 512, 768, 2);
        GpuConstantPool pool(256, 512, 768, 2, 128, 4, 1e-6f, 4, 1, 256, 10000.f);
        ao_seq *seq = ao_seq_create(t.om, 64, 1);
        std::vector<float> ref(1000);
        uint32_t tok = 5;
        for (int step = 0; step < 4; step++) {
            const std::vector<float> a = encode_full_token_gpu(ctx, t.w, gd, sd, pool, tok);
            const std::vector<float> b = encode_full_token_gpu(ctx, w, gg, sg, pool, tok);
            EXPECT(a == b, "step %d: logits differ from the direct upload", step);
            ao_forward_token(t.om, seq, tok, ref.data(), 0);
            double num = 0, den = 0;
            for (size_t i = 0; i < 1000; i++) num += (b[i] - ref[i]) * (b[i] - ref[i]), den += ref[i] * ref[i];
            EXPECT(std::sqrt(num / den) < 1e-3, "step %d rel_l2 %g", step, std::sqrt(num / den));
            tok = greedy_sample(b);
        }
        ao_seq_destroy(seq);
        ao_model_destroy(t.om);
    });

    std::printf("%s (%d failed)\n", failures ? "FAILED" : "OK", failures);
    return failures ? 1 : 0;
}
