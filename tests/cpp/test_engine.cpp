// Tests of the C++ engine API (ane-infer_amd/engine), named and shaped after
// the reference's own tests of the API it mirrors:
//   test_gpu_context_creation / test_upload_weights / test_graph_single_gemv
//     crates/engine/src/metal_graph.rs:543-594
//   test_q8_gemv_identity / test_q8_gemv_parallel   crates/engine/src/q8_gemv.rs:257-314
// plus the SiLU-mul graph op, graph replays over new inputs, the from_raw
// shape checks, and encode_full_token_gpu on a tiny seeded hybrid model
// against the CPU oracle (test infrastructure, oracle/ane_oracle.h).
// Prints one line per test; exit status 0 iff all pass.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "ane_engine.hpp"
#include "ane_oracle.h"

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

    std::printf("%s (%d failed)\n", failures ? "FAILED" : "OK", failures);
    return failures ? 1 : 0;
}
