// decode.hip — model weights, per-sequence state and the decode step.
//
// Replaces upload_model_weights (crates/engine/src/gpu_decode.rs:152-283),
// GpuLayerScratch / GpuConstantPool (gpu_full_decode.rs:18-217) and
// encode_full_token_gpu (gpu_full_decode.rs:221-1044), whose CPU counterpart
// is qwen35_forward_token (crates/cli/src/main.rs:953-1023).
//
// Differences from the reference design, all deliberate:
//   * one hipGraph per step (captured once per state allocation) replaces the
//     per-token command buffer with its ~506 encodes and ~150 buffer
//     allocations; every per-step scalar (token ids, positions) is read from
//     device memory, and a tail kernel advances the positions, so the graph
//     is replayed unchanged;
//   * projections that read the same input are stored stacked in one matrix
//     ([qkv; attn_gate; ssm_beta; ssm_alpha], [wq; wk; wv], [ffn_gate;
//     ffn_up]) so each is one streaming pass over its weights;
//   * residual adds, the next layer's RMSNorm and SiLU-mul are fused into the
//     kernel that also reduces the K-split GEMV partials;
//   * state is per sequence ([batch] leading dim), so batch 1..32 decodes
//     independent sequences (the reference is batch-1 only);
//   * the KV cache is fp16 (RNE), [kv_head][max_seq][head_dim] per sequence;
//   * positions are range-checked (the reference writes past the KV buffer
//     when pos >= max_seq, gpu_full_decode.rs:805).
#include "common.h"

#include <algorithm>

#include <cmath>
#include <cstring>

using namespace anehip;

namespace {

constexpr uint32_t kDk = 128;
constexpr uint32_t kConvK = 4;
constexpr uint32_t kHd = 256;

// A quantised matrix: GGUF blocks (d, as uploaded) and, once a step has run,
// its panel copy (p) that the step's GEMV / GEMM kernels read; `stale` marks
// a panel copy that has to be rebuilt from d before the next step.
// A stacked quantised matrix: d = GGUF blocks (as uploaded), p = the panel
// copy the step reads.  d is freed once p is built, unless a caller holds a
// pointer into it (anehip_tensor_ptr: keep); it is rebuilt from p by the
// inverse permutation when a later upload or tensor_ptr needs it.
struct QMat {
    void *d = nullptr, *p = nullptr;
    uint32_t type = 0, rows = 0, cols = 0;
    uint32_t il = 0;  // > 0: a stacked [gate; up] matrix of il features each, its panel rows interleaved
    bool stale = true;
    bool keep = false;
};

struct Layer {
    uint32_t type = 0;
    QMat mix_in, mix_out, ffn_gu, ffn_down;
    float *attn_norm = nullptr, *post_attn_norm = nullptr;
    float *ssm_a = nullptr, *conv1d = nullptr, *dt_bias = nullptr, *ssm_norm = nullptr;
    float *q_norm = nullptr, *k_norm = nullptr;
    uint64_t have = 0;  // bit per uploaded kind
    // state
    float *conv_state = nullptr, *S = nullptr;
    __half *kc = nullptr, *vc = nullptr;
};

}  // namespace

// Tokens per prefill chunk: the rows of the chunk's GEMMs (launched per
// 32-row group) and of its element-wise, DeltaNet and attention kernels.
constexpr uint32_t kPrefillRows = 256;
constexpr uint32_t kPrefillGroups = kPrefillRows / 32;

struct Model {
    anehip_model_desc desc{};
    std::vector<uint8_t> types;
    std::vector<Layer> layers;
    float *embedding = nullptr, *final_norm = nullptr;
    QMat lm_head;
    uint64_t glob_have = 0;
    float *inv_freq = nullptr;
    uint32_t rows_dn = 0, rows_attn = 0;  // stacked mix_in rows
    // state
    uint32_t batch = 0, max_seq = 0;
    std::vector<uint32_t> host_pos;
    uint32_t *d_pos = nullptr, *d_tokens = nullptr, *d_sampled = nullptr;
    // sampled tokens by (sequence, position of the step's input): [batch][max_seq]
    uint32_t *d_hist = nullptr;
    uint32_t *h_tokens = nullptr;  // pinned staging
    // scratch
    float *x0 = nullptr, *x1 = nullptr;                  // residual stream (two buffers, alternating)
    float *pmix = nullptr, *p0 = nullptr, *p1 = nullptr;  // GEMV outputs as K-split partial slices
    float *heads = nullptr, *attn_out = nullptr, *logits = nullptr, *attn_part = nullptr;
    // batch 1 with the fused DeltaNet + ssm_out kernel: the DeltaNet layers'
    // pending state updates (kDnPendFloats each, in layer order), committed
    // by one apply launch at the end of the step; null otherwise
    float *dn_pend = nullptr;
    // batch > 1: the residual norms' per-row sums of squares when their
    // scale is left to the consuming GEMM (Planes::rs), [32][kMaxRsParts]
    float *norm_ss = nullptr;
    float *xin = nullptr;        // GEMM input planes (batch > 1): hi then lo, xin_len halves each,
                                 // then the group exponents (xe_cnt bytes)
    size_t xin_len = 0;          // fragment-order plane of the widest GEMM input (32 rows)
    size_t xe_cnt = 0;
    size_t part_len = 0;         // floats per partial buffer
    void *argmax_ws = nullptr;
    // prefill scratch for chunks of up to kPrefillRows tokens of one sequence
    // (allocated by the first anehip_prefill; rows = tokens)
    struct {
        float *x = nullptr, *xn = nullptr, *pmix = nullptr, *p0 = nullptr, *p1 = nullptr, *attn_part = nullptr;
        float *logits = nullptr;
        _Float16 *xin = nullptr;  // planes: hi then lo, xin_len halves each, then xe_cnt exponents
        uint32_t *d_tokens = nullptr, *d_pos = nullptr;
    } pf;
    static Planes planes_at(void *base, size_t len) {
        Planes p;
        p.hi = static_cast<_Float16 *>(base);
        p.lo = p.hi + len;
        p.xe = reinterpret_cast<int8_t *>(p.lo + len);
        return p;
    }
    size_t planes_bytes() const { return 2 * xin_len * sizeof(_Float16) + xe_cnt; }
    Planes planes() const { return planes_at(xin, xin_len); }
    // prefill: kPrefillGroups 32-row planes of each (Planes::group)
    size_t pf_planes_bytes() const { return kPrefillGroups * planes_bytes(); }
    Planes pf_planes() const { return planes_at(pf.xin, kPrefillGroups * xin_len); }
    // graph
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool use_graph = true;
    // prefill: graph of one full chunk (kPrefillRows tokens, no logits) of
    // sequence pf_graph_seq, and pinned staging of a call's token / position
    // rows ([chunk][tokens | positions], kPrefillRows each)
    hipGraph_t pf_graph = nullptr;
    hipGraphExec_t pf_exec = nullptr;
    uint32_t pf_graph_seq = 0;
    uint32_t *pf_stage = nullptr;
    size_t pf_stage_chunks = 0;
};

namespace {

size_t qrow_bytes(uint32_t type, uint32_t cols) {
    return (size_t)(cols / 32) * (type == ANEHIP_GGML_Q8_0 ? 34 : 18);
}

void free_ptr(void *p) {
    if (p) (void)hipFree(p);
}

void drop_graph(Model *M) {
    if (M->exec) (void)hipGraphExecDestroy(M->exec);
    if (M->graph) (void)hipGraphDestroy(M->graph);
    if (M->pf_exec) (void)hipGraphExecDestroy(M->pf_exec);
    if (M->pf_graph) (void)hipGraphDestroy(M->pf_graph);
    M->exec = M->pf_exec = nullptr;
    M->graph = M->pf_graph = nullptr;
}

void free_state(Model *M) {
    drop_graph(M);
    for (Layer &L : M->layers) {
        free_ptr(L.conv_state);
        free_ptr(L.S);
        free_ptr(L.kc);
        free_ptr(L.vc);
        L.conv_state = L.S = nullptr;
        L.kc = L.vc = nullptr;
    }
    void *bufs[] = {M->d_pos, M->d_tokens, M->d_sampled, M->d_hist,    M->x0,        M->x1,  M->pmix,   M->p0,
                    M->p1,    M->heads,    M->attn_out,  M->logits, M->attn_part, M->argmax_ws, M->xin, M->dn_pend,
                    M->norm_ss};
    for (void *p : bufs) free_ptr(p);
    void *pfb[] = {M->pf.x, M->pf.xn, M->pf.pmix, M->pf.p0, M->pf.p1, M->pf.attn_part, M->pf.logits, M->pf.xin,
                   M->pf.d_tokens, M->pf.d_pos};
    for (void *p : pfb) free_ptr(p);
    M->pf = {};
    if (M->h_tokens) (void)hipHostFree(M->h_tokens);
    if (M->pf_stage) (void)hipHostFree(M->pf_stage);
    M->pf_stage = nullptr;
    M->pf_stage_chunks = 0;
    M->d_pos = M->d_tokens = M->d_sampled = M->d_hist = M->h_tokens = nullptr;
    M->x0 = M->x1 = M->pmix = M->p0 = M->p1 = M->heads = M->attn_out = M->logits = M->attn_part = nullptr;
    M->xin = nullptr;
    M->dn_pend = nullptr;
    M->norm_ss = nullptr;
    M->argmax_ws = nullptr;
    M->batch = M->max_seq = 0;
    M->host_pos.clear();
}

// Expected shape of a kind: {rows, cols, is_quant}; rows == 0 means the kind
// does not belong to this layer type.
struct KindShape {
    uint32_t rows, cols;
    bool quant;
};

KindShape kind_shape(const Model *M, int layer, uint32_t kind) {
    const anehip_model_desc &D = M->desc;
    const uint32_t d = D.dim, F = D.hidden_dim, H = D.ssm_group_count, C = 3 * d;
    const uint32_t qd = D.n_heads * D.head_dim, kvd = D.n_kv_heads * D.head_dim;
    if (layer < 0) {
        switch (kind) {
            case ANEHIP_T_EMBEDDING: return {D.vocab_size, d, false};
            case ANEHIP_T_FINAL_NORM: return {1, d, false};
            case ANEHIP_T_LM_HEAD: return {D.vocab_size, d, true};
            default: return {0, 0, false};
        }
    }
    const bool dn = M->types[layer] == ANEHIP_LAYER_DELTANET;
    switch (kind) {
        case ANEHIP_T_ATTN_NORM:
        case ANEHIP_T_POST_ATTN_NORM: return {1, d, false};
        case ANEHIP_T_FFN_GATE:
        case ANEHIP_T_FFN_UP: return {F, d, true};
        case ANEHIP_T_FFN_DOWN: return {d, F, true};
        default: break;
    }
    if (dn) {
        switch (kind) {
            case ANEHIP_T_QKV: return {C, d, true};
            case ANEHIP_T_ATTN_GATE: return {d, d, true};
            case ANEHIP_T_SSM_A:
            case ANEHIP_T_SSM_DT_BIAS: return {1, H, false};
            case ANEHIP_T_SSM_ALPHA:
            case ANEHIP_T_SSM_BETA: return {H, d, true};
            case ANEHIP_T_SSM_CONV1D: return {C, D.ssm_conv_kernel, false};
            case ANEHIP_T_SSM_NORM: return {1, D.ssm_state_size, false};
            case ANEHIP_T_SSM_OUT: return {d, d, true};
            default: return {0, 0, false};
        }
    }
    switch (kind) {
        case ANEHIP_T_WQ: return {2 * qd, d, true};
        case ANEHIP_T_WK:
        case ANEHIP_T_WV: return {kvd, d, true};
        case ANEHIP_T_WO: return {d, qd, true};
        case ANEHIP_T_Q_NORM:
        case ANEHIP_T_K_NORM: return {1, D.head_dim, false};
        default: return {0, 0, false};
    }
}

uint64_t required_mask(const Model *M, int layer) {
    uint64_t m = 0;
    for (uint32_t k = 0; k < ANEHIP_T_COUNT; k++)
        if (kind_shape(M, layer, k).rows) m |= 1ull << k;
    return m;
}

const char *kind_name(uint32_t k) {
    static const char *names[] = {"attn_norm", "post_attn_norm", "ffn_gate", "ffn_up", "ffn_down", "qkv",
                                  "attn_gate", "ssm_a", "ssm_alpha", "ssm_beta", "ssm_conv1d", "ssm_dt_bias",
                                  "ssm_norm", "ssm_out", "wq", "wk", "wv", "wo", "q_norm", "k_norm",
                                  "embedding", "final_norm", "lm_head"};
    return k < ANEHIP_T_COUNT ? names[k] : "?";
}

// Where a quant kind lives: target matrix, its total rows, row offset.
struct QSlot {
    QMat *mat;
    uint32_t total_rows, row_off;
};

QSlot quant_slot(Model *M, int layer, uint32_t kind) {
    const anehip_model_desc &D = M->desc;
    if (layer < 0) return {&M->lm_head, D.vocab_size, 0};
    Layer &L = M->layers[layer];
    const uint32_t d = D.dim, F = D.hidden_dim, H = D.ssm_group_count, C = 3 * d;
    const uint32_t qd2 = 2 * D.n_heads * D.head_dim, kvd = D.n_kv_heads * D.head_dim;
    switch (kind) {
        case ANEHIP_T_FFN_GATE: return {&L.ffn_gu, 2 * F, 0};
        case ANEHIP_T_FFN_UP: return {&L.ffn_gu, 2 * F, F};
        case ANEHIP_T_FFN_DOWN: return {&L.ffn_down, d, 0};
        case ANEHIP_T_QKV: return {&L.mix_in, M->rows_dn, 0};
        case ANEHIP_T_ATTN_GATE: return {&L.mix_in, M->rows_dn, C};
        case ANEHIP_T_SSM_BETA: return {&L.mix_in, M->rows_dn, C + d};
        case ANEHIP_T_SSM_ALPHA: return {&L.mix_in, M->rows_dn, C + d + H};
        case ANEHIP_T_SSM_OUT: return {&L.mix_out, d, 0};
        case ANEHIP_T_WQ: return {&L.mix_in, M->rows_attn, 0};
        case ANEHIP_T_WK: return {&L.mix_in, M->rows_attn, qd2};
        case ANEHIP_T_WV: return {&L.mix_in, M->rows_attn, qd2 + kvd};
        case ANEHIP_T_WO: return {&L.mix_out, d, 0};
        default: return {nullptr, 0, 0};
    }
}

float **f32_slot(Model *M, int layer, uint32_t kind) {
    if (layer < 0) {
        if (kind == ANEHIP_T_EMBEDDING) return &M->embedding;
        if (kind == ANEHIP_T_FINAL_NORM) return &M->final_norm;
        return nullptr;
    }
    Layer &L = M->layers[layer];
    switch (kind) {
        case ANEHIP_T_ATTN_NORM: return &L.attn_norm;
        case ANEHIP_T_POST_ATTN_NORM: return &L.post_attn_norm;
        case ANEHIP_T_SSM_A: return &L.ssm_a;
        case ANEHIP_T_SSM_CONV1D: return &L.conv1d;
        case ANEHIP_T_SSM_DT_BIAS: return &L.dt_bias;
        case ANEHIP_T_SSM_NORM: return &L.ssm_norm;
        case ANEHIP_T_Q_NORM: return &L.q_norm;
        case ANEHIP_T_K_NORM: return &L.k_norm;
        default: return nullptr;
    }
}

int check_model(anehip_ctx *ctx, Model *M) {
    for (uint32_t l = 0; l < M->desc.n_layers; l++) {
        uint64_t miss = required_mask(M, (int)l) & ~M->layers[l].have;
        if (miss) {
            uint32_t k = (uint32_t)__builtin_ctzll(miss);
            return set_error(ctx->err, ANEHIP_ESTATE, "layer %u: tensor %s not uploaded", l, kind_name(k));
        }
    }
    uint64_t miss = required_mask(M, -1) & ~M->glob_have;
    if (miss)
        return set_error(ctx->err, ANEHIP_ESTATE, "model tensor %s not uploaded",
                         kind_name((uint32_t)__builtin_ctzll(miss)));
    if (!M->batch) return set_error(ctx->err, ANEHIP_ESTATE, "no state: call anehip_alloc_state first");
    return ANEHIP_OK;
}

#define TRY(expr)                   \
    do {                            \
        int _rc = (expr);           \
        if (_rc) return _rc;        \
    } while (0)

// Batch 1: every projection is one GEMV launch whose prologue forms its input
// (embedding / residual sum + RMSNorm, gated RMSNorm, SiLU-mul, the
// attention's chunk merge) from what the previous kernels left, so a DeltaNet
// layer is 5 launches (mixer-in GEMV, DeltaNet, ssm_out GEMV, gate/up GEMV,
// down GEMV) and so is an attention layer when o_proj has one head per split.
int enqueue_step_b1(anehip_ctx *ctx, Model *M, hipStream_t s) {
    const anehip_model_desc &D = M->desc;
    const uint32_t d = D.dim, F = D.hidden_dim, H = D.ssm_group_count, C = 3 * d;
    const uint32_t qd = D.n_heads * D.head_dim;
    const float eps = D.rms_norm_eps;
    float *cur = M->x0, *nxt = M->x1;
    const float *prev_part = nullptr;
    int prev_kp = 0;
    DnApplyTab tab;  // the fused DeltaNet layers' pending updates
    for (uint32_t l = 0; l < D.n_layers; l++) {
        Layer &L = M->layers[l];
        const bool dn = L.type == ANEHIP_LAYER_DELTANET;
        const uint32_t rows_in = dn ? M->rows_dn : M->rows_attn;
        // 1. mixer input projections, input = RMSNorm(residual)
        GemvInput in1;
        in1.mode = l == 0 ? GEMV_IN_EMBED_RMSNORM : GEMV_IN_RESID_RMSNORM;
        in1.x = cur;
        in1.part = prev_part;
        in1.kp = prev_kp;
        in1.part_stride = d;
        in1.w = L.attn_norm;
        in1.eps = eps;
        in1.x_out = nxt;
        in1.token = M->d_tokens;
        in1.emb = M->embedding;
        in1.vocab = D.vocab_size;
        const int k1 = gemv_packed_ksplit(ctx, rows_in, d, GEMV_IN_RESID_RMSNORM);
        TRY(launch_gemv_packed(ctx, s, L.mix_in.type, L.mix_in.p, rows_in, d, in1, M->pmix, k1));
        std::swap(cur, nxt);
        MixIn mix;
        mix.p = M->pmix;
        mix.kp = k1;
        mix.split = rows_in;
        mix.stride = (int)rows_in;
        // 2. mixer core, 3. output projection (its input formed in the prologue)
        GemvInput in3;
        uint32_t cols3;
        if (dn && M->dn_pend) {
            // DeltaNet step fused into ssm_out; its state update is committed
            // after the last layer (launch_deltanet_apply)
            float *pend = M->dn_pend + (size_t)tab.n * kDnPendFloats(d, H);
            TRY(launch_dn_ssm(ctx, s, L.mix_out.type, L.mix_out.p, d, H, mix, L.conv1d, L.conv_state, L.ssm_a,
                              L.dt_bias, L.S, L.ssm_norm, eps, pend, M->p0));
            tab.S[tab.n] = L.S;
            tab.conv[tab.n] = L.conv_state;
            tab.pend[tab.n] = pend;
            tab.n++;
            cols3 = d;
        } else if (dn) {
            TRY(launch_deltanet_step(ctx, s, 1, (int)H, mix, mix.shifted((int)(C + d)), mix.shifted((int)(C + d + H)),
                                     L.conv1d, L.ssm_a, L.dt_bias, L.conv_state, L.S, M->heads));
            in3.mode = GEMV_IN_GATED_NORM;
            in3.x = M->heads;
            in3.part = M->pmix;
            in3.kp = k1;
            in3.part_stride = rows_in;
            in3.w = L.ssm_norm;
            in3.eps = eps;
            in3.gate_off = (int)C;
            in3.conv_state = L.conv_state;
            cols3 = d;
        } else {
            cols3 = qd;
            // with one head per K split the o_proj prologue merges the
            // attention's chunk partials (no combine kernel)
            const bool fuse = gemv_packed_ksplit(ctx, d, cols3) == (int)(qd / 256);
            TRY(launch_attention(ctx, s, 1, (int)D.n_heads, (int)D.n_kv_heads, (int)M->max_seq, mix, L.q_norm,
                                 L.k_norm, M->inv_freq, M->d_pos, L.kc, L.vc, M->attn_part,
                                 fuse ? nullptr : M->attn_out, Planes{}));
            if (fuse) {
                const int G = (int)(D.n_heads / D.n_kv_heads);
                const int nch = attn_chunks((int)M->max_seq, 1, (int)D.n_kv_heads);
                in3.mode = GEMV_IN_ATTN_COMBINE;
                in3.part = M->pmix;
                in3.kp = k1;
                in3.part_stride = rows_in;
                in3.att_o = M->attn_part;
                in3.att_ml = M->attn_part + (size_t)D.n_kv_heads * nch * G * 256;
                in3.att_nch = nch;
                in3.att_g = G;
                in3.att_pos = M->d_pos;
            } else {
                in3.mode = GEMV_IN_PLAIN;
                in3.x = M->attn_out;
            }
        }
        const int k3 = dn && M->dn_pend ? (int)(d / 256) : gemv_packed_ksplit(ctx, d, cols3);
        if (!(dn && M->dn_pend)) TRY(launch_gemv_packed(ctx, s, L.mix_out.type, L.mix_out.p, d, cols3, in3, M->p0, k3));
        // 4. FFN gate/up, input = RMSNorm(residual + mixer output)
        GemvInput in4;
        in4.mode = GEMV_IN_RESID_RMSNORM;
        in4.x = cur;
        in4.part = M->p0;
        in4.kp = k3;
        in4.part_stride = d;
        in4.w = L.post_attn_norm;
        in4.eps = eps;
        in4.x_out = nxt;
        const int k4 = gemv_packed_ksplit(ctx, 2 * F, d, GEMV_IN_RESID_RMSNORM);
        TRY(launch_gemv_packed(ctx, s, L.ffn_gu.type, L.ffn_gu.p, 2 * F, d, in4, M->p1, k4));
        std::swap(cur, nxt);
        // 5. FFN down, input = SiLU(gate) * up
        GemvInput in5;
        in5.mode = GEMV_IN_SILU_MUL;
        in5.part = M->p1;
        in5.kp = k4;
        in5.part_stride = 2 * F;
        const int k5 = gemv_packed_ksplit(ctx, d, F, GEMV_IN_SILU_MUL);
        TRY(launch_gemv_packed(ctx, s, L.ffn_down.type, L.ffn_down.p, d, F, in5, M->p0, k5));
        prev_part = M->p0;
        prev_kp = k5;
    }
    if (tab.n) TRY(launch_deltanet_apply(ctx, s, tab, (int)H, (int)d));
    // lm_head, input = final RMSNorm(residual + last FFN output), formed once
    // by its own kernel: as a prologue each of the lm_head's ~1200 workgroups
    // would re-read the residual and every partial slice (measured 19 us)
    TRY(launch_residual_rmsnorm(ctx, s, 1, (int)d, cur, prev_part, prev_kp, M->final_norm, M->heads, eps));
    GemvInput inf;
    inf.mode = GEMV_IN_PLAIN;
    inf.x = M->heads;
    const int kf = gemv_packed_ksplit(ctx, D.vocab_size, d);
    if (kf == 1) {
        TRY(launch_gemv_packed(ctx, s, M->lm_head.type, M->lm_head.p, D.vocab_size, d, inf, M->logits, 1));
    } else {
        TRY(launch_gemv_packed(ctx, s, M->lm_head.type, M->lm_head.p, D.vocab_size, d, inf, M->pmix, kf));
        TRY(launch_sum_partials(ctx, s, M->pmix, M->logits, D.vocab_size, kf));
    }
    return ANEHIP_OK;
}

// Batch 2..32: element-wise kernels (residual + RMSNorm, gated norm, SiLU-mul,
// attention combine) write the next GEMM's input as fp16 hi / lo planes;
// projections run on the panel MFMA GEMM.
int enqueue_step_bn(anehip_ctx *ctx, Model *M, hipStream_t s) {
    const anehip_model_desc &D = M->desc;
    const int B = (int)M->batch;
    const uint32_t d = D.dim, F = D.hidden_dim, H = D.ssm_group_count, C = 3 * d;
    const uint32_t qd = D.n_heads * D.head_dim;
    const float eps = D.rms_norm_eps;
    const Planes xp = M->planes();  // GEMM input planes
    // The residual norms whose consumer is the 17..32-row x-stationary GEMM
    // write r (.) w planes and leave the scale to it (Planes::rs): one wave
    // per 256 columns of a row, so that a row's partial slices are read by
    // 8 CUs instead of one.  Measured on MI355X, batch 32, ctx 1k, the same
    // box: 1.592-1.597 ms per step against 1.636-1.638 with the full-row
    // norm kernel (the deferred scale costs the gate / up product a little).
    Planes xs = xp;
    xs.rs = M->norm_ss;
    xs.rs_parts = (int)(d / 256);
    xs.rs_eps = eps;
    const bool parts_ok = M->norm_ss && d % 256 == 0 && d / 256 <= (uint32_t)kMaxRsParts;
    float *x = M->x0;
    // the planes of the next mixer input carry a deferred scale
    bool in_scaled = parts_ok && gemm_takes_norm_scale(ctx, M->layers[0].type == ANEHIP_LAYER_DELTANET ? M->rows_dn
                                                                                                       : M->rows_attn,
                                                       d, B);
    if (in_scaled)
        TRY(launch_embed_rmsnorm_parts(ctx, s, B, (int)d, M->d_tokens, M->embedding, D.vocab_size, x,
                                       M->layers[0].attn_norm, xs));
    else
        TRY(launch_embed_rmsnorm(ctx, s, B, (int)d, M->d_tokens, M->embedding, D.vocab_size, x,
                                 M->layers[0].attn_norm, nullptr, eps, xp));
    for (uint32_t l = 0; l < D.n_layers; l++) {
        Layer &L = M->layers[l];
        const bool dn = L.type == ANEHIP_LAYER_DELTANET;
        const uint32_t rows_in = dn ? M->rows_dn : M->rows_attn;
        const int k1 = gemm_packed_ksplit(ctx, rows_in, d, B);
        TRY(launch_gemm_packed(ctx, s, L.mix_in.type, L.mix_in.p, rows_in, d, in_scaled ? xs : xp, B, M->pmix, k1));
        MixIn mix;
        mix.p = M->pmix;
        mix.kp = k1;
        mix.split = (size_t)B * rows_in;
        mix.stride = (int)rows_in;
        uint32_t cols3;
        if (dn) {
            TRY(launch_deltanet_head(ctx, s, B, (int)H, mix, mix.shifted((int)(C + d)), mix.shifted((int)(C + d + H)),
                                     L.conv1d, L.ssm_a, L.dt_bias, L.conv_state, L.S, nullptr, (int)C, L.ssm_norm,
                                     eps, xp));
            cols3 = d;
        } else {
            TRY(launch_attention(ctx, s, B, (int)D.n_heads, (int)D.n_kv_heads, (int)M->max_seq, mix, L.q_norm,
                                 L.k_norm, M->inv_freq, M->d_pos, L.kc, L.vc, M->attn_part, nullptr, xp));
            cols3 = qd;
        }
        const int k3 = gemm_packed_ksplit(ctx, d, cols3, B);
        TRY(launch_gemm_packed(ctx, s, L.mix_out.type, L.mix_out.p, d, cols3, xp, B, M->p0, k3));
        const int k5 = gemm_packed_ksplit(ctx, d, F, B);
        const bool silu_fused = gemm_gate_up_silu_ok(ctx, 2 * F, d, B) && gemm_is_xs(ctx, d, F, B);
        const bool ffn_scaled = parts_ok && (silu_fused || gemm_takes_norm_scale(ctx, 2 * F, d, B));
        if (ffn_scaled)
            TRY(launch_residual_rmsnorm_parts(ctx, s, B, (int)d, x, M->p0, k3, L.post_attn_norm, xs));
        else
            TRY(launch_residual_rmsnorm(ctx, s, B, (int)d, x, M->p0, k3, L.post_attn_norm, nullptr, eps, xp));
        const Planes &xf = ffn_scaled ? xs : xp;
        if (silu_fused) {
            // the SiLU-mul in the gate / up product's epilogue (h as fp32
            // rows in p1), the down product splitting those rows itself:
            // one launch less per layer
            TRY(launch_gemm_gate_up_silu(ctx, s, L.ffn_gu.type, L.ffn_gu.p, 2 * F, d, xf, B, M->p1));
            TRY(launch_gemm_xs_rows(ctx, s, L.ffn_down.type, L.ffn_down.p, d, F, M->p1, B, M->p0));
        } else {
            const int k4 = gemm_packed_ksplit(ctx, 2 * F, d, B);
            TRY(launch_gemm_packed(ctx, s, L.ffn_gu.type, L.ffn_gu.p, 2 * F, d, xf, B, M->p1, k4));
            TRY(launch_silu_mul_stacked(ctx, s, B, (int)F, M->p1, k4, nullptr, xp));
            TRY(launch_gemm_packed(ctx, s, L.ffn_down.type, L.ffn_down.p, d, F, xp, B, M->p0, k5));
        }
        const bool last = l + 1 == D.n_layers;
        const float *next_norm = last ? M->final_norm : M->layers[l + 1].attn_norm;
        const uint32_t next_rows = last ? D.vocab_size
                                        : M->layers[l + 1].type == ANEHIP_LAYER_DELTANET ? M->rows_dn : M->rows_attn;
        in_scaled = parts_ok && gemm_takes_norm_scale(ctx, next_rows, d, B);
        if (in_scaled)
            TRY(launch_residual_rmsnorm_parts(ctx, s, B, (int)d, x, M->p0, k5, next_norm, xs));
        else
            TRY(launch_residual_rmsnorm(ctx, s, B, (int)d, x, M->p0, k5, next_norm, nullptr, eps, xp));
    }
    const int kf = gemm_packed_ksplit(ctx, D.vocab_size, d, B);
    const Planes &xl = in_scaled ? xs : xp;
    if (kf == 1) {
        TRY(launch_gemm_packed(ctx, s, M->lm_head.type, M->lm_head.p, D.vocab_size, d, xl, B, M->logits, 1));
    } else {
        TRY(launch_gemm_packed(ctx, s, M->lm_head.type, M->lm_head.p, D.vocab_size, d, xl, B, M->pmix, kf));
        TRY(launch_sum_partials(ctx, s, M->pmix, M->logits, (size_t)B * D.vocab_size, kf));
    }
    return ANEHIP_OK;
}

// Enqueues one decode step for all sequences on `s` (captured or eager):
// the projections, greedy argmax of the logits and the position advance.
int enqueue_step(anehip_ctx *ctx, Model *M, hipStream_t s) {
    TRY(M->batch == 1 ? enqueue_step_b1(ctx, M, s) : enqueue_step_bn(ctx, M, s));
    // greedy argmax: the sampled tokens also become the next step's input
    // (greedy feedback on device) and are recorded by position; each
    // sequence's position is advanced by the same kernel
    return launch_argmax(ctx, s, (int)M->batch, M->desc.vocab_size, M->logits, M->argmax_ws, M->d_sampled,
                         M->d_pos, M->d_tokens, M->d_hist, M->max_seq);
}

// Largest K-split partial buffer any GEMM of the step needs.
size_t part_floats(anehip_ctx *ctx, Model *M) {
    const anehip_model_desc &D = M->desc;
    const uint32_t d = D.dim, F = D.hidden_dim;
    struct {
        uint32_t m, n;
        int mode;  // the batch-1 GEMV's input prologue
    } g[] = {{M->rows_dn, d, GEMV_IN_RESID_RMSNORM},
             {M->rows_attn, d, GEMV_IN_RESID_RMSNORM},
             {d, d, GEMV_IN_GATED_NORM},
             {d, D.n_heads * D.head_dim, GEMV_IN_PLAIN},
             {2 * F, d, GEMV_IN_RESID_RMSNORM},
             {d, F, GEMV_IN_SILU_MUL},
             {D.vocab_size, d, GEMV_IN_PLAIN}};
    size_t mx = 0;
    for (auto &e : g) {
        if (!e.m) continue;
        const int k = M->batch == 1 ? gemv_packed_ksplit(ctx, e.m, e.n, e.mode)
                                    : gemm_packed_ksplit(ctx, e.m, e.n, M->batch);
        size_t need = (size_t)k * M->batch * e.m;
        if (need > mx) mx = need;
    }
    return mx;
}

// Builds the panel copy of every matrix whose GGUF blocks changed since the
// last step (all of them on the first step).
int pack_mat(anehip_ctx *ctx, QMat &Q) {
    if (!Q.d || !Q.stale) return ANEHIP_OK;
    if (!Q.p) {
        const size_t bytes = packed_bytes(Q.type, Q.rows, Q.cols);
        if (hipMalloc(&Q.p, bytes) != hipSuccess) {
            Q.p = nullptr;
            return set_error(ctx->err, ANEHIP_ENOMEM, "decode: cannot allocate %zu bytes of panel weights", bytes);
        }
    }
    TRY(launch_repack(ctx, ctx->stream, Q.type, Q.d, Q.rows, Q.cols, Q.p, Q.il));
    Q.stale = false;
    if (!Q.keep) {
        // the panel copy is the only one the step reads: drop the GGUF copy
        // (not while the stream is being captured: the free would wait on it)
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        ANEHIP_HIP_TRY(ctx->err, hipStreamIsCapturing(ctx->stream, &cs));
        if (cs == hipStreamCaptureStatusNone) {
            ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
            ANEHIP_HIP_TRY(ctx->err, hipFree(Q.d));
            Q.d = nullptr;
        }
    }
    return ANEHIP_OK;
}

// Makes Q's GGUF copy exist (allocated for total_rows x cols of ggml_type,
// or rebuilt from the panel copy if it was dropped after packing).
int gguf_copy(anehip_ctx *ctx, QMat &Q, uint32_t ggml_type, uint32_t total_rows, uint32_t cols, const char *who) {
    if (Q.d) return ANEHIP_OK;
    const size_t bytes = (size_t)total_rows * qrow_bytes(ggml_type, cols);
    if (hipMalloc(&Q.d, bytes) != hipSuccess) {
        Q.d = nullptr;
        return set_error(ctx->err, ANEHIP_ENOMEM, "%s: cannot allocate %zu bytes", who, bytes);
    }
    if (Q.p) {
        TRY(launch_unpack(ctx, ctx->stream, Q.type, Q.p, Q.rows, Q.cols, Q.d, Q.il));
        ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
    } else {
        Q.type = ggml_type;
        Q.rows = total_rows;
        Q.cols = cols;
    }
    return ANEHIP_OK;
}

int pack_weights(anehip_ctx *ctx, Model *M) {
    for (Layer &L : M->layers) {
        TRY(pack_mat(ctx, L.mix_in));
        TRY(pack_mat(ctx, L.mix_out));
        TRY(pack_mat(ctx, L.ffn_gu));
        TRY(pack_mat(ctx, L.ffn_down));
    }
    return pack_mat(ctx, M->lm_head);
}


// K-split partial floats of the prefill's GEMMs at up to kPrefillRows rows
// (the split depends on the rows only through rows <= 16, <= 32, or the
// number of 128-row blocks above 32), of the
// batch-1 lm_head GEMV, and the DeltaNet scan's per-token inputs (q, k, v,
// beta, decay; kept in the ffn partial buffer, which is free at that point).
size_t prefill_part_floats(anehip_ctx *ctx, Model *M) {
    const anehip_model_desc &D = M->desc;
    const uint32_t d = D.dim, F = D.hidden_dim;
    const uint32_t g[][2] = {{M->rows_dn, d}, {M->rows_attn, d}, {d, d}, {d, D.n_heads * D.head_dim}, {2 * F, d}, {d, F}};
    size_t mx = (size_t)gemv_packed_ksplit(ctx, D.vocab_size, d) * D.vocab_size;
    mx = std::max(mx, (size_t)kPrefillRows * (3 * d + 2 * D.ssm_group_count));
    for (auto &e : g)
        for (uint32_t rows : {16u, 32u, kPrefillRows})  // the split depends on rows <= 16, <= 32 or above
            if (e[0]) mx = std::max(mx, (size_t)gemm_rows_ksplit(ctx, e[0], e[1], rows) * rows * e[0]);
    return mx;
}

int alloc_prefill(anehip_ctx *ctx, Model *M) {
    if (M->pf.x) return ANEHIP_OK;
    const anehip_model_desc &D = M->desc;
    const size_t d = D.dim;
    const size_t part = prefill_part_floats(ctx, M);
    size_t attn = 0;
    if (M->rows_attn) {
        const int G = (int)(D.n_heads / D.n_kv_heads);
        for (uint32_t r = 1; r <= kPrefillRows; r++)
            attn = std::max(attn, attn_partial_floats((int)r, (int)D.n_kv_heads, (int)M->max_seq, G));
    }
    struct {
        void **p;
        size_t bytes;
    } a[] = {{(void **)&M->pf.x, kPrefillRows * d * 4}, {(void **)&M->pf.xn, kPrefillRows * d * 4},
             {(void **)&M->pf.pmix, part * 4}, {(void **)&M->pf.p0, part * 4}, {(void **)&M->pf.p1, part * 4},
             {(void **)&M->pf.attn_part, std::max<size_t>(attn, 1) * 4}, {(void **)&M->pf.logits, (size_t)D.vocab_size * 4},
             {(void **)&M->pf.xin, M->pf_planes_bytes()}, {(void **)&M->pf.d_tokens, kPrefillRows * 4},
             {(void **)&M->pf.d_pos, kPrefillRows * 4}};
    for (auto &e : a) {
        if (hipMalloc(e.p, e.bytes) != hipSuccess) {
            *e.p = nullptr;
            (void)hipGetLastError();
            return set_error(ctx->err, ANEHIP_ENOMEM, "prefill: cannot allocate %zu bytes", e.bytes);
        }
    }
    return ANEHIP_OK;
}

// One chunk of T <= kPrefillRows tokens of sequence `seq` (tokens and their
// positions already in pf.d_tokens / pf.d_pos): the batched step's kernels
// with one row per token, except the DeltaNet recurrence (a scan over the
// rows, deltanet_scan) and attention (k / v of every row appended first,
// then row t attends over positions <= its own).  With `logits`, the final
// RMSNorm of the last row and the lm_head GEMV into pf.logits.
int enqueue_prefill_chunk(anehip_ctx *ctx, Model *M, hipStream_t s, uint32_t seq, int T, bool logits) {
    const anehip_model_desc &D = M->desc;
    const uint32_t d = D.dim, F = D.hidden_dim, H = D.ssm_group_count, C = 3 * d;
    const float eps = D.rms_norm_eps;
    const Planes xp = M->pf_planes();
    float *x = M->pf.x;
    TRY(launch_embed_rmsnorm(ctx, s, T, (int)d, M->pf.d_tokens, M->embedding, D.vocab_size, x,
                             M->layers[0].attn_norm, nullptr, eps, xp));
    for (uint32_t l = 0; l < D.n_layers; l++) {
        Layer &L = M->layers[l];
        const bool dn = L.type == ANEHIP_LAYER_DELTANET;
        const uint32_t rows_in = dn ? M->rows_dn : M->rows_attn;
        const int k1 = gemm_rows_ksplit(ctx, rows_in, d, T);
        TRY(launch_gemm_rows(ctx, s, L.mix_in.type, L.mix_in.p, rows_in, d, xp, T, M->pf.pmix, k1));
        MixIn mix;
        mix.p = M->pf.pmix;
        mix.kp = k1;
        mix.split = (size_t)T * rows_in;
        mix.stride = (int)rows_in;
        uint32_t cols3;
        if (dn) {
            TRY(launch_deltanet_scan(ctx, s, T, (int)H, mix, mix.shifted((int)(C + d)), mix.shifted((int)(C + d + H)),
                                     L.conv1d, L.ssm_a, L.dt_bias, L.conv_state + (size_t)seq * C * kConvK,
                                     L.S + (size_t)seq * H * kDk * kDk, M->pf.p1, M->pf.xn, (int)C, L.ssm_norm,
                                     eps, xp));
            cols3 = d;
        } else {
            const size_t cache_off = (size_t)seq * D.n_kv_heads * M->max_seq * D.head_dim;
            TRY(launch_attention_prefill(ctx, s, T, (int)D.n_heads, (int)D.n_kv_heads, (int)M->max_seq, mix, L.q_norm,
                                         L.k_norm, M->inv_freq, M->pf.d_pos, L.kc, L.vc, cache_off, M->pf.attn_part,
                                         xp));
            cols3 = D.n_heads * D.head_dim;
        }
        const int k3 = gemm_rows_ksplit(ctx, d, cols3, T);
        TRY(launch_gemm_rows(ctx, s, L.mix_out.type, L.mix_out.p, d, cols3, xp, T, M->pf.p0, k3));
        TRY(launch_residual_rmsnorm(ctx, s, T, (int)d, x, M->pf.p0, k3, L.post_attn_norm, nullptr, eps, xp));
        const int k4 = gemm_rows_ksplit(ctx, 2 * F, d, T);
        TRY(launch_gemm_rows(ctx, s, L.ffn_gu.type, L.ffn_gu.p, 2 * F, d, xp, T, M->pf.p1, k4));
        TRY(launch_silu_mul_stacked(ctx, s, T, (int)F, M->pf.p1, k4, nullptr, xp));
        const int k5 = gemm_rows_ksplit(ctx, d, F, T);
        TRY(launch_gemm_rows(ctx, s, L.ffn_down.type, L.ffn_down.p, d, F, xp, T, M->pf.p0, k5));
        if (l + 1 < D.n_layers)
            TRY(launch_residual_rmsnorm(ctx, s, T, (int)d, x, M->pf.p0, k5, M->layers[l + 1].attn_norm, nullptr, eps,
                                        xp));
        else if (logits)  // final RMSNorm as fp32 rows
            TRY(launch_residual_rmsnorm(ctx, s, T, (int)d, x, M->pf.p0, k5, M->final_norm, M->pf.xn, eps));
    }
    if (!logits) return ANEHIP_OK;
    GemvInput inf;
    inf.mode = GEMV_IN_PLAIN;
    inf.x = M->pf.xn + (size_t)(T - 1) * d;
    const int kf = gemv_packed_ksplit(ctx, D.vocab_size, d);
    if (kf == 1) {
        TRY(launch_gemv_packed(ctx, s, M->lm_head.type, M->lm_head.p, D.vocab_size, d, inf, M->pf.logits, 1));
    } else {
        TRY(launch_gemv_packed(ctx, s, M->lm_head.type, M->lm_head.p, D.vocab_size, d, inf, M->pf.pmix, kf));
        TRY(launch_sum_partials(ctx, s, M->pf.pmix, M->pf.logits, D.vocab_size, kf));
    }
    return ANEHIP_OK;
}

int launch_step(anehip_ctx *ctx, Model *M) {
    hipStream_t s = ctx->stream;
    TRY(pack_weights(ctx, M));
    if (!M->use_graph) return enqueue_step(ctx, M, s);
    if (!M->exec) {
        ANEHIP_HIP_TRY(ctx->err, hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        int rc = enqueue_step(ctx, M, s);
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamEndCapture(s, &g);
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess)
            return set_error(ctx->err, ANEHIP_EHIP, "graph capture failed: %s", hipGetErrorString(e));
        M->graph = g;
        e = hipGraphInstantiate(&M->exec, g, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            drop_graph(M);
            return set_error(ctx->err, ANEHIP_EHIP, "graph instantiate failed: %s", hipGetErrorString(e));
        }
    }
    ANEHIP_HIP_TRY(ctx->err, hipGraphLaunch(M->exec, s));
    return ANEHIP_OK;
}

int stage_tokens(anehip_ctx *ctx, Model *M, const uint32_t *tokens, uint32_t batch) {
    if (!tokens) return set_error(ctx->err, ANEHIP_EINVAL, "decode_step: tokens is NULL");
    if (batch != M->batch)
        return set_error(ctx->err, ANEHIP_ESHAPE, "decode_step: batch %u, state was allocated for %u", batch,
                         M->batch);
    for (uint32_t b = 0; b < batch; b++)
        if (M->host_pos[b] >= M->max_seq)
            return set_error(ctx->err, ANEHIP_ERANGE, "decode_step: sequence %u at pos %u, KV capacity %u", b,
                             M->host_pos[b], M->max_seq);
    // the previous step may still read the staging buffer
    ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
    std::memcpy(M->h_tokens, tokens, batch * sizeof(uint32_t));
    ANEHIP_HIP_TRY(ctx->err, hipMemcpyAsync(M->d_tokens, M->h_tokens, batch * sizeof(uint32_t),
                                            hipMemcpyHostToDevice, ctx->stream));
    return ANEHIP_OK;
}

Model *model_of(anehip_ctx *ctx, int *rc) {
    if (!ctx) {
        *rc = set_error(global_error(), ANEHIP_EINVAL, "ctx is NULL");
        return nullptr;
    }
    if (!ctx->model) {
        *rc = set_error(ctx->err, ANEHIP_ESTATE, "context was created without a model description");
        return nullptr;
    }
    *rc = ANEHIP_OK;
    return ctx->model;
}

}  // namespace

namespace anehip {
void rope_inv_freq(float base, int head_dim, float *out) {
    for (int i = 0; i < head_dim; i += 2) out[i / 2] = 1.0f / powf(base, (float)i / (float)head_dim);
}
}  // namespace anehip

extern "C" {

__attribute__((visibility("hidden"))) int anehip_model_setup(anehip_ctx *ctx, const anehip_model_desc *desc) {
    const anehip_model_desc &D = *desc;
    if (!D.layer_types || D.n_layers == 0)
        return set_error(ctx->err, ANEHIP_EINVAL, "model: layer_types NULL or n_layers 0");
    for (uint32_t l = 0; l < D.n_layers; l++)
        if (D.layer_types[l] > ANEHIP_LAYER_FULL_ATTENTION)
            return set_error(ctx->err, ANEHIP_EINVAL, "model: layer %u has type %u", l, D.layer_types[l]);
    if (D.dim == 0 || D.dim % 256 || D.hidden_dim == 0 || D.hidden_dim % 256 || D.vocab_size == 0)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "model: dim %u / hidden_dim %u must be multiples of 256",
                         D.dim, D.hidden_dim);
    if (D.ssm_state_size != kDk || D.ssm_conv_kernel != kConvK || D.ssm_group_count * kDk != D.dim)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED,
                         "model: DeltaNet kernels need ssm_state_size 128, conv kernel 4 and "
                         "ssm_group_count*128 == dim (got %u, %u, %u)",
                         D.ssm_state_size, D.ssm_conv_kernel, D.ssm_group_count);
    bool has_attn = false;
    for (uint32_t l = 0; l < D.n_layers; l++) has_attn |= D.layer_types[l] == ANEHIP_LAYER_FULL_ATTENTION;
    if (has_attn) {
        if (D.head_dim != kHd || D.n_kv_heads == 0 || D.n_heads % D.n_kv_heads ||
            (D.n_heads / D.n_kv_heads != 1 && D.n_heads / D.n_kv_heads != 2 && D.n_heads / D.n_kv_heads != 4) ||
            (D.n_heads * D.head_dim) % 256)
            return set_error(ctx->err, ANEHIP_EUNSUPPORTED,
                             "model: attention kernels need head_dim 256 and 1, 2 or 4 query heads per kv head "
                             "(got head_dim %u, %u/%u heads)",
                             D.head_dim, D.n_heads, D.n_kv_heads);
        if (!(D.rope_freq_base > 0.0f))
            return set_error(ctx->err, ANEHIP_EINVAL, "model: rope_freq_base must be > 0");
    }
    Model *M = new Model();
    M->desc = D;
    M->types.assign(D.layer_types, D.layer_types + D.n_layers);
    M->desc.layer_types = M->types.data();
    M->layers.resize(D.n_layers);
    for (uint32_t l = 0; l < D.n_layers; l++) {
        M->layers[l].type = D.layer_types[l];
        // the FFN's gate / up products come out in groups of 32 features
        // (gate sums, then the matching up sums): gu_index()
        M->layers[l].ffn_gu.il = D.hidden_dim;
    }
    M->rows_dn = 3 * D.dim + D.dim + 2 * D.ssm_group_count;
    M->rows_attn = has_attn ? 2 * D.n_heads * D.head_dim + 2 * D.n_kv_heads * D.head_dim : 0;
    ctx->model = M;
    if (has_attn) {
        std::vector<float> f(kHd / 2);
        rope_inv_freq(D.rope_freq_base, (int)kHd, f.data());
        if (hipMalloc(&M->inv_freq, f.size() * sizeof(float)) != hipSuccess)
            return set_error(ctx->err, ANEHIP_ENOMEM, "model: inv_freq allocation failed");
        ANEHIP_HIP_TRY(ctx->err, hipMemcpy(M->inv_freq, f.data(), f.size() * sizeof(float), hipMemcpyHostToDevice));
    }
    return ANEHIP_OK;
}

__attribute__((visibility("hidden"))) void anehip_model_teardown(anehip_ctx *ctx) {
    Model *M = ctx->model;
    if (!M) return;
    free_state(M);
    for (Layer &L : M->layers) {
        void *ps[] = {L.mix_in.d, L.mix_out.d, L.ffn_gu.d, L.ffn_down.d, L.mix_in.p, L.mix_out.p,
                      L.ffn_gu.p, L.ffn_down.p, L.attn_norm, L.post_attn_norm, L.ssm_a, L.conv1d,
                      L.dt_bias, L.ssm_norm, L.q_norm, L.k_norm};
        for (void *p : ps) free_ptr(p);
    }
    free_ptr(M->embedding);
    free_ptr(M->final_norm);
    free_ptr(M->lm_head.d);
    free_ptr(M->lm_head.p);
    free_ptr(M->inv_freq);
    delete M;
    ctx->model = nullptr;
}

int anehip_upload_quant(anehip_ctx *ctx, int32_t layer, uint32_t kind, const uint8_t *blocks, size_t nbytes,
                        uint32_t m, uint32_t n, uint32_t ggml_type) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    if (!blocks) return set_error(ctx->err, ANEHIP_EINVAL, "upload_quant: blocks is NULL");
    if (layer < -1 || layer >= (int32_t)M->desc.n_layers)
        return set_error(ctx->err, ANEHIP_EINVAL, "upload_quant: layer %d out of range", layer);
    if (ggml_type != ANEHIP_GGML_Q8_0 && ggml_type != ANEHIP_GGML_Q4_0)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "upload_quant: ggml type %u (Q4_0=2, Q8_0=8)", ggml_type);
    // Q8Tensor::from_raw checks (q8_gemv.rs:41-50)
    if (n % 32) return set_error(ctx->err, ANEHIP_ESHAPE, "upload_quant: n=%u not divisible by 32", n);
    const size_t expected = (size_t)m * (n / 32) * (ggml_type == ANEHIP_GGML_Q8_0 ? 34 : 18);
    if (nbytes != expected)
        return set_error(ctx->err, ANEHIP_ESHAPE, "upload_quant: got %zu bytes, expected %zu (m=%u, n=%u, type=%u)",
                         nbytes, expected, m, n, ggml_type);
    KindShape ks = kind_shape(M, layer, kind);
    if (!ks.rows || !ks.quant)
        return set_error(ctx->err, ANEHIP_EINVAL, "upload_quant: kind %s is not a quantised tensor of layer %d",
                         kind_name(kind), layer);
    if (ks.rows != m || ks.cols != n)
        return set_error(ctx->err, ANEHIP_ESHAPE, "upload_quant: %s of layer %d is [%u x %u], got [%u x %u]",
                         kind_name(kind), layer, ks.rows, ks.cols, m, n);
    QSlot slot = quant_slot(M, layer, kind);
    QMat &Q = *slot.mat;
    if ((Q.d || Q.p) && Q.type != ggml_type)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED,
                         "upload_quant: %s of layer %d is type %u but its stacked matrix holds type %u",
                         kind_name(kind), layer, ggml_type, Q.type);
    TRY(gguf_copy(ctx, Q, ggml_type, slot.total_rows, n, "upload_quant"));
    char *dst = static_cast<char *>(Q.d) + (size_t)slot.row_off * qrow_bytes(ggml_type, n);
    ANEHIP_HIP_TRY(ctx->err, hipMemcpy(dst, blocks, nbytes, hipMemcpyHostToDevice));
    Q.stale = true;
    if (layer < 0) M->glob_have |= 1ull << kind;
    else M->layers[layer].have |= 1ull << kind;
    return ANEHIP_OK;
}

int anehip_upload_f32(anehip_ctx *ctx, int32_t layer, uint32_t kind, const float *data, size_t n) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    if (!data) return set_error(ctx->err, ANEHIP_EINVAL, "upload_f32: data is NULL");
    if (layer < -1 || layer >= (int32_t)M->desc.n_layers)
        return set_error(ctx->err, ANEHIP_EINVAL, "upload_f32: layer %d out of range", layer);
    KindShape ks = kind_shape(M, layer, kind);
    if (!ks.rows || ks.quant)
        return set_error(ctx->err, ANEHIP_EINVAL, "upload_f32: kind %s is not an f32 tensor of layer %d",
                         kind_name(kind), layer);
    const size_t want = (size_t)ks.rows * ks.cols;
    if (n != want)
        return set_error(ctx->err, ANEHIP_ESHAPE, "upload_f32: %s of layer %d has %zu values, got %zu",
                         kind_name(kind), layer, want, n);
    float **slot = f32_slot(M, layer, kind);
    if (!*slot && hipMalloc((void **)slot, want * sizeof(float)) != hipSuccess) {
        *slot = nullptr;
        return set_error(ctx->err, ANEHIP_ENOMEM, "upload_f32: cannot allocate %zu floats", want);
    }
    ANEHIP_HIP_TRY(ctx->err, hipMemcpy(*slot, data, want * sizeof(float), hipMemcpyHostToDevice));
    if (layer < 0) M->glob_have |= 1ull << kind;
    else M->layers[layer].have |= 1ull << kind;
    return ANEHIP_OK;
}

int anehip_tensor_ptr(anehip_ctx *ctx, int32_t layer, uint32_t kind, uint32_t ggml_type, void **dptr,
                      size_t *nbytes) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    if (!dptr || !nbytes || layer < -1 || layer >= (int32_t)M->desc.n_layers)
        return set_error(ctx->err, ANEHIP_EINVAL, "tensor_ptr: bad argument");
    KindShape ks = kind_shape(M, layer, kind);
    if (!ks.rows) return set_error(ctx->err, ANEHIP_EINVAL, "tensor_ptr: layer %d has no %s", layer, kind_name(kind));
    if (ks.quant) {
        if (ggml_type != ANEHIP_GGML_Q8_0 && ggml_type != ANEHIP_GGML_Q4_0)
            return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "tensor_ptr: ggml type %u", ggml_type);
        QSlot slot = quant_slot(M, layer, kind);
        QMat &Q = *slot.mat;
        if ((Q.d || Q.p) && Q.type != ggml_type)
            return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "tensor_ptr: stacked matrix of %s holds type %u",
                             kind_name(kind), Q.type);
        TRY(gguf_copy(ctx, Q, ggml_type, slot.total_rows, ks.cols, "tensor_ptr"));
        Q.keep = true;  // the caller may read or write through *dptr at any time
        *dptr = static_cast<char *>(Q.d) + (size_t)slot.row_off * qrow_bytes(ggml_type, ks.cols);
        Q.stale = true;  // writes through *dptr reach the step's panel copy at the next step
        *nbytes = (size_t)ks.rows * qrow_bytes(ggml_type, ks.cols);
    } else {
        float **slot = f32_slot(M, layer, kind);
        const size_t want = (size_t)ks.rows * ks.cols;
        if (!*slot && hipMalloc((void **)slot, want * sizeof(float)) != hipSuccess) {
            *slot = nullptr;
            return set_error(ctx->err, ANEHIP_ENOMEM, "tensor_ptr: cannot allocate %zu floats", want);
        }
        *dptr = *slot;
        *nbytes = want * sizeof(float);
    }
    if (layer < 0) M->glob_have |= 1ull << kind;
    else M->layers[layer].have |= 1ull << kind;
    return ANEHIP_OK;
}

int anehip_alloc_state(anehip_ctx *ctx, uint32_t batch, uint32_t max_seq) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    if (batch == 0 || batch > 32) return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "alloc_state: batch %u outside 1..32", batch);
    if (max_seq == 0) return set_error(ctx->err, ANEHIP_EINVAL, "alloc_state: max_seq is 0");
    // batch > 1 runs the projections on the panel MFMA GEMM (16-byte output stores)
    if (batch > 1 && M->desc.vocab_size % 4)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "alloc_state: batch > 1 needs vocab_size %% 4 == 0 (got %u)",
                         M->desc.vocab_size);
    ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
    free_state(M);
    const anehip_model_desc &D = M->desc;
    const size_t d = D.dim, F = D.hidden_dim, H = D.ssm_group_count, C = 3 * d;
    const size_t kvd = (size_t)D.n_kv_heads * D.head_dim;
    auto alloc = [&](void **p, size_t bytes) -> int {
        if (hipMalloc(p, bytes) != hipSuccess) {
            *p = nullptr;
            (void)hipGetLastError();
            return set_error(ctx->err, ANEHIP_ENOMEM, "alloc_state: cannot allocate %zu bytes", bytes);
        }
        if (hipMemset(*p, 0, bytes) != hipSuccess)
            return set_error(ctx->err, ANEHIP_EHIP, "alloc_state: memset failed");
        return ANEHIP_OK;
    };
    M->batch = batch;
    M->max_seq = max_seq;
    int r = ANEHIP_OK;
    for (Layer &L : M->layers) {
        if (L.type == ANEHIP_LAYER_DELTANET) {
            r = r ? r : alloc((void **)&L.conv_state, batch * C * kConvK * sizeof(float));
            r = r ? r : alloc((void **)&L.S, batch * H * kDk * kDk * sizeof(float));
        } else {
            r = r ? r : alloc((void **)&L.kc, batch * kvd * max_seq * sizeof(__half));
            r = r ? r : alloc((void **)&L.vc, batch * kvd * max_seq * sizeof(__half));
        }
    }
    const size_t qd = (size_t)D.n_heads * D.head_dim;
    size_t nmax = d > F ? d : F;
    if (qd > nmax) nmax = qd;
    M->xin_len = xf_plane_len(nmax);
    M->xe_cnt = xe_bytes(nmax);
    M->part_len = part_floats(ctx, M);
    r = r ? r : alloc((void **)&M->d_pos, 64 * sizeof(uint32_t));
    r = r ? r : alloc((void **)&M->d_tokens, 64 * sizeof(uint32_t));
    r = r ? r : alloc((void **)&M->d_sampled, 64 * sizeof(uint32_t));
    r = r ? r : alloc((void **)&M->d_hist, (size_t)batch * max_seq * sizeof(uint32_t));
    r = r ? r : alloc((void **)&M->x0, batch * d * sizeof(float));
    r = r ? r : alloc((void **)&M->x1, batch * d * sizeof(float));
    r = r ? r : alloc((void **)&M->pmix, M->part_len * sizeof(float));
    r = r ? r : alloc((void **)&M->p0, M->part_len * sizeof(float));
    r = r ? r : alloc((void **)&M->p1, M->part_len * sizeof(float));
    r = r ? r : alloc((void **)&M->heads, batch * d * sizeof(float));
    r = r ? r : alloc((void **)&M->attn_out, batch * (qd ? qd : 1) * sizeof(float));
    r = r ? r : alloc((void **)&M->xin, M->planes_bytes());
    r = r ? r : alloc((void **)&M->logits, batch * (size_t)D.vocab_size * sizeof(float));
    r = r ? r : alloc(&M->argmax_ws, argmax_workspace_bytes((int)batch));
    if (batch > 1) r = r ? r : alloc((void **)&M->norm_ss, 32 * kMaxRsParts * sizeof(float));
    if (M->rows_attn) {
        const int G = (int)(D.n_heads / D.n_kv_heads);
        r = r ? r : alloc((void **)&M->attn_part, attn_partial_floats((int)batch, (int)D.n_kv_heads, (int)max_seq, G) * sizeof(float));
    }
    if (batch == 1 && M->rows_dn && dn_ssm_fusable(ctx, (uint32_t)d, (uint32_t)H)) {
        size_t n_dn = 0;
        for (const Layer &L : M->layers) n_dn += L.type == ANEHIP_LAYER_DELTANET;
        if (n_dn <= (size_t)kMaxDnApplyLayers)
            r = r ? r : alloc((void **)&M->dn_pend, n_dn * kDnPendFloats(d, H) * sizeof(float));
    }
    if (!r && hipHostMalloc((void **)&M->h_tokens, 64 * sizeof(uint32_t), 0) != hipSuccess) {
        M->h_tokens = nullptr;
        r = set_error(ctx->err, ANEHIP_ENOMEM, "alloc_state: pinned staging allocation failed");
    }
    if (r) {
        free_state(M);
        return r;
    }
    M->host_pos.assign(batch, 0);
    return ANEHIP_OK;
}

int anehip_reset_state(anehip_ctx *ctx) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    if (!M->batch) return set_error(ctx->err, ANEHIP_ESTATE, "reset_state: no state allocated");
    ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
    const anehip_model_desc &D = M->desc;
    const size_t C = 3 * (size_t)D.dim, kvd = (size_t)D.n_kv_heads * D.head_dim;
    for (Layer &L : M->layers) {
        if (L.type == ANEHIP_LAYER_DELTANET) {
            ANEHIP_HIP_TRY(ctx->err, hipMemset(L.conv_state, 0, M->batch * C * kConvK * sizeof(float)));
            ANEHIP_HIP_TRY(ctx->err, hipMemset(L.S, 0, M->batch * (size_t)D.ssm_group_count * kDk * kDk * sizeof(float)));
        } else {
            ANEHIP_HIP_TRY(ctx->err, hipMemset(L.kc, 0, M->batch * kvd * M->max_seq * sizeof(__half)));
            ANEHIP_HIP_TRY(ctx->err, hipMemset(L.vc, 0, M->batch * kvd * M->max_seq * sizeof(__half)));
        }
    }
    ANEHIP_HIP_TRY(ctx->err, hipMemset(M->d_pos, 0, 64 * sizeof(uint32_t)));
    M->host_pos.assign(M->batch, 0);
    return ANEHIP_OK;
}

int anehip_set_pos(anehip_ctx *ctx, uint32_t seq, uint32_t pos) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    if (seq >= M->batch) return set_error(ctx->err, ANEHIP_EINVAL, "set_pos: sequence %u of %u", seq, M->batch);
    if (pos >= M->max_seq) return set_error(ctx->err, ANEHIP_ERANGE, "set_pos: pos %u >= capacity %u", pos, M->max_seq);
    ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
    ANEHIP_HIP_TRY(ctx->err, hipMemcpy(M->d_pos + seq, &pos, sizeof(uint32_t), hipMemcpyHostToDevice));
    M->host_pos[seq] = pos;
    return ANEHIP_OK;
}

int anehip_get_pos(anehip_ctx *ctx, uint32_t seq, uint32_t *pos) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    if (!pos || seq >= M->batch) return set_error(ctx->err, ANEHIP_EINVAL, "get_pos: bad argument");
    *pos = M->host_pos[seq];
    return ANEHIP_OK;
}

int anehip_state_ptr(anehip_ctx *ctx, uint32_t layer, uint32_t which, void **dptr, size_t *nbytes) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    if (!dptr || !nbytes || layer >= M->desc.n_layers || which > 3)
        return set_error(ctx->err, ANEHIP_EINVAL, "state_ptr: bad argument");
    if (!M->batch) return set_error(ctx->err, ANEHIP_ESTATE, "state_ptr: no state allocated");
    Layer &L = M->layers[layer];
    const anehip_model_desc &D = M->desc;
    const bool dn = L.type == ANEHIP_LAYER_DELTANET;
    if (dn != (which < 2))
        return set_error(ctx->err, ANEHIP_EINVAL, "state_ptr: layer %u has no state kind %u", layer, which);
    switch (which) {
        case 0: *dptr = L.conv_state; *nbytes = M->batch * 3 * (size_t)D.dim * kConvK * sizeof(float); break;
        case 1: *dptr = L.S; *nbytes = M->batch * (size_t)D.ssm_group_count * kDk * kDk * sizeof(float); break;
        case 2: *dptr = L.kc; *nbytes = M->batch * (size_t)D.n_kv_heads * D.head_dim * M->max_seq * sizeof(__half); break;
        default: *dptr = L.vc; *nbytes = M->batch * (size_t)D.n_kv_heads * D.head_dim * M->max_seq * sizeof(__half); break;
    }
    return ANEHIP_OK;
}

int anehip_set_graph(anehip_ctx *ctx, int enabled) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
    drop_graph(M);
    M->use_graph = enabled != 0;
    return ANEHIP_OK;
}

int anehip_decode_step_async(anehip_ctx *ctx, const uint32_t *tokens, uint32_t batch) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    if ((rc = check_model(ctx, M))) return rc;
    if ((rc = stage_tokens(ctx, M, tokens, batch))) return rc;
    if ((rc = launch_step(ctx, M))) return rc;
    for (uint32_t b = 0; b < batch; b++) M->host_pos[b]++;
    return ANEHIP_OK;
}

int anehip_decode_step(anehip_ctx *ctx, const uint32_t *tokens, uint32_t batch, float *logits_out) {
    int rc = anehip_decode_step_async(ctx, tokens, batch);
    if (rc) return rc;
    Model *M = ctx->model;
    if (logits_out)
        ANEHIP_HIP_TRY(ctx->err, hipMemcpyAsync(logits_out, M->logits, (size_t)batch * M->desc.vocab_size * sizeof(float),
                                                hipMemcpyDeviceToHost, ctx->stream));
    ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
    return ANEHIP_OK;
}

int anehip_prefill(anehip_ctx *ctx, uint32_t seq, const uint32_t *tokens, uint32_t n_tokens, float *logits_out) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    if ((rc = check_model(ctx, M))) return rc;
    if (!tokens || n_tokens == 0) return set_error(ctx->err, ANEHIP_EINVAL, "prefill: no tokens");
    if (seq >= M->batch) return set_error(ctx->err, ANEHIP_EINVAL, "prefill: sequence %u of %u", seq, M->batch);
    const uint32_t p0 = M->host_pos[seq];
    if ((uint64_t)p0 + n_tokens > M->max_seq)
        return set_error(ctx->err, ANEHIP_ERANGE, "prefill: sequence %u at pos %u + %u tokens exceeds capacity %u", seq,
                         p0, n_tokens, M->max_seq);
    hipStream_t s = ctx->stream;
    TRY(pack_weights(ctx, M));
    TRY(alloc_prefill(ctx, M));
    // every chunk's rows staged in pinned memory up front, copied in stream
    // order before its kernels (no host wait between chunks); an earlier
    // call's copies may still read the staging buffer, hence the one sync
    const size_t chunks = (n_tokens + kPrefillRows - 1) / kPrefillRows;
    ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(s));
    if (M->pf_stage_chunks < chunks) {
        if (M->pf_stage) (void)hipHostFree(M->pf_stage);
        M->pf_stage = nullptr;
        M->pf_stage_chunks = 0;
        if (hipHostMalloc((void **)&M->pf_stage, chunks * 2 * kPrefillRows * sizeof(uint32_t), 0) != hipSuccess) {
            M->pf_stage = nullptr;
            return set_error(ctx->err, ANEHIP_ENOMEM, "prefill: cannot allocate %zu chunks of pinned staging", chunks);
        }
        M->pf_stage_chunks = chunks;
    }
    for (uint32_t c0 = 0, c = 0; c0 < n_tokens; c0 += kPrefillRows, c++) {
        const uint32_t T = std::min(kPrefillRows, n_tokens - c0);
        uint32_t *st = M->pf_stage + (size_t)c * 2 * kPrefillRows;
        for (uint32_t t = 0; t < T; t++) {
            st[t] = tokens[c0 + t];
            st[kPrefillRows + t] = p0 + c0 + t;
        }
        ANEHIP_HIP_TRY(ctx->err, hipMemcpyAsync(M->pf.d_tokens, st, T * 4, hipMemcpyHostToDevice, s));
        ANEHIP_HIP_TRY(ctx->err, hipMemcpyAsync(M->pf.d_pos, st + kPrefillRows, T * 4, hipMemcpyHostToDevice, s));
        const bool last = c0 + T == n_tokens;
        if (T != kPrefillRows || last || !M->use_graph) {
            TRY(enqueue_prefill_chunk(ctx, M, s, seq, (int)T, last));
            continue;
        }
        // full chunks replay one captured graph (per sequence: its state blocks)
        if (M->pf_exec && M->pf_graph_seq != seq) {
            (void)hipGraphExecDestroy(M->pf_exec);
            (void)hipGraphDestroy(M->pf_graph);
            M->pf_exec = nullptr;
            M->pf_graph = nullptr;
        }
        if (!M->pf_exec) {
            ANEHIP_HIP_TRY(ctx->err, hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            int rc2 = enqueue_prefill_chunk(ctx, M, s, seq, (int)kPrefillRows, false);
            hipGraph_t g = nullptr;
            hipError_t e = hipStreamEndCapture(s, &g);
            if (rc2) {
                if (g) (void)hipGraphDestroy(g);
                return rc2;
            }
            if (e != hipSuccess)
                return set_error(ctx->err, ANEHIP_EHIP, "prefill graph capture failed: %s", hipGetErrorString(e));
            e = hipGraphInstantiate(&M->pf_exec, g, nullptr, nullptr, 0);
            if (e != hipSuccess) {
                (void)hipGraphDestroy(g);
                M->pf_exec = nullptr;
                return set_error(ctx->err, ANEHIP_EHIP, "prefill graph instantiate failed: %s", hipGetErrorString(e));
            }
            M->pf_graph = g;
            M->pf_graph_seq = seq;
        }
        ANEHIP_HIP_TRY(ctx->err, hipGraphLaunch(M->pf_exec, s));
    }
    // the sequence continues at p0 + n_tokens (device copy for the step graph)
    const uint32_t pos = p0 + n_tokens;
    ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(s));
    ANEHIP_HIP_TRY(ctx->err, hipMemcpy(M->d_pos + seq, &pos, sizeof(uint32_t), hipMemcpyHostToDevice));
    M->host_pos[seq] = pos;
    if (logits_out)
        ANEHIP_HIP_TRY(ctx->err, hipMemcpy(logits_out, M->pf.logits, (size_t)M->desc.vocab_size * sizeof(float),
                                           hipMemcpyDeviceToHost));
    return ANEHIP_OK;
}

int anehip_logits_ptr(anehip_ctx *ctx, const float **dptr) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    if (!dptr || !M->batch) return set_error(ctx->err, ANEHIP_ESTATE, "logits_ptr: no state");
    *dptr = M->logits;
    return ANEHIP_OK;
}

int anehip_sampled_tokens(anehip_ctx *ctx, uint32_t *out) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    if (!out || !M->batch) return set_error(ctx->err, ANEHIP_ESTATE, "sampled_tokens: no state");
    ANEHIP_HIP_TRY(ctx->err, hipMemcpyAsync(out, M->d_sampled, M->batch * sizeof(uint32_t), hipMemcpyDeviceToHost,
                                            ctx->stream));
    ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
    return ANEHIP_OK;
}

int anehip_generate(anehip_ctx *ctx, const uint32_t *first_tokens, uint32_t batch, uint32_t steps,
                    uint32_t *out_tokens) {
    int rc;
    Model *M = model_of(ctx, &rc);
    if (!M) return rc;
    if (!out_tokens || steps == 0) return set_error(ctx->err, ANEHIP_EINVAL, "generate: bad argument");
    if ((rc = check_model(ctx, M))) return rc;
    for (uint32_t b = 0; b < M->batch && b < batch; b++)
        if ((uint64_t)M->host_pos[b] + steps > M->max_seq)
            return set_error(ctx->err, ANEHIP_ERANGE, "generate: sequence %u at pos %u + %u steps > capacity %u", b,
                             M->host_pos[b], steps, M->max_seq);
    if ((rc = stage_tokens(ctx, M, first_tokens, batch))) return rc;
    // each step's argmax feeds its tokens to the next step and records them
    // at the sequence's position (d_hist), all inside the step: nothing is
    // enqueued between steps
    const std::vector<uint32_t> start(M->host_pos.begin(), M->host_pos.begin() + batch);
    for (uint32_t i = 0; i < steps; i++) {
        if ((rc = launch_step(ctx, M))) break;
        for (uint32_t b = 0; b < batch; b++) M->host_pos[b]++;
    }
    std::vector<uint32_t> hist(rc ? 0 : (size_t)batch * steps);
    for (uint32_t b = 0; b < batch && !rc; b++)
        if (hipMemcpyAsync(hist.data() + (size_t)b * steps, M->d_hist + (size_t)b * M->max_seq + start[b],
                           (size_t)steps * sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->stream) != hipSuccess)
            rc = set_error(ctx->err, ANEHIP_EHIP, "generate: copy-out failed");
    ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
    if (!rc)
        for (uint32_t i = 0; i < steps; i++)
            for (uint32_t b = 0; b < batch; b++) out_tokens[(size_t)i * batch + b] = hist[(size_t)b * steps + i];
    return rc;
}

}  // extern "C"
