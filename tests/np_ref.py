"""Independent float64 numpy statement of the decode math (test helper).

Written from the mathematics of the reference's decode step, vectorised and in
float64, so that it shares no code or loop structure with the C oracle.  Tests
use it to pin the oracle: an index, sign or dropped-term mistake in either one
shows up as a disagreement far above float32 rounding.
"""
import numpy as np

Q4_0, Q8_0 = 2, 8


def f16_bits_to_f64(lo, hi):
    return np.frombuffer(np.asarray(lo | (hi << 8), np.uint16).tobytes(), np.float16).astype(np.float64)


def dequant(t, w, m, n):
    nb = n // 32
    if t == Q8_0:
        blk = np.asarray(w, np.uint8).reshape(m, nb, 34)
        d = f16_bits_to_f64(blk[:, :, 0].astype(np.uint16), blk[:, :, 1].astype(np.uint16)).reshape(m, nb, 1)
        q = blk[:, :, 2:].view(np.int8).astype(np.float64)
        return (q * d).reshape(m, n)
    blk = np.asarray(w, np.uint8).reshape(m, nb, 18)
    d = f16_bits_to_f64(blk[:, :, 0].astype(np.uint16), blk[:, :, 1].astype(np.uint16)).reshape(m, nb, 1)
    b = blk[:, :, 2:].astype(np.int64)
    q = np.concatenate([(b & 15) - 8, (b >> 4) - 8], axis=2).astype(np.float64)
    return (q * d).reshape(m, n)


def silu(x):
    return x / (1.0 + np.exp(-x))


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def rmsnorm(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * w


def deltanet_core(qkv, beta_raw, alpha_raw, conv_w, ssm_a, dt_bias, conv_state, S, n_heads, dk):
    """Returns (out_heads, new_conv_state, new_S), all float64.

    conv_state / conv_w: [C, K]; S: [H, dk, dv]."""
    conv_state = np.asarray(conv_state, np.float64)
    cs = np.concatenate([conv_state[:, 1:], np.asarray(qkv, np.float64)[:, None]], axis=1)
    co = silu((cs * np.asarray(conv_w, np.float64)).sum(axis=1))
    chunk = n_heads * dk
    q = co[:chunk].reshape(n_heads, dk)
    k = co[chunk:2 * chunk].reshape(n_heads, dk)
    v = co[2 * chunk:].reshape(n_heads, dk)
    q = q / np.sqrt((q * q).sum(1, keepdims=True) + 1e-12) / np.sqrt(dk)
    k = k / np.sqrt((k * k).sum(1, keepdims=True) + 1e-12)
    beta = sigmoid(np.asarray(beta_raw, np.float64))
    decay = np.exp(np.asarray(ssm_a, np.float64) * np.log1p(np.exp(np.asarray(alpha_raw, np.float64) + dt_bias)))
    S = np.asarray(S, np.float64) * decay[:, None, None]
    sk = np.einsum("hij,hi->hj", S, k)
    delta = beta[:, None] * (v - sk)
    S = S + k[:, :, None] * delta[:, None, :]
    o = np.einsum("hij,hi->hj", S, q)
    return o.reshape(-1), cs, S


def rope(x, pos, base):
    """x: [nh, hd]; rotates adjacent pairs (2p, 2p+1) by pos * base^(-2p/hd)."""
    nh, hd = x.shape
    inv = 1.0 / np.power(np.float64(base), np.arange(0, hd, 2, dtype=np.float64) / hd)
    ang = pos * inv
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[:, 0::2], x[:, 1::2]
    out = np.empty_like(x)
    out[:, 0::2] = a * c - b * s
    out[:, 1::2] = a * s + b * c
    return out


def attention_core(q_full, k_in, v_in, q_norm, k_norm, k_hist, v_hist, pos, n_heads, n_kv, hd, base=10000.0,
                   kv_round=None):
    """k_hist/v_hist: [n_kv, pos, hd] float64 history (positions < pos).
    Returns (attn_out [n_heads*hd], k_new [n_kv, hd], v_new)."""
    qf = np.asarray(q_full, np.float64).reshape(n_heads, 2, hd)
    q, gate = qf[:, 0, :], qf[:, 1, :]
    k = np.asarray(k_in, np.float64).reshape(n_kv, hd)
    v = np.asarray(v_in, np.float64).reshape(n_kv, hd)
    q = np.stack([rmsnorm(q[h], q_norm, 1e-6) for h in range(n_heads)])
    k = np.stack([rmsnorm(k[h], k_norm, 1e-6) for h in range(n_kv)])
    q = rope(q, pos, base)
    k = rope(k, pos, base)
    if kv_round is not None:
        k, v = kv_round(k), kv_round(v)
    K = np.concatenate([k_hist, k[:, None, :]], axis=1)
    V = np.concatenate([v_hist, v[:, None, :]], axis=1)
    hpk = n_heads // n_kv
    out = np.empty((n_heads, hd))
    for h in range(n_heads):
        sc = K[h // hpk] @ q[h] / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        out[h] = p @ V[h // hpk]
    return (out * sigmoid(gate)).reshape(-1), k, v


def ffn(x, w_gate, w_up, w_down):
    """ffn_forward (main.rs:1115-1135): down(silu(gate x) * up x), float64."""
    return w_down @ (silu(w_gate @ x) * (w_up @ x))


class Forward64:
    """The decode step composed in float64 from the functions above, following
    qwen35_forward_token (crates/cli/src/main.rs:953-1023):

        x = embedding[token]
        per layer l:  x += mixer_l(rmsnorm(x, attn_norm_l))
                      x += ffn_l(rmsnorm(x, post_attn_norm_l))
        logits = lm_head @ rmsnorm(x, final_norm)

    with the DeltaNet mixer of deltanet.rs:429-539 (qkv / beta / alpha / gate
    projections of the normed input, the core above, per-head RMSNorm times
    SiLU(gate), ssm_out) and the attention mixer of deltanet.rs:541-675
    (wq -> q | gate per head, q / k RMSNorm with eps 1e-6, RoPE, K/V history
    kept exact as the reference's fp32 cache does, or rounded to fp16 with
    `kv_f16`, softmax, sigmoid(gate), wo).

    `weights(layer, name)` returns float64 arrays: dequantised matrices
    [rows, cols] or fp32 vectors; names are the model's tensor names
    (attn_norm, qkv, ssm_conv1d [C, K], ...).  State is float64 and lives here:
    conv windows [C, K], S [H, dk, dk], K / V history [n_kv, pos, hd]."""

    def __init__(self, weights, layer_types, cfg, kv_f16=True):
        self.w, self.types, self.cfg = weights, list(layer_types), dict(cfg)
        self.kv_f16 = kv_f16
        self.pos = 0
        self.conv, self.S, self.K, self.V = {}, {}, {}, {}
        c = self.cfg
        for l, t in enumerate(self.types):
            if t == 0:
                self.conv[l] = np.zeros((3 * c["dim"], c["ksize"]))
                self.S[l] = np.zeros((c["H"], c["dk"], c["dk"]))
            else:
                self.K[l] = np.zeros((c["n_kv"], 0, c["hd"]))
                self.V[l] = np.zeros((c["n_kv"], 0, c["hd"]))

    def forward(self, token):
        c, w = self.cfg, self.w
        eps = c["eps"]
        x = np.array(w(-1, "embedding")[token], np.float64) if token < c["vocab"] else np.zeros(c["dim"])
        for l, t in enumerate(self.types):
            xn = rmsnorm(x, w(l, "attn_norm"), eps)
            if t == 0:
                qkv = w(l, "qkv") @ xn
                heads, self.conv[l], self.S[l] = deltanet_core(
                    qkv, w(l, "ssm_beta") @ xn, w(l, "ssm_alpha") @ xn, w(l, "ssm_conv1d"), w(l, "ssm_a"),
                    w(l, "ssm_dt_bias"), self.conv[l], self.S[l], c["H"], c["dk"])
                gate = w(l, "attn_gate") @ xn
                hs = heads.reshape(c["H"], c["dk"])
                normed = np.concatenate([rmsnorm(hs[h], w(l, "ssm_norm"), eps) for h in range(c["H"])])
                mix = w(l, "ssm_out") @ (normed * silu(gate))
            else:
                f16 = (lambda a: np.asarray(a, np.float64).astype(np.float16).astype(np.float64)) \
                    if self.kv_f16 else None
                out, k_new, v_new = attention_core(
                    w(l, "wq") @ xn, w(l, "wk") @ xn, w(l, "wv") @ xn, w(l, "q_norm"), w(l, "k_norm"),
                    self.K[l], self.V[l], self.pos, c["n_heads"], c["n_kv"], c["hd"], c["rope_base"],
                    kv_round=f16)
                self.K[l] = np.concatenate([self.K[l], k_new[:, None, :]], axis=1)
                self.V[l] = np.concatenate([self.V[l], v_new[:, None, :]], axis=1)
                mix = w(l, "wo") @ out
            x = x + mix
            x = x + ffn(rmsnorm(x, w(l, "post_attn_norm"), eps), w(l, "ffn_gate"), w(l, "ffn_up"),
                        w(l, "ffn_down"))
        self.pos += 1
        return w(-1, "lm_head") @ rmsnorm(x, w(-1, "final_norm"), eps)
