"""GPU parity of the decode-step kernels against the CPU oracle, through the
C ABI (include/anehip.h).  Bounds: DeltaNet state after 256 steps <= 1e-3
relative; attention / norms <= 1e-4 relative
unless stated."""
import numpy as np
import pytest

import np_ref
from conftest import rel_errs

pytestmark = pytest.mark.gpu

H, DK = 16, 128
CH = 3 * H * DK


def f32(a):
    return np.ascontiguousarray(a, np.float32)


# ------------------------------------------------------------ DeltaNet ----

@pytest.mark.parametrize("batch", [1, 8, 32])
def test_deltanet_256_steps_state_parity(gpu_ctx, oracle_lib, batch):
    """Config 3: 16 heads, dk = dv = 128, S0 ~ N(0, 0.01), conv width 4 over a
    [B, 4, 6144] window, fresh N(0,1) qkv / beta / alpha inputs per step,
    ssm_a = -U(0,1); 256 steps.  S after 256 steps within 1e-3 (rel L2 and
    max-abs/max) per checked sequence; outputs checked every 32 steps."""
    seed = 300 + batch
    conv_w = oracle_lib.normal(seed, 1, CH * 4, std=0.5)
    ssm_a = -oracle_lib.uniform(seed, 2, H)
    dt_bias = oracle_lib.normal(seed, 3, H)
    S0 = oracle_lib.normal(seed, 4, batch * H * DK * DK, std=0.01)
    win0 = oracle_lib.normal(seed, 5, batch * CH * 4)
    check = sorted({0, batch // 2, batch - 1})
    o_S = {b: S0.reshape(batch, -1)[b].copy() for b in check}
    o_cs = {b: win0.reshape(batch, -1)[b].copy() for b in check}

    d_S, d_cs = gpu_ctx.to_device(S0), gpu_ctx.to_device(win0)
    d_cw, d_a, d_dt = gpu_ctx.to_device(conv_w), gpu_ctx.to_device(ssm_a), gpu_ctx.to_device(dt_bias)
    d_qkv, d_b, d_al = gpu_ctx.alloc(batch * CH * 4), gpu_ctx.alloc(batch * H * 4), gpu_ctx.alloc(batch * H * 4)
    d_out = gpu_ctx.alloc(batch * H * DK * 4)
    worst = 0.0
    for step in range(256):
        qkv = oracle_lib.normal(seed, 1000 + step, batch * CH).reshape(batch, CH)
        br = oracle_lib.normal(seed, 2000 + step, batch * H).reshape(batch, H)
        ar = oracle_lib.normal(seed, 3000 + step, batch * H).reshape(batch, H)
        d_qkv.upload(qkv)
        d_b.upload(br)
        d_al.upload(ar)
        gpu_ctx.call("deltanet_step", batch, H, d_qkv, d_b, d_al, d_cw, d_a, d_dt, d_cs, d_S, d_out)
        outs = {}
        for b in check:
            outs[b] = oracle_lib.deltanet_core(qkv[b], br[b], ar[b], conv_w, ssm_a, dt_bias, o_cs[b], o_S[b], H, DK)
        if step % 32 == 31:
            g = d_out.download(np.float32, batch * H * DK).reshape(batch, -1)
            for b in check:
                worst = max(worst, max(rel_errs(g[b], outs[b])))
    gS = d_S.download(np.float32, batch * H * DK * DK).reshape(batch, -1)
    gcs = d_cs.download(np.float32, batch * CH * 4).reshape(batch, -1)
    for b in check:
        l2, mx = rel_errs(gS[b], o_S[b])
        print(f"B={batch} seq {b}: S rel_l2={l2:.2e} rel_max={mx:.2e}; outputs worst {worst:.2e}", flush=True)
        assert l2 <= 1e-3 and mx <= 1e-3
        assert np.array_equal(gcs[b], o_cs[b])  # the window is a pure shift/append
    assert worst <= 1e-3
    for buf in (d_S, d_cs, d_cw, d_a, d_dt, d_qkv, d_b, d_al, d_out):
        buf.free()


def test_deltanet_many_heads_batch1(gpu_ctx, oracle_lib):
    """Batch 1 with more heads than the in-kernel window commit has counters
    for (256 per head, 65536 in all): the step kernel without counters, then
    the window-commit launch.  260 heads, 4 steps: outputs every step, S and
    the conv windows (bit-exact) after the last, against the oracle."""
    h = 260
    ch = 3 * h * DK
    seed = 77
    conv_w = oracle_lib.normal(seed, 1, ch * 4, std=0.5)
    ssm_a = -oracle_lib.uniform(seed, 2, h)
    dt_bias = oracle_lib.normal(seed, 3, h)
    S0 = oracle_lib.normal(seed, 4, h * DK * DK, std=0.01)
    win0 = oracle_lib.normal(seed, 5, ch * 4)
    o_S, o_cs = S0.copy(), win0.copy()
    d_S, d_cs = gpu_ctx.to_device(S0), gpu_ctx.to_device(win0)
    d_cw, d_a, d_dt = gpu_ctx.to_device(conv_w), gpu_ctx.to_device(ssm_a), gpu_ctx.to_device(dt_bias)
    d_qkv, d_b, d_al = gpu_ctx.alloc(ch * 4), gpu_ctx.alloc(h * 4), gpu_ctx.alloc(h * 4)
    d_out = gpu_ctx.alloc(h * DK * 4)
    worst = 0.0
    for step in range(4):
        qkv = oracle_lib.normal(seed, 1000 + step, ch)
        br = oracle_lib.normal(seed, 2000 + step, h)
        ar = oracle_lib.normal(seed, 3000 + step, h)
        d_qkv.upload(qkv)
        d_b.upload(br)
        d_al.upload(ar)
        gpu_ctx.call("deltanet_step", 1, h, d_qkv, d_b, d_al, d_cw, d_a, d_dt, d_cs, d_S, d_out)
        ref = oracle_lib.deltanet_core(qkv, br, ar, conv_w, ssm_a, dt_bias, o_cs, o_S, h, DK)
        worst = max(worst, max(rel_errs(d_out.download(np.float32, h * DK), ref)))
    l2, mx = rel_errs(d_S.download(np.float32, h * DK * DK), o_S)
    print(f"260 heads: S rel_l2={l2:.2e} rel_max={mx:.2e}; outputs worst {worst:.2e}", flush=True)
    assert l2 <= 1e-3 and mx <= 1e-3 and worst <= 1e-3
    assert np.array_equal(d_cs.download(np.float32, ch * 4), o_cs)
    for buf in (d_S, d_cs, d_cw, d_a, d_dt, d_qkv, d_b, d_al, d_out):
        buf.free()


def test_deltanet_exact_recall_on_gpu(gpu_ctx, oracle_lib):
    """decay = 1 (ssm_a = 0), beta = 1 (beta_raw = 40): after one step S^T k = v."""
    conv_w = np.zeros((CH, 4), np.float32)
    conv_w[:, 3] = 1.0
    qkv = oracle_lib.normal(7, 1, CH)
    S = oracle_lib.normal(7, 2, H * DK * DK, std=0.01)
    d_S, d_cs = gpu_ctx.to_device(S), gpu_ctx.to_device(np.zeros(CH * 4, np.float32))
    d_out = gpu_ctx.alloc(H * DK * 4)
    gpu_ctx.call("deltanet_step", 1, H, gpu_ctx.to_device(qkv), gpu_ctx.to_device(np.full(H, 40.0, np.float32)),
                 gpu_ctx.to_device(np.zeros(H, np.float32)), gpu_ctx.to_device(conv_w),
                 gpu_ctx.to_device(np.zeros(H, np.float32)), gpu_ctx.to_device(np.zeros(H, np.float32)), d_cs, d_S,
                 d_out)
    Sg = d_S.download(np.float32, H * DK * DK).reshape(H, DK, DK).astype(np.float64)
    co = np_ref.silu(qkv.astype(np.float64))
    k = co[H * DK:2 * H * DK].reshape(H, DK)
    k /= np.linalg.norm(k, axis=1, keepdims=True)
    v = co[2 * H * DK:].reshape(H, DK)
    assert np.max(np.abs(np.einsum("hij,hi->hj", Sg, k) - v)) < 1e-5 * max(1.0, np.abs(v).max())


def test_gated_rmsnorm_parity(gpu_ctx, oracle_lib):
    B = 3
    heads = oracle_lib.normal(8, 1, B * H * DK)
    gate = oracle_lib.normal(8, 2, B * H * DK)
    w = oracle_lib.normal(8, 3, DK, mean=1.0, std=0.1)
    d_out = gpu_ctx.alloc(heads.nbytes)
    gpu_ctx.call("gated_rmsnorm", B, H, gpu_ctx.to_device(heads), gpu_ctx.to_device(gate), gpu_ctx.to_device(w),
                 1e-6, d_out)
    g = d_out.download(np.float32, heads.size).reshape(B, -1)
    for b in range(B):
        ref = oracle_lib.gated_rmsnorm(heads.reshape(B, -1)[b], gate.reshape(B, -1)[b], w, H, 1e-6)
        assert max(rel_errs(g[b], ref)) <= 1e-5


# ------------------------------------------------------------ attention ---

def _attn_case(gpu_ctx, oracle_lib, batch, n_heads, n_kv, max_seq, positions, seed, tol=2e-4):
    hd = 256
    stride = n_heads * 2 * hd + 2 * n_kv * hd
    qkv = oracle_lib.normal(seed, 1, batch * stride).reshape(batch, stride)
    qn = oracle_lib.normal(seed, 2, hd, mean=1.0, std=0.1)
    kn = oracle_lib.normal(seed, 3, hd, mean=1.0, std=0.1)
    hist = oracle_lib.normal(seed, 4, batch * n_kv * max_seq * hd)
    kc = oracle_lib.f32_to_f16(hist).reshape(batch, n_kv, max_seq, hd)
    vc = oracle_lib.f32_to_f16(oracle_lib.normal(seed, 5, batch * n_kv * max_seq * hd)).reshape(kc.shape)
    pos = np.array(positions, np.uint32)
    d_k, d_v = gpu_ctx.to_device(kc), gpu_ctx.to_device(vc)
    d_out = gpu_ctx.alloc(batch * n_heads * hd * 4)
    gpu_ctx.call("attention_step", batch, n_heads, n_kv, max_seq, gpu_ctx.to_device(qkv), gpu_ctx.to_device(qn),
                 gpu_ctx.to_device(kn), 10000.0, gpu_ctx.to_device(pos), d_k, d_v, d_out)
    out = d_out.download(np.float32, batch * n_heads * hd).reshape(batch, -1)
    gk = d_k.download(np.uint16, kc.size).reshape(kc.shape)
    gv = d_v.download(np.uint16, vc.size).reshape(vc.shape)
    for b in range(batch):
        p = int(pos[b])
        okc, ovc = kc[b].copy(), vc[b].copy()
        q_full = qkv[b, :n_heads * 2 * hd]
        k_in = qkv[b, n_heads * 2 * hd:n_heads * 2 * hd + n_kv * hd]
        v_in = qkv[b, n_heads * 2 * hd + n_kv * hd:]
        ref = oracle_lib.attention_core(q_full, k_in, v_in, qn, kn, okc, ovc, p, n_heads, n_kv, hd)
        l2, mx = rel_errs(out[b], ref)
        print(f"attn b={b} pos={p} heads={n_heads}/{n_kv}: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
        assert l2 <= tol and mx <= tol
        # appended rows: v exact, k within one fp16 ulp (sin/cos/sqrt rounding)
        assert np.array_equal(gv[b, :, p], ovc[:, p])
        kd = np.abs(oracle_lib.f16_to_f32(gk[b, :, p]).astype(np.float64) - oracle_lib.f16_to_f32(okc[:, p]))
        assert np.all(kd <= np.abs(oracle_lib.f16_to_f32(okc[:, p])) * 2 ** -10 + 1e-7)
        # nothing else of the cache changed
        mask = np.ones(max_seq, bool)
        mask[p] = False
        assert np.array_equal(gk[b][:, mask], kc[b][:, mask]) and np.array_equal(gv[b][:, mask], vc[b][:, mask])


@pytest.mark.parametrize("positions", [[0, 1], [63, 64], [65, 127], [128, 299]])
def test_attention_chunk_boundaries(gpu_ctx, oracle_lib, positions):
    _attn_case(gpu_ctx, oracle_lib, 2, 8, 2, 300, positions, seed=sum(positions) + 11)


def test_attention_live_length_split(gpu_ctx, oracle_lib):
    """An 8192-position cache at batch 8 (16 chunks per sequence and kv head)
    holding ragged live lengths: fewer live tiles than chunks, uneven splits
    of the live tiles over all chunks, the cache's last position."""
    _attn_case(gpu_ctx, oracle_lib, 8, 8, 2, 8192, [0, 63, 64, 700, 4095, 5000, 8000, 8191], seed=77, tol=5e-4)


@pytest.mark.parametrize("n_heads,n_kv", [(8, 2), (4, 2), (2, 2)])
def test_attention_gqa_ratios(gpu_ctx, oracle_lib, n_heads, n_kv):
    _attn_case(gpu_ctx, oracle_lib, 1, n_heads, n_kv, 200, [150], seed=n_heads * 10 + n_kv)


@pytest.mark.parametrize("ctx_len", [1024, 8192, 32768])
def test_attention_long_context(gpu_ctx, oracle_lib, ctx_len):
    """Config 4 contexts: the step at pos = ctx - 1 over a full fp16 cache."""
    _attn_case(gpu_ctx, oracle_lib, 1, 8, 2, ctx_len, [ctx_len - 1], seed=ctx_len, tol=5e-4)


# ------------------------------------------------------------ elementwise -

def test_rmsnorm_rows(gpu_ctx, oracle_lib):
    rows, n = 5, 2048
    x = oracle_lib.normal(9, 1, rows * n, std=2.0)
    w = oracle_lib.normal(9, 2, n, mean=1.0, std=0.1)
    d_out = gpu_ctx.alloc(x.nbytes)
    gpu_ctx.call("rmsnorm", gpu_ctx.to_device(x), gpu_ctx.to_device(w), d_out, rows, n, 1e-6)
    g = d_out.download(np.float32, x.size).reshape(rows, n)
    for r in range(rows):
        assert max(rel_errs(g[r], oracle_lib.rmsnorm(x.reshape(rows, n)[r], w, 1e-6))) <= 1e-6


def test_silu_mul_and_residual(gpu_ctx, oracle_lib):
    n = 6144 * 3 + 17
    a = oracle_lib.normal(10, 1, n, std=3.0)
    b = oracle_lib.normal(10, 2, n)
    da, db = gpu_ctx.to_device(a), gpu_ctx.to_device(b)
    gpu_ctx.call("silu_mul", da, db, n)
    ref = a.copy()
    oracle_lib.lib().ao_silu_mul_inplace(ref, b, n)
    assert max(rel_errs(da.download(np.float32, n), ref)) <= 1e-6
    x = oracle_lib.normal(10, 3, n)
    dx = gpu_ctx.to_device(x)
    gpu_ctx.call("residual_add", dx, db, n)
    assert np.array_equal(dx.download(np.float32, n), x + b)


def test_argmax_total_cmp(gpu_ctx, oracle_lib):
    rows, n = 4, 151936
    lg = oracle_lib.normal(11, 1, rows * n).reshape(rows, n)
    lg[1, 5] = lg[1, 70000] = lg[1, 151935] = 50.0   # ties: last index wins
    lg[2, :] = -np.inf
    lg[2, 1234] = np.nan                                # positive NaN is the maximum
    lg[3, :] = 0.0
    lg[3, 100] = -0.0                                   # -0.0 < +0.0
    d_out = gpu_ctx.alloc(rows * 4)
    gpu_ctx.call("argmax", gpu_ctx.to_device(lg), rows, n, d_out)
    got = d_out.download(np.uint32, rows)
    exp = [oracle_lib.argmax(lg[r]) for r in range(rows)]
    assert list(got) == exp
    assert exp[1] == 151935 and exp[2] == 1234 and exp[3] == n - 1


@pytest.mark.parametrize("n", [1000, 131072, 131073])
def test_argmax_row_lengths(gpu_ctx, oracle_lib, n):
    """Rows shorter than one strided pass of the 64 x 256 threads (8 values
    each) and rows ending exactly at, or one past, a pass: the maximum at the
    last index, a tie with it earlier, and a row whose maximum sits in the
    second pass's only value."""
    rows = 3
    lg = oracle_lib.normal(13, n, rows * n).reshape(rows, n)
    lg[0, n - 1] = 40.0
    lg[1, 7] = lg[1, n - 1] = 40.0
    lg[2, :] = -1.0
    lg[2, n - 1] = 2.0
    d_out = gpu_ctx.alloc(rows * 4)
    gpu_ctx.call("argmax", gpu_ctx.to_device(lg), rows, n, d_out)
    got = d_out.download(np.uint32, rows)
    assert list(got) == [oracle_lib.argmax(lg[r]) for r in range(rows)] == [n - 1] * rows


# ------------------------------------------------------------ utilities ---

@pytest.mark.parametrize("t", [8, 2])
def test_device_quantiser_matches_oracle_bits(gpu_ctx, oracle_lib, t):
    m, n = 96, 2048
    w = oracle_lib.normal(12, t, m * n, std=0.02).reshape(m, n)
    w[0, :32] = 0.0
    w[1, 5] = 1e-30
    out = gpu_ctx.alloc(oracle_lib.quant_bytes(t, m, n))
    gpu_ctx.call("quantize", t, gpu_ctx.to_device(w), m, n, out)
    assert np.array_equal(out.download(np.uint8, oracle_lib.quant_bytes(t, m, n)), oracle_lib.quantize(t, w))


def test_fill_random_is_deterministic(gpu_ctx):
    n = 1 << 20
    a, b = gpu_ctx.alloc(4 * n), gpu_ctx.alloc(4 * n)
    gpu_ctx.call("fill_random", a, n, 0, 0, 5, 0.0, 1.0)
    gpu_ctx.call("fill_random", b, n, 0, 0, 5, 0.0, 1.0)
    x, y = a.download(np.float32, n), b.download(np.float32, n)
    assert np.array_equal(x, y)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    gpu_ctx.call("fill_random", a, n, 1, 0, 6, -1.0, 0.0)
    u = a.download(np.float32, n)
    assert u.min() > -1.0 and u.max() < 0.0 and abs(u.mean() + 0.5) < 0.01
