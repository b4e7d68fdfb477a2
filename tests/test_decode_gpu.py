"""GPU parity of the full decode step (anehip_decode_step) against the oracle's
restatement of qwen35_forward_token (crates/cli/src/main.rs:953-1023).
Bound: logits within 1e-3 relative (rel L2 and max-abs / max |ref|)."""
import numpy as np
import pytest

import anehip
import oracle
from conftest import rel_errs
from model_util import MID, SMALL, WIDE, HostModel, copy_state_to_oracle

pytestmark = pytest.mark.gpu

TOL = 1e-3


@pytest.fixture(scope="module")
def small_host():
    return HostModel(anehip.Spec(**SMALL), seed=3)


def _model(host, batch, max_seq, graph=True):
    gm = anehip.Model(host.spec)
    host.upload(gm)
    gm.alloc_state(batch, max_seq)
    gm.set_graph(graph)
    return gm


def test_small_model_steps_from_zero(small_host):
    gm = _model(small_host, 1, 64)
    oseq = small_host.seq(64)
    toks = oracle.randint(5, 1, 10, small_host.spec.vocab_size)
    for i, t in enumerate(toks):
        g = gm.step([t])[0]
        r = oseq.forward(int(t))
        l2, mx = rel_errs(g, r)
        print(f"step {i}: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
        assert l2 <= TOL and mx <= TOL
    assert gm.get_pos(0) == 10 and oseq.pos == 10
    # recurrent states, conv windows and KV rows after 10 steps (at batch 1
    # the DeltaNet updates are committed by the step's last kernels)
    _check_state(gm, oseq, 0, small_host.spec, "after 10 steps")
    gm.close()
    oseq.close()


def test_batch_is_independent_sequences(small_host):
    B = 3
    gm = _model(small_host, B, 32)
    seqs = [small_host.seq(32) for _ in range(B)]
    toks = oracle.randint(6, 2, 5 * B, small_host.spec.vocab_size).reshape(5, B)
    for step in range(5):
        g = gm.step(toks[step])
        for b in range(B):
            l2, mx = rel_errs(g[b], seqs[b].forward(int(toks[step, b])))
            assert l2 <= TOL and mx <= TOL
    gm.close()


@pytest.fixture(scope="module")
def mid_host():
    return HostModel(anehip.Spec(**MID), seed=5)


@pytest.mark.parametrize("B", [2, 7, 20, 32])
def test_mid_model_batched_steps(mid_host, B):
    """Every sequence of a batched step vs the oracle over 4 steps (graph
    replays), on the mid-size model: K-split partial sums of 2 and 4 splits
    read by the DeltaNet / attention kernels, SiLU-mul and residual RMSNorm
    (at 20 and 32 rows sliced per row, the norm's scale applied by the
    consuming GEMM; batch rows past 20 of its 32-row tiles unused)."""
    steps = 4
    toks = oracle.randint(21, B, steps * B, mid_host.spec.vocab_size).reshape(steps, B)
    gm = _model(mid_host, B, 32)
    seqs = [mid_host.seq(32) for _ in range(B)]
    for step in range(steps):
        g = gm.step(toks[step])
        for b in range(B):
            l2, mx = rel_errs(g[b], seqs[b].forward(int(toks[step, b])))
            assert l2 <= TOL and mx <= TOL, (step, b, l2, mx)
    gm.close()
    for q in seqs:
        q.close()


@pytest.mark.parametrize("B", [1, 2])
def test_wide_model_unfused_deltanet_step(B):
    """The 2304-wide model (model_util.WIDE): at batch 1 the DeltaNet step is
    deltanet_step_kernel followed by ssm_out with the gated-norm prologue that
    commits the conv windows (the path models up to 2048 wide never take);
    at batch 2 the 9-panel projections run on uneven K splits.  4 steps from
    position 0 vs the oracle per sequence: logits, then every layer's
    DeltaNet state, conv window and KV rows."""
    host = HostModel(anehip.Spec(**WIDE), seed=9)
    spec = host.spec
    gm = _model(host, B, 64)
    seqs = [host.seq(64) for _ in range(B)]
    toks = oracle.randint(37, B, 4 * B, spec.vocab_size).reshape(4, B)
    for step in range(4):
        g = gm.step(toks[step])
        for b in range(B):
            l2, mx = rel_errs(g[b], seqs[b].forward(int(toks[step, b])))
            print(f"wide B={B} step {step} seq {b}: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
            assert l2 <= TOL and mx <= TOL, (step, b)
    for b in range(B):
        _check_state(gm, seqs[b], b, spec, f"wide B={B} seq {b} after 4 steps")
    gm.close()
    for q in seqs:
        q.close()


def _check_state(gm, oseq, b, spec, what):
    """Sequence b's DeltaNet states / conv windows / KV rows against an oracle sequence."""
    for l in range(spec.n_layers):
        if spec.layer_types[l] == anehip.LAYER_DELTANET:
            for which in (0, 1):
                g = gm.get_state(l, which, b)
                r = oseq.view(l, which, g.size, np.float32)
                assert max(rel_errs(g, r)) <= TOL, (what, l, which)
        else:
            p = gm.get_pos(b)
            for which in (2, 3):
                g = gm.get_state(l, which, b).reshape(spec.n_kv_heads, -1, spec.head_dim)[:, :p]
                r = oseq.view(l, which, spec.n_kv_heads * oseq.max_seq * spec.head_dim,
                              np.uint16).reshape(spec.n_kv_heads, -1, spec.head_dim)[:, :p]
                gf = g.view(np.float16).astype(np.float32)
                rf = r.view(np.float16).astype(np.float32)
                assert max(rel_errs(gf, rf)) <= TOL, (what, l, which)


@pytest.mark.parametrize("n", [1, 13, 45])
def test_prefill_matches_token_steps(small_host, n):
    """anehip_prefill of n prompt tokens (one chunk; 45 rows run the chunk
    GEMM, 1 and 13 the decode GEMMs) from position 0 vs the oracle run token
    by token: the last token's logits, the DeltaNet states / conv windows and
    the KV rows written, then 3 decode steps continuing the sequence."""
    spec = small_host.spec
    gm = _model(small_host, 1, 64)
    oseq = small_host.seq(64)
    toks = oracle.randint(31, n, n, spec.vocab_size)
    g = gm.prefill(0, toks)
    for t in toks:
        r = oseq.forward(int(t))
    l2, mx = rel_errs(g, r)
    print(f"prefill n={n}: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
    assert l2 <= TOL and mx <= TOL
    assert gm.get_pos(0) == n
    _check_state(gm, oseq, 0, spec, "after prefill")
    for t in oracle.randint(32, n, 3, spec.vocab_size):
        assert max(rel_errs(gm.step([t])[0], oseq.forward(int(t)))) <= TOL
    _check_state(gm, oseq, 0, spec, "after prefill and 3 steps")
    gm.close()
    oseq.close()


def test_prefill_one_sequence_of_a_batch(mid_host):
    """On the mid-size model (K-split projections), batch 3: after two decode
    steps of every sequence, sequence 1 prefills 40 tokens (one chunk) from
    position 2; its logits and state follow the oracle, sequences 0 and 2 keep
    their state and positions, and a batched step afterwards matches the
    oracle for every sequence."""
    spec = mid_host.spec
    B = 3
    gm = _model(mid_host, B, 64)
    seqs = [mid_host.seq(64) for _ in range(B)]
    for step in range(2):
        toks = oracle.randint(40 + step, B, B, spec.vocab_size)
        g = gm.step(toks)
        for b in range(B):
            assert max(rel_errs(g[b], seqs[b].forward(int(toks[b])))) <= TOL
    before = {b: [gm.get_state(l, 1).reshape(B, -1)[b].copy() for l in (0, 1)] for b in (0, 2)}
    prompt = oracle.randint(50, 40, 40, spec.vocab_size)
    g1 = gm.prefill(1, prompt)
    for t in prompt:
        r1 = seqs[1].forward(int(t))
    assert max(rel_errs(g1, r1)) <= TOL
    assert [gm.get_pos(b) for b in range(B)] == [2, 42, 2]
    for b in (0, 2):
        for i, l in enumerate((0, 1)):
            assert np.array_equal(gm.get_state(l, 1).reshape(B, -1)[b], before[b][i])
    _check_state(gm, seqs[1], 1, spec, "after prefill")
    toks = oracle.randint(60, B, B, spec.vocab_size)
    g = gm.step(toks)
    for b in range(B):
        assert max(rel_errs(g[b], seqs[b].forward(int(toks[b])))) <= TOL
    gm.close()
    for q in seqs:
        q.close()


@pytest.mark.parametrize("which,B", [("small", 1), ("small", 2), ("small", 32), ("mid", 1), ("mid", 2), ("mid", 7),
                                     ("mid", 32)])
def test_activations_beyond_fp16_range(which, B):
    """Steps whose GEMM inputs leave fp16's range: post-attention and
    DeltaNet output norm weights scaled by 3e4 (FFN inputs, SiLU-mul outputs
    and gated-norm outputs reach 1e5 - 1e9) and q-norm weights by 1e5 (the
    attention's q operand).  At batch > 1 the element-wise kernels write
    range-safe planes and the GEMMs / attention scale them back; at batch 1
    the GEMV prologues digitise each block with its own exponent: logits
    match the fp32 oracle (1e-3) over 3 steps for every sequence."""
    spec = anehip.Spec(**(SMALL if which == "small" else MID))
    host = HostModel(spec, seed=41)
    scale = {anehip.T["POST_ATTN_NORM"]: 3e4, anehip.T["SSM_NORM"]: 3e4, anehip.T["Q_NORM"]: 1e5}
    for (layer, kind), (arr, rows, cols, quant) in host.tensors.items():
        if kind in scale:
            arr *= np.float32(scale[kind])
            host.om.set_f32(layer, kind, arr)
    gm = _model(host, B, 16)
    seqs = [host.seq(16) for _ in range(B)]
    for step in range(3):
        toks = oracle.randint(42, step, B, spec.vocab_size)
        g = gm.step(toks)
        assert np.all(np.isfinite(g))
        for b in range(B):
            l2, mx = rel_errs(g[b], seqs[b].forward(int(toks[b])))
            assert l2 <= TOL and mx <= TOL, (step, b, l2, mx)
    gm.close()
    for q in seqs:
        q.close()


def test_prefill_rejects_bad_arguments(small_host):
    gm = _model(small_host, 2, 16)
    with pytest.raises(anehip.AnehipError) as e:
        gm.prefill(2, [1, 2, 3])
    assert e.value.code == -1  # ANEHIP_EINVAL
    with pytest.raises(anehip.AnehipError) as e:
        gm.prefill(0, np.arange(17))
    assert e.value.code == -7  # ANEHIP_ERANGE
    assert gm.get_pos(0) == 0
    gm.close()


def test_graph_replay_matches_eager_bits(small_host):
    toks = oracle.randint(7, 3, 6, small_host.spec.vocab_size)
    outs = []
    for graph in (False, True):
        gm = _model(small_host, 1, 16, graph=graph)
        outs.append(np.stack([gm.step([t])[0] for t in toks]))
        gm.close()
    assert np.array_equal(outs[0], outs[1])


def test_token_beyond_vocab_uses_zero_embedding(small_host):
    gm = _model(small_host, 1, 8)
    oseq = small_host.seq(8)
    g = gm.step([small_host.spec.vocab_size + 5])[0]
    r = oseq.forward(small_host.spec.vocab_size + 5)
    assert max(rel_errs(g, r)) <= TOL
    gm.close()


def test_token_beyond_vocab_batch32(mid_host):
    """The same at batch 32 on the mid-size model, where the embedding gather
    runs one wave per 256-column slice and leaves the RMSNorm scale to the
    first projection: every sequence over 2 steps, tokens past the
    vocabulary in a few of them."""
    B = 32
    V = mid_host.spec.vocab_size
    gm = _model(mid_host, B, 8)
    seqs = [mid_host.seq(8) for _ in range(B)]
    for step in range(2):
        toks = oracle.randint(77, step, B, V)
        toks[3 + step] = V + 5
        toks[31] = V + 1000 * step
        g = gm.step(toks)
        for b in range(B):
            assert max(rel_errs(g[b], seqs[b].forward(int(toks[b])))) <= TOL, (step, b)
    gm.close()
    for q in seqs:
        q.close()


def test_generate_feeds_back_on_device(small_host):
    gm = _model(small_host, 2, 40)
    out = gm.generate([1, 2], 12)
    gm2 = _model(small_host, 2, 40)
    tok = np.array([1, 2], np.uint32)
    for i in range(12):
        gm2.step(tok, want_logits=False)
        tok = gm2.sampled()
        assert np.array_equal(out[i], tok)
    # the greedy choice is the oracle's argmax of the same logits
    oseq = small_host.seq(40)
    t = 1
    for i in range(4):
        t = oracle.argmax(oseq.forward(t))
        assert t == out[i, 0]
    gm.close()
    gm2.close()


def test_generate_ragged_positions_and_continuation(small_host):
    """Greedy feedback and the token record stay inside the step graph: from
    ragged start positions, one generate of 10 steps equals generate(4) +
    generate(6) continued from the last sampled tokens, and equals stepping
    one token at a time."""
    def fresh():
        gm = _model(small_host, 3, 48)
        for b, p in enumerate((0, 5, 17)):
            gm.set_pos(b, p)
        return gm

    first = [3, 7, 11]
    gm = fresh()
    out = gm.generate(first, 10)
    assert [gm.get_pos(b) for b in range(3)] == [10, 15, 27]
    gm2 = fresh()
    a = gm2.generate(first, 4)
    b = gm2.generate(a[-1], 6)
    assert np.array_equal(np.concatenate([a, b]), out)
    gm3 = fresh()
    tok = np.array(first, np.uint32)
    for i in range(10):
        gm3.step(tok, want_logits=False)
        tok = gm3.sampled()
        assert np.array_equal(out[i], tok), i
    for g in (gm, gm2, gm3):
        g.close()


def test_gguf_copy_dropped_and_rebuilt(small_host):
    """After the first step the GGUF copy of each matrix is dropped (the step
    reads the panel copy); re-uploading one part of a stacked matrix rebuilds
    it from the panels (the inverse permutation) and the step then matches a
    model uploaded with the new part from the start; a tensor read back after
    the drop equals what was uploaded."""
    T = anehip.T
    s = small_host.spec
    rows, cols, _ = s.shapes(0)[T["FFN_UP"]]
    new_up = oracle.gen_quant(8, 77, 78, rows, cols, std=anehip.WEIGHT_STD)
    gm = _model(small_host, 1, 16)
    gm.step([1], want_logits=False)  # packs the weights, drops the GGUF copies
    got = gm.download_tensor(0, T["FFN_GATE"])
    assert np.array_equal(got, small_host.tensors[(0, T["FFN_GATE"])][0])
    gm.upload_quant(0, T["FFN_UP"], new_up, rows, cols)
    gm.reset_state()
    y = gm.step([2])
    ref = anehip.Model(s)
    small_host.upload(ref)
    ref.upload_quant(0, T["FFN_UP"], new_up, rows, cols)
    ref.alloc_state(1, 16)
    y_ref = ref.step([2])
    assert np.array_equal(y, y_ref)
    gm.close()
    ref.close()


def test_errors(small_host):
    gm = anehip.Model(small_host.spec)
    with pytest.raises(anehip.AnehipError) as e:
        gm.alloc_state(1, 4)
        gm.step([1])
    assert e.value.code == -6 and "not uploaded" in str(e.value)
    small_host.upload(gm)
    gm.alloc_state(1, 2)
    gm.step([1])
    gm.step([2])
    with pytest.raises(anehip.AnehipError) as e:
        gm.step([3])
    assert e.value.code == -7
    with pytest.raises(anehip.AnehipError) as e:
        gm.step([1, 2])
    assert e.value.code == -2
    with pytest.raises(anehip.AnehipError) as e:
        gm.upload_quant(0, anehip.T["QKV"], np.zeros(10, np.uint8), 768, 256)
    assert e.value.code == -2
    gm.close()


def test_q4_0_model(small_host):
    host = HostModel(anehip.Spec(**SMALL), seed=4, ggml_type=2)
    gm = _model(host, 1, 16)
    oseq = host.seq(16)
    for t in (3, 999, 0, 500):
        assert max(rel_errs(gm.step([t])[0], oseq.forward(t))) <= TOL
    gm.close()


def test_q4_0_model_prefill():
    """A Q4_0 model's 70-token prefill (the chunk GEMM on Q4_0 panels at 70
    rows) vs the oracle run token by token: last logits and states."""
    host = HostModel(anehip.Spec(**SMALL), seed=5, ggml_type=2)
    spec = host.spec
    gm = _model(host, 1, 128)
    oseq = host.seq(128)
    toks = oracle.randint(35, 70, 70, spec.vocab_size)
    g = gm.prefill(0, toks)
    for t in toks:
        r = oseq.forward(int(t))
    l2, mx = rel_errs(g, r)
    print(f"Q4_0 prefill 70: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
    assert l2 <= TOL and mx <= TOL
    _check_state(gm, oseq, 0, spec, "Q4_0 after prefill")
    gm.close()
    oseq.close()


# ---------------------------------------------- Qwen3.5-2B shape (config 4) --

@pytest.fixture(scope="module")
def big_host():
    return HostModel(anehip.Spec(), seed=11)


def _fill_state(gm, spec, seed=0):
    """DeltaNet states N(0, 0.01), conv windows N(0, 1), fp16 KV N(0, 1)."""
    for l in range(spec.n_layers):
        if spec.layer_types[l] == anehip.LAYER_DELTANET:
            p, n = gm.state_ptr(l, 0)
            gm.fill_random(p, n // 4, 0, seed + 100 + l, 0.0, 1.0)
            p, n = gm.state_ptr(l, 1)
            gm.fill_random(p, n // 4, 0, seed + 200 + l, 0.0, 0.01)
        else:
            for which in (2, 3):
                p, n = gm.state_ptr(l, which)
                gm.fill_random(p, n // 2, 0, seed + 300 + 10 * l + which, 0.0, 1.0, f16=True)


def _step_vs_oracle(host, gm, positions, check, tok_seed, steps=1, label="", dn_state=False):
    """Sets every sequence's position, copies the checked sequences' state to
    oracle sequences and compares `steps` decode steps' logits (and with
    dn_state, the checked sequences' DeltaNet states and conv windows after
    the last step)."""
    spec = host.spec
    for b, p in enumerate(positions):
        gm.set_pos(b, int(p))
    seqs = {}
    for b in check:
        seqs[b] = host.seq(gm.max_seq)
        copy_state_to_oracle(gm, seqs[b], b)
    for step in range(steps):
        toks = oracle.randint(tok_seed, step, len(positions), spec.vocab_size)
        g = gm.step(toks)
        for b in check:
            r = seqs[b].forward(int(toks[b]))
            l2, mx = rel_errs(g[b], r)
            print(f"{label} step {step} seq {b} pos {int(positions[b]) + step}: rel_l2={l2:.2e} rel_max={mx:.2e}",
                  flush=True)
            assert l2 <= TOL and mx <= TOL, (label, step, b)
    if dn_state:
        for b in check:
            for l in range(spec.n_layers):
                if spec.layer_types[l] == anehip.LAYER_DELTANET:
                    for which in (0, 1):
                        g = gm.get_state(l, which, b)
                        assert max(rel_errs(g, seqs[b].view(l, which, g.size, np.float32))) <= TOL, (label, l, which)
    for q in seqs.values():
        q.close()


@pytest.mark.parametrize("ctx_len,batch", [(1024, 1), (8192, 1), (32768, 1), (1024, 32), (8192, 32),
                                           (32768, 32)])
def test_qwen35_2b_shape_step(big_host, ctx_len, batch):
    """Random-init 24-layer Qwen3.5-2B shape, Q8_0 weights, fp16 KV cache
    filled with N(0,1) at positions < ctx-1, DeltaNet states N(0, 0.01)
    (windows N(0,1)); one step at pos = ctx-1 (cache capacity = ctx) vs the
    oracle, sequences 0 and batch-1: logits, then the DeltaNet states and
    conv windows."""
    gm = _model(big_host, batch, ctx_len)
    _fill_state(gm, big_host.spec)
    _step_vs_oracle(big_host, gm, [ctx_len - 1] * batch, sorted({0, batch - 1}), 12,
                    label=f"2B ctx={ctx_len} B={batch}", dn_state=True)
    gm.close()


@pytest.fixture(scope="module")
def big_host_q4():
    return HostModel(anehip.Spec(), seed=12, ggml_type=2)


@pytest.mark.parametrize("batch", [1, 32])
def test_qwen35_2b_shape_q4_0_step(big_host_q4, batch):
    """The 2B shape with Q4_0 weights on every linear layer (the model the
    bench's decode_q4 times): one step at pos 1023 (cache capacity 1024) vs
    the oracle, sequences 0 and batch - 1: logits, then the DeltaNet states
    and conv windows."""
    gm = _model(big_host_q4, batch, 1024)
    _fill_state(gm, big_host_q4.spec, seed=3)
    _step_vs_oracle(big_host_q4, gm, [1023] * batch, sorted({0, batch - 1}), 15, label=f"2B Q4_0 B={batch}",
                    dn_state=True)
    gm.close()


@pytest.mark.parametrize("batch,positions,check", [
    (1, [1023], [0]),
    (1, [8191], [0]),
    # ragged live lengths in one batch: a single position, a partial first
    # tile, tile and chunk boundaries, mid-tile / mid-chunk positions and the
    # cache's last position
    (32, [1023, 0, 5, 63, 64, 3000, 8191, 8192, 12345, 20000, 32767] + [1000 + 977 * i for i in range(21)],
     [0, 1, 2, 5, 6, 7, 10, 31]),
])
def test_qwen35_2b_shape_live_length(big_host, batch, positions, check):
    """2B shape with a 32k-position cache holding shorter live contexts: the
    attention splits the live tiles, not the capacity, over its chunks; one
    step per sequence vs the oracle."""
    gm = _model(big_host, batch, 32768)
    _fill_state(gm, big_host.spec, seed=7)
    _step_vs_oracle(big_host, gm, positions, check, 13, label=f"2B cap=32k B={batch}")
    gm.close()


def test_ragged_positions_across_chunk_boundaries(mid_host):
    """Mid-size model, batch 4, 4096-position cache, positions 5 / 3000 / 63 /
    4090: 4 steps per sequence, so live lengths cross tile boundaries and the
    split of the live tiles over the chunks changes from step to step."""
    gm = _model(mid_host, 4, 4096)
    _fill_state(gm, mid_host.spec, seed=21)
    _step_vs_oracle(mid_host, gm, [5, 3000, 63, 4090], [0, 1, 2, 3], 14, steps=4, label="mid ragged")
    gm.close()


@pytest.mark.parametrize("n", [100, 300, 600])
def test_prefill_long_prompt_large_cache(mid_host, n):
    """anehip_prefill into a 2048-position cache of a 100-token prompt (one
    chunk on the chunk GEMM at 100 rows), a 300-token one (chunks of 256 and
    44) and a 600-token one (256, 256, 88: the second full chunk replays the
    graph the first captured; the DeltaNet scan runs 256 tokens per launch);
    chunk rows see up to 10 live tiles of attention; the last logits, states
    and KV rows vs the oracle run token by token, then 2 decode steps."""
    spec = mid_host.spec
    gm = _model(mid_host, 1, 2048)
    oseq = mid_host.seq(2048)
    toks = oracle.randint(33, n, n, spec.vocab_size)
    g = gm.prefill(0, toks)
    for t in toks:
        r = oseq.forward(int(t))
    l2, mx = rel_errs(g, r)
    print(f"prefill n={n} cap 2048: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
    assert l2 <= TOL and mx <= TOL
    _check_state(gm, oseq, 0, spec, "after prefill")
    for t in oracle.randint(34, n, 2, spec.vocab_size):
        assert max(rel_errs(gm.step([t])[0], oseq.forward(int(t)))) <= TOL
    gm.close()
    oseq.close()


@pytest.mark.parametrize("n", [40, 300])
def test_qwen35_2b_shape_prefill(big_host, n):
    """Random-init 24-layer Qwen3.5-2B shape: a 40-token prompt (one chunk) and
    a 300-token one (a full 256-token chunk, recorded as the prefill's chunk
    graph and replayed for it, then 44 rows) prefilled from position 0 vs the
    oracle run token by token: the last logits, every layer's DeltaNet state,
    conv window and KV rows, then one decode step continuing the sequence."""
    spec = big_host.spec
    gm = _model(big_host, 1, 512)
    oseq = big_host.seq(512)
    prompt = oracle.randint(70, n, n, spec.vocab_size)
    g = gm.prefill(0, prompt)
    for i, t in enumerate(prompt):
        r = oseq.forward(int(t))
        if i % 64 == 63:
            print(f"2B prefill {n}: oracle at token {i + 1}", flush=True)
    l2, mx = rel_errs(g, r)
    print(f"2B prefill {n}: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
    assert l2 <= TOL and mx <= TOL
    _check_state(gm, oseq, 0, spec, f"2B after prefill {n}")
    t = int(oracle.randint(71, 1, 1, spec.vocab_size)[0])
    assert max(rel_errs(gm.step([t])[0], oseq.forward(t))) <= TOL
    gm.close()
    oseq.close()
