"""anehip_attention_step_noalloc (the attention step on a static device
scratch, no allocation) against anehip_attention_step on the same inputs:
two calls in a row, the second smaller, bit-identical outputs and caches;
the call captured into a graph as the first call of a fresh context and
replayed, with calls of another rope_base between the replays; a call whose
partials exceed the scratch is refused before any launch."""
import ctypes as C

import numpy as np
import pytest

from conftest import rel_errs

pytestmark = pytest.mark.gpu

HD = 256


def _inputs(oracle_lib, batch, n_heads, n_kv, max_seq, positions, seed):
    stride = n_heads * 2 * HD + 2 * n_kv * HD
    qkv = oracle_lib.normal(seed, 1, batch * stride)
    qn = oracle_lib.normal(seed, 2, HD, mean=1.0, std=0.1)
    kn = oracle_lib.normal(seed, 3, HD, mean=1.0, std=0.1)
    kc = oracle_lib.f32_to_f16(oracle_lib.normal(seed, 4, batch * n_kv * max_seq * HD))
    vc = oracle_lib.f32_to_f16(oracle_lib.normal(seed, 5, batch * n_kv * max_seq * HD))
    return qkv, qn, kn, kc, vc, np.array(positions, np.uint32)


def _run(ctx, name, case, inputs, rope_base=10000.0):
    batch, n_heads, n_kv, max_seq = case
    qkv, qn, kn, kc, vc, pos = inputs
    d_k, d_v = ctx.to_device(kc), ctx.to_device(vc)
    d_out = ctx.alloc(batch * n_heads * HD * 4)
    ctx.call(name, batch, n_heads, n_kv, max_seq, ctx.to_device(qkv), ctx.to_device(qn), ctx.to_device(kn),
             rope_base, ctx.to_device(pos), d_k, d_v, d_out)
    ctx.sync()
    return (d_out.download(np.float32, batch * n_heads * HD), d_k.download(np.uint16, kc.size),
            d_v.download(np.uint16, vc.size))


def test_noalloc_matches_allocating_entry_point(gpu_ctx, oracle_lib):
    big = (4, 8, 2, 4096)
    small = (2, 8, 2, 300)
    in_big = _inputs(oracle_lib, *big, [4095, 0, 2000, 63], seed=81)
    in_small = _inputs(oracle_lib, *small, [299, 64], seed=82)
    print("noalloc: big then small", flush=True)
    got = [_run(gpu_ctx, "attention_step_noalloc", big, in_big),
           _run(gpu_ctx, "attention_step_noalloc", small, in_small)]
    print("allocating entry point: big then small", flush=True)
    ref = [_run(gpu_ctx, "attention_step", big, in_big), _run(gpu_ctx, "attention_step", small, in_small)]
    for g, r in zip(got, ref):
        for a, b in zip(g, r):
            assert np.array_equal(a, b)
    # and the small call against the oracle (the attention tests' bound)
    qkv, qn, kn, kc, vc, pos = in_small
    batch, n_heads, n_kv, max_seq = small
    out = got[1][0].reshape(batch, -1)
    for b in range(batch):
        row = qkv.reshape(batch, -1)[b]
        okc = kc.reshape(batch, n_kv, max_seq, HD)[b].copy()
        ovc = vc.reshape(batch, n_kv, max_seq, HD)[b].copy()
        r = oracle_lib.attention_core(row[:n_heads * 2 * HD], row[n_heads * 2 * HD:n_heads * 2 * HD + n_kv * HD],
                                      row[n_heads * 2 * HD + n_kv * HD:], qn, kn, okc, ovc, int(pos[b]), n_heads,
                                      n_kv, HD)
        assert max(rel_errs(out[b], r)) <= 2e-4


def test_noalloc_captured_as_first_call(gpu_ctx, oracle_lib, anehip_mod):
    """A fresh context's first noalloc call, recorded under graph capture,
    replays bit-identically to the allocating entry point at its own
    rope_base, also after eager noalloc calls with another rope_base (which
    rewrite the shared table) between the replays."""
    case = (2, 8, 2, 512)
    batch, n_heads, n_kv, max_seq = case
    qkv, qn, kn, kc, vc, pos = _inputs(oracle_lib, *case, [511, 70], seed=83)
    other = _inputs(oracle_lib, *case, [100, 3], seed=84)
    ref = _run(gpu_ctx, "attention_step", case, (qkv, qn, kn, kc, vc, pos), rope_base=5.0e5)
    ctx = anehip_mod.Context(0)
    try:
        d_q, d_qn, d_kn, d_pos = ctx.to_device(qkv), ctx.to_device(qn), ctx.to_device(kn), ctx.to_device(pos)
        d_k, d_v = ctx.to_device(kc), ctx.to_device(vc)
        d_out = ctx.alloc(batch * n_heads * HD * 4)
        ctx.sync()
        print("noalloc: capture as the context's first call", flush=True)
        ctx.capture_begin()
        ctx.call("attention_step_noalloc", batch, n_heads, n_kv, max_seq, d_q, d_qn, d_kn, 5.0e5, d_pos, d_k, d_v,
                 d_out)
        g = ctx.capture_end()
        try:
            for rep in range(3):
                ctx.call("dev_memset", d_out, 0xFF, d_out.nbytes)  # poison the output between replays
                _run(ctx, "attention_step_noalloc", case, other, rope_base=10000.0)  # rewrites the shared table
                print(f"noalloc: replay {rep}", flush=True)
                ctx.graph_launch(g)
                ctx.sync()
                got = (d_out.download(np.float32, batch * n_heads * HD), d_k.download(np.uint16, kc.size),
                       d_v.download(np.uint16, vc.size))
                for a, b in zip(got, ref):
                    assert np.array_equal(a, b), f"replay {rep}"
        finally:
            ctx.graph_destroy(g)
    finally:
        ctx.close()


def test_noalloc_refuses_oversized_call(gpu_ctx, anehip_mod):
    # batch 600 x 2 kv heads x 1 chunk x 4 heads x 258 floats > the 1,048,320-float scratch
    buf = gpu_ctx.alloc(1 << 20)
    p = C.c_void_p(buf.ptr)
    rc = anehip_mod.lib().anehip_attention_step_noalloc(gpu_ctx.h, 600, 8, 2, 64, p, p, p, C.c_float(10000.0), p, p,
                                                        p, p)
    assert rc == -7  # ANEHIP_ERANGE
    assert b"static scratch" in anehip_mod.lib().anehip_last_error(gpu_ctx.h)
