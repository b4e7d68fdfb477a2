"""Graph capture of kernel-level calls (anehip_capture_begin / _end /
anehip_graph_launch): every replay reproduces the eager results bit for bit,
also with other eager work and synchronisations between replays, and a call
that would have to grow the workspace is refused during capture."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_replays_match_eager_bits(gpu_ctx, oracle_lib, anehip_mod):
    ctx = gpu_ctx
    m, n, rows = 2048, 6144, 4
    w = oracle_lib.gen_quant(8, 31, 32, m, n, std=0.02)
    x = oracle_lib.normal(31, 33, rows * n).astype(np.float32)
    nw = oracle_lib.normal(31, 34, m).astype(np.float32)
    dw, dx, dnw = ctx.to_device(w), ctx.to_device(x), ctx.to_device(nw)
    nbytes = int(anehip_mod.lib().anehip_quant_packed_bytes(8, m, n))
    dp = ctx.alloc(nbytes)
    ctx.call("quant_pack", 8, dw, m, n, dp)
    y4, y1, yn = ctx.alloc(rows * m * 4), ctx.alloc(m * 4), ctx.alloc(m * 4)

    def enqueue():
        ctx.quant_gemm(8, dw, m, n, dx, rows, y4)
        ctx.call("quant_gemv_packed", 8, dp, m, n, dx, y1)
        ctx.call("rmsnorm", y1, dnw, yn, 1, m, 1e-6)

    def read():
        return (y4.download(np.float32, rows * m), y1.download(np.float32, m), yn.download(np.float32, m))

    enqueue()
    eager = read()
    ctx.capture_begin()
    enqueue()
    g = ctx.capture_end()
    scratch = ctx.alloc(rows * m * 4)
    try:
        for rep in range(4):
            for buf in (y4, y1, yn):
                ctx.call("dev_memset", buf, 0xFF, buf.nbytes)  # poison between replays
            ctx.quant_gemm(8, dw, m, n, dx, 2, scratch)       # unrelated eager work
            ctx.sync()
            ctx.graph_launch(g)
            ctx.sync()
            for a, b in zip(read(), eager):
                assert np.array_equal(a, b), f"replay {rep}"
    finally:
        ctx.graph_destroy(g)
    for b in (dw, dx, dnw, dp, y4, y1, yn, scratch):
        b.free()


def test_workspace_growth_refused_during_capture(oracle_lib, anehip_mod):
    ctx = anehip_mod.Context(0)  # fresh context: empty workspace
    try:
        m, n = 4096, 6144
        w = oracle_lib.gen_quant(8, 41, 42, m, n)
        dw, dx, dy = ctx.to_device(w), ctx.to_device(np.ones(32 * n, np.float32)), ctx.alloc(32 * m * 4)
        ctx.capture_begin()
        with pytest.raises(anehip_mod.AnehipError) as e:
            ctx.quant_gemm(8, dw, m, n, dx, 16, dy)
        assert e.value.code == -6 and "capture" in str(e.value)
        g = ctx.capture_end()
        ctx.graph_destroy(g)
        ctx.quant_gemm(8, dw, m, n, dx, 16, dy)  # eager: grows the workspace, runs
        ctx.sync()
    finally:
        ctx.close()


def test_memset_refused_during_capture(gpu_ctx, anehip_mod):
    ctx = gpu_ctx
    buf = ctx.alloc(4096)
    ctx.capture_begin()
    with pytest.raises(anehip_mod.AnehipError) as e:
        ctx.call("dev_memset", buf, 0, 4096)
    assert e.value.code == -6 and "captur" in str(e.value)
    g = ctx.capture_end()
    ctx.graph_destroy(g)
    ctx.call("dev_memset", buf, 0, 4096)
    ctx.sync()
    buf.free()
