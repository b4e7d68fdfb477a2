"""GPU parity of the Q8_0 / Q4_0 GEMV and small-batch GEMM (anehip_quant_gemm)
against the CPU oracle's restatement of q8_gemv / q4_gemv_cpu
(crates/engine/src/q8_gemv.rs:67-148).  Bound: relative error <= 1e-4 in L2
and in max-abs / max |ref| (fp32 accumulate)."""
import json
import os

import numpy as np
import pytest

from conftest import rel_errs

pytestmark = pytest.mark.gpu

TOL = 1e-4
HERE = os.path.dirname(os.path.abspath(__file__))


def _run(ctx, t, w, m, n, x):
    batch = x.shape[0] if x.ndim == 2 else 1
    dw = ctx.to_device(w)
    dx = ctx.to_device(x.astype(np.float32))
    dy = ctx.alloc(batch * m * 4)
    ctx.quant_gemm(t, dw, m, n, dx, batch, dy)
    y = dy.download(np.float32, batch * m).reshape(batch, m)
    for b in (dw, dx, dy):
        b.free()
    return y


def test_reference_kat_identity_gemv(gpu_ctx, oracle_lib):
    """q8_gemv.rs:257-281 through the GPU path (padded to n = 256 with zero blocks)."""
    with open(os.path.join(HERE, "golden", "reference_kats.json")) as f:
        kat = json.load(f)["q8_gemv_identity"]
    m, n = kat["m"], 256
    blocks = np.zeros((m, n // 32, 34), np.uint8)
    blocks[:, 0, :] = np.array(kat["w"], np.uint8).reshape(m, 34)
    one = np.array([1.0], np.float16).view(np.uint16)[0]
    blocks[:, 1:, 0], blocks[:, 1:, 1] = one & 0xFF, one >> 8
    x = np.zeros(n, np.float32)
    x[:32] = kat["x"]
    y = _run(gpu_ctx, 8, blocks.reshape(-1), m, n, x[None])
    assert np.all(np.abs(y[0] - np.array(kat["expected"])) < 0.01)


def test_reference_kat_patterned_gemv(gpu_ctx, oracle_lib):
    """q8_gemv.rs:283-314 pattern (m=256, n=1024): integer-valued, exact in fp32."""
    from test_oracle import _patterned_w

    m, n = 256, 1024
    w = _patterned_w(m, n)
    x = (np.arange(n) % 100).astype(np.float32)
    y = _run(gpu_ctx, 8, w, m, n, x[None])[0]
    ref = oracle_lib.gemv(8, w, m, n, x)
    assert np.all(np.abs(y - ref) < 1e-3)


SHAPES = [(6144, 2048), (2048, 6144), (151936, 2048), (16, 2048), (100, 256), (4096, 2048), (512, 2048)]


@pytest.mark.parametrize("t", [8, 2])
@pytest.mark.parametrize("m,n", SHAPES)
def test_gemv_parity(gpu_ctx, oracle_lib, t, m, n):
    w = oracle_lib.gen_quant(t, 1234, m * 7 + n + t, m, n, std=0.02)
    x = oracle_lib.normal(1234, 99 + n, n)
    y = _run(gpu_ctx, t, w, m, n, x[None])[0]
    ref = oracle_lib.gemv(t, w, m, n, x)
    l2, mx = rel_errs(y, ref)
    print(f"type={t} m={m} n={n}: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
    assert l2 <= TOL and mx <= TOL


@pytest.mark.parametrize("t", [8, 2])
@pytest.mark.parametrize("batch", [1, 3, 4, 7, 16, 17, 32])
@pytest.mark.parametrize("m,n", [(6144, 2048), (2048, 6144)])
def test_small_batch_gemm_parity(gpu_ctx, oracle_lib, t, batch, m, n):
    """Ragged batches: batch is not padded to any tile; rows are read exactly
    (17 and 32 rows: two 16-row passes, the second of 1 or 16 rows)."""
    w = oracle_lib.gen_quant(t, 77, m + n + t, m, n, std=0.02)
    x = oracle_lib.normal(77, 1000 + batch, batch * n).reshape(batch, n)
    y = _run(gpu_ctx, t, w, m, n, x)
    ref = oracle_lib.gemm(t, w, m, n, x)
    l2, mx = rel_errs(y, ref)
    print(f"type={t} m={m} n={n} batch={batch}: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
    assert l2 <= TOL and mx <= TOL


@pytest.mark.parametrize("t", [8, 2])
@pytest.mark.parametrize("m,batch", [(151936, 2), (151936, 16), (65570, 9), (151936, 17), (151936, 32), (65570, 24)])
def test_gguf_gemm_many_tiles(gpu_ctx, oracle_lib, t, m, batch):
    """GGUF-layout GEMM at batch 2..32 on matrices of at least 4 row tiles per
    CU: the x-stationary kernels (8 waves; up to 16 rows one super-block's x
    fragments per wave, 17-32 rows two super-blocks' for one 16-row half,
    the pair's weights shared through LDS), the workgroup walking the row
    tiles; 65570 rows end in a ragged tile of 34 rows.  First, middle and
    last batch rows against the oracle."""
    n = 2048
    w = oracle_lib.gen_quant(t, 21, m % 97 + t, m, n, std=0.02)
    x = oracle_lib.normal(21, 300 + batch, batch * n).reshape(batch, n)
    y = _run(gpu_ctx, t, w, m, n, x)
    for b in sorted({0, batch // 2, batch - 1}):
        l2, mx = rel_errs(y[b], oracle_lib.gemv(t, w, m, n, x[b]))
        print(f"type={t} m={m} batch={batch} row={b}: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
        assert l2 <= TOL and mx <= TOL


@pytest.mark.parametrize("t", [8, 2])
@pytest.mark.parametrize("batch", [16, 24])
def test_gguf_gemm_many_tiles_input_range(gpu_ctx, oracle_lib, t, batch):
    """The x-stationary GGUF-layout kernels on rows far outside fp16's range
    (the extreme rows of the panel GEMM's range test), 16 and 24 rows."""
    from test_packed_gpu import check_extreme, extreme_rows

    m, n = 65570, 2048
    w = oracle_lib.gen_quant(t, 23, 5 + t, m, n, std=0.02)
    x = extreme_rows(oracle_lib, batch, n, 901)
    y = _run(gpu_ctx, t, w, m, n, x)
    check_extreme(y, x, w, t, m, n, oracle_lib)


@pytest.mark.parametrize("t", [8, 2])
def test_gguf_gemv_many_tiles_input_range(gpu_ctx, oracle_lib, t):
    """Batch 1 on a GGUF-layout matrix of at least 4 row tiles per CU (the
    x-stationary GEMV: x as int8 digits with a power-of-two exponent per
    32-block, digitised once per workgroup): each kind of extreme row as its
    own call, against the oracle; 65570 rows end in a ragged tile."""
    from test_packed_gpu import check_extreme, extreme_rows

    m, n = 65570, 2048
    w = oracle_lib.gen_quant(t, 29, 3 + t, m, n, std=0.02)
    x = extreme_rows(oracle_lib, 8, n, 903)
    y = np.stack([_run(gpu_ctx, t, w, m, n, x[b][None])[0] for b in range(x.shape[0])])
    check_extreme(y, x, w, t, m, n, oracle_lib)


def test_gemm_lm_head_batch32(gpu_ctx, oracle_lib):
    m, n, batch = 151936, 2048, 32
    w = oracle_lib.gen_quant(8, 5, 5, m, n, std=0.02)
    x = oracle_lib.normal(5, 6, batch * n).reshape(batch, n)
    y = _run(gpu_ctx, 8, w, m, n, x)
    for b in (0, 13, 31):
        ref = oracle_lib.gemv(8, w, m, n, x[b])
        l2, mx = rel_errs(y[b], ref)
        assert l2 <= TOL and mx <= TOL


def test_repeated_split_k_calls_are_deterministic(gpu_ctx, oracle_lib):
    """The GGUF-layout GEMV (anehip_quant_gemm at batch 1) on a K-split shape:
    gemv_fused writes its partial slices, a sum_partials launch adds them in
    split order, so repeated calls give identical bits."""
    m, n = 2048, 6144
    w = oracle_lib.gen_quant(8, 8, 8, m, n)
    x = oracle_lib.normal(8, 9, n)
    dw, dx, dy = gpu_ctx.to_device(w), gpu_ctx.to_device(x), gpu_ctx.alloc(m * 4)
    outs = []
    for _ in range(5):
        gpu_ctx.quant_gemm(8, dw, m, n, dx, 1, dy)
        outs.append(dy.download(np.float32, m))
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    for b in (dw, dx, dy):
        b.free()


def test_rejects_bad_shapes(gpu_ctx, anehip_mod):
    dw = gpu_ctx.alloc(34 * 8)
    dx = gpu_ctx.alloc(4 * 256)
    dy = gpu_ctx.alloc(4 * 8)
    with pytest.raises(anehip_mod.AnehipError) as e:
        gpu_ctx.quant_gemm(8, dw, 1, 100, dx, 1, dy)
    assert e.value.code == -2
    with pytest.raises(anehip_mod.AnehipError) as e:
        gpu_ctx.quant_gemm(14, dw, 1, 256, dx, 1, dy)
    assert e.value.code == -3
    with pytest.raises(anehip_mod.AnehipError) as e:
        gpu_ctx.quant_gemm(8, dw, 1, 256, dx, 33, dy)
    assert e.value.code == -3
    for b in (dw, dx, dy):
        b.free()
