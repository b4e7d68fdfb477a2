"""The panel weight layout of the batch-1 decode path (anehip_quant_pack /
anehip_quant_gemv_packed): the repack is a pure byte permutation, pinned here
bit-exactly against an independent numpy statement of the layout, and the
GEMV over panels matches the oracle's q8_gemv / q4_gemv_cpu restatement
(crates/engine/src/q8_gemv.rs:67-148) to 1e-4 relative, including ragged row
counts and K ranges long enough to take several rounds per workgroup."""
import numpy as np
import pytest

from conftest import rel_errs

TOL = 1e-4


def pack_ref(t, w, m, n):
    """Panel layout: row tiles of 64 (zero rows past m), 256-column panels;
    a panel is [chunk][64 rows][16 B] quant bytes then [64 rows][8 fp16] scales.
    Q8_0 chunk c = half (c % 2) of block c // 2; Q4_0 chunk c = block c's nibbles."""
    bb = 34 if t == 8 else 18
    nb, nsb, tiles = n // 32, n // 256, (m + 63) // 64
    pad = np.zeros((tiles * 64, nb, bb), np.uint8)
    pad[:m] = w.reshape(m, nb, bb)
    b = pad.reshape(tiles, 64, nsb, 8, bb)
    if t == 8:
        q = b[..., 2:34].reshape(tiles, 64, nsb, 16, 16)
    else:
        q = b[..., 2:18]
    q = q.transpose(0, 2, 3, 1, 4)                                   # tile, sb, chunk, row, byte
    sc = b[..., 0:2].reshape(tiles, 64, nsb, 16).transpose(0, 2, 1, 3)  # tile, sb, row, scale bytes
    return np.concatenate([q.reshape(tiles, nsb, -1), sc.reshape(tiles, nsb, -1)], axis=2).reshape(-1)


def test_packed_bytes(anehip_mod):
    f = anehip_mod.lib().anehip_quant_packed_bytes
    assert f(8, 64, 256) == 17 * 1024
    assert f(2, 64, 256) == 9 * 1024
    assert f(8, 65, 512) == 2 * 2 * 17 * 1024
    assert f(8, 64, 100) == 0 and f(14, 64, 256) == 0 and f(8, 0, 256) == 0


def test_pack_ref_is_a_permutation(oracle_lib):
    """The numpy layout keeps every byte once (rows padded with zeros)."""
    m, n = 70, 512
    w = oracle_lib.gen_quant(8, 1, 2, m, n)
    p = pack_ref(8, w, m, n)
    assert p.size == 2 * 2 * 17 * 1024
    assert np.array_equal(np.sort(p[p != 0]), np.sort(w[w != 0]))


def _pack(ctx, t, w, m, n):
    import anehip

    nbytes = int(anehip.lib().anehip_quant_packed_bytes(t, m, n))
    dw, dp = ctx.to_device(w), ctx.alloc(nbytes)
    ctx.call("quant_pack", t, dw, m, n, dp)
    return dw, dp, nbytes


@pytest.mark.gpu
@pytest.mark.parametrize("t", [8, 2])
@pytest.mark.parametrize("m,n", [(64, 256), (100, 512), (130, 2048), (1, 256)])
def test_repack_bit_exact(gpu_ctx, oracle_lib, t, m, n):
    w = oracle_lib.gen_quant(t, 21, m + n + t, m, n, std=0.02)
    dw, dp, nbytes = _pack(gpu_ctx, t, w, m, n)
    got = dp.download(np.uint8, nbytes)
    assert np.array_equal(got, pack_ref(t, w, m, n))
    dw.free()
    dp.free()


SHAPES = [(6144, 2048), (2048, 6144), (248320, 2048), (16, 2048), (100, 256), (8224, 2048), (300, 20480),
          (64, 32768)]


@pytest.mark.gpu
@pytest.mark.parametrize("t", [8, 2])
@pytest.mark.parametrize("m,n", SHAPES)
def test_packed_gemv_parity(gpu_ctx, oracle_lib, t, m, n):
    w = oracle_lib.gen_quant(t, 4321, m * 3 + n + t, m, n, std=0.02)
    x = oracle_lib.normal(4321, 7 + n, n)
    dw, dp, _ = _pack(gpu_ctx, t, w, m, n)
    dx, dy = gpu_ctx.to_device(x), gpu_ctx.alloc(m * 4)
    gpu_ctx.call("quant_gemv_packed", t, dp, m, n, dx, dy)
    y = dy.download(np.float32, m)
    ref = oracle_lib.gemv(t, w, m, n, x)
    l2, mx = rel_errs(y, ref)
    print(f"type={t} m={m} n={n}: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
    assert l2 <= TOL and mx <= TOL
    for b in (dw, dp, dx, dy):
        b.free()


@pytest.mark.gpu
def test_packed_gemv_back_to_back_splits(gpu_ctx, oracle_lib):
    """Batch-1 panel GEMVs queued back to back on matrices of different tile
    and split counts share the context's workspace: few-tile matrices run on
    gemv_rows (one launch, whole K range per workgroup, no partial sums),
    the others as a K-split gemv_packed launch followed by a sum_partials
    launch over the workspace's partial slices.  Each input used twice, all
    outputs match the oracle and repeated calls give identical bits."""
    t = 8
    cases = []
    for i, (m, n) in enumerate([(6144, 2048), (2048, 6144), (100, 2048), (6144, 2048), (2048, 2048)]):
        w = oracle_lib.gen_quant(t, 90 + i, 91, m, n, std=0.02)
        dw, dp, _ = _pack(gpu_ctx, t, w, m, n)
        xs = [oracle_lib.normal(92 + i, r, n) for r in range(2)]
        dxs = [gpu_ctx.to_device(x) for x in xs]
        dys = [gpu_ctx.alloc(m * 4) for _ in range(4)]
        cases.append((m, n, w, dw, dp, xs, dxs, dys))
    for rep in range(2):
        for m, n, w, dw, dp, xs, dxs, dys in cases:
            for r in range(2):
                gpu_ctx.call("quant_gemv_packed", t, dp, m, n, dxs[r], dys[2 * rep + r])
    for m, n, w, dw, dp, xs, dxs, dys in cases:
        for rep in range(2):
            for r in range(2):
                y = dys[2 * rep + r].download(np.float32, m)
                l2, mx = rel_errs(y, oracle_lib.gemv(t, w, m, n, xs[r]))
                assert l2 <= TOL and mx <= TOL, (m, n, rep, r, l2, mx)
        assert np.array_equal(dys[0].download(np.float32, m), dys[2].download(np.float32, m))
        for b in [dw, dp, *dxs, *dys]:
            b.free()


@pytest.mark.gpu
def test_packed_rejects_bad_shapes(gpu_ctx, anehip_mod):
    d = gpu_ctx.alloc(17 * 1024)
    with pytest.raises(anehip_mod.AnehipError) as e:
        gpu_ctx.call("quant_pack", 8, d, 64, 100, d)
    assert e.value.code == -2
    with pytest.raises(anehip_mod.AnehipError) as e:
        gpu_ctx.call("quant_gemv_packed", 14, d, 64, 256, d, d)
    assert e.value.code == -3
    # batch > 1 needs m % 4 == 0 (16-byte output stores)
    with pytest.raises(anehip_mod.AnehipError) as e:
        gpu_ctx.call("quant_gemm_packed", 8, d, 62, 256, d, 2, d)
    assert e.value.code == -3
    d.free()


@pytest.mark.gpu
@pytest.mark.parametrize("t", [8, 2])
@pytest.mark.parametrize("batch", [2, 3, 4, 7, 16, 17, 32])
@pytest.mark.parametrize("m,n", [(6144, 2048), (2048, 6144), (100, 256), (8224, 2048), (12288, 1792), (2048, 2048),
                                 (100, 512), (1024, 8192), (20480, 2048)])
def test_packed_gemm_parity(gpu_ctx, oracle_lib, t, batch, m, n):
    """Panel MFMA GEMM, ragged batch (not padded to the 32-row MFMA tile), at
    the decode shapes, a tiny matrix and an odd panel count (12288 x 1792).
    Batch <= 16 runs on the 16-wide x-stationary kernel wherever the split
    has 1, 2, 4 or 8 panels; batch 17 and 32 on the 8-wave x-stationary kernel
    for splits of 2 panels, the 4-wave one for single-panel splits and the
    persistent kernel otherwise.  Shapes: 2 panels per K split
    (6144 x 2048, 2048 x 6144 at 12 splits, 8224 x 2048 with a ragged last
    tile), 1 panel (2048 x 2048, 100 x 512, the odd 12288 x 1792), the
    persistent kernel (100 x 256; 1024 x 8192, whose 32 single-panel splits
    exceed the x-stationary limit), and a matrix of more tiles than CUs split
    by the balance model (20480 x 2048)."""
    w = oracle_lib.gen_quant(t, 99, m + 5 * n + t, m, n, std=0.02)
    x = oracle_lib.normal(99, 300 + batch, batch * n).reshape(batch, n)
    dw, dp, _ = _pack(gpu_ctx, t, w, m, n)
    dx, dy = gpu_ctx.to_device(x), gpu_ctx.alloc(batch * m * 4)
    gpu_ctx.call("quant_gemm_packed", t, dp, m, n, dx, batch, dy)
    y = dy.download(np.float32, batch * m).reshape(batch, m)
    ref = oracle_lib.gemm(t, w, m, n, x)
    l2, mx = rel_errs(y, ref)
    print(f"type={t} m={m} n={n} batch={batch}: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
    assert l2 <= TOL and mx <= TOL
    for b in (dw, dp, dx, dy):
        b.free()


@pytest.mark.gpu
@pytest.mark.parametrize("t", [8, 2])
@pytest.mark.parametrize("batch", [33, 100, 256])
@pytest.mark.parametrize("m,n", [(6144, 2048), (2048, 6144), (8224, 2048), (2048, 2048), (12288, 1792), (100, 256),
                                 (32968, 256)])
def test_packed_gemm_tall(gpu_ctx, oracle_lib, t, batch, m, n):
    """More than 32 rows (the prefill's chunk GEMM, gemm_tall): 32-row groups
    of planes, one per compute wave (33: one full group and one row, six
    waves without rows; 100 and 256: partial and full), a ragged last weight
    tile (8224 rows; 100 rows: two tiles, the second ragged), K splits that
    divide the panel count (12288 x 1792: 7 panels; 2048 x 2048: 8 splits),
    and workgroups walking several items (32968 x 256: 516 one-panel items,
    2 or 3 per workgroup, the last tile ragged)."""
    w = oracle_lib.gen_quant(t, 77, m + 3 * n + t, m, n, std=0.02)
    x = oracle_lib.normal(77, 900 + batch, batch * n).reshape(batch, n)
    dw, dp, _ = _pack(gpu_ctx, t, w, m, n)
    dx, dy = gpu_ctx.to_device(x), gpu_ctx.alloc(batch * m * 4)
    gpu_ctx.call("quant_gemm_packed", t, dp, m, n, dx, batch, dy)
    y = dy.download(np.float32, batch * m).reshape(batch, m)
    ref = oracle_lib.gemm(t, w, m, n, x)
    l2, mx = rel_errs(y, ref)
    print(f"type={t} m={m} n={n} batch={batch}: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
    assert l2 <= TOL and mx <= TOL
    for b in (dw, dp, dx, dy):
        b.free()


@pytest.mark.gpu
@pytest.mark.parametrize("t,m,n,batch", [(8, 151936, 2048, 32), (2, 151936, 2048, 19), (8, 151936, 2048, 4),
                                         (8, 151936, 2048, 16), (2, 151936, 2048, 11), (8, 65600, 1024, 16),
                                         (2, 65600, 1024, 5)])
def test_packed_gemm_many_tiles(gpu_ctx, oracle_lib, t, m, n, batch):
    """Matrices of at least 4 row tiles per CU: lm_head unsplit on the 16-wide
    x-stationary kernel with 8 panels per workgroup at batch <= 16 (splitting
    the fp32 rows itself), and at batch 17-32 unsplit on the 8-wave kernel
    (gemm_xsh, 4 panels per wave, after a planes launch); n = 1024 (4
    panels, unsplit at batch <= 16) with a ragged last tile.  Checked on the
    first, a middle and the last batch row."""
    w = oracle_lib.gen_quant(t, 6, 6 + m % 7, m, n, std=0.02)
    x = oracle_lib.normal(6, 7 + batch, batch * n).reshape(batch, n)
    dw, dp, _ = _pack(gpu_ctx, t, w, m, n)
    dx, dy = gpu_ctx.to_device(x), gpu_ctx.alloc(batch * m * 4)
    gpu_ctx.call("quant_gemm_packed", t, dp, m, n, dx, batch, dy)
    y = dy.download(np.float32, batch * m).reshape(batch, m)
    for b in sorted({0, batch // 2, batch - 1}):
        l2, mx = rel_errs(y[b], oracle_lib.gemv(t, w, m, n, x[b]))
        print(f"type={t} m={m} n={n} batch={batch} row={b}: rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
        assert l2 <= TOL and mx <= TOL
    for buf in (dw, dp, dx, dy):
        buf.free()


def extreme_rows(oracle_lib, batch, n, seed):
    """Batch rows outside fp16's range, cycled: N(0, 1) with +-7e4 / +-1e5
    entries in several 128-column groups; whole rows scaled to 1e5, 1e-6 and
    1e-30; a row of zeros; groups alternating 1e4 and 1e-4; fp32 subnormals
    (1e-40); a plain N(0, 1) row."""
    x = oracle_lib.normal(seed, 1, batch * n).reshape(batch, n).astype(np.float64)
    out = np.empty_like(x)
    for b in range(batch):
        r, kind = x[b].copy(), b % 8
        if kind == 0:
            idx = np.arange(3, n, 97)
            r[idx] = np.where(idx % 2, 7e4, -1e5) * np.where(idx % 3, 1.0, -1.0)
        elif kind == 1:
            r *= 1e5
        elif kind == 2:
            r *= 1e-6
        elif kind == 3:
            r *= 1e-30
        elif kind == 4:
            r[:] = 0.0
        elif kind == 5:
            r *= np.where((np.arange(n) // 128) % 2, 1e4, 1e-4)
        elif kind == 6:
            r *= 1e-40
        out[b] = r
    return out.astype(np.float32)


def check_extreme(y, x, w, t, m, n, oracle_lib):
    """Every row against the oracle (1e-4 relative, rel L2 and max-abs /
    max |ref|); zero rows exactly zero; the subnormal row, where the oracle's
    own fp32 products lose bits, against float64."""
    import np_ref

    ref = oracle_lib.gemm(t, w, m, n, x)
    for b in range(x.shape[0]):
        assert np.all(np.isfinite(y[b])), b
        if not np.any(x[b]):
            assert not np.any(y[b]), b
            continue
        if b % 8 == 6:
            r = np_ref.dequant(t, w, m, n) @ x[b].astype(np.float64)
        else:
            r = ref[b]
        l2, mx = rel_errs(y[b], r)
        print(f"row {b} (kind {b % 8}): rel_l2={l2:.2e} rel_max={mx:.2e}", flush=True)
        assert l2 <= TOL and mx <= TOL, (b, l2, mx)


@pytest.mark.gpu
@pytest.mark.parametrize("t", [8, 2])
@pytest.mark.parametrize("batch", [2, 17, 32, 72])
@pytest.mark.parametrize("m,n", [(6144, 2048), (2048, 2048), (100, 256), (2048, 6144)])
def test_packed_gemm_input_range(gpu_ctx, oracle_lib, t, batch, m, n):
    """The batch > 1 GEMMs split fp32 x into fp16 hi + lo: rows far outside
    fp16's range (overflow, underflow, subnormal, zero, mixed groups) match
    the fp32 oracle, on the x-stationary kernels (fp32 rows, per-row scaling
    over the split), on the persistent kernel (range-safe planes) and above
    32 rows on gemm_tall (range-safe planes, per-row scaling over the split)."""
    w = oracle_lib.gen_quant(t, 55, m + n + t, m, n, std=0.02)
    x = extreme_rows(oracle_lib, batch, n, 500 + batch)
    dw, dp, _ = _pack(gpu_ctx, t, w, m, n)
    dx, dy = gpu_ctx.to_device(x), gpu_ctx.alloc(batch * m * 4)
    gpu_ctx.call("quant_gemm_packed", t, dp, m, n, dx, batch, dy)
    y = dy.download(np.float32, batch * m).reshape(batch, m)
    check_extreme(y, x, w, t, m, n, oracle_lib)
    for b in (dw, dp, dx, dy):
        b.free()


@pytest.mark.gpu
@pytest.mark.parametrize("t", [8, 2])
@pytest.mark.parametrize("batch", [5, 16, 24])
def test_packed_gemm_many_tiles_input_range(gpu_ctx, oracle_lib, t, batch):
    """The extreme rows of the test above on a matrix of at least 4 row tiles
    per CU (65600 x 2048: one split of 8 panels): at batch <= 16 the 16-wide
    kernel splits the fp32 rows itself over all 8 panels, at batch 24 the
    8-wave kernel reads range-safe planes."""
    m, n = 65600, 2048
    w = oracle_lib.gen_quant(t, 57, 11 + t, m, n, std=0.02)
    x = extreme_rows(oracle_lib, batch, n, 700 + batch)
    dw, dp, _ = _pack(gpu_ctx, t, w, m, n)
    dx, dy = gpu_ctx.to_device(x), gpu_ctx.alloc(batch * m * 4)
    gpu_ctx.call("quant_gemm_packed", t, dp, m, n, dx, batch, dy)
    y = dy.download(np.float32, batch * m).reshape(batch, m)
    check_extreme(y, x, w, t, m, n, oracle_lib)
    for b in (dw, dp, dx, dy):
        b.free()


@pytest.mark.gpu
@pytest.mark.parametrize("t", [8, 2])
@pytest.mark.parametrize("m,n", [(6144, 2048), (2048, 6144), (16384, 256), (100, 256)])
@pytest.mark.parametrize("layout", ["panel", "gguf"])
def test_gemv_input_range(gpu_ctx, oracle_lib, t, m, n, layout):
    """Batch 1 (x as int8 digits with a power-of-two exponent per 32-block):
    each kind of extreme row of the batched test as its own call, on every
    batch-1 kernel (6144 x 2048 and 2048 x 6144: the one-launch row GEMV;
    16384 x 256: the panel GEMV without a K split; the GGUF-layout GEMV)."""
    w = oracle_lib.gen_quant(t, 57, m + n + t, m, n, std=0.02)
    x = extreme_rows(oracle_lib, 8, n, 700 + n)
    if layout == "panel":
        dw, dp, _ = _pack(gpu_ctx, t, w, m, n)
    else:
        dw, dp = gpu_ctx.to_device(w), None
    y = np.empty((8, m), np.float32)
    for b in range(8):
        dx, dy = gpu_ctx.to_device(x[b:b + 1]), gpu_ctx.alloc(m * 4)
        if layout == "panel":
            gpu_ctx.call("quant_gemm_packed", t, dp, m, n, dx, 1, dy)
        else:
            gpu_ctx.quant_gemm(t, dw, m, n, dx, 1, dy)
        y[b] = dy.download(np.float32, m)
        dx.free()
        dy.free()
    check_extreme(y, x, w, t, m, n, oracle_lib)
    dw.free()
    if dp is not None:
        dp.free()


@pytest.mark.gpu
@pytest.mark.parametrize("t", [8, 2])
@pytest.mark.parametrize("layout", ["panel", "gguf"])
@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
def test_gemv_nonfinite_input(gpu_ctx, oracle_lib, t, layout, bad):
    """An inf or NaN in x makes every output non-finite, as in the reference
    (q8_gemv.rs:234-242: the product with a nonzero weight is +-inf, with a
    zero weight NaN, and either swamps the row's sum); this build returns NaN
    for each row whose block holds it, i.e. every row."""
    m, n = 2048, 2048
    w = oracle_lib.gen_quant(t, 58, 3, m, n, std=0.02)
    x = oracle_lib.normal(9, 4, n).reshape(1, n)
    x[0, 777] = bad
    ref = oracle_lib.gemm(t, w, m, n, x)
    assert not np.any(np.isfinite(ref))
    dx, dy = gpu_ctx.to_device(x), gpu_ctx.alloc(m * 4)
    if layout == "panel":
        dw, dp, _ = _pack(gpu_ctx, t, w, m, n)
        gpu_ctx.call("quant_gemm_packed", t, dp, m, n, dx, 1, dy)
        dp.free()
    else:
        dw = gpu_ctx.to_device(w)
        gpu_ctx.quant_gemm(t, dw, m, n, dx, 1, dy)
    y = dy.download(np.float32, m)
    assert not np.any(np.isfinite(y))
    for b in (dw, dx, dy):
        b.free()


@pytest.mark.gpu
@pytest.mark.parametrize("t", [8, 2])
@pytest.mark.parametrize("batch", [2, 17, 32])
@pytest.mark.parametrize("m,n", [(2048, 2048), (100, 256)])
def test_gguf_gemm_input_range(gpu_ctx, oracle_lib, t, batch, m, n):
    """The same rows through anehip_quant_gemm (GGUF blocks, row-major
    range-safe planes)."""
    w = oracle_lib.gen_quant(t, 56, m + n + t, m, n, std=0.02)
    x = extreme_rows(oracle_lib, batch, n, 600 + batch)
    dw, dx, dy = gpu_ctx.to_device(w), gpu_ctx.to_device(x), gpu_ctx.alloc(batch * m * 4)
    gpu_ctx.quant_gemm(t, dw, m, n, dx, batch, dy)
    y = dy.download(np.float32, batch * m).reshape(batch, m)
    check_extreme(y, x, w, t, m, n, oracle_lib)
    for b in (dw, dx, dy):
        b.free()
