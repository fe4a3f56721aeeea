"""GPU parity: dense block-scaled FP8 linear (small-M and tiled kernels)."""

import numpy as np
import pytest

from oracle import fp8 as ofp8
from golden_inputs import bf16_normal, block_weights, exact_codes, rel_fro

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(dev)


# M values exercise every kernel path: small-M (1..64, MT=1/2/4), tiled
# 128x128 (65..), the 256x128 tile (large M) and ragged tails.
EXACT_CASES = [(1, 256, 128), (5, 512, 256), (16, 2048, 384), (33, 384, 128), (64, 256, 512),
               (65, 256, 256), (100, 384, 384), (300, 256, 640), (2049, 256, 1024)]


@pytest.mark.parametrize("m,k,n", EXACT_CASES)
def test_projection_exact_products(dev, m, k, n):
    """Exact-product operands: the device result equals the float64 oracle
    bit for bit, whatever the accumulation order."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(m * 7 + n)
    x = exact_codes(rng, (m, k))
    w = exact_codes(rng, (n, k))
    xs = np.full((m, k // 128), 0.125, np.float32)
    ws = np.full(((n + 127) // 128, k // 128), 0.125, np.float32)
    out = ops.projection_partial(_t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev))
    torch.cuda.synchronize()
    exp = ofp8.fp8_linear(x, w, ws, activation_scales=xs)
    np.testing.assert_array_equal(out.cpu().numpy(), exp)


# 2048-deep products with 16 < M <= 256 (the weight-stationary split-K
# kernel): ragged M, 48-column tiles that straddle 128-column scale blocks
# (N = 240, 480), and every m-tile height.
SPLIT_CASES = [(17, 2048, 96), (40, 2048, 480), (64, 2048, 144), (100, 2048, 240),
               (129, 2048, 192), (256, 2048, 336),
               # N not a multiple of 48: 16-column tiles, and 32-column tiles
               # from 2048 columns, for four- and eight-wave row tiles
               (17, 2048, 16), (40, 2048, 512), (33, 2048, 1040), (64, 2048, 2080),
               (100, 2048, 2080), (200, 2048, 1040), (256, 2048, 16)]


@pytest.mark.parametrize("m,k,n", SPLIT_CASES)
def test_projection_exact_products_split(dev, m, k, n):
    test_projection_exact_products(dev, m, k, n)


# Up to 16 rows the wide kernel picks its columns per workgroup from N:
# 24 at N = 6144 and 7680 (a 16-column tile with 8 valid columns, and tiles
# straddling 128-column scale blocks), 16 at 4096, 8 at 2048 and below.
WIDE_CASES = [(1, 2048, 6144), (16, 2048, 6144), (7, 256, 7680), (4, 512, 4096), (16, 1024, 2048)]


@pytest.mark.parametrize("m,k,n", WIDE_CASES)
def test_projection_exact_products_wide(dev, m, k, n):
    test_projection_exact_products(dev, m, k, n)


@pytest.mark.parametrize("m,k,n", WIDE_CASES)
def test_fp8_linear_fused_equals_quantize_then_gemm(dev, m, k, n):
    """The one-launch fused path (the wide kernel quantizing its own slab)
    equals quantize -> projection_partial bit for bit."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(5 * m + n)
    x = _t(bf16_normal(rng, (m, k)), dev, torch.bfloat16)
    w, ws = ofp8.quantize_weight_blocks(rng.normal(0, 0.02, (n, k)).astype(np.float32))
    wt, wst = _t(w, dev), _t(ws, dev)
    fused = ops.fp8_linear(x, wt, wst)
    q, qs = ops.quantize(x)
    ref = ops.projection_partial(q, qs, wt, wst)
    torch.cuda.synchronize()
    assert torch.equal(fused, ref)


@pytest.mark.parametrize("m,k,n", EXACT_CASES[:6] + SPLIT_CASES + WIDE_CASES)
def test_projection_varying_scales(dev, m, k, n):
    """Distinct per-row / per-block scales catch a wrong scale index."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(11 + m)
    x = exact_codes(rng, (m, k))
    w = exact_codes(rng, (n, k))
    xs = (2.0 ** rng.integers(-6, 2, (m, k // 128))).astype(np.float32)
    ws = (2.0 ** rng.integers(-6, 2, ((n + 127) // 128, k // 128))).astype(np.float32)
    out = ops.projection_partial(_t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev))
    torch.cuda.synchronize()
    exp = ofp8.fp8_linear(x, w, ws, activation_scales=xs)
    np.testing.assert_array_equal(out.cpu().numpy(), exp)


@pytest.mark.parametrize("m", [1, 4, 16, 64, 256])
@pytest.mark.parametrize("scale_dtype", ["float32", "bfloat16"])
def test_fp8_linear_decode_shapes(dev, m, scale_dtype):
    """Decode sweep shape K=2048, N=6144 with 1% x20 outliers: relative
    Frobenius error vs the float64 oracle within 1e-2 (observed ~1e-7)."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(0)
    codes, scales = block_weights(rng, (6144, 2048), scale_dtype=scale_dtype)
    x = bf16_normal(rng, (m, 2048), outliers=0.01)
    sdt = torch.float32 if scale_dtype == "float32" else torch.bfloat16
    y = ops.fp8_linear(_t(x, dev, torch.bfloat16), _t(codes, dev), _t(scales, dev, sdt),
                       out_dtype=torch.float32)
    torch.cuda.synchronize()
    exp = ofp8.fp8_linear(x, codes, scales)
    err = rel_fro(y.cpu().numpy(), exp)
    assert err < 1e-2
    # f32 accumulation; the FP8 MFMA sums each 128-deep block with its own
    # internal precision (~1e-5 relative on random data, exact on exact products)
    assert err < 1e-4, err


@pytest.mark.parametrize("m,n", [(64, 512), (20, 1040), (48, 2080)])
def test_fp8_linear_narrow_tiles_match_two_step(dev, m, n):
    """Narrow column tiles (N not a multiple of 48, up to 64 rows):
    fp8_linear's fragment-major path equals quantize -> projection_partial
    bit for bit, and both match the oracle."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(m + n)
    codes, scales = block_weights(rng, (n, 2048))
    x = bf16_normal(rng, (m, 2048), outliers=0.01)
    xt = _t(x, dev, torch.bfloat16)
    w, s = _t(codes, dev), _t(scales, dev)
    y = ops.fp8_linear(xt, w, s, out_dtype=torch.float32)
    q, qs = ops.quantize(xt)
    y2 = ops.projection_partial(q, qs, w, s, out_dtype=torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), y2.cpu().numpy())
    assert rel_fro(y.cpu().numpy(), ofp8.fp8_linear(x, codes, scales)) < 1e-4


@pytest.mark.parametrize("m,k,n", [(1, 8192, 2048), (8, 8192, 2048), (16, 4096, 6144)])
def test_fp8_linear_deep_k_fused_small(dev, m, k, n):
    """Up to 16 rows the wide kernel quantizes the whole activation slab into
    LDS, deep K included (K=8192: a 132 KB slab), within the oracle bound."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(m + k)
    codes, scales = block_weights(rng, (n, k))
    x = bf16_normal(rng, (m, k), outliers=0.01)
    y = ops.fp8_linear(_t(x, dev, torch.bfloat16), _t(codes, dev), _t(scales, dev),
                       out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rel_fro(y.cpu().numpy(), ofp8.fp8_linear(x, codes, scales)) < 1e-4


@pytest.mark.parametrize("m,k,n", [(64, 8192, 2048), (17, 4096, 512), (40, 4096, 1040),
                                   (256, 4096, 6144), (100, 6144, 480), (128, 8192, 2048)])
def test_fp8_linear_deep_k_partitions(dev, m, k, n):
    """Deeper than 2048 at 17-256 rows: fp8_linear runs 2048-deep partitions
    with f32 partials and the serial merge -- bit for bit the
    projection_partial(partitions) -> projection_merge pair on the same codes
    -- and matches the oracle."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(m + k + n)
    codes, scales = block_weights(rng, (n, k))
    x = bf16_normal(rng, (m, k), outliers=0.01)
    xt = _t(x, dev, torch.bfloat16)
    w, s = _t(codes, dev), _t(scales, dev)
    y = ops.fp8_linear(xt, w, s, out_dtype=torch.float32)
    q, qs = ops.quantize(xt)
    partial = ops.projection_partial(q, qs, w, s, partitions=k // 2048)
    y2 = ops.projection_merge(partial, out_dtype=torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), y2.cpu().numpy())
    assert rel_fro(y.cpu().numpy(), ofp8.fp8_linear(x, codes, scales)) < 1e-4


@pytest.mark.parametrize("m", [1, 5, 16, 17, 33, 64, 100, 129, 256])
@pytest.mark.parametrize("x_dtype", ["float32", "float16", "bfloat16"])
def test_fp8_linear_fused_quantize_matches_two_step(dev, m, x_dtype):
    """fp8_linear quantizes x inside the GEMM (up to 16 rows) or into
    fragment-major tiles (17-256 rows); either way the result is bit for bit
    quantize -> projection_partial on row-major codes, and those codes equal
    the oracle's (stress rows included)."""
    import torch
    from akas_amd import ops
    from golden_inputs import stress_rows

    rng = np.random.default_rng(m)
    codes, scales = block_weights(rng, (768, 2048))
    x = np.concatenate([bf16_normal(rng, (max(m - 2, 1), 2048), outliers=0.01),
                        stress_rows(2048, 2, rng)])[:m]
    xt = _t(x, dev, getattr(torch, x_dtype))
    w, s = _t(codes, dev), _t(scales, dev)
    y = ops.fp8_linear(xt, w, s, out_dtype=torch.float32)
    q, qs = ops.quantize(xt)
    y2 = ops.projection_partial(q, qs, w, s, out_dtype=torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), y2.cpu().numpy())
    xq = ofp8.round_to(x, x_dtype)
    ec, es = ofp8.quantize(xq)
    np.testing.assert_array_equal(q.cpu().numpy(), ec)
    assert rel_fro(y.cpu().numpy(), ofp8.fp8_linear(xq, codes, scales)) < 1e-4


@pytest.mark.parametrize("out_dtype", ["float32", "bfloat16", "float16"])
def test_fp8_linear_config1_and_out_dtypes(dev, out_dtype):
    """Config: x bf16 [16,2048] ~N(0,1), W N(0,0.02) block-quantized, seed 0."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(0)
    codes, scales = block_weights(rng, (2048, 2048))
    x = bf16_normal(rng, (16, 2048))
    y = ops.fp8_linear(_t(x, dev, torch.bfloat16), _t(codes, dev), _t(scales, dev),
                       out_dtype=getattr(torch, out_dtype))
    torch.cuda.synchronize()
    exp = ofp8.fp8_linear(x, codes, scales, out_dtype="float32")
    got = y.float().cpu().numpy()
    assert rel_fro(got, exp) < (1e-4 if out_dtype == "float32" else 4e-3)


# Shapes that select the DMA-fed 256x256 prefill kernel (more than 256 rows,
# N a multiple of 128, at least 240 tiles): ragged last row tiles (M % 256 of
# 1, 16 and 208 rows) and a half-width last column tile (N % 256 == 128).
DMA_CASES = [(2000, 512, 7808), (1537, 384, 10112), (4097, 256, 3840), (2304, 1024, 6784)]


@pytest.mark.parametrize("m,k,n", DMA_CASES)
def test_projection_exact_products_dma(dev, m, k, n):
    """The prefill kernel on exact products with distinct per-row and
    per-block binary scales: the whole output equals the float64 oracle bit
    for bit, so a misplaced row, column, k-block or scale index fails."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(m + 3 * n)
    x = exact_codes(rng, (m, k))
    w = exact_codes(rng, (n, k))
    xs = (2.0 ** rng.integers(-6, 2, (m, k // 128))).astype(np.float32)
    ws = (2.0 ** rng.integers(-6, 2, ((n + 127) // 128, k // 128))).astype(np.float32)
    exp = ofp8.fp8_linear(x, w, ws, activation_scales=xs)
    xt, xst, wt = _t(x, dev), _t(xs, dev), _t(w, dev)
    for sdt in (torch.float32, torch.bfloat16):  # binary scales are exact in bf16
        out = ops.projection_partial(xt, xst, wt, _t(ws, dev, sdt))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), exp)
    for odt in ("bfloat16", "float16"):  # 16-bit tiles go out through LDS
        out = ops.projection_partial(xt, xst, wt, _t(ws, dev), out_dtype=getattr(torch, odt))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.float().cpu().numpy(), ofp8.round_to(exp, odt))


def test_projection_dma_deepest_k(dev):
    """The prefill kernel at the deepest k range it takes (K = 16384: 128
    k-blocks, a full weight-scale table) on a ragged 4000 x 3840 output (240
    tiles).  Scales 2^-2 or 2^-1 keep every partial sum exact in float32 while
    a wrong k-block or scale index still changes the result; rows from every
    row tile (the ragged last one included) are compared bit for bit."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(16384)
    m, k, n = 4000, 16384, 3840
    x = exact_codes(rng, (m, k))
    w = exact_codes(rng, (n, k))
    xs = (2.0 ** rng.integers(-2, 0, (m, k // 128))).astype(np.float32)
    ws = (2.0 ** rng.integers(-2, 0, (n // 128, k // 128))).astype(np.float32)
    out = ops.projection_partial(_t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev))
    torch.cuda.synchronize()
    rows = np.array([0, 1, 255, 256, 1023, 2049, 3839, 3840, 3999])
    exp = ofp8.fp8_linear(x[rows], w, ws, activation_scales=xs[rows])
    np.testing.assert_array_equal(out.cpu().numpy()[rows], exp)


def test_projection_dma_partitions(dev):
    """K-partitions on the prefill kernel (2 x 128 tiles >= 240 workgroups):
    each partition's f32 partial lands at its own offset, bit-exact."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(21)
    m, k, n, parts = 2048, 1024, 4096, 2
    x = exact_codes(rng, (m, k))
    w = exact_codes(rng, (n, k))
    xs = (2.0 ** rng.integers(-6, 2, (m, k // 128))).astype(np.float32)
    ws = (2.0 ** rng.integers(-6, 2, (n // 128, k // 128))).astype(np.float32)
    part = ops.projection_partial(_t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev),
                                  partitions=parts)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(part.cpu().numpy(), ofp8.projection_partial(x, xs, w, ws, parts))


@pytest.mark.parametrize("m,k,n", [(8192, 2048, 6144), (8192, 2048, 8192), (8192, 8192, 2048)])
def test_fp8_linear_prefill_config_shapes_full(dev, m, k, n):
    """The three prefill GEMM shapes of the benchmark, whole output: f32 out
    within 1e-4 relative Frobenius of the float64 oracle (bar 1e-2), and the
    bf16 output equal to the f32 output rounded to nearest even, element for
    element (one accumulation, two stores)."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(m + k + n)
    codes, scales = block_weights(rng, (n, k))
    x = bf16_normal(rng, (m, k))
    xt, w, s = _t(x, dev, torch.bfloat16), _t(codes, dev), _t(scales, dev)
    y32 = ops.fp8_linear(xt, w, s, out_dtype=torch.float32)
    y16 = ops.fp8_linear(xt, w, s, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    got = y32.cpu().numpy()
    del y32
    np.testing.assert_array_equal(y16.float().cpu().numpy(), ofp8.bf16_round(got))
    del y16
    assert rel_fro(got, ofp8.fp8_linear(x, codes, scales)) < 1e-4


@pytest.mark.parametrize("m,k,n", [(8192, 2048, 6144), (8192, 8192, 2048), (512, 2048, 8192)])
def test_fp8_linear_prefill_shapes(dev, m, k, n):
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(1)
    codes, scales = block_weights(rng, (n, k))
    x = bf16_normal(rng, (m, k))
    y = ops.fp8_linear(_t(x, dev, torch.bfloat16), _t(codes, dev), _t(scales, dev),
                       out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    # oracle on a row sample keeps the CPU time bounded
    rows = np.unique(np.concatenate([np.arange(8), rng.integers(0, m, 56), [m - 1]]))
    exp = ofp8.fp8_linear(x[rows], codes, scales)
    got = y.float().cpu().numpy()[rows]
    assert rel_fro(got, exp) < 4e-3


@pytest.mark.parametrize("m,n", [(40, 480), (256, 96)])
@pytest.mark.parametrize("out_dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("scale_dtype", ["float32", "bfloat16"])
def test_projection_split_out_and_scale_dtypes(dev, m, n, out_dtype, scale_dtype):
    """16-bit outputs of exact products: the device rounding of each exact
    sum equals the oracle's round-to-nearest-even, element for element."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(m + n)
    k = 2048
    x = exact_codes(rng, (m, k))
    w = exact_codes(rng, (n, k))
    xs = (2.0 ** rng.integers(-6, 2, (m, k // 128))).astype(np.float32)
    ws = (2.0 ** rng.integers(-6, 2, ((n + 127) // 128, k // 128))).astype(np.float32)
    out = ops.projection_partial(_t(x, dev), _t(xs, dev), _t(w, dev),
                                 _t(ws, dev, getattr(torch, scale_dtype)),
                                 out_dtype=getattr(torch, out_dtype))
    torch.cuda.synchronize()
    exp = ofp8.round_to(ofp8.fp8_linear(x, w, ws, activation_scales=xs), out_dtype)
    np.testing.assert_array_equal(out.float().cpu().numpy(), exp)


@pytest.mark.parametrize("parts", [2, 4])
def test_projection_partitions_and_merge(dev, parts):
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(parts)
    m, k, n = 20, 1024, 256
    x = exact_codes(rng, (m, k))
    w = exact_codes(rng, (n, k))
    xs = np.full((m, k // 128), 0.125, np.float32)
    ws = np.full((n // 128, k // 128), 0.125, np.float32)
    part = ops.projection_partial(_t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev),
                                  partitions=parts)
    merged = ops.projection_merge(part)
    torch.cuda.synchronize()
    exp = ofp8.projection_partial(x, xs, w, ws, parts)
    np.testing.assert_array_equal(part.cpu().numpy(), exp)
    np.testing.assert_array_equal(merged.cpu().numpy(), ofp8.projection_merge(exp))


def test_projection_split_partitions(dev):
    """2048-deep partitions of a 4096-deep product run one split-K workgroup
    grid per partition; each partition's tile lands at its own offset."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(5)
    m, k, n = 40, 4096, 96
    x = exact_codes(rng, (m, k))
    w = exact_codes(rng, (n, k))
    xs = (2.0 ** rng.integers(-6, 2, (m, k // 128))).astype(np.float32)
    ws = (2.0 ** rng.integers(-6, 2, (1, k // 128))).astype(np.float32)
    part = ops.projection_partial(_t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev), partitions=2)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(part.cpu().numpy(), ofp8.projection_partial(x, xs, w, ws, 2))


def test_linear_rejects_bad_geometry(dev):
    import torch
    from akas_amd import ops

    x = torch.zeros((4, 200), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((128, 200), dtype=torch.uint8, device=dev)
    s = torch.zeros((1, 1), dtype=torch.float32, device=dev)
    with pytest.raises(ValueError):
        ops.fp8_linear(x, w, s)


def test_fp8_linear_default_workspace_per_stream(dev):
    """fp8_linear without an explicit workspace on two streams at once: each
    stream has its own cached workspace, so concurrent calls do not share
    codes and scales, and every result equals the one-stream result."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(17)
    codes, scales = block_weights(rng, (6144, 2048))
    w, s = _t(codes, dev), _t(scales, dev)
    xs = [_t(bf16_normal(rng, (m, 2048), outliers=0.01), dev, torch.bfloat16)
          for m in (64, 200, 64, 256)]
    ref = [ops.fp8_linear(x, w, s, out_dtype=torch.float32) for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    assert (ops.linear_workspace(64, 2048, 6144, dev, streams[0]).data_ptr() !=
            ops.linear_workspace(64, 2048, 6144, dev, streams[1]).data_ptr())
    outs = [[None] * len(xs) for _ in streams]
    for rep in range(20):
        for j, st in enumerate(streams):
            with torch.cuda.stream(st):
                for i, x in enumerate(xs):
                    outs[j][i] = ops.fp8_linear(x, w, s, out_dtype=torch.float32)
    torch.cuda.synchronize()
    for j in range(len(streams)):
        for i in range(len(xs)):
            np.testing.assert_array_equal(outs[j][i].cpu().numpy(), ref[i].cpu().numpy())


@pytest.mark.parametrize("m", [16, 8192])
def test_fp8_linear_prequantized_binding(dev, m):
    """``fp8_linear`` bound as the reference's block-FP8 prefill registration
    binds it (u8 codes ``x`` plus ``activation_scales``,
    src/akas/ops/linear/definition.py:558-568, :942-963) equals
    ``projection_partial`` with one partition bit for bit, and the oracle to
    the GEMM bar."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(101 + m)
    codes, scales = block_weights(rng, (6144, 2048))
    w, s = _t(codes, dev), _t(scales, dev)
    x = bf16_normal(rng, (m, 2048), outliers=0.01)
    xc, xs = ops.quantize(_t(x, dev, torch.bfloat16))
    got = ops.fp8_linear(xc, w, s, xs, out_dtype=torch.bfloat16)
    ref = ops.projection_partial(xc, xs, w, s, partitions=1, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert got.dtype == torch.bfloat16 and tuple(got.shape) == (m, 6144)
    assert torch.equal(got, ref)
    rows = slice(0, m) if m <= 256 else np.r_[0:64, m - 64:m]
    exp = ofp8.fp8_linear(x[rows], codes, scales)
    assert rel_fro(got.float().cpu().numpy()[rows], exp) < 4e-3
    # the same kind into a caller-owned f32 output
    out = torch.empty((m, 6144), dtype=torch.float32, device=dev)
    ops.fp8_linear(xc, w, s, activation_scales=xs, out=out)
    torch.cuda.synchronize()
    assert torch.equal(out, ops.projection_partial(xc, xs, w, s, out_dtype=torch.float32))
    with pytest.raises(ValueError):  # codes must be u8 when scales are bound
        ops.fp8_linear(_t(x, dev, torch.bfloat16), w, s, xs)


def test_fp8_linear_graph_replays(dev):
    """fp8_linear at every kernel path (fused wide, split with its quantizer,
    deep-k partitions and merge, tiled, the DMA-fed prefill tiles, and the
    entry point without allocation) captured in one HIP graph, as a decode
    or prefill program captures a step: every replay, each on new input
    values written between replays and with eager calls and
    synchronizations in between, equals the eager result bit for bit."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(57)
    shapes = [(1, 2048, 6144), (16, 2048, 6144), (256, 2048, 6144), (64, 4096, 2048),
              (300, 512, 1024), (4096, 2048, 4096)]
    cases = []
    for m, k, n in shapes:
        codes, scales = block_weights(rng, (n, k))
        x = _t(bf16_normal(rng, (m, k), outliers=0.01), dev, torch.bfloat16)
        cases.append((x, _t(codes, dev), _t(scales, dev),
                      torch.empty((m, n), dtype=torch.bfloat16, device=dev)))
    m0, k0, n0 = shapes[0]
    noalloc_out = torch.empty((m0, n0), dtype=torch.bfloat16, device=dev)

    def step():
        for x, w, s, out in cases:
            ops.fp8_linear(x, w, s, out=out)
        x, w, s, _ = cases[0]
        ops.fp8_linear_noalloc(x, w, s, out=noalloc_out)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm the per-stream caches outside capture
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for rep in range(3):
        for x, _, _, out in cases:
            x.copy_(_t(bf16_normal(rng, tuple(x.shape), outliers=0.01), dev, torch.bfloat16))
            out.zero_()
        noalloc_out.zero_()
        g.replay()
        torch.cuda.synchronize()
        got = [out.clone() for *_, out in cases] + [noalloc_out.clone()]
        step()  # eager on the same inputs, between replays
        torch.cuda.synchronize()
        for (_, _, _, out), r in zip(cases, got):
            assert torch.equal(r, out), rep
        assert torch.equal(got[-1], cases[0][3]), rep


def test_zero_row_calls(dev):
    """Empty batches (zero rows) through the dense entry points: each returns
    correctly shaped empty outputs without error, and a later non-empty call
    on the same stream is unaffected."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(61)
    codes, scales = block_weights(rng, (512, 1024))
    w, s = _t(codes, dev), _t(scales, dev)
    x0 = torch.empty((0, 1024), dtype=torch.bfloat16, device=dev)
    q, qs = ops.quantize(x0)
    assert tuple(q.shape) == (0, 1024) and tuple(qs.shape) == (0, 8)
    assert tuple(ops.fp8_linear(x0, w, s, out_dtype=torch.bfloat16).shape) == (0, 512)
    assert tuple(ops.fp8_linear(q, w, s, qs).shape) == (0, 512)
    assert tuple(ops.projection_partial(q, qs, w, s).shape) == (0, 512)
    assert tuple(ops.fp8_linear_noalloc(x0, w, s, out_dtype=torch.bfloat16).shape) == (0, 512)
    norm_w = _t(np.ones(1024, np.float32), dev)
    rc, rs, rn = ops.rms_quantize(x0, norm_w, eps=1e-6)
    assert tuple(rc.shape) == (0, 1024) and tuple(rs.shape) == (0, 8) and tuple(rn.shape) == (0, 1024)
    x = bf16_normal(rng, (5, 1024))
    y = ops.fp8_linear(_t(x, dev, torch.bfloat16), w, s, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rel_fro(y.cpu().numpy(), ofp8.fp8_linear(x, codes, scales)) < 1e-4


def test_linear_workspace_cache_is_bounded(dev):
    """Calls cycling through more streams than the per-device cache keeps
    leave at most that many workspaces cached, and every result equals the
    one-stream result (a dropped workspace is freed in its stream's order)."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(23)
    codes, scales = block_weights(rng, (2048, 2048))
    w, s = _t(codes, dev), _t(scales, dev)
    x = _t(bf16_normal(rng, (64, 2048)), dev, torch.bfloat16)
    ref = ops.fp8_linear(x, w, s)
    torch.cuda.synchronize()
    limit = ops._StreamBuffers.LIMIT
    streams = [torch.cuda.Stream() for _ in range(limit + 8)]
    outs = []
    for rep in range(2):
        for st in streams:
            st.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(st):
                outs.append(ops.fp8_linear(x, w, s))
    torch.cuda.synchronize()
    assert sum(1 for key in ops._WORKSPACES._entries if key[0] == dev.index) <= limit
    for out in outs:
        assert torch.equal(out, ref)
