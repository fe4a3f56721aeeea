"""GPU parity: the FP8 activation quantizer is bit-exact against the oracle."""

import numpy as np
import pytest

from oracle import fp8 as ofp8
from golden_inputs import bf16_normal, stress_rows

pytestmark = pytest.mark.gpu

DT = {"float32": "float32", "float16": "float16", "bfloat16": "bfloat16"}


def _to_device(x, dtype, dev):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(x, np.float32))
    return t.to(getattr(torch, dtype)).to(dev)


def _run(x_np, dtype, dev, top=None):
    import torch
    from akas_amd import ops

    x = _to_device(x_np, dtype, dev)
    codes, scales = ops.quantize(x, top=top)
    torch.cuda.synchronize()
    # the oracle sees exactly the values the device read
    xin = x.float().cpu().numpy()
    ec, es = ofp8.quantize(xin)
    return codes.cpu().numpy(), scales.cpu().numpy(), ec, es


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("top", [None, 4])
def test_quantize_stress_and_random(dev, dtype, top):
    rng = np.random.default_rng(17)
    rows, k = 3, 384
    x = stress_rows(k, rows * (top or 1), rng)
    if top:
        x = x.reshape(rows, top, k)
    c, s, ec, es = _run(x, dtype, dev, top)
    np.testing.assert_array_equal(c, ec)
    np.testing.assert_array_equal(s, es)
    # zero group: scale 1e-12/448, all codes +0
    assert s.reshape(-1)[0] == np.float32(1e-12) / np.float32(448)
    assert not c.reshape(-1, 128)[0].any()


@pytest.mark.parametrize("shape", [(1, 2048), (16, 2048), (257, 1536), (8192, 2048),
                                   (4099, 2048)])
def test_quantize_large_bit_exact(dev, shape):
    """4099 rows: a ragged last grid-stride pass."""
    rng = np.random.default_rng(0)
    x = bf16_normal(rng, shape, outliers=0.01)
    c, s, ec, es = _run(x, "bfloat16", dev)
    np.testing.assert_array_equal(s, es)
    np.testing.assert_array_equal(c, ec)


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_quantize_large_other_dtypes(dev, dtype):
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (4100, 2048)).astype(np.float32)
    if dtype == "float16":
        x = x.astype(np.float16).astype(np.float32)
    c, s, ec, es = _run(x, dtype, dev)
    np.testing.assert_array_equal(s, es)
    np.testing.assert_array_equal(c, ec)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("rows,top", [(5, None), (3, 4), (4099, None)])
def test_quantize_groups_holding_infinity(dev, dtype, rows, top):
    """A group holding +-inf gets scale inf (max|x| / 448) and its finite
    values the codes of x / inf = +-0 (IEEE division, as the reference's
    ``values[j] / scale``, activations/fp8/cuda.py:37-43); an infinite value
    divides to NaN, which the encoder saturates to magnitude code 126 (the
    sign of that NaN is the platform's, so only the magnitude is compared).
    The other groups of the same rows are unaffected."""
    rng = np.random.default_rng(23)
    k = 512
    x = rng.normal(0, 2, (rows * (top or 1), k)).astype(np.float32)
    x[0, 3] = np.inf
    x[1, 130] = -np.inf
    x[2, 256], x[2, 300] = np.inf, -np.inf
    x[-1, 384:] = np.inf  # a group of infinities only
    x[-1, 0] = np.inf
    if top:
        x = x.reshape(rows, top, k)
    c, s, ec, es = _run(x, dtype, dev, top)
    np.testing.assert_array_equal(s, es)
    assert np.isinf(s.reshape(-1, k // 128)[[0, 1, 2], [0, 1, 2]]).all()
    finite = np.isfinite(x)
    np.testing.assert_array_equal(c[finite], ec[finite])
    assert (c[~finite] & 0x7F == 126).all()
    # the finite values of the infinite groups are the signed zero codes
    grp = np.isinf(np.abs(x.reshape(-1, k // 128, 128)).max(-1))
    in_inf_group = np.repeat(grp, 128, axis=-1).reshape(x.shape) & finite
    assert in_inf_group.sum() > 100
    assert (c[in_inf_group] & 0x7F == 0).all()


def test_quantize_midpoints_and_subnormals(dev):
    """Values placed exactly on and one ulp around e4m3 rounding midpoints,
    after scaling, and in the e4m3 subnormal range."""
    rng = np.random.default_rng(5)
    codes = np.arange(0, 126, dtype=np.uint8)
    lo, hi = ofp8.decode_e4m3(codes), ofp8.decode_e4m3(codes + 1)
    mids = ((lo.astype(np.float64) + hi) / 2).astype(np.float32)
    vals = np.concatenate([mids, np.nextafter(mids, 0), np.nextafter(mids, 1000),
                           -mids, rng.uniform(-2 ** -6, 2 ** -6, 1000).astype(np.float32)])
    vals = np.resize(vals, (64, 128 * 4)).astype(np.float32)
    vals[:, ::128] = 448.0  # amax 448 -> scale exactly 1: values pass through unscaled
    c, s, ec, es = _run(vals, "float32", dev)
    np.testing.assert_array_equal(s, es)
    np.testing.assert_array_equal(c, ec)


def test_quantize_group_scale_every_mantissa(dev):
    """The group scale max(max|x|, 1e-12) / 448 is the oracle's float32
    division for every float32 mantissa, at the exponent where the 1e-12
    floor sits, at two ordinary exponents and at the largest finite one, and
    at the ends of the range: groups holding one value (either sign) among
    zeros, through quantize.  (The device forms it without a division
    sequence, from RN(1/448) and one FMA correction.)"""
    import torch
    from akas_amd import ops

    n = 1 << 21
    mant = torch.arange(1 << 23, dtype=torch.int32, device=dev)
    for e in (87, 107, 130, 254):  # biased exponents: 2^-40, 2^-20, 2^3, 2^127
        for c0 in range(0, 1 << 23, n):
            a = (mant[c0:c0 + n] | (e << 23)).view(torch.float32)
            x = torch.zeros((n, 128), dtype=torch.float32, device=dev)
            x[:, 37] = a
            x[::2, 37] *= -1
            _, s = ops.quantize(x)
            got = s.view(-1).cpu().numpy()
            want = ofp8.group_scales(x[:, 37:38].cpu().numpy())
            bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
            assert bad.size == 0, (e, c0 + bad[:8], got[bad[:8]], want[bad[:8]])
    f32 = np.finfo(np.float32)
    ends = np.array([0.0, 1e-45, 1e-13, np.nextafter(np.float32(1e-12), 0), 1e-12,
                     np.nextafter(np.float32(1e-12), 1), 1.0, 448.0, f32.max, np.inf], np.float32)
    x = np.zeros((ends.size, 128), np.float32)
    x[:, 5] = ends
    c, s, ec, es = _run(x, "float32", dev)
    np.testing.assert_array_equal(s.view(np.uint32), es.view(np.uint32))
    # inf / inf is a NaN whose sign is the platform's: magnitude code only
    finite = np.isfinite(x)
    np.testing.assert_array_equal(c[finite], ec[finite])
    assert (c[~finite] & 0x7F == 126).all() and (ec[~finite] & 0x7F == 126).all()


def _numerics_probe(dev, name):
    """Run an exhaustive check of the numerics probe (libakas_probe.so):
    returns the mismatch count and the first mismatching bit patterns."""
    import ctypes

    import torch
    from akas_amd import build

    fn = getattr(ctypes.CDLL(build.PROBE_LIBRARY), name)
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    out = torch.zeros(9, dtype=torch.int64, device=dev)
    assert fn(out.data_ptr(), torch.cuda.current_stream().cuda_stream) == 0
    res = out.cpu().numpy()
    return int(res[0]), [hex(int(b)) for b in res[1:1 + min(int(res[0]), 8)]]


def test_group_scale_every_input(dev):
    """The device's group scale and its reciprocal (formed without a division
    sequence) equal IEEE float32 division for every group maximum from the
    1e-12 floor to FLT_MAX and for +inf: the numerics probe runs the same
    device function over all of them (about 360 million inputs)."""
    n, first = _numerics_probe(dev, "akas_probe_group_scale_check")
    assert n == 0, first


def test_e4m3_hardware_pack_every_input(dev):
    """The hardware e4m3 pack the quantizers use equals the integer
    restatement of the reference encoder (_shared/e4m3.py:16-29) for every
    float32 of magnitude below 464, both signs (about 2.3 billion inputs)."""
    n, first = _numerics_probe(dev, "akas_probe_e4m3_pack_check")
    assert n == 0, first


def test_bf16_hardware_pack_every_input(dev):
    """The packed bf16 conversion equals the reference's integer round to
    nearest even (_shared/rounding.py:43-54) for every non-NaN float32."""
    n, first = _numerics_probe(dev, "akas_probe_bf16_pack_check")
    assert n == 0, first


def test_dequantize_round_trip(dev):
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(3)
    x = bf16_normal(rng, (33, 1024))
    c, s = ops.quantize(_to_device(x, "bfloat16", dev))
    d = ops.dequantize_fp8(c, s).cpu().numpy()
    exp = ofp8.dequantize_activation(c.cpu().numpy(), s.cpu().numpy())
    np.testing.assert_array_equal(d, exp)


@pytest.mark.parametrize("scale_dtype", ["float32", "bfloat16"])
def test_weight_block_quantizer(dev, scale_dtype):
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(0)
    w = rng.normal(0, 0.02, (2, 300, 512)).astype(np.float32)
    codes, scales = ops.quantize_weight_blocks(torch.from_numpy(w).to(dev),
                                               scale_dtype=getattr(torch, scale_dtype))
    ec, es = ofp8.quantize_weight_blocks(w, scale_dtype)
    np.testing.assert_array_equal(scales.float().cpu().numpy(), es)
    np.testing.assert_array_equal(codes.cpu().numpy(), ec)
