"""Pins the oracle's FP8 codec, quantizer, weight blocks and dense linear.

Every check here is independent of the oracle's own formula: torch's
float8_e4m3fn / bfloat16 casts, a brute-force nearest-even search over the
finite e4m3 magnitudes, float64 quotients (exact after rounding to float32 by
the double-rounding theorem for division, 53 >= 2*24 + 2), hand-derived known
answers from the reference's stress row, and integer brute force on
exact-product inputs.  CPU only.
"""

import numpy as np
import pytest
import torch

from golden_inputs import bf16_normal, exact_codes, rel_fro, stress_rows
from oracle import fp8 as ofp8


def _torch_e4m3_decode(codes):
    t = torch.from_numpy(np.asarray(codes, np.uint8).copy()).view(torch.float8_e4m3fn)
    return t.float().numpy()


def _finite_magnitudes():
    """The 127 finite non-negative e4m3 values (codes 0..126) from torch."""
    return _torch_e4m3_decode(np.arange(127, dtype=np.uint8)).astype(np.float64)


def _nearest_even_encode(values):
    """Independent encoder: nearest finite magnitude, ties to the even code,
    saturating at 448, sign bit copied from the float32 pattern."""
    v = np.asarray(values, np.float32)
    mag = np.abs(v).astype(np.float64)
    table = _finite_magnitudes()
    hi = np.clip(np.searchsorted(table, mag, side="left"), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    d_hi, d_lo = np.abs(table[hi] - mag), np.abs(mag - table[lo])
    code = np.where(d_lo < d_hi, lo, hi)
    tie = d_lo == d_hi
    code = np.where(tie, np.where(lo % 2 == 0, lo, hi), code)
    sign = (v.view(np.uint32) >> 31).astype(np.uint8) << 7
    return code.astype(np.uint8) | sign


def test_decode_every_code_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    finite = (codes & 127) != 127
    np.testing.assert_array_equal(ofp8.decode_e4m3(codes)[finite], _torch_e4m3_decode(codes)[finite])
    # codes 0x7F / 0xFF are NaN in OCP e4m3; the reference's closed form reads
    # them as +-480 and its weight storage never emits them (&127 != 127).
    assert ofp8.decode_e4m3(np.uint8(0x7F)) == 480.0


def _encode_inputs():
    rng = np.random.default_rng(2)
    every_bf16 = (np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32)
    every_bf16 = every_bf16[np.isfinite(every_bf16)]
    table = _finite_magnitudes()
    mids = ((table[1:] + table[:-1]) / 2).astype(np.float32)  # exact ties
    nudged = np.concatenate([np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9))])
    wide = (rng.choice([-1, 1], 200000) * np.exp2(rng.uniform(-14, 10, 200000))).astype(np.float32)
    return np.concatenate([every_bf16, mids, -mids, nudged, -nudged, wide,
                           np.float32([0.0, -0.0, 448, 464, 479, 480, 1e30, -1e30])])


def test_encode_matches_nearest_even_search():
    v = _encode_inputs()
    np.testing.assert_array_equal(ofp8.encode_e4m3(v), _nearest_even_encode(v))


def test_encode_matches_torch_cast_on_finite_range():
    v = _encode_inputs()
    v = v[np.abs(v) <= 448]
    got = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ofp8.encode_e4m3(v), got)


def test_quantize_stress_row_known_answers():
    """Stress row of src/akas/quantization/activations/fp8/validation.py:24:
    max 448 -> scale exactly 1, and the codes derived by hand from the OCP
    e4m3 grid: 1.0625 is the 1|1.125 midpoint (even: 1.0 = 0x38), 1.1875 the
    1.125|1.25 midpoint (even: 1.25 = 0x3A), 2^-10 rounds to zero at the
    2^-9 subnormal spacing; signs are kept, zeros included."""
    row = np.zeros((1, 128), np.float32)
    row[0, :8] = [448, -448, 1.0625, 1.1875, 2.0**-10, -(2.0**-10), 0.0, -0.0]
    codes, scales = ofp8.quantize(row)
    assert scales[0, 0] == np.float32(1.0)
    assert list(codes[0, :8]) == [0x7E, 0xFE, 0x38, 0x3A, 0x00, 0x80, 0x00, 0x80]
    assert (codes[0, 8:] == 0).all()


def test_quantize_zero_row_scale():
    codes, scales = ofp8.quantize(np.zeros((2, 256), np.float32))
    assert (scales == np.float32(np.float32(1e-12) / np.float32(448))).all()
    assert (codes == 0).all()


def test_quantize_is_float32_division_and_scale():
    rng = np.random.default_rng(3)
    x = np.concatenate([bf16_normal(rng, (64, 2048), outliers=0.01), stress_rows(2048, 4, rng)])
    codes, scales = ofp8.quantize(x)
    blocks = x.astype(np.float64).reshape(x.shape[0], -1, 128)
    amax = np.abs(blocks).max(axis=-1)
    exp_scales = (np.maximum(amax, np.float64(np.float32(1e-12))) / 448.0).astype(np.float32)
    np.testing.assert_array_equal(scales, exp_scales)
    quot = (blocks / exp_scales.astype(np.float64)[..., None]).astype(np.float32)
    np.testing.assert_array_equal(codes, _nearest_even_encode(quot).reshape(x.shape))


def test_device_division_method_is_exact():
    """The device divides by a group scale with one reciprocal and one FMA
    correction (Markstein); the C oracle checks that against IEEE float32
    division on 2M random (x, s) pairs drawn like real groups."""
    import ctypes

    from oracle import native

    lib = native.load()
    bad = ctypes.c_int64(0)
    n = lib.ref_check_exact_quotient(2_000_000, 12345, ctypes.byref(bad))
    assert n == 0 and bad.value == 0


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(4)
    v = rng.normal(0, 1, 200000).astype(np.float32) * np.exp2(rng.integers(-20, 20, 200000)).astype(np.float32)
    ties = ((rng.integers(0, 1 << 15, 5000, dtype=np.uint32) << 16) | 0x8000).view(np.float32)
    v = np.concatenate([v, ties[np.isfinite(ties)], np.float32([0.0, -0.0, 1e-40, -1e-40])])
    np.testing.assert_array_equal(ofp8.bf16_round(v), torch.from_numpy(v).to(torch.bfloat16).float().numpy())


@pytest.mark.parametrize("scale_dtype", ["float32", "bfloat16"])
def test_weight_blocks(scale_dtype):
    rng = np.random.default_rng(5)
    w = rng.normal(0, 0.02, (300, 384)).astype(np.float32)  # ragged last row block
    codes, scales = ofp8.quantize_weight_blocks(w, scale_dtype)
    assert scales.shape == (3, 3) and ((codes & 127) != 127).all()
    pad = np.zeros((384, 384), np.float64)
    pad[:300] = w
    amax = np.abs(pad.reshape(3, 128, 3, 128)).max(axis=(1, 3))
    exp = (amax / 448.0).astype(np.float32)
    if scale_dtype == "bfloat16":
        exp = torch.from_numpy(exp).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(scales, exp)
    full = np.repeat(np.repeat(exp.astype(np.float64), 128, 0), 128, 1)[:300]
    quot = (w.astype(np.float64) / full).astype(np.float32)
    np.testing.assert_array_equal(codes, _nearest_even_encode(quot))


def _exact_case(rng, r, k, o):
    x = exact_codes(rng, (r, k))
    w = exact_codes(rng, (o, k))
    xs = (2.0 ** rng.integers(-4, 2, (r, k // 128))).astype(np.float32)
    ws = (2.0 ** rng.integers(-4, 2, ((o + 127) // 128, k // 128))).astype(np.float32)
    return x, xs, w, ws


def test_linear_exact_products_brute_force():
    """Triple loop in Python integers x powers of two: exact, with per-block
    scales that differ along both axes (a transposed operand or a wrong block
    index changes the result)."""
    rng = np.random.default_rng(6)
    r, k, o = 3, 384, 260
    x, xs, w, ws = _exact_case(rng, r, k, o)
    got = ofp8.fp8_linear(x, w, ws, activation_scales=xs)
    dx, dw = ofp8.decode_e4m3(x).astype(np.float64), ofp8.decode_e4m3(w).astype(np.float64)
    for i in range(r):
        for n in range(0, o, 37):
            acc = 0.0
            for kk in range(k):
                acc += dx[i, kk] * xs[i, kk // 128] * dw[n, kk] * ws[n // 128, kk // 128]
            assert got[i, n] == np.float32(acc)


def test_linear_quantizes_then_multiplies():
    """fp8_linear on float input equals the product of the independently
    quantized operands, and stays within FP8 rounding of the float product."""
    rng = np.random.default_rng(7)
    x = bf16_normal(rng, (16, 512))
    wf = rng.normal(0, 0.02, (256, 512)).astype(np.float32)
    w, ws = ofp8.quantize_weight_blocks(wf)
    y = ofp8.fp8_linear(x, w, ws)
    xq = (x.astype(np.float64).reshape(16, 4, 128))
    s = (np.abs(xq).max(-1) / 448.0).astype(np.float32).astype(np.float64)
    # activations dequantize in float32 (validation.py:15-17: decode * scale,
    # a product of up to 28 significant bits, rounded); weights in float64
    xd = (_torch_e4m3_decode(_nearest_even_encode((xq / s[..., None]).astype(np.float32)))
          * s[..., None].astype(np.float32)).astype(np.float32).astype(np.float64)
    wd = _torch_e4m3_decode(w).astype(np.float64) * np.repeat(np.repeat(ws, 128, 0), 128, 1)
    np.testing.assert_allclose(y, (xd.reshape(16, 512) @ wd.T).astype(np.float32), rtol=1e-6, atol=1e-9)
    assert rel_fro(y, x.astype(np.float64) @ wf.astype(np.float64).T) < 0.08


def test_projection_partitions_known_answers():
    """src/akas/ops/linear/definition.py:13-40: smallest divisor of K/128 that
    reaches the minimum workgroup count."""
    # 16 k-blocks, 1 row tile x 96 column tiles: 256 groups need >= 3 -> 4
    assert ofp8.projection_partitions(1, 2048, 6144, 16, 256, 16, 64) == 4
    # already enough groups -> 1
    assert ofp8.projection_partitions(256, 2048, 6144, 16, 64, 16, 64) == 1
    # the requirement exceeds every divisor -> the largest allowed one
    assert ofp8.projection_partitions(1, 768, 128, 4, 10_000, 16, 64) == 3
    # no minimum: the ceiling itself, which must divide the blocks
    assert ofp8.projection_partitions(1, 1024, 128, 4, None, 16, 64) == 4
    with pytest.raises(ValueError):
        ofp8.projection_partitions(1, 1000, 128, 4, 8, 16, 64)
    with pytest.raises(ValueError):
        ofp8.projection_partitions(1, 768, 128, 4, None, 16, 64)


def test_projection_partial_slices_and_merge():
    rng = np.random.default_rng(8)
    x, xs, w, ws = _exact_case(rng, 5, 512, 256)
    part = ofp8.projection_partial(x, xs, w, ws, 4)
    for p in range(4):
        seg = slice(p * 128, (p + 1) * 128)
        exp = ofp8.fp8_linear(x[:, seg], w[:, seg], ws[:, p:p + 1], activation_scales=xs[:, p:p + 1])
        np.testing.assert_array_equal(part[:, p], exp)
    np.testing.assert_array_equal(ofp8.projection_merge(part),
                                  ofp8.fp8_linear(x, w, ws, activation_scales=xs))


def test_c_oracle_matches_numpy_oracle():
    """oracle/cpu_ref.c (the timed CPU baseline) agrees with the NumPy oracle:
    codes and scales bit for bit, outputs within float32 accumulation."""
    from oracle import native

    lib = native.load()
    rng = np.random.default_rng(0)
    x = ofp8.bf16_round(np.concatenate([bf16_normal(rng, (12, 2048), outliers=0.01),
                                        stress_rows(2048, 4, rng)]))
    xb = ofp8.bf16_bits(x)
    codes = np.zeros(x.shape, np.uint8)
    scales = np.zeros((x.shape[0], 16), np.float32)
    assert lib.ref_quantize_bf16(native.ptr(xb), native.ptr(codes), native.ptr(scales), x.shape[0], 2048, 1) == 0
    ec, es = ofp8.quantize(x)
    np.testing.assert_array_equal(codes, ec)
    np.testing.assert_array_equal(scales, es)
    w, ws = ofp8.quantize_weight_blocks(rng.normal(0, 0.02, (384, 2048)).astype(np.float32))
    y = np.zeros((x.shape[0], 384), np.float32)
    assert lib.ref_fp8_linear_bf16(native.ptr(xb), native.ptr(w), native.ptr(ws), native.ptr(y), 0,
                                   x.shape[0], 2048, 384, 2) == 0
    assert rel_fro(y, ofp8.fp8_linear(x, w, ws)) < 1e-6
