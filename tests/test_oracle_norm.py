"""Pins the RMSNorm oracle with closed forms and invariants (no retyping of
its formula): constant rows, unit mean square, row-scale invariance,
zero-centred weights and the zero row."""

import numpy as np

from oracle import norm


def test_constant_row_closed_form():
    c, eps = np.float32(3.0), 1e-3
    x = np.full((1, 256), c, np.float32)
    w = np.linspace(0.5, 1.5, 256).astype(np.float32)
    y = norm.rms_norm(x, w, eps)
    exp = (3.0 / np.sqrt(9.0 + eps)) * w.astype(np.float64)
    np.testing.assert_allclose(y[0], exp, rtol=1e-6)
    np.testing.assert_allclose(norm.rms_norm(-x, w, 0.0)[0], -w, rtol=1e-6)


def test_unit_mean_square_and_scale_invariance():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (5, 384)).astype(np.float32)
    ones = np.ones(384, np.float32)
    y = norm.rms_norm(x, ones, 0.0).astype(np.float64)
    np.testing.assert_allclose(np.mean(y * y, axis=1), 1.0, rtol=1e-6)
    np.testing.assert_allclose(norm.rms_norm(x * np.float32(37.5), ones, 0.0), y, rtol=1e-6)
    # each row is positively homogeneous of degree 1 in w
    w = rng.uniform(0.5, 2.0, 384).astype(np.float32)
    np.testing.assert_allclose(norm.rms_norm(x, w, 0.0), y * w, rtol=1e-6)


def test_zero_centered_and_zero_row():
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, (3, 128)).astype(np.float32)
    w = rng.normal(0, 0.1, 128).astype(np.float32)
    np.testing.assert_allclose(norm.rms_norm(x, w, 1e-5, zero_centered=True),
                               norm.rms_norm(x, (1.0 + w.astype(np.float64)).astype(np.float32), 1e-5),
                               rtol=1e-6)
    z = norm.rms_norm(np.zeros((2, 128), np.float32), w, 1e-6)
    assert np.all(z == 0)


def test_rounding_to_storage_dtype():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (4, 256)).astype(np.float32)
    w = np.ones(256, np.float32)
    y32 = norm.rms_norm(x, w, 1e-6)
    ybf = norm.rms_norm(x, w, 1e-6, out_dtype="bfloat16")
    assert np.all((ybf.view(np.uint32) & 0xFFFF) == 0)
    assert np.max(np.abs(ybf - y32) / np.maximum(np.abs(y32), 1e-30)) <= 2.0 ** -8
