"""Seeded input recipes shared by the CPU oracle tests, the GPU parity tests,
the golden fixtures and the benchmark (numpy only; no device code)."""

import numpy as np

from oracle import fp8 as ofp8


def bf16_normal(rng, shape, std=1.0, outliers=0.0, factor=20.0):
    """float32 values on the bfloat16 grid, ~N(0, std) with an optional
    fraction of entries multiplied by ``factor`` (before bf16 rounding)."""
    x = rng.normal(0.0, std, shape).astype(np.float32)
    if outliers:
        mask = rng.random(shape) < outliers
        x = np.where(mask, x * np.float32(factor), x).astype(np.float32)
    return ofp8.bf16_round(x)


def block_weights(rng, shape, std=0.02, scale_dtype="float32"):
    """e4m3 codes + 128x128 block scales from N(0, std) float32 weights."""
    w = rng.normal(0.0, std, shape).astype(np.float32)
    return ofp8.quantize_weight_blocks(w, scale_dtype)


def exact_codes(rng, shape):
    """Signed codes from {56, 64} (values +-1, +-2): with binary scales every
    product and partial sum of a block-scaled dot product is exact in float32
    (src/akas/ops/moe/validation.py:353-360)."""
    c = rng.choice(np.array([56, 64], dtype=np.uint8), shape)
    return (c | (rng.integers(0, 2, shape, dtype=np.uint8) * 128)).astype(np.uint8)


def random_codes(rng, shape, lo=32, hi=81):
    """Finite signed codes with magnitude codes in [lo, hi)."""
    c = rng.integers(lo, hi, shape, dtype=np.uint8)
    return (c | (rng.integers(0, 2, shape, dtype=np.uint8) * 128)).astype(np.uint8)


def rel_fro(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def stress_rows(k, rows, rng):
    """Quantizer stress input: a zero group and the reference's special values
    (src/akas/quantization/activations/fp8/validation.py:21-26)."""
    x = rng.normal(0, 0.15, (rows, k)).astype(np.float32)
    g = x.reshape(-1, 128)
    g[0] = 0
    if len(g) > 1:
        g[1, :8] = [448, -448, 1.0625, 1.1875, 2 ** -10, -(2 ** -10), 0, -0.0]
    return x
