"""RMSNorm and its fusion with the activation quantizer (oracle).

Test infrastructure only; see ``oracle/__init__.py``.
"""

import numpy as np

from .fp8 import quantize, round_to


def rms_norm(x, w, eps, zero_centered=False, out_dtype="float32"):
    """``x / sqrt(mean(x^2) + eps) * w`` per row in float64, then rounded to
    ``out_dtype``; ``1 + w`` when ``zero_centered``.  Follows
    ``src/akas/ops/normalization/validation.py:31-52`` (kind ``rms``)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    if zero_centered:
        w = 1.0 + w
    y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w
    return round_to(y.astype(np.float32), out_dtype)


def rms_quantize_of(normalized):
    """The codes/scales the fused kernel must produce for the normalized rows
    it returns: ``quantize`` of exactly those values
    (``src/akas/quantization/activations/fp8/cuda.py:10-56``)."""
    return quantize(np.asarray(normalized, np.float32))
