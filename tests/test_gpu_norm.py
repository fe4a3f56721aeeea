"""GPU parity of the fused RMSNorm + quantizer (``rms_quantize``): the
normalized rows against the float64 oracle (within one unit in the last place
of the output dtype: float32 accumulation against float64), and the codes and
scales bit-exact against the quantizer applied to exactly the rows returned."""

import numpy as np
import pytest

from golden_inputs import bf16_normal
from oracle import norm as onorm

pytestmark = pytest.mark.gpu

ULP = {"bfloat16": 2.0 ** -7, "float16": 2.0 ** -10, "float32": 2.0 ** -21}


def _t(a, dev, dtype):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(getattr(torch, dtype))


def _np(t):
    import torch

    torch.cuda.synchronize()
    return t.float().cpu().numpy() if t.dtype in (torch.bfloat16, torch.float16) else t.cpu().numpy()


@pytest.mark.parametrize("rows,cols", [(1, 128), (7, 384), (300, 2048), (33, 8192), (64, 640),
                                       (5, 2176), (9, 4224)])
@pytest.mark.parametrize("x_dtype,w_dtype,y_dtype", [("bfloat16", "float32", "bfloat16"),
                                                      ("float32", "bfloat16", "float32"),
                                                      ("float16", "float32", "float16")])
@pytest.mark.parametrize("zero_centered", [False, True])
def test_rms_quantize(dev, rows, cols, x_dtype, w_dtype, y_dtype, zero_centered):
    from akas_amd import ops

    rng = np.random.default_rng(rows * 7 + cols)
    x = bf16_normal(rng, (rows, cols), std=2.0, outliers=0.01)
    if x_dtype == "float16":
        x = x.astype(np.float16).astype(np.float32)
    w = (rng.normal(0, 0.1, cols) if zero_centered else rng.uniform(0.5, 1.5, cols)).astype(np.float32)
    xt, wt = _t(x, dev, x_dtype), _t(w, dev, w_dtype)
    codes, scales, y = ops.rms_quantize(xt, wt, eps=1e-5, zero_centered=zero_centered,
                                        normalized_dtype=y_dtype)
    got = _np(y)
    exp = onorm.rms_norm(_np(xt), _np(wt), 1e-5, zero_centered, y_dtype)
    err = np.abs(got - exp) / np.maximum(np.abs(exp), 1e-30)
    assert float(err.max()) <= ULP[y_dtype]
    ec, es = onorm.rms_quantize_of(got)
    np.testing.assert_array_equal(_np(codes), ec)
    np.testing.assert_array_equal(_np(scales), es)
    c2, s2 = ops.quantize(y)
    np.testing.assert_array_equal(_np(codes), _np(c2))
    np.testing.assert_array_equal(_np(scales), _np(s2))
    c3, s3 = ops.rms_quantize(xt, wt, eps=1e-5, zero_centered=zero_centered,
                              normalized_dtype=y_dtype, return_normalized=False)
    np.testing.assert_array_equal(_np(c3), _np(codes))
    np.testing.assert_array_equal(_np(s3), _np(scales))


def test_rms_quantize_zero_rows_and_eps(dev):
    from akas_amd import ops

    x = np.zeros((4, 256), np.float32)
    x[1] = 1e-20
    w = np.ones(256, np.float32)
    codes, scales, y = ops.rms_quantize(_t(x, dev, "float32"), _t(w, dev, "float32"), eps=1e-6,
                                        normalized_dtype="float32")
    exp = onorm.rms_norm(x, w, 1e-6)
    np.testing.assert_allclose(_np(y), exp, rtol=2.0 ** -21, atol=0)
    assert np.all(_np(codes)[[0, 2, 3]] == 0)
    np.testing.assert_array_equal(_np(scales)[0], np.full(2, np.float32(1e-12) / np.float32(448)))


def test_rms_quantize_rejects_bad_geometry(dev):
    from akas_amd import ops

    w = _t(np.ones(100, np.float32), dev, "float32")
    with pytest.raises(ValueError):
        ops.rms_quantize(_t(np.ones((2, 100), np.float32), dev, "float32"), w, eps=1e-5)
    big = _t(np.ones((1, 8320), np.float32), dev, "bfloat16")
    with pytest.raises(ValueError):
        ops.rms_quantize(big, _t(np.ones(8320, np.float32), dev, "float32"), eps=1e-5)
    x = _t(np.ones((2, 128), np.float32), dev, "bfloat16")
    with pytest.raises(ValueError):
        ops.rms_quantize(x, _t(np.ones(128, np.float32), dev, "float32"), eps=-1.0)
    with pytest.raises(ValueError):
        ops.rms_quantize(x, _t(np.ones(256, np.float32), dev, "float32"), eps=1e-5)
