"""FP8 codec, activation quantizer and block-scaled dense linear (oracle).

Test infrastructure only; see ``oracle/__init__.py``.
"""

import numpy as np

BLOCK = 128
F32_EPS_SCALE = np.float32(1e-12)
E4M3_MAX = np.float32(448)


# --------------------------------------------------------------------------
# scalar codecs
# --------------------------------------------------------------------------

def bf16_round(values):
    """Round float32 values to the nearest bfloat16, ties to even; f32 out.

    Follows ``src/akas/quantization/_shared/rounding.py:43-54``
    (``(bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000``); finite inputs.
    """
    v = np.ascontiguousarray(values, dtype=np.float32)
    bits = v.view(np.uint32).astype(np.uint64)
    out = ((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return out.view(np.float32).reshape(v.shape)


def f16_round(values):
    """Round float32 to float16 and back (IEEE nearest-even)."""
    with np.errstate(over="ignore"):  # beyond the f16 range rounds to inf, as in IEEE
        return np.asarray(values, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(values, dtype):
    """Round to the storage dtype named by the reference ('float32', 'float16', 'bfloat16')."""
    if dtype == "bfloat16":
        return bf16_round(values)
    if dtype == "float16":
        return f16_round(values)
    if dtype == "float32":
        return np.asarray(values, dtype=np.float32)
    raise ValueError(f"unsupported rounding dtype {dtype}")


def bf16_bits(values):
    """float32 values -> uint16 bfloat16 storage bits (nearest-even)."""
    return (bf16_round(values).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits):
    """uint16 bfloat16 storage bits -> float32 values."""
    b = np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def decode_e4m3(bits):
    """OCP e4m3 byte -> float32: ``exp==0 ? f/512 : (1+f/8)*2^(exp-7)``, signed.

    Follows ``src/akas/quantization/_shared/e4m3.py:4-13``.
    """
    bits = np.asarray(bits, dtype=np.uint8)
    exponent = ((bits >> 3) & 15).astype(np.int32)
    fraction = (bits & 7).astype(np.float32)
    magnitude = np.where(
        exponent == 0,
        fraction / np.float32(512),
        (np.float32(1) + fraction / np.float32(8)) * np.exp2(exponent - 7).astype(np.float32),
    ).astype(np.float32)
    return np.where(bits & 128, -magnitude, magnitude).astype(np.float32)


def encode_e4m3(values):
    """float32 -> OCP e4m3 byte, nearest-even, finite saturation at 448.

    Follows ``src/akas/quantization/_shared/e4m3.py:16-29``: normals round the
    f32 bit pattern at mantissa bit 20 (``+0x7FFFF + bit20``) and rebias by
    ``960 = 120 << 3``; magnitudes below ``2^-6`` use ``rint(|v| * 512)``;
    the magnitude code is clipped to ``[0, 126]`` and the sign bit ORed in.
    """
    v = np.asarray(values, dtype=np.float32)
    bits = np.ascontiguousarray(v).view(np.uint32).reshape(v.shape)
    magnitude = np.abs(v)
    rounded = (bits & np.uint32(0x7FFFFFFF)) + np.uint32(0x7FFFF) + ((bits >> 20) & 1)
    normal = (rounded >> 20).astype(np.int64) - 960
    with np.errstate(over="ignore", invalid="ignore"):  # only taken below 2^-6
        subnormal = np.rint(magnitude * np.float32(512)).astype(np.int64)
    code = np.clip(np.where(magnitude < np.float32(0.015625), subnormal, normal), 0, 126)
    return code.astype(np.uint8) | ((bits >> 24) & 128).astype(np.uint8)


# --------------------------------------------------------------------------
# activation quantizer (1 x 128 groups)
# --------------------------------------------------------------------------

def group_scales(blocks):
    """Per-group scale ``max(max|x|, 1e-12) / 448`` in float32.

    Follows ``src/akas/quantization/activations/fp8/cuda.py:39`` and
    ``validation.py:29-31``.
    """
    amax = np.max(np.abs(blocks.astype(np.float32)), axis=-1)
    return (np.maximum(amax, F32_EPS_SCALE) / E4M3_MAX).astype(np.float32)


def quantize(x):
    """Per-token, per-128-group FP8 quantizer (reference kind ``quantize``).

    ``x`` has shape ``[..., k]`` (``[r, k]`` or ``[r, top, k]``), any float
    dtype; it is widened to float32 exactly as the device kernel does.
    Returns ``(codes uint8 [..., k], scales float32 [..., k/128])`` where
    ``codes = enc(x / s)`` with IEEE float32 division.

    Follows ``src/akas/quantization/activations/fp8/cuda.py:10-56`` and the
    oracle ``src/akas/quantization/activations/fp8/validation.py:27-36``.
    """
    x = np.asarray(x, dtype=np.float32)
    k = x.shape[-1]
    if k % BLOCK:
        raise ValueError("FP8 channels must be divisible by 128")
    blocks = x.reshape(*x.shape[:-1], k // BLOCK, BLOCK)
    scales = group_scales(blocks)
    with np.errstate(invalid="ignore"):  # inf / inf in a group holding inf gives NaN, as on the GPU
        codes = encode_e4m3(blocks / scales[..., None]).reshape(x.shape)
    return codes, scales


def dequantize_activation(codes, scales):
    """``decode(codes) * scale`` per 128-group, float32 (validation.py:15-17)."""
    codes = np.asarray(codes, dtype=np.uint8)
    k = codes.shape[-1]
    d = decode_e4m3(codes).reshape(*codes.shape[:-1], k // BLOCK, BLOCK)
    return (d * np.asarray(scales, np.float32)[..., None]).reshape(codes.shape)


def fake_quantize(x):
    """``dec(enc(x/s))*s`` (``tests/support/native_fp8_reference.py:84-89``)."""
    codes, scales = quantize(x)
    return dequantize_activation(codes, scales)


# --------------------------------------------------------------------------
# block-scaled weights (128 x 128 blocks)
# --------------------------------------------------------------------------

def quantize_weight_blocks(w, scale_dtype="float32"):
    """Block-quantize float32 weights ``[..., N, K]`` to e4m3 + block scales.

    Scale per 128x128 block is ``max(|block|, 1e-12) / 448`` in float32
    (the measured workloads' weight recipe); ``scale_dtype='bfloat16'`` rounds
    each scale to bf16 *before* encoding, which is the reference's resident
    storage (``src/akas/quantization/weights/fp8/definition.py:24-27``,
    ``kernel.py:53``).  Codes are finite (``&127 != 127``, ``kernel.py:48-49``).
    Returns ``(codes uint8 [..., N, K], scales float32 [..., ceil(N/128), K/128])``.
    """
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape[-2:]
    if k % BLOCK:
        raise ValueError("FP8 weight channels must be divisible by 128")
    nb = (n + BLOCK - 1) // BLOCK
    pad = nb * BLOCK - n
    wp = np.pad(w, [(0, 0)] * (w.ndim - 2) + [(0, pad), (0, 0)]) if pad else w
    blocks = wp.reshape(*w.shape[:-2], nb, BLOCK, k // BLOCK, BLOCK)
    amax = np.max(np.abs(blocks), axis=(-3, -1))
    scales = (np.maximum(amax, F32_EPS_SCALE) / E4M3_MAX).astype(np.float32)
    if scale_dtype == "bfloat16":
        scales = bf16_round(scales)
    elif scale_dtype != "float32":
        raise ValueError("scale dtype must be float32 or bfloat16")
    expanded = expand_block_scales(scales, n, k)
    codes = encode_e4m3(w / expanded)
    return codes, scales


def expand_block_scales(scales, n, k):
    """Repeat ``[..., ceil(N/128), K/128]`` block scales to ``[..., N, K]``."""
    s = np.asarray(scales, dtype=np.float32)
    return np.repeat(np.repeat(s, BLOCK, axis=-2), BLOCK, axis=-1)[..., :n, :k]


def dequantize_weight(codes, scales):
    """Decoded weight ``dec(w) * scales[n//128, k//128]`` in float64.

    Follows ``src/akas/ops/linear/validation.py:214-217`` and
    ``src/akas/quantization/weights/fp8/validation.py:17-23``.
    """
    codes = np.asarray(codes, dtype=np.uint8)
    n, k = codes.shape[-2:]
    return decode_e4m3(codes).astype(np.float64) * expand_block_scales(scales, n, k)


# --------------------------------------------------------------------------
# dense linear
# --------------------------------------------------------------------------

def fp8_linear(x, w, scales, activation_scales=None, out_dtype="float32"):
    """Block-scaled FP8 linear ``y = deq(quantize(x)) @ deq(W).T``.

    * ``x``: float activations ``[r, k]`` (quantized per 1x128 group first), or
      uint8 codes when ``activation_scales`` is given (prequantized input,
      ``projection_partial`` with one partition).
    * ``w``: uint8 ``[o, k]``; ``scales``: float ``[ceil(o/128), k/128]``.

    Accumulates in float64 and rounds once to ``out_dtype``.  Follows
    ``src/akas/ops/linear/validation.py:206-230``.
    """
    if activation_scales is None:
        xq = fake_quantize(x).astype(np.float64)
    else:
        xq = dequantize_activation(x, activation_scales).astype(np.float64)
    y = xq @ dequantize_weight(w, scales).T
    return round_to(y.astype(np.float32), out_dtype)


def projection_partitions(rows, depth, width, ceiling, minimum_groups, block_m, columns):
    """Smallest legal K-partition count that fills an under-occupied launch.

    Follows ``src/akas/ops/linear/definition.py:13-40``.
    """
    from math import isqrt

    if depth < 128 or depth % 128:
        raise ValueError("split projection requires whole block-128 partitions")
    blocks = depth // 128
    ceiling = min(ceiling, blocks)
    if minimum_groups is None:
        if blocks % ceiling:
            raise ValueError("split projection requires whole block-128 partitions")
        return ceiling
    groups = ((rows + block_m - 1) // block_m) * ((width + columns - 1) // columns)
    required = (minimum_groups + groups - 1) // groups
    choices = sorted({v for f in range(1, isqrt(blocks) + 1) if blocks % f == 0
                      for v in (f, blocks // f) if v <= ceiling})
    return next((v for v in choices if v >= required), choices[-1])


def projection_partial(codes, activation_scales, w, scales, partitions):
    """Split-K partial products ``[r, parts, o]`` (float32).

    Follows ``src/akas/ops/linear/validation.py:76-111``.
    """
    x = dequantize_activation(codes, activation_scales).astype(np.float64)
    weight = dequantize_weight(w, scales)
    r, k = x.shape
    o = weight.shape[0]
    span = k // partitions
    out = np.zeros((r, partitions, o), np.float32)
    for part in range(partitions):
        seg = slice(part * span, (part + 1) * span)
        out[:, part] = x[:, seg] @ weight[:, seg].T
    return out


def projection_merge(partial, out_dtype="float32"):
    """Serial float32 sum over partitions (``src/akas/ops/linear/cuda.py:1369-1402``)."""
    partial = np.asarray(partial, np.float32)
    total = np.zeros(partial.shape[:-2] + partial.shape[-1:], np.float32)
    for part in range(partial.shape[-2]):
        total += partial[..., part, :]
    return round_to(total, out_dtype)
