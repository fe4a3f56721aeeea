"""Operator kinds of the block-scaled FP8 path, on PyTorch-ROCm device tensors.

Each function mirrors one graph call kind of the reference (same name, same
parameter meaning, same buffer names and output order) and calls the gfx950
C ABI of ``include/akas_fp8.h`` on the current HIP stream of its tensors'
device (made current for the call when it is not).  Outputs may be
passed in (caller-owned buffers, as in the reference runtime) or are
allocated here with torch.  Invalid geometry raises ``ValueError`` before any
launch, like the reference factories.  There is no CPU fallback.
"""

import collections
import functools

import torch

from . import _lib
from ._lib import BF16, F16, F32, check

BLOCK = 128

_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
_NAME_TO_TORCH = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def _dt(dtype):
    """torch dtype or reference dtype name -> ABI code."""
    if isinstance(dtype, str):
        dtype = _NAME_TO_TORCH.get(dtype)
    if dtype not in _DTYPE_CODE:
        raise ValueError(f"unsupported dtype {dtype}")
    return _DTYPE_CODE[dtype]


def _torch_dtype(dtype):
    return _NAME_TO_TORCH[dtype] if isinstance(dtype, str) else dtype


def _stream():
    """hipStream_t of torch's current stream on the current device."""
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _on_tensor_device(fn):
    """Run an op on the device of its tensor arguments.  The library launches
    on the current device and its current stream, so that device is made
    current for the call when it is not already; device tensors on two
    different devices raise ``ValueError``."""
    @functools.wraps(fn)
    def call(*args, **kwargs):
        dev = None
        for a in (*args, *kwargs.values()):
            if isinstance(a, torch.Tensor) and a.is_cuda:
                if dev is None:
                    dev = a.device
                elif a.device != dev:
                    raise ValueError(f"{fn.__name__}: tensors on {dev} and {a.device}")
        if dev is None or dev.index == torch.cuda.current_device():
            return fn(*args, **kwargs)
        with torch.cuda.device(dev):
            return fn(*args, **kwargs)
    return call


def _need(t, name, dtype=None, shape=None):
    if t is None:
        raise ValueError(f"{name} is required")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtype is not None and t.dtype not in (dtype if isinstance(dtype, tuple) else (dtype,)):
        raise ValueError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    return t


def _out(t, name, shape, dtype, like):
    if t is None:
        return torch.empty(shape, dtype=dtype, device=like.device)
    return _need(t, name, dtype, shape)


def _out_dtype(out, out_dtype, default=torch.float32):
    """Output dtype: explicit, else that of a caller-provided ``out``, else f32."""
    if out_dtype is not None:
        return _torch_dtype(out_dtype)
    return out.dtype if out is not None else default


_FLOATS = (torch.float32, torch.float16, torch.bfloat16)
_SCALES = (torch.float32, torch.bfloat16)


# ---------------------------------------------------------------------------
# activation / weight codecs
# ---------------------------------------------------------------------------

@_on_tensor_device
def quantize(x, *, top=None, out=None, scales=None):
    """``quantize(r, k[, top, input_dtype]): x -> out, scales``.

    ``x``: f32/f16/bf16 ``[r, k]`` or ``[r, top, k]``.  Returns e4m3 codes
    (uint8, same shape) and f32 scales ``[..., k/128]``.
    (src/akas/quantization/activations/fp8/cuda.py:10-56)
    """
    _need(x, "x", _FLOATS)
    if top is not None and (x.dim() != 3 or x.shape[1] != top):
        raise ValueError("routed quantize input must be [r, top, k]")
    k = x.shape[-1]
    if k % BLOCK:
        raise ValueError("FP8 channels must be divisible by 128")
    rows = x.numel() // k
    out = _out(out, "out", tuple(x.shape), torch.uint8, x)
    scales = _out(scales, "scales", (*x.shape[:-1], k // BLOCK), torch.float32, x)
    check(_lib.load().akas_quantize(_ptr(x), _dt(x.dtype), _ptr(out), _ptr(scales), rows, k,
                                    _stream()), "quantize")
    return out, scales


@_on_tensor_device
def rms_quantize(x, weight, *, eps, zero_centered=False, normalized_dtype=torch.bfloat16,
                 return_normalized=True, normalized=None, out=None, scales=None):
    """RMSNorm fused with ``quantize``: ``x [r, c]`` (f32/f16/bf16), ``weight [c]``
    (f32/bf16) -> e4m3 codes ``[r, c]``, f32 scales ``[r, c/128]`` and, with
    ``return_normalized``, the normalized rows in ``normalized_dtype``.

    ``y = x / sqrt(mean(x^2) + eps) * w`` (``1 + w`` when ``zero_centered``) is
    rounded to ``normalized_dtype`` and the codes are ``quantize(y)`` of those
    rounded values, bit for bit.  Fuses the kinds ``rms``
    (src/akas/ops/normalization/definition.py:10-31) and ``quantize``
    (src/akas/quantization/activations/fp8/cuda.py:10-56).
    """
    _need(x, "x", _FLOATS)
    _need(weight, "weight", (torch.float32, torch.bfloat16))
    if x.dim() != 2 or tuple(weight.shape) != (x.shape[1],):
        raise ValueError("rms_quantize takes x [r, c] and weight [c]")
    rows, cols = x.shape
    if cols % BLOCK or cols > 8192:
        raise ValueError("RMSNorm-quantize channels must be a multiple of 128, at most 8192")
    if not (eps >= 0.0) or eps == float("inf"):
        raise ValueError("eps must be finite and non-negative")
    ydt = _torch_dtype(normalized_dtype)
    if ydt not in _FLOATS:
        raise ValueError("normalized_dtype must be float32, float16 or bfloat16")
    y = _out(normalized, "normalized", (rows, cols), ydt, x) if return_normalized else None
    out = _out(out, "out", (rows, cols), torch.uint8, x)
    scales = _out(scales, "scales", (rows, cols // BLOCK), torch.float32, x)
    check(_lib.load().akas_rms_quantize(_ptr(x), _dt(x.dtype), _ptr(weight), _dt(weight.dtype),
                                        float(eps), int(bool(zero_centered)),
                                        _ptr(y) if y is not None else None, _dt(ydt), _ptr(out),
                                        _ptr(scales), rows, cols, _stream()), "rms_quantize")
    return (out, scales, y) if return_normalized else (out, scales)


@_on_tensor_device
def dequantize_fp8(codes, scales, *, out=None, out_dtype=None):
    """``dequantize_fp8``: ``decode(codes) * scale`` per 128-group."""
    _need(codes, "codes", torch.uint8)
    k = codes.shape[-1]
    _need(scales, "scales", torch.float32, (*codes.shape[:-1], k // BLOCK))
    out = _out(out, "out", tuple(codes.shape), _out_dtype(out, out_dtype), codes)
    check(_lib.load().akas_dequantize_fp8(_ptr(codes), _ptr(scales), _ptr(out), _dt(out.dtype),
                                          codes.numel() // k, k, _stream()), "dequantize_fp8")
    return out


@_on_tensor_device
def quantize_weight_blocks(w, *, scale_dtype=torch.float32):
    """Block-quantize f32 weights ``[(E,) n, k]`` to e4m3 codes and 128x128 scales.

    Device form of the reference's host weight preparation
    (src/akas/quantization/weights/fp8/kernel.py:34-59).
    """
    _need(w, "w", torch.float32)
    n, k = w.shape[-2:]
    if k % BLOCK:
        raise ValueError("FP8 weight channels must be divisible by 128")
    batch = w.numel() // (n * k) if n * k else 0
    codes = torch.empty(w.shape, dtype=torch.uint8, device=w.device)
    scales = torch.empty((*w.shape[:-2], (n + BLOCK - 1) // BLOCK, k // BLOCK),
                         dtype=_torch_dtype(scale_dtype), device=w.device)
    check(_lib.load().akas_quantize_weight_blocks(_ptr(w), _ptr(codes), _ptr(scales),
                                                  _dt(scales.dtype), batch, n, k, _stream()),
          "quantize_weight_blocks")
    return codes, scales


# ---------------------------------------------------------------------------
# dense linear
# ---------------------------------------------------------------------------

class _StreamBuffers:
    """Device buffers cached per (device, stream): calls sharing a buffer must
    be ordered on one stream, so each stream gets its own.

    At most ``LIMIT`` streams per device keep a buffer; the least recently
    used one is dropped beyond that, and a buffer outgrown by its stream is
    replaced.  Each buffer is allocated with its own stream current, so
    dropping it is stream-ordered: torch's caching allocator hands that
    memory only to later allocations on the same stream.  A buffer that was
    used while a HIP graph was being captured is retired instead, never
    freed, since a replay of that graph still addresses it.

    Streams are told apart by their handle.  torch's streams come from pools
    that are never destroyed; a caller who destroys an external stream must
    first synchronize it, or a new stream given the same handle would share
    the buffer with work still in flight.
    """

    LIMIT = 16

    def __init__(self, make):
        self._make = make  # (elements, device index) -> new tensor
        self._entries = collections.OrderedDict()  # key -> [tensor, used under capture]

    def get(self, need, device, stream=None):
        device = torch.device(device)
        index = device.index if device.index is not None else torch.cuda.current_device()
        if stream is None:
            stream = torch.cuda.current_stream(index)
        key = (index, stream.cuda_stream)
        capturing = torch.cuda.is_current_stream_capturing()
        entry = self._entries.get(key)
        if entry is not None:
            self._entries.move_to_end(key)
            if entry[0].numel() >= need:
                entry[1] = entry[1] or capturing
                return entry[0]
            self._drop(self._entries.pop(key))
        with torch.cuda.stream(stream):
            buf = self._make(need, index)
        self._entries[key] = [buf, capturing]
        mine = [k for k in self._entries if k[0] == index]
        for old in mine[:max(0, len(mine) - self.LIMIT)]:
            self._drop(self._entries.pop(old))
        return buf

    def __len__(self):
        return len(self._entries)

    @staticmethod
    def _drop(entry):
        if entry[1]:
            _RETIRED.append(entry[0])


_RETIRED = []  # buffers a captured graph may still address, kept for good
_WORKSPACES = _StreamBuffers(
    lambda need, index: torch.empty(max(need, 1 << 20), dtype=torch.uint8,
                                    device=torch.device("cuda", index)))


def linear_workspace(r, k, o, device, stream=None):
    """Cached workspace for :func:`fp8_linear`, one per device and stream
    (see ``_StreamBuffers``).  The contents need no initialization."""
    need = _lib.load().akas_fp8_linear_workspace_size(r, k, o)
    return _WORKSPACES.get(need, device, stream)


@_on_tensor_device
def fp8_linear(x, w, scales, activation_scales=None, *, out=None, out_dtype=None,
               workspace=None):
    """``fp8_linear(r, k, o[, input_dtype]): x, w, scales[, activation_scales] -> out``.

    ``x`` f32/f16/bf16 ``[r, k]`` is quantized per 1x128 group, multiplied by
    the e4m3 weight ``[o, k]`` with 128x128 block ``scales`` (f32 or bf16,
    ``[ceil(o/128), k/128]``), f32 accumulation, stored as ``out_dtype``
    (src/akas/ops/linear/cuda.py:642-646, :757-828).

    With ``activation_scales`` (f32 ``[r, k/128]``), ``x`` holds e4m3 codes
    (uint8 ``[r, k]``) already quantized, as the reference binds its block-FP8
    prefill registration (``fp8_prequantized``,
    src/akas/ops/linear/definition.py:558-568, :942-963): the product then
    runs on ``akas_projection_partial`` with one partition and no workspace.
    """
    if activation_scales is not None:
        if workspace is not None:
            raise ValueError("prequantized fp8_linear takes no workspace")
        _need(x, "x", torch.uint8)
        return projection_partial(x, activation_scales, w, scales, partitions=1, out=out,
                                  out_dtype=out_dtype)
    _need(x, "x", _FLOATS)
    _need(w, "w", torch.uint8)
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError("fp8_linear expects x [r, k] and w [o, k]")
    r, k = x.shape
    o = w.shape[0]
    if k % BLOCK or o % 16:
        raise ValueError("invalid FP8 projection geometry")
    _need(scales, "scales", _SCALES, ((o + BLOCK - 1) // BLOCK, k // BLOCK))
    out = _out(out, "out", (r, o), _out_dtype(out, out_dtype), x)
    if workspace is None:
        workspace = linear_workspace(r, k, o, x.device)  # this stream's own
    check(_lib.load().akas_fp8_linear(
        _ptr(x), _dt(x.dtype), _ptr(w), _ptr(scales), _dt(scales.dtype), _ptr(out),
        _dt(out.dtype), _ptr(workspace), workspace.numel(), r, k, o, _stream()), "fp8_linear")
    return out


@_on_tensor_device
def fp8_linear_noalloc(x, w, scales, *, out=None, out_dtype=None):
    """:func:`fp8_linear` on the library's static device scratch
    (``akas_fp8_linear_noalloc``): no workspace argument and no device
    allocation inside the call when ``out`` is given.  Problems whose
    workspace exceeds the scratch raise ``ValueError``; calls overlapping in
    time on one GPU race on the shared scratch."""
    _need(x, "x", _FLOATS)
    _need(w, "w", torch.uint8)
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError("fp8_linear expects x [r, k] and w [o, k]")
    r, k = x.shape
    o = w.shape[0]
    if k % BLOCK or o % 16:
        raise ValueError("invalid FP8 projection geometry")
    _need(scales, "scales", _SCALES, ((o + BLOCK - 1) // BLOCK, k // BLOCK))
    out = _out(out, "out", (r, o), _out_dtype(out, out_dtype), x)
    check(_lib.load().akas_fp8_linear_noalloc(
        _ptr(x), _dt(x.dtype), _ptr(w), _ptr(scales), _dt(scales.dtype), _ptr(out),
        _dt(out.dtype), r, k, o, _stream()), "fp8_linear_noalloc")
    return out


@_on_tensor_device
def projection_partial(x, activation_scales, w, scales, *, partitions=1, out=None,
                       out_dtype=None):
    """``projection_partial(r, k, o, partitions)`` on prequantized codes.

    ``partitions == 1``: ``out [r, o]``; otherwise f32 ``[r, partitions, o]``.
    (src/akas/ops/linear/cuda.py:649-653)
    """
    _need(x, "x", torch.uint8)
    _need(w, "w", torch.uint8)
    r, k = x.shape
    o = w.shape[0]
    if w.shape[1] != k or k % BLOCK or o % 16 or partitions < 1 or (k // BLOCK) % partitions:
        raise ValueError("invalid FP8 projection geometry")
    _need(activation_scales, "activation_scales", torch.float32, (r, k // BLOCK))
    _need(scales, "scales", _SCALES, ((o + BLOCK - 1) // BLOCK, k // BLOCK))
    shape = (r, partitions, o) if partitions > 1 else (r, o)
    dtype = torch.float32 if partitions > 1 else _out_dtype(out, out_dtype)
    out = _out(out, "out", shape, dtype, x)
    check(_lib.load().akas_projection_partial(
        _ptr(x), _ptr(activation_scales), _ptr(w), _ptr(scales), _dt(scales.dtype), _ptr(out),
        _dt(out.dtype), r, k, o, partitions, _stream()), "projection_partial")
    return out


@_on_tensor_device
def projection_merge(partial, *, out=None, out_dtype=None):
    """``projection_merge(r, o, partitions)``: serial f32 sum over partitions."""
    _need(partial, "partial", torch.float32)
    parts, o = partial.shape[-2:]
    rows = partial.numel() // (parts * o) if parts * o else 0
    out = _out(out, "out", (*partial.shape[:-2], o), _out_dtype(out, out_dtype), partial)
    check(_lib.load().akas_projection_merge(_ptr(partial), _ptr(out), _dt(out.dtype), rows, o,
                                            parts, _stream()), "projection_merge")
    return out


@_on_tensor_device
def expert_merge(partial, *, out=None, output_dtype=None):
    """``expert_merge(r, top, o, partitions)``: ``[r, top, parts, o] -> [r, top, o]``."""
    if partial.dim() != 4:
        raise ValueError("expert_merge expects [r, top, partitions, o]")
    return projection_merge(partial, out=out, out_dtype=output_dtype)


# ---------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------

@_on_tensor_device
def biased_router(logits, bias, *, top, scale=1.0, normalize=True, ids=None, weights=None):
    """``biased_router(r, experts, top, scale, normalize): logits, bias -> ids, weights``.

    (src/akas/ops/moe/kernel.py:154-203)
    """
    _need(logits, "logits", torch.float32)
    r, experts = logits.shape
    if bias is not None:
        _need(bias, "bias", torch.float32, (experts,))
    ids = _out(ids, "ids", (r, top), torch.int32, logits)
    weights = _out(weights, "weights", (r, top), torch.float32, logits)
    check(_lib.load().akas_biased_router(_ptr(logits), _ptr(bias), _ptr(ids), _ptr(weights), r,
                                         experts, top, float(scale), int(bool(normalize)),
                                         _stream()), "biased_router")
    return ids, weights


@_on_tensor_device
def biased_softmax_router(logits, bias, *, top, scale=1.0, ids=None, weights=None):
    """``biased_softmax_router(r, experts, top, scale)`` (src/akas/ops/moe/kernel.py:444-499)."""
    _need(logits, "logits", torch.float32)
    r, experts = logits.shape
    if bias is not None:
        _need(bias, "bias", torch.float32, (experts,))
    ids = _out(ids, "ids", (r, top), torch.int32, logits)
    weights = _out(weights, "weights", (r, top), torch.float32, logits)
    check(_lib.load().akas_biased_softmax_router(_ptr(logits), _ptr(bias), _ptr(ids),
                                                 _ptr(weights), r, experts, top, float(scale),
                                                 _stream()), "biased_softmax_router")
    return ids, weights


@_on_tensor_device
def router(logits, *, top, ids=None, weights=None):
    """``router(r, experts, top): logits -> ids, weights``, the block-fp8
    decode variant's router: selection on the bf16-rounded f32 logits, softmax
    over the selected ones (src/akas/ops/moe/cuda.py:2011-2050)."""
    _need(logits, "logits", torch.float32)
    r, experts = logits.shape
    ids = _out(ids, "ids", (r, top), torch.int32, logits)
    weights = _out(weights, "weights", (r, top), torch.float32, logits)
    check(_lib.load().akas_router(_ptr(logits), _ptr(ids), _ptr(weights), r, experts, top,
                                  _stream()), "router")
    return ids, weights


@_on_tensor_device
def router_quantize(logits, bias, x, *, top, softmax=True, scale=1.0, normalize=True):
    """The MoE block's router (``biased_softmax_router`` when ``softmax``,
    else ``biased_router``) and ``quantize(x)`` in one launch; up to 64
    experts and top 8.  Returns ``(ids, weights, codes, scales)``, each
    bit-identical to the separate kinds' outputs."""
    _need(logits, "logits", torch.float32)
    _need(x, "x", _FLOATS)
    r, experts = logits.shape
    if x.dim() != 2 or x.shape[0] != r:
        raise ValueError("router_quantize expects x [r, k] with the logits' rows")
    k = x.shape[1]
    if bias is not None:
        _need(bias, "bias", torch.float32, (experts,))
    ids = torch.empty((r, top), dtype=torch.int32, device=logits.device)
    weights = torch.empty((r, top), dtype=torch.float32, device=logits.device)
    codes = torch.empty((r, k), dtype=torch.uint8, device=x.device)
    scales = torch.empty((r, k // BLOCK), dtype=torch.float32, device=x.device)
    check(_lib.load().akas_router_quantize(
        _ptr(logits), _ptr(bias), _ptr(ids), _ptr(weights), r, experts, top, float(scale),
        int(bool(softmax)), int(bool(normalize)), _ptr(x), _dt(x.dtype), _ptr(codes), _ptr(scales),
        k, _stream()), "router_quantize")
    return ids, weights, codes, scales


@_on_tensor_device
def moe_groups(ids, *, experts=None, routes=None):
    """``moe_groups(r, top): ids -> experts, routes``, the block-fp8 decode
    variant's route tables (src/akas/ops/moe/cuda.py:1978-2008): per (row,
    rank) group the expert it owns (first occurrence) or -1, and per owning
    group the rank at which each row selected it, or -1."""
    _need(ids, "ids", torch.int32)
    r, top = ids.shape
    experts = _out(experts, "experts", (r * top,), torch.int32, ids)
    routes = _out(routes, "routes", (r * top, r), torch.int32, ids)
    check(_lib.load().akas_moe_groups(_ptr(ids), _ptr(experts), _ptr(routes), r, top,
                                      _stream()), "moe_groups")
    return experts, routes


@_on_tensor_device
def quantized_routes(ids, active, *, experts, counts=None, routes=None):
    """``quantized_routes(r, experts, top): ids, active -> counts, routes``.

    (src/akas/ops/moe/kernel.py:121-151)
    """
    _need(ids, "ids", torch.int32)
    r, top = ids.shape
    _need(active, "active", torch.int32, (r,))
    counts = _out(counts, "counts", (experts,), torch.int32, ids)
    routes = _out(routes, "routes", (experts, r), torch.int32, ids)
    check(_lib.load().akas_quantized_routes(_ptr(ids), _ptr(active), _ptr(counts), _ptr(routes),
                                            r, experts, top, _stream()), "quantized_routes")
    return counts, routes


def tile_capacity(rows, top, experts, block_m):
    """Non-empty expert tile bound (src/akas/ops/moe/definition.py:9-16)."""
    if any(type(v) is not int or v < 1 for v in (rows, top, experts, block_m)):
        raise ValueError("expert tile geometry must contain positive integers")
    routes = rows * top
    return min(routes, (routes + block_m - 1) // block_m + experts - 1)


def tile_layouts(max_block_m=64):
    """Row layouts 4..max_block_m (src/akas/ops/moe/definition.py:19-26)."""
    if type(max_block_m) is not int or max_block_m not in (4, 8, 16, 32, 64, 128):
        raise ValueError(
            "expert maximum row tile must be a supported power of two from 4 through 128")
    return max_block_m.bit_length() - 2


def map_capacity(rows, top, experts):
    return (rows * top + 3) // 4 + experts


@_on_tensor_device
def expert_tile_map(counts, *, r, top, max_block_m=64, tile_experts=None, tile_rows=None):
    """``expert_tile_map(r, experts, top[, max_block_m]): counts -> tile_experts, tile_rows``.

    (src/akas/ops/moe/kernel.py:79-118)
    """
    _need(counts, "counts", torch.int32)
    experts = counts.shape[0]
    shape = (tile_layouts(max_block_m), map_capacity(r, top, experts))
    tile_experts = _out(tile_experts, "tile_experts", shape, torch.int32, counts)
    tile_rows = _out(tile_rows, "tile_rows", shape, torch.int32, counts)
    check(_lib.load().akas_expert_tile_map(_ptr(counts), _ptr(tile_experts), _ptr(tile_rows), r,
                                           experts, top, max_block_m, _stream()),
          "expert_tile_map")
    return tile_experts, tile_rows


@_on_tensor_device
def expert_pack(x, activation_scales, counts, routes, tile_experts, tile_offsets, *, top,
                max_block_m=64, routed_input=False, packed=None, packed_scales=None,
                expert_offsets=None):
    """``expert_pack(r, top, experts, k, max_block_m[, routed_input])``.

    Returns ``(packed, packed_scales, expert_offsets)``; padding rows hold codes
    0 and scale 1 (src/akas/ops/moe/cuda.py:2423-2502).
    """
    _need(x, "x", torch.uint8)
    _need(counts, "counts", torch.int32)
    experts = counts.shape[0]
    r = x.shape[0]
    k = x.shape[-1]
    if routed_input and (x.dim() != 3 or x.shape[1] != top):
        raise ValueError("routed pack input must be [r, top, k]")
    _need(activation_scales, "activation_scales", torch.float32, (*x.shape[:-1], k // BLOCK))
    _need(routes, "routes", torch.int32, (experts, r))
    rows = tile_capacity(r, top, experts, max_block_m) * max_block_m
    packed = _out(packed, "packed", (rows, k), torch.uint8, x)
    packed_scales = _out(packed_scales, "packed_scales", (rows, k // BLOCK), torch.float32, x)
    if expert_offsets is None:
        expert_offsets = torch.zeros((experts,), dtype=torch.int32, device=x.device)
    _need(expert_offsets, "expert_offsets", torch.int32, (experts,))
    check(_lib.load().akas_expert_pack(
        _ptr(x), _ptr(activation_scales), _ptr(counts), _ptr(routes), _ptr(tile_experts),
        _ptr(tile_offsets), _ptr(packed), _ptr(packed_scales), _ptr(expert_offsets), r, top,
        experts, k, max_block_m, int(bool(routed_input)), _stream()), "expert_pack")
    return packed, packed_scales, expert_offsets


# ---------------------------------------------------------------------------
# grouped expert products
# ---------------------------------------------------------------------------

@_on_tensor_device
def expert_partial(x, activation_scales, w, scales, counts, routes, tile_experts=None,
                   tile_offsets=None, expert_offsets=None, *, r, top, routed_input=False,
                   partitions=1, output_dtype=torch.float32, max_block_m=64,
                   packed_input=False, out=None):
    """``expert_partial``: grouped FP8 projection scattered to ``out[row, rank]``.

    ``out`` is ``[r, top, o]`` (``partitions == 1``) or f32
    ``[r, top, partitions, o]``; only routed entries are written
    (src/akas/ops/moe/cuda.py:541-1354).
    """
    _need(x, "x", torch.uint8)
    _need(w, "w", torch.uint8)
    experts, o, k = w.shape
    _need(scales, "scales", _SCALES, (experts, (o + BLOCK - 1) // BLOCK, k // BLOCK))
    _need(counts, "counts", torch.int32, (experts,))
    _need(routes, "routes", torch.int32, (experts, r))
    if x.shape[-1] != k:
        raise ValueError("activation depth differs from the expert weights")
    _need(activation_scales, "activation_scales", torch.float32, (*x.shape[:-1], k // BLOCK))
    if packed_input and expert_offsets is None:
        raise ValueError("packed expert input requires expert_offsets")
    shape = (r, top, partitions, o) if partitions > 1 else (r, top, o)
    dtype = torch.float32 if partitions > 1 else _torch_dtype(output_dtype)
    if out is None:
        out = torch.zeros(shape, dtype=dtype, device=x.device)
    _need(out, "out", dtype, shape)
    check(_lib.load().akas_expert_partial(
        _ptr(x), _ptr(activation_scales), _ptr(w), _ptr(scales), _dt(scales.dtype), _ptr(counts),
        _ptr(routes), _ptr(tile_experts), _ptr(tile_offsets), _ptr(expert_offsets), _ptr(out),
        _dt(out.dtype), r, top, experts, o, k, int(bool(routed_input)), partitions, max_block_m,
        int(bool(packed_input)), _stream()), "expert_partial")
    return out


_ARRIVALS = _StreamBuffers(
    lambda need, index: torch.zeros(max(need, 1 << 16), dtype=torch.int32,
                                    device=torch.device("cuda", index)))


def combine_arrivals(r, o, device, stream=None):
    """Arrival counters of :func:`expert_combine`, one zeroed buffer per device
    and stream (see ``_StreamBuffers``); every call leaves its counters zero
    again, so calls ordered on one stream share it."""
    return _ARRIVALS.get(r * (o // BLOCK), device, stream)


@_on_tensor_device
def expert_combine(x, activation_scales, w, scales, counts, routes, ids, weights, active=None,
                   expert_offsets=None, *, r, top, routed_input=False, packed_input=False,
                   contribution_dtype=torch.float32, max_block_m=64, contributions=None,
                   out=None, arrivals=None):
    """The down projection with ``routed_combine`` folded into its epilogue:
    ``expert_partial`` (``partitions`` 1, ``contribution_dtype``) and
    ``routed_combine`` in one launch, bit-identical to that pair
    (src/akas/ops/moe/cuda.py:541-1354 scatter :956-966;
    src/akas/ops/moe/kernel.py:206-267).

    Returns ``(out, contributions)``: f32 ``[r, o]`` and the ``[r, top, o]``
    contributions in ``contribution_dtype``.  ``counts``/``routes`` must be
    ``quantized_routes(ids, active)``; a rank is folded when its id is in
    ``[0, experts)``.
    """
    _need(x, "x", torch.uint8)
    _need(w, "w", torch.uint8)
    experts, o, k = w.shape
    _need(scales, "scales", _SCALES, (experts, (o + BLOCK - 1) // BLOCK, k // BLOCK))
    _need(counts, "counts", torch.int32, (experts,))
    _need(routes, "routes", torch.int32, (experts, r))
    _need(ids, "ids", torch.int32, (r, top))
    _need(weights, "weights", torch.float32, (r, top))
    if active is not None:
        _need(active, "active", torch.int32, (r,))
    if x.shape[-1] != k:
        raise ValueError("activation depth differs from the expert weights")
    _need(activation_scales, "activation_scales", torch.float32, (*x.shape[:-1], k // BLOCK))
    if packed_input and expert_offsets is None:
        raise ValueError("packed expert input requires expert_offsets")
    cdt = _torch_dtype(contribution_dtype)
    if contributions is None:
        contributions = torch.empty((r, top, o), dtype=cdt, device=x.device)
    _need(contributions, "contributions", cdt, (r, top, o))
    out = _out(out, "out", (r, o), torch.float32, x)
    if arrivals is None:
        arrivals = combine_arrivals(r, o, x.device)
    _need(arrivals, "arrivals", torch.int32)
    if arrivals.numel() < r * (o // BLOCK):
        raise ValueError("arrivals holds fewer than r * o / 128 counters")
    check(_lib.load().akas_expert_combine(
        _ptr(x), _ptr(activation_scales), _ptr(w), _ptr(scales), _dt(scales.dtype), _ptr(counts),
        _ptr(routes), _ptr(expert_offsets), _ptr(ids), _ptr(weights), _ptr(active),
        _ptr(contributions), _dt(cdt), _ptr(out), _ptr(arrivals), r, top, experts, o, k,
        int(bool(routed_input)), max_block_m, int(bool(packed_input)), _stream()),
        "expert_combine")
    return out, contributions


def fp8_experts_workspace(r, top, experts, k, routed_input, device):
    """Workspace of :func:`fp8_experts` (quantized input and the per-expert
    route tables built from the group tables)."""
    n = _lib.load().akas_fp8_experts_workspace_size(r, top, experts, k, int(bool(routed_input)))
    return torch.empty(max(int(n), 1), dtype=torch.uint8, device=device)


@_on_tensor_device
def fp8_experts(x, w, scales, experts, routes, *, top, routed_input=False, out=None,
                output_dtype=torch.float32, workspace=None):
    """``fp8_experts(r, experts, top, o, k, routed_input)``: the block-fp8
    decode variant's expert products over moe_groups' tables
    (src/akas/ops/moe/cuda.py:439-531).

    ``x`` f32/f16/bf16 ``[r, k]`` (``[r, top, k]`` routed) is quantized per
    1x128 group; ``out[b, rank] = x_row . dequant(w[e])^T`` for every group of
    expert ``e`` and row ``b`` it routes; ``out`` ``[r, top, o]`` entries that
    no group routes are left as they are.
    """
    _need(x, "x", _FLOATS)
    _need(w, "w", torch.uint8)
    num_experts, o, k = w.shape
    r = x.shape[0]
    if routed_input and (x.dim() != 3 or x.shape[1] != top):
        raise ValueError("routed fp8_experts input must be [r, top, k]")
    if not routed_input and x.dim() != 2:
        raise ValueError("fp8_experts input must be [r, k]")
    if x.shape[-1] != k:
        raise ValueError("x and w disagree on k")
    _need(scales, "scales", _SCALES, (num_experts, (o + BLOCK - 1) // BLOCK, k // BLOCK))
    _need(experts, "experts", torch.int32, (r * top,))
    _need(routes, "routes", torch.int32, (r * top, r))
    if out is None:
        out = torch.zeros((r, top, o), dtype=output_dtype, device=x.device)
    _need(out, "out", _FLOATS, (r, top, o))
    if workspace is None:
        workspace = fp8_experts_workspace(r, top, num_experts, k, routed_input, x.device)
    check(_lib.load().akas_fp8_experts(
        _ptr(x), _dt(x.dtype), _ptr(w), _ptr(scales), _dt(scales.dtype), _ptr(experts),
        _ptr(routes), _ptr(out), _dt(out.dtype), _ptr(workspace), workspace.numel(), r, top,
        num_experts, o, k, int(bool(routed_input)), _stream()), "fp8_experts")
    return out


@_on_tensor_device
def fp8_expert_swiglu(x, activation_scales, w, scales, w2, scales2, counts, routes,
                      tile_experts=None, tile_offsets=None, expert_offsets=None, *, r, top,
                      product_dtype=torch.float32, activation_dtype=torch.float32,
                      max_block_m=64, packed_input=False, packed_output=False, out=None,
                      output_scales=None):
    """``fp8_expert_swiglu``: gate/up products, SwiGLU, FP8 re-quantization.

    Returns ``(out, output_scales)``: codes ``[r, top, o]`` and scales
    ``[r, top, o/128]`` (packed ``[cap*A, ...]`` with ``packed_output``)
    (src/akas/ops/moe/cuda.py:823-946).
    """
    _need(x, "x", torch.uint8)
    _need(w, "w", torch.uint8)
    _need(w2, "w2", torch.uint8, tuple(w.shape))
    experts, o, k = w.shape
    sshape = (experts, (o + BLOCK - 1) // BLOCK, k // BLOCK)
    _need(scales, "scales", _SCALES, sshape)
    _need(scales2, "scales2", scales.dtype, sshape)
    _need(counts, "counts", torch.int32, (experts,))
    _need(routes, "routes", torch.int32, (experts, r))
    _need(activation_scales, "activation_scales", torch.float32, (*x.shape[:-1], k // BLOCK))
    if (packed_input or packed_output) and expert_offsets is None:
        raise ValueError("packed experts require expert_offsets")
    if packed_output and not packed_input:
        raise ValueError("packed expert output requires a packed paired projection")
    if packed_output:
        rows = tile_capacity(r, top, experts, max_block_m) * max_block_m
        oshape, sshape_out = (rows, o), (rows, o // BLOCK)
    else:
        oshape, sshape_out = (r, top, o), (r, top, o // BLOCK)
    if out is None:
        out = torch.zeros(oshape, dtype=torch.uint8, device=x.device)
    if output_scales is None:
        output_scales = torch.zeros(sshape_out, dtype=torch.float32, device=x.device)
    _need(out, "out", torch.uint8, oshape)
    _need(output_scales, "output_scales", torch.float32, sshape_out)
    check(_lib.load().akas_fp8_expert_swiglu(
        _ptr(x), _ptr(activation_scales), _ptr(w), _ptr(scales), _ptr(w2), _ptr(scales2),
        _dt(scales.dtype), _ptr(counts), _ptr(routes), _ptr(tile_experts), _ptr(tile_offsets),
        _ptr(expert_offsets), _ptr(out), _ptr(output_scales), r, top, experts, o, k,
        _dt(product_dtype), _dt(activation_dtype), max_block_m, int(bool(packed_input)),
        int(bool(packed_output)), _stream()), "fp8_expert_swiglu")
    return out, output_scales


@_on_tensor_device
def routed_fp8_expert_swiglu(ids, active, x, activation_scales, w, scales, w2, scales2, *,
                             product_dtype=torch.float32, activation_dtype=torch.float32,
                             counts=None, routes=None, out=None, output_scales=None):
    """``quantized_routes`` then ``fp8_expert_swiglu`` (unpacked rows) as one
    call: ``(counts, routes, out, output_scales)``, each bit-identical to the
    two kinds run in turn (src/akas/ops/moe/kernel.py:121-151,
    src/akas/ops/moe/cuda.py:823-946).  ``active`` may be None (every row
    active).  Decode batches (up to 512 experts, top 64, 4096 routes, 48 per expert
    on average) take one launch, in which every workgroup scans ``ids`` itself.
    """
    _need(ids, "ids", torch.int32)
    r, top = ids.shape
    if active is not None:
        _need(active, "active", torch.int32, (r,))
    _need(w, "w", torch.uint8)
    _need(w2, "w2", torch.uint8, tuple(w.shape))
    experts, o, k = w.shape
    sshape = (experts, (o + BLOCK - 1) // BLOCK, k // BLOCK)
    _need(scales, "scales", _SCALES, sshape)
    _need(scales2, "scales2", scales.dtype, sshape)
    _need(x, "x", torch.uint8, (r, k))
    _need(activation_scales, "activation_scales", torch.float32, (r, k // BLOCK))
    counts = _out(counts, "counts", (experts,), torch.int32, ids)
    routes = _out(routes, "routes", (experts, r), torch.int32, ids)
    out = _out(out, "out", (r, top, o), torch.uint8, x)
    output_scales = _out(output_scales, "output_scales", (r, top, o // BLOCK), torch.float32, x)
    check(_lib.load().akas_routed_fp8_expert_swiglu(
        _ptr(ids), _ptr(active), _ptr(counts), _ptr(routes), _ptr(x), _ptr(activation_scales),
        _ptr(w), _ptr(scales), _ptr(w2), _ptr(scales2), _dt(scales.dtype), _ptr(out),
        _ptr(output_scales), r, top, experts, o, k, _dt(product_dtype), _dt(activation_dtype),
        _stream()), "routed_fp8_expert_swiglu")
    return counts, routes, out, output_scales


def _paired_inputs(x, activation_scales, w, scales, w2, scales2, counts, routes, r):
    _need(x, "x", torch.uint8)
    _need(w, "w", torch.uint8)
    _need(w2, "w2", torch.uint8, tuple(w.shape))
    experts, o, k = w.shape
    sshape = (experts, (o + BLOCK - 1) // BLOCK, k // BLOCK)
    _need(scales, "scales", _SCALES, sshape)
    _need(scales2, "scales2", scales.dtype, sshape)
    _need(counts, "counts", torch.int32, (experts,))
    _need(routes, "routes", torch.int32, (experts, r))
    _need(activation_scales, "activation_scales", torch.float32, (*x.shape[:-1], k // BLOCK))
    return experts, o, k


@_on_tensor_device
def expert_swiglu(x, activation_scales, w, scales, w2, scales2, counts, routes,
                  tile_experts=None, tile_offsets=None, expert_offsets=None, *, r, top,
                  product_dtype=torch.float32, activation_dtype=torch.float32,
                  output_dtype=torch.float32, max_block_m=64, packed_input=False,
                  packed_output=False, out=None):
    """``expert_swiglu`` (FP8 paired): gate and up products of one tile,
    SwiGLU, stored unquantized in ``output_dtype`` -- ``[r, top, o]``, or
    packed ``[cap*A, o]`` with ``packed_output``.  Bit-identical to
    ``expert_partial`` x2 -> ``swiglu_experts`` with the same dtypes
    (src/akas/ops/moe/cuda.py:1531-1534)."""
    experts, o, k = _paired_inputs(x, activation_scales, w, scales, w2, scales2, counts, routes, r)
    if (packed_input or packed_output) and expert_offsets is None:
        raise ValueError("packed experts require expert_offsets")
    if packed_output and not packed_input:
        raise ValueError("packed expert output requires a packed paired projection")
    oshape = ((tile_capacity(r, top, experts, max_block_m) * max_block_m, o) if packed_output
              else (r, top, o))
    out = _out(out, "out", oshape, _torch_dtype(output_dtype), x)
    check(_lib.load().akas_expert_swiglu(
        _ptr(x), _ptr(activation_scales), _ptr(w), _ptr(scales), _ptr(w2), _ptr(scales2),
        _dt(scales.dtype), _ptr(counts), _ptr(routes), _ptr(tile_experts), _ptr(tile_offsets),
        _ptr(expert_offsets), _ptr(out), _dt(out.dtype), r, top, experts, o, k,
        _dt(product_dtype), _dt(activation_dtype), max_block_m, int(bool(packed_input)),
        int(bool(packed_output)), _stream()), "expert_swiglu")
    return out


@_on_tensor_device
def expert_pair_partial(x, activation_scales, w, scales, w2, scales2, counts, routes,
                        tile_experts=None, tile_offsets=None, *, r, top, partitions=1,
                        max_block_m=64, gate=None, up=None):
    """``expert_pair_partial``: the gate (``w``) and up (``w2``) products of
    one paired tile as f32 K-partition partials, ``(gate, up)`` each
    ``[r, top, partitions, o]``; only routed entries are written
    (src/akas/ops/moe/cuda.py:1537-1542, OutputABI ``("gate", "up")``)."""
    experts, o, k = _paired_inputs(x, activation_scales, w, scales, w2, scales2, counts, routes, r)
    if x.dim() != 2 or x.shape[0] != r:
        raise ValueError("paired partial input must be [r, k] codes")
    if partitions < 1 or (k // BLOCK) % partitions:
        raise ValueError("partitions must divide the k-blocks")
    shape = (r, top, partitions, o)
    gate = torch.zeros(shape, dtype=torch.float32, device=x.device) if gate is None else gate
    up = torch.zeros(shape, dtype=torch.float32, device=x.device) if up is None else up
    _need(gate, "gate", torch.float32, shape)
    _need(up, "up", torch.float32, shape)
    check(_lib.load().akas_expert_pair_partial(
        _ptr(x), _ptr(activation_scales), _ptr(w), _ptr(scales), _ptr(w2), _ptr(scales2),
        _dt(scales.dtype), _ptr(counts), _ptr(routes), _ptr(tile_experts), _ptr(tile_offsets),
        _ptr(gate), _ptr(up), r, top, experts, o, k, partitions, max_block_m, _stream()),
        "expert_pair_partial")
    return gate, up


@_on_tensor_device
def swiglu_experts(g, u, *, round_inputs=False, round_dtype=torch.float32,
                   output_dtype=torch.float32, out=None):
    """``swiglu_experts``: ``g / (1 + exp(-g)) * u`` on ``[r, top, (parts,) c]``.

    (src/akas/ops/activation/kernel.py:28-88)
    """
    _need(g, "g", _FLOATS)
    _need(u, "u", g.dtype, tuple(g.shape))
    if g.dim() == 4:
        r, top, parts, c = g.shape
    elif g.dim() == 3:
        (r, top, c), parts = g.shape, 1
    else:
        raise ValueError("expert SwiGLU expects [r, top, c] or [r, top, parts, c]")
    out = _out(out, "out", (r, top, c), _torch_dtype(output_dtype), g)
    check(_lib.load().akas_swiglu_experts(
        _ptr(g), _ptr(u), _dt(g.dtype), _ptr(out), _dt(out.dtype), r, top, c, parts,
        int(bool(round_inputs)), _dt(round_dtype), _stream()), "swiglu_experts")
    return out


@_on_tensor_device
def moe_combine(experts, weights, shared, gate, *, out=None):
    """``moe_combine(r, top, c): experts, weights, shared, gate -> out``: the
    weighted top-k combine plus a sigmoid-gated shared expert,
    ``sum_rank bf16(e) * w + bf16(shared) / (1 + exp(-bf16(gate)))`` in f32.

    ``experts`` ``[r, top, c]``, ``shared`` ``[r, c]`` and ``gate`` ``[r]`` or
    ``[r, 1]`` (f32/f16/bf16), ``weights`` f32 ``[r, top]``.
    (src/akas/ops/moe/cuda.py:392-422)
    """
    _need(experts, "experts", _FLOATS)
    r, top, c = experts.shape
    if c % 8:
        raise ValueError("moe_combine channels must be a multiple of 8")
    _need(weights, "weights", torch.float32, (r, top))
    _need(shared, "shared", _FLOATS, (r, c))
    _need(gate, "gate", _FLOATS)
    if gate.numel() != r or gate.dim() > 2:
        raise ValueError("moe_combine gate must be [r] or [r, 1]")
    out = _out(out, "out", (r, c), torch.float32, experts)
    check(_lib.load().akas_moe_combine(_ptr(experts), _dt(experts.dtype), _ptr(weights),
                                       _ptr(shared), _dt(shared.dtype), _ptr(gate),
                                       _dt(gate.dtype), _ptr(out), r, top, c, _stream()),
          "moe_combine")
    return out


def shared_expert_moe_workspace(r, experts, top, h, f, device):
    """Workspace of :func:`shared_expert_moe_block` (route tables, x's codes,
    the activations' codes and the bf16 contributions of top + 1 ranks)."""
    n = _lib.load().akas_shared_expert_moe_workspace_size(r, experts, top, h, f)
    return torch.empty(max(int(n), 1), dtype=torch.uint8, device=device)


@_on_tensor_device
def shared_expert_moe_block(x, logits, shared_gate, w1, s1, w3, s3, w2, s2, sw1, ss1, sw3, ss3,
                            sw2, ss2, *, top, out=None, workspace=None):
    """The shared-expert MoE block in one call: ``x [r, h]``, router
    ``logits`` f32 ``[r, E]``, ``shared_gate [r]`` -> f32 ``[r, h]``.

    decode_router (src/akas/ops/moe/cuda.py:2011-2050), the routed experts
    (bank ``w1``/``w3`` ``[E, f, h]``, ``w2`` ``[E, h, f]``) and the shared
    expert (``sw1``/``sw3`` ``[f, h]``, ``sw2`` ``[h, f]``) with f32
    products and activations, and moe_combine with the sigmoid gate
    (cuda.py:392-422), all six weights' block scales of one dtype.  The
    shared expert is computed as one more expert of the routed launches.
    """
    _need(x, "x", _FLOATS)
    _need(logits, "logits", torch.float32)
    if x.dim() != 2 or logits.dim() != 2 or logits.shape[0] != x.shape[0]:
        raise ValueError("shared_expert_moe_block expects x [r, h] and logits [r, E]")
    r, h = x.shape
    experts = logits.shape[1]
    _need(shared_gate, "shared_gate", _FLOATS)
    if shared_gate.numel() != r or shared_gate.dim() > 2:
        raise ValueError("shared_gate must be [r] or [r, 1]")
    _need(w1, "w1", torch.uint8)
    if w1.dim() != 3 or w1.shape[0] != experts or w1.shape[2] != h:
        raise ValueError("w1 must be [E, f, h]")
    f = w1.shape[1]
    if h % BLOCK or f % BLOCK:
        raise ValueError("shared_expert_moe_block widths must be multiples of 128")
    _need(w3, "w3", torch.uint8, (experts, f, h))
    _need(w2, "w2", torch.uint8, (experts, h, f))
    _need(s1, "s1", _SCALES, (experts, f // BLOCK, h // BLOCK))
    _need(s3, "s3", s1.dtype, (experts, f // BLOCK, h // BLOCK))
    _need(s2, "s2", s1.dtype, (experts, h // BLOCK, f // BLOCK))
    _need(sw1, "sw1", torch.uint8, (f, h))
    _need(sw3, "sw3", torch.uint8, (f, h))
    _need(sw2, "sw2", torch.uint8, (h, f))
    _need(ss1, "ss1", s1.dtype, (f // BLOCK, h // BLOCK))
    _need(ss3, "ss3", s1.dtype, (f // BLOCK, h // BLOCK))
    _need(ss2, "ss2", s1.dtype, (h // BLOCK, f // BLOCK))
    out = _out(out, "out", (r, h), torch.float32, x)
    if workspace is None:
        workspace = shared_expert_moe_workspace(r, experts, top, h, f, x.device)
    _need(workspace, "workspace", torch.uint8)
    check(_lib.load().akas_shared_expert_moe(
        _ptr(x), _dt(x.dtype), _ptr(logits), _ptr(shared_gate), _dt(shared_gate.dtype),
        _ptr(w1), _ptr(s1), _ptr(w3), _ptr(s3), _ptr(w2), _ptr(s2), _ptr(sw1), _ptr(ss1),
        _ptr(sw3), _ptr(ss3), _ptr(sw2), _ptr(ss2), _dt(s1.dtype), _ptr(out), _ptr(workspace),
        workspace.numel(), r, experts, top, h, f, _stream()), "shared_expert_moe")
    return out


@_on_tensor_device
def routed_combine(experts, weights, active, *, out=None):
    """``routed_combine(r, top, c[, input_dtype]): experts, weights, active -> out``.

    (src/akas/ops/moe/kernel.py:206-267)
    """
    _need(experts, "experts", _FLOATS)
    r, top, c = experts.shape
    _need(weights, "weights", torch.float32, (r, top))
    if active is not None:
        _need(active, "active", torch.int32, (r,))
    out = _out(out, "out", (r, c), torch.float32, experts)
    check(_lib.load().akas_routed_combine(_ptr(experts), _dt(experts.dtype), _ptr(weights),
                                          _ptr(active), _ptr(out), r, top, c, _stream()),
          "routed_combine")
    return out
