"""Block-FP8 safetensors checkpoints (compressed-tensors format) -> device layout.

The on-disk side of the path: a checkpoint stores each quantized linear as
an F8_E4M3 ``weight`` ``[N, K]`` and a BF16 ``weight_scale``
``[ceil(N/128), K/128]`` (static 128x128 weight blocks, dynamic 1x128
activation groups).  The loader validates every header and extent on the
host before any device allocation, then uploads the raw bits -- no decoded
copy -- in the layout the kernels read: expert banks grouped ``[E, N, K]``
(uint8 codes) with ``[E, ceil(N/128), K/128]`` bf16 scales, dense linears
``[N, K]`` with ``[ceil(N/128), K/128]``.

Follows src/akas/checkpoints/safetensors.py (``block_fp8_config`` :21-41,
``inspect_tensors`` :62-132, ``read_tensor`` :135-143, ``tensor_index``
:163-186) and the LFM2-MoE grouping of src/akas/models/lfm2/weights.py:95-200
(``model.layers.{L}.feed_forward.experts.{e}.{w1,w3,w2}.weight`` plus their
``weight_scale``, ``feed_forward.gate.weight`` and ``expert_bias``).  Errors
are ``ValueError`` raised before allocation, as there.
"""

from dataclasses import dataclass
import json
import math
from pathlib import Path
import struct
from types import MappingProxyType

import numpy as np

# safetensors dtype -> (numpy storage dtype, bytes per element)
STORAGE = {
    "F8_E4M3": (np.dtype(np.uint8), 1),
    "BF16": (np.dtype(np.uint16), 2),
    "F16": (np.dtype(np.float16), 2),
    "F32": (np.dtype(np.float32), 4),
}
_HEADER_LIMIT = 100_000_000


def _no_duplicates(pairs):
    out = {}
    for key, value in pairs:
        if key in out:
            raise ValueError(f"duplicate checkpoint JSON key: {key}")
        out[key] = value
    return out


def json_document(text):
    """JSON with duplicate keys rejected (a duplicated tensor entry would
    otherwise silently shadow the first)."""
    return json.loads(text, object_pairs_hook=_no_duplicates)


def block_fp8_config(config):
    """``False`` for an unquantized checkpoint, ``True`` for the supported
    block-FP8 contract (static symmetric 128x128 float8 weight blocks,
    dynamic symmetric float8 activation groups of 128), ``ValueError`` for
    any other quantization (safetensors.py:21-41)."""
    q = config.get("quantization_config")
    if q is None:
        return False
    groups = q.get("config_groups") or {}
    if (q.get("quant_method") != "compressed-tensors" or q.get("format") != "float-quantized"
            or len(groups) != 1 or q.get("kv_cache_scheme") is not None):
        raise ValueError("unsupported block-FP8 checkpoint quantization")
    group = next(iter(groups.values()))
    w = group.get("weights") or {}
    a = group.get("input_activations") or {}
    weights_ok = (w.get("num_bits") == 8 and w.get("type") == "float" and w.get("strategy") == "block"
                  and w.get("block_structure") == [128, 128] and w.get("dynamic") is False
                  and w.get("symmetric") is True)
    acts_ok = (a.get("num_bits") == 8 and a.get("type") == "float" and a.get("strategy") == "group"
               and a.get("group_size") == 128 and a.get("dynamic") is True
               and a.get("symmetric") is True)
    if not (weights_ok and acts_ok):
        raise ValueError("FP8 requires static 128x128 weights and dynamic group-128 activations")
    return True


def _read_header(path):
    size = path.stat().st_size
    with path.open("rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise ValueError("truncated safetensors header")
        length = struct.unpack("<Q", head)[0]
        if not 2 <= length <= min(size - 8, _HEADER_LIMIT):
            raise ValueError("invalid safetensors header length")
        header = json_document(f.read(length))
    if not isinstance(header, dict):
        raise ValueError("invalid safetensors header object")
    return header, length, size


def tensor_index(directory):
    """Tensor name -> shard file name: ``model.safetensors.index.json`` when
    present, else the directory's single ``*.safetensors`` file."""
    directory = Path(directory)
    index = directory / "model.safetensors.index.json"
    if index.is_file():
        weight_map = json_document(index.read_text()).get("weight_map")
        if not isinstance(weight_map, dict):
            raise ValueError("invalid checkpoint weight map")
        return weight_map
    shards = sorted(directory.glob("*.safetensors"))
    if len(shards) != 1:
        raise ValueError("checkpoint requires an index or exactly one safetensors shard")
    header, _, _ = _read_header(shards[0])
    return {name: shards[0].name for name in header if name != "__metadata__"}


@dataclass(frozen=True)
class TensorInfo:
    shard: Path
    dtype: str
    shape: tuple
    offset: int  # absolute byte offset of the data in the shard
    nbytes: int


def inspect_tensors(directory, index, shapes, dtypes):
    """Check the selected tensors' dtype, shape and extent, and that no two
    extents of a shard overlap, before anything is read or allocated.
    ``shapes``/``dtypes`` map tensor names to the expected shape and
    safetensors dtype (safetensors.py:62-132)."""
    directory = Path(directory).resolve()
    if shapes.keys() != dtypes.keys() or any(name not in index for name in shapes):
        raise ValueError("incomplete checkpoint tensor contract")
    found = {}
    for filename in sorted({index[name] for name in shapes}):
        shard = (directory / filename).resolve()
        if shard.parent != directory or not shard.is_file():
            raise ValueError("checkpoint shard must be a local file within its directory")
        header, length, size = _read_header(shard)
        data_bytes = size - 8 - length
        extents = []
        for name, entry in header.items():
            if name == "__metadata__":
                continue
            if not isinstance(entry, dict):
                raise ValueError(f"invalid safetensors tensor entry: {name}")
            shape, span = entry.get("shape"), entry.get("data_offsets")
            if (not isinstance(shape, list) or any(type(d) is not int or d < 0 for d in shape)
                    or not isinstance(span, list) or len(span) != 2
                    or any(type(v) is not int for v in span)
                    or not 0 <= span[0] <= span[1] <= data_bytes):
                raise ValueError(f"invalid safetensors extent: {name}")
            extents.append((span[0], span[1]))
            if name not in shapes:
                continue
            dtype = entry.get("dtype")
            if (name in found or index[name] != filename or dtype not in STORAGE
                    or tuple(shape) != tuple(shapes[name])
                    or span[1] - span[0] != math.prod(shape) * STORAGE[dtype][1]):
                raise ValueError(f"invalid checkpoint tensor layout: {name}")
            if dtype != dtypes[name]:
                raise ValueError(f"unsupported checkpoint tensor dtype: {name}: {dtype}")
            found[name] = TensorInfo(shard, dtype, tuple(shape), 8 + length + span[0],
                                     span[1] - span[0])
        extents.sort()
        if any(a[1] > b[0] for a, b in zip(extents, extents[1:])):
            raise ValueError("overlapping safetensors storage")
    if found.keys() != shapes.keys():
        raise ValueError("index references missing safetensors tensors")
    return MappingProxyType(found)


def read_tensor(info):
    """The stored bits as a numpy array of the storage dtype (BF16 as uint16,
    F8_E4M3 as uint8), without numeric interpretation (safetensors.py:135-143)."""
    with info.shard.open("rb") as f:
        f.seek(info.offset)
        raw = f.read(info.nbytes)
    if len(raw) != info.nbytes:
        raise ValueError("checkpoint changed after validation")
    return np.frombuffer(raw, dtype=STORAGE[info.dtype][0]).reshape(info.shape)


def bf16_values(bits):
    """float32 values of raw bf16 bits."""
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _check_codes(name, codes):
    if np.any((codes & 127) == 127):
        raise ValueError(f"resident FP8 storage must be finite: {name}")


def _check_scales(name, bits):
    values = bf16_values(bits)
    if not np.isfinite(values).all() or (values <= 0).any():
        raise ValueError(f"invalid FP8 weight scale: {name}")


def _scale_shape(n, k):
    return ((n + 127) // 128, k // 128)


class BlockFP8Checkpoint:
    """A directory holding ``config.json`` and block-FP8 safetensors shards.

    ``expert_weights(layer, device)`` returns the layer's grouped expert banks
    (``akas_amd.moe.ExpertWeights`` with bf16 scales); ``linear_weight(name,
    device)`` one dense quantized linear; ``router_weights(layer, device)``
    the router projection and selection bias; ``moe_options()`` the
    ``routed_moe`` keyword arguments the config implies.
    """

    def __init__(self, path):
        self.path = Path(path)
        if not self.path.is_dir():
            raise ValueError("block-FP8 checkpoint must be a directory")
        self.config = json_document((self.path / "config.json").read_text())
        if not block_fp8_config(self.config):
            raise ValueError("checkpoint is not block-FP8 quantized")
        self.index = tensor_index(self.path)
        c = self.config
        self.hidden = c.get("hidden_size")
        self.experts = c.get("num_experts")
        self.top = c.get("num_experts_per_tok")
        self.width = c.get("moe_intermediate_size")
        if self.experts is not None:
            if not (isinstance(self.top, int) and 1 <= self.top <= self.experts):
                raise ValueError("experts per token must be between 1 and the expert count")
            if c.get("use_expert_bias") is not True:
                raise ValueError("LFM2-MoE routing requires the expert selection bias")
            if self.hidden % 128 or self.width % 128:
                raise ValueError("block-FP8 expert dimensions must be multiples of 128")

    def _prefix(self, layer):
        return f"model.layers.{layer}.feed_forward."

    def moe_options(self):
        """The sigmoid + bias router and its normalization/scale (LFM2-MoE:
        ``norm_topk_prob``, ``routed_scaling_factor``)."""
        return dict(top=self.top, router="biased_router",
                    scale=float(self.config.get("routed_scaling_factor", 1.0)),
                    normalize=bool(self.config.get("norm_topk_prob", True)))

    def expert_weights(self, layer, device):
        """Grouped gate ``w1`` / up ``w3`` ``[E, F, H]`` and down ``w2``
        ``[E, H, F]`` codes with bf16 block scales, uploaded after every
        tensor of the layer was validated."""
        import torch

        from .moe import ExpertWeights

        if self.experts is None:
            raise ValueError("checkpoint has no routed experts")
        E, H, F = self.experts, self.hidden, self.width
        base = self._prefix(layer) + "experts."
        dims = {"w1": (F, H), "w3": (F, H), "w2": (H, F)}
        shapes, dtypes = {}, {}
        for e in range(E):
            for w, (n, k) in dims.items():
                shapes[f"{base}{e}.{w}.weight"], dtypes[f"{base}{e}.{w}.weight"] = (n, k), "F8_E4M3"
                name = f"{base}{e}.{w}.weight_scale"
                shapes[name], dtypes[name] = _scale_shape(n, k), "BF16"
        infos = inspect_tensors(self.path, self.index, shapes, dtypes)
        banks = {}
        for w, (n, k) in dims.items():
            codes = np.empty((E, n, k), np.uint8)
            scales = np.empty((E, *_scale_shape(n, k)), np.uint16)
            for e in range(E):
                name = f"{base}{e}.{w}.weight"
                codes[e] = read_tensor(infos[name])
                _check_codes(name, codes[e])
                scales[e] = read_tensor(infos[name + "_scale"])
                _check_scales(name + "_scale", scales[e])
            banks[w] = (torch.from_numpy(codes).to(device),
                        torch.from_numpy(scales.view(np.int16)).view(torch.bfloat16).to(device))
        return ExpertWeights(*banks["w1"], *banks["w3"], *banks["w2"])

    def linear_weight(self, name, device):
        """One dense quantized linear ``name`` (without the ``.weight``
        suffix): codes ``[N, K]`` uint8 and bf16 scales."""
        import torch

        header = self._shape_of(name + ".weight")
        if len(header) != 2 or header[1] % 128:
            raise ValueError(f"invalid FP8 linear shape: {name}")
        n, k = header
        shapes = {name + ".weight": (n, k), name + ".weight_scale": _scale_shape(n, k)}
        dtypes = {name + ".weight": "F8_E4M3", name + ".weight_scale": "BF16"}
        infos = inspect_tensors(self.path, self.index, shapes, dtypes)
        codes = read_tensor(infos[name + ".weight"]).copy()
        _check_codes(name, codes)
        scales = read_tensor(infos[name + ".weight_scale"]).copy()
        _check_scales(name + ".weight_scale", scales)
        return (torch.from_numpy(codes).to(device),
                torch.from_numpy(scales.view(np.int16)).view(torch.bfloat16).to(device))

    def router_weights(self, layer, device):
        """Router projection ``gate.weight`` ``[E, H]`` (BF16 in the file)
        and ``expert_bias`` ``[E]`` (F32), both as float32 device tensors."""
        import torch

        base = self._prefix(layer)
        gate, bias = base + "gate.weight", base + "expert_bias"
        infos = inspect_tensors(self.path, self.index,
                                {gate: (self.experts, self.hidden), bias: (self.experts,)},
                                {gate: "BF16", bias: "F32"})
        g = bf16_values(read_tensor(infos[gate]))
        b = np.array(read_tensor(infos[bias]), np.float32)
        return torch.from_numpy(np.ascontiguousarray(g)).to(device), torch.from_numpy(b).to(device)

    def _shape_of(self, name):
        if name not in self.index:
            raise ValueError(f"index references missing safetensors tensors: {name}")
        shard = (self.path / self.index[name]).resolve()
        if shard.parent != self.path.resolve() or not shard.is_file():
            raise ValueError("checkpoint shard must be a local file within its directory")
        header, _, _ = _read_header(shard)
        entry = header.get(name)
        if not isinstance(entry, dict) or not isinstance(entry.get("shape"), list):
            raise ValueError(f"invalid safetensors tensor entry: {name}")
        return tuple(entry["shape"])
