"""Block-FP8 checkpoints on disk -> the device layout of the FP8 kernels.

A checkpoint directory holds ``config.json`` and one or more safetensors
shards (with ``model.safetensors.index.json`` when there are several).  Its
``quantization_config`` is the compressed-tensors block-FP8 scheme: every
quantized linear is an ``F8_E4M3`` ``weight [N, K]`` with a ``BF16``
``weight_scale [ceil(N/128), K/128]`` (static 128x128 weight blocks; the
activations are quantized at run time in 1x128 groups).  The checkpoint
contract is the reference's (src/akas/checkpoints/safetensors.py:21-41 for
the scheme, src/akas/models/lfm2/weights.py:95-200 for the LFM2-MoE tensor
names: ``model.layers.{L}.feed_forward.experts.{e}.{w1,w3,w2}.weight`` and
``weight_scale``, ``feed_forward.gate.weight``, ``feed_forward.expert_bias``).

Layers of this module:

* ``Shard`` -- one safetensors file.  Its header is parsed and every entry
  checked when it is opened (dtype, shape, byte count, bounds, no two
  tensors sharing bytes); reads go through ``os.pread`` on the open file and
  fail if the file got shorter since.
* ``TensorStore`` -- tensor name -> shard, through the index or the
  directory's single shard; shards outside the directory are refused.
* ``BlockFP8Checkpoint`` -- the model view: the scheme and the LFM2-MoE
  shape from ``config.json``, and loaders that resolve and check every
  tensor a request needs before any of them is read or any device memory is
  allocated, then upload the stored bits unchanged (no decoded copy).

Every failure is a ``CheckpointError``, a ``ValueError``, as the reference
raises.
"""

from dataclasses import dataclass
import json
import math
import os
from pathlib import Path
import struct

import numpy as np


class CheckpointError(ValueError):
    """A checkpoint this loader cannot use, found before anything is uploaded."""


# Element sizes of the safetensors dtypes (needed to check every entry of a
# header, including tensors this loader never reads).
_ELEMENT_BYTES = {"BOOL": 1, "U8": 1, "I8": 1, "F8_E4M3": 1, "F8_E5M2": 1, "U16": 2, "I16": 2,
                  "F16": 2, "BF16": 2, "U32": 4, "I32": 4, "F32": 4, "U64": 8, "I64": 8, "F64": 8}
# Host storage of the dtypes this loader reads: raw bits for the 8- and
# 16-bit float formats numpy has no type for.
_HOST_TYPE = {"F8_E4M3": np.uint8, "BF16": np.uint16, "F16": np.float16, "F32": np.float32}
_MAX_HEADER_BYTES = 64 << 20


def json_document(text):
    """Parse JSON, refusing any object that names a key twice (a repeated
    tensor entry would otherwise replace the first one unnoticed)."""

    def build(pairs):
        keys = [k for k, _ in pairs]
        if len(set(keys)) != len(keys):
            repeated = sorted({k for k in keys if keys.count(k) > 1})
            raise CheckpointError(f"JSON object repeats key(s) {repeated}")
        return dict(pairs)

    try:
        return json.loads(text, object_pairs_hook=build)
    except json.JSONDecodeError as err:
        raise CheckpointError(f"malformed JSON: {err}") from None


def bf16_values(bits):
    """float32 values of stored bf16 bit patterns (a bf16 is the top half of
    a float32)."""
    return np.left_shift(np.asarray(bits, np.uint16).astype(np.uint32), 16).view(np.float32)


# ---------------------------------------------------------------------------
# safetensors files
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class Entry:
    """One tensor of a shard: bytes [begin, end) of the data area."""

    name: str
    dtype: str
    shape: tuple
    begin: int
    end: int


def _is_count(v):
    return type(v) is int and v >= 0


def _entry(name, fields, data_bytes, where):
    if not isinstance(fields, dict) or not {"dtype", "shape", "data_offsets"} <= fields.keys():
        raise CheckpointError(f"{where}: entry {name!r} lacks dtype, shape or data_offsets")
    dtype, shape, offsets = fields["dtype"], fields["shape"], fields["data_offsets"]
    if dtype not in _ELEMENT_BYTES:
        raise CheckpointError(f"{where}: entry {name!r} has unknown dtype {dtype!r}")
    if not isinstance(shape, list) or not all(map(_is_count, shape)):
        raise CheckpointError(f"{where}: entry {name!r} has shape {shape!r}")
    if not (isinstance(offsets, list) and len(offsets) == 2 and all(map(_is_count, offsets))):
        raise CheckpointError(f"{where}: entry {name!r} has data_offsets {offsets!r}")
    begin, end = offsets
    if begin > end or end > data_bytes:
        raise CheckpointError(f"{where}: entry {name!r} spans bytes {begin}..{end} of a "
                              f"{data_bytes}-byte data area")
    if end - begin != math.prod(shape) * _ELEMENT_BYTES[dtype]:
        raise CheckpointError(f"{where}: entry {name!r} holds {end - begin} bytes for a "
                              f"{dtype} tensor of shape {shape}")
    return Entry(name, dtype, tuple(shape), begin, end)


class Shard:
    """A safetensors file: little-endian u64 header length, JSON header,
    data area.  Opening it checks the whole header."""

    def __init__(self, path):
        self.path = Path(path)
        self._fd = os.open(self.path, os.O_RDONLY)
        try:
            self._size = os.fstat(self._fd).st_size
            head = os.pread(self._fd, 8, 0)
            if len(head) < 8:
                raise CheckpointError(f"{self.path.name}: shorter than a safetensors preamble")
            (length,) = struct.unpack("<Q", head)
            if length < 2 or length > _MAX_HEADER_BYTES or 8 + length > self._size:
                raise CheckpointError(f"{self.path.name}: header length {length} does not fit "
                                      f"a {self._size}-byte file")
            raw = os.pread(self._fd, length, 8)
            try:
                text = raw.decode("utf-8")
            except UnicodeDecodeError:
                raise CheckpointError(f"{self.path.name}: header is not UTF-8") from None
            header = json_document(text)
            if not isinstance(header, dict):
                raise CheckpointError(f"{self.path.name}: header is not a JSON object")
            self._data_at = 8 + length
            data_bytes = self._size - self._data_at
            meta = header.pop("__metadata__", {})
            if not isinstance(meta, dict):
                raise CheckpointError(f"{self.path.name}: __metadata__ is not an object")
            self.entries = {n: _entry(n, f, data_bytes, self.path.name) for n, f in header.items()}
            spans = sorted(self.entries.values(), key=lambda e: (e.begin, e.end))
            for a, b in zip(spans, spans[1:]):
                if b.begin < a.end:
                    raise CheckpointError(f"{self.path.name}: tensors {a.name!r} and {b.name!r} "
                                          f"share bytes")
        except BaseException:
            self.close()
            raise

    def read(self, entry):
        """The entry's stored elements (raw bits for F8_E4M3 and BF16)."""
        if os.fstat(self._fd).st_size != self._size:
            raise CheckpointError(f"{self.path.name}: file size changed since it was opened")
        raw = os.pread(self._fd, entry.end - entry.begin, self._data_at + entry.begin)
        if len(raw) != entry.end - entry.begin:
            raise CheckpointError(f"{self.path.name}: {entry.name!r} is cut short")
        return np.frombuffer(raw, dtype=_HOST_TYPE[entry.dtype]).reshape(entry.shape)

    def close(self):
        fd, self._fd = getattr(self, "_fd", -1), -1
        if fd >= 0:
            os.close(fd)

    def __del__(self):
        self.close()


class TensorStore:
    """The tensors of a checkpoint directory by name."""

    INDEX = "model.safetensors.index.json"

    def __init__(self, directory):
        self.root = Path(directory).resolve()
        index = self.root / self.INDEX
        if index.is_file():
            doc = json_document(index.read_text())
            owner = doc.get("weight_map") if isinstance(doc, dict) else None
            if not isinstance(owner, dict) or not all(isinstance(v, str) for v in owner.values()):
                raise CheckpointError(f"{self.INDEX}: weight_map must map names to file names")
            self._owner = owner
            self._shards = {}
        else:
            files = sorted(self.root.glob("*.safetensors"))
            if len(files) != 1:
                raise CheckpointError(f"{self.root}: no {self.INDEX} and {len(files)} "
                                      f"safetensors files (one is needed)")
            shard = Shard(files[0])
            self._owner = {name: files[0].name for name in shard.entries}
            self._shards = {files[0].name: shard}

    def __contains__(self, name):
        return name in self._owner

    def _shard(self, filename):
        if filename not in self._shards:
            path = (self.root / filename).resolve()
            if path.parent != self.root or not path.is_file():
                raise CheckpointError(f"shard {filename!r} is not a file inside {self.root}")
            self._shards[filename] = Shard(path)
        return self._shards[filename]

    def locate(self, name, dtype=None, shape=None):
        """(shard, entry) of ``name``, checked against the expected dtype and
        shape when given."""
        if name not in self._owner:
            raise CheckpointError(f"tensor {name!r} is not in the checkpoint")
        shard = self._shard(self._owner[name])
        entry = shard.entries.get(name)
        if entry is None:
            raise CheckpointError(f"tensor {name!r} is indexed to {shard.path.name} but absent there")
        if dtype is not None and entry.dtype != dtype:
            raise CheckpointError(f"tensor {name!r} is {entry.dtype}, expected {dtype}")
        if shape is not None and entry.shape != tuple(shape):
            raise CheckpointError(f"tensor {name!r} has shape {list(entry.shape)}, "
                                  f"expected {list(shape)}")
        return shard, entry


# ---------------------------------------------------------------------------
# the block-FP8 scheme and the LFM2-MoE model config
# ---------------------------------------------------------------------------

# compressed-tensors fields of the one supported config group.
_WEIGHT_SCHEME = dict(num_bits=8, type="float", strategy="block", block_structure=[128, 128],
                      dynamic=False, symmetric=True)
_ACTIVATION_SCHEME = dict(num_bits=8, type="float", strategy="group", group_size=128,
                          dynamic=True, symmetric=True)


def _same(value, expected):
    # type-strict: 0 is not False and 1.0 is not 1
    return type(value) is type(expected) and value == expected


def block_fp8_config(config):
    """False when ``config`` has no ``quantization_config``; True when it is
    the block-FP8 scheme; ``CheckpointError`` naming every difference
    otherwise."""
    quant = config.get("quantization_config")
    if quant is None:
        return False
    problems = []
    if not isinstance(quant, dict):
        raise CheckpointError("quantization_config is not an object")
    if quant.get("quant_method") != "compressed-tensors":
        problems.append(f"quant_method {quant.get('quant_method')!r} (need 'compressed-tensors')")
    if quant.get("format") != "float-quantized":
        problems.append(f"format {quant.get('format')!r} (need 'float-quantized')")
    if quant.get("kv_cache_scheme") is not None:
        problems.append("a KV-cache quantization scheme")
    groups = quant.get("config_groups")
    if not isinstance(groups, dict) or len(groups) != 1:
        problems.append(f"{len(groups) if isinstance(groups, dict) else 'no'} config groups "
                        f"(need exactly one)")
    else:
        (scheme,) = groups.values()
        scheme = scheme if isinstance(scheme, dict) else {}
        for part, wanted in (("weights", _WEIGHT_SCHEME), ("input_activations", _ACTIVATION_SCHEME)):
            fields = scheme.get(part) if isinstance(scheme.get(part), dict) else {}
            for key, value in wanted.items():
                if not _same(fields.get(key), value):
                    problems.append(f"{part}.{key} = {fields.get(key)!r} (need {value!r})")
    if problems:
        raise CheckpointError("unsupported checkpoint quantization: " + "; ".join(problems))
    return True


@dataclass(frozen=True)
class MoEShape:
    """The routed-expert dimensions and router options of an LFM2-MoE config."""

    experts: int
    top: int
    hidden: int
    width: int
    scale: float
    normalize: bool

    @classmethod
    def from_config(cls, c):
        experts, top = c.get("num_experts"), c.get("num_experts_per_tok")
        hidden, width = c.get("hidden_size"), c.get("moe_intermediate_size")
        if not all(type(v) is int and v > 0 for v in (experts, hidden, width)):
            raise CheckpointError("num_experts, hidden_size and moe_intermediate_size must be "
                                  "positive integers")
        if type(top) is not int or not 1 <= top <= experts:
            raise CheckpointError(f"num_experts_per_tok {top!r} is outside 1..{experts}")
        if hidden % 128 or width % 128:
            raise CheckpointError(f"hidden_size {hidden} and moe_intermediate_size {width} must "
                                  f"be multiples of the 128-wide FP8 blocks")
        if c.get("use_expert_bias") is not True:
            raise CheckpointError("the LFM2-MoE router selects with an expert bias; "
                                  "use_expert_bias must be true")
        return cls(experts, top, hidden, width, float(c.get("routed_scaling_factor", 1.0)),
                   bool(c.get("norm_topk_prob", True)))


def _scale_grid(n, k):
    return (-(-n // 128), k // 128)


def _checked_codes(name, codes):
    # e4m3 has one NaN pattern per sign and no infinities
    if np.count_nonzero((codes | 0x80) == 0xFF):
        raise CheckpointError(f"{name}: e4m3 codes include NaN")
    return codes


def _checked_scales(name, bits):
    # positive finite bf16 patterns are exactly 0x0001 .. 0x7F7F
    if np.count_nonzero((bits == 0) | (bits >= 0x7F80)):
        raise CheckpointError(f"{name}: block scales must be positive and finite")
    return bits


def _bf16_tensor(torch, bits, device):
    return torch.from_numpy(np.array(bits, np.uint16).view(np.int16)).view(torch.bfloat16).to(device)


class BlockFP8Checkpoint:
    """A block-FP8 LFM2-MoE checkpoint directory.

    ``expert_weights(layer, device)`` -> ``akas_amd.moe.ExpertWeights``
    (grouped ``[E, N, K]`` codes, bf16 ``[E, ceil(N/128), K/128]`` scales);
    ``linear_weight(name, device)`` -> one dense quantized linear's codes
    and scales; ``router_weights(layer, device)`` -> the router projection
    and the selection bias as float32; ``moe_options()`` -> the
    ``moe.routed_moe`` keyword arguments the config implies.
    """

    def __init__(self, path):
        root = Path(path)
        if not root.is_dir():
            raise CheckpointError(f"{root} is not a checkpoint directory")
        self.config = json_document((root / "config.json").read_text())
        if not isinstance(self.config, dict) or not block_fp8_config(self.config):
            raise CheckpointError(f"{root} is not a block-FP8 quantized checkpoint")
        self.moe = MoEShape.from_config(self.config) if "num_experts" in self.config else None
        self.store = TensorStore(root)

    def _moe(self):
        if self.moe is None:
            raise CheckpointError("the checkpoint has no routed experts")
        return self.moe

    def moe_options(self):
        m = self._moe()
        return dict(top=m.top, router="biased_router", scale=m.scale, normalize=m.normalize)

    def _linear_entries(self, name, n, k):
        return (self.store.locate(name + ".weight", "F8_E4M3", (n, k)),
                self.store.locate(name + ".weight_scale", "BF16", _scale_grid(n, k)))

    def expert_weights(self, layer, device):
        import torch

        from .moe import ExpertWeights

        m = self._moe()
        prefix = f"model.layers.{layer}.feed_forward.experts."
        dims = {"w1": (m.width, m.hidden), "w3": (m.width, m.hidden), "w2": (m.hidden, m.width)}
        # every tensor of the layer is located and checked before any is read
        plan = {w: [self._linear_entries(f"{prefix}{e}.{w}", *nk) for e in range(m.experts)]
                for w, nk in dims.items()}
        banks = []
        for w, (n, k) in dims.items():
            codes = np.empty((m.experts, n, k), np.uint8)
            scales = np.empty((m.experts, *_scale_grid(n, k)), np.uint16)
            for e, ((cs, ce), (ss, se)) in enumerate(plan[w]):
                codes[e] = _checked_codes(ce.name, cs.read(ce))
                scales[e] = _checked_scales(se.name, ss.read(se))
            banks += [torch.from_numpy(codes).to(device), _bf16_tensor(torch, scales, device)]
        return ExpertWeights(*banks)

    def linear_weight(self, name, device):
        """``name`` without the ``.weight`` suffix."""
        import torch

        _, entry = self.store.locate(name + ".weight", "F8_E4M3")
        if len(entry.shape) != 2 or entry.shape[1] % 128:
            raise CheckpointError(f"{name}.weight has shape {list(entry.shape)}; an FP8 linear "
                                  f"is [N, K] with K a multiple of 128")
        (cs, ce), (ss, se) = self._linear_entries(name, *entry.shape)
        codes = _checked_codes(ce.name, cs.read(ce))
        scales = _checked_scales(se.name, ss.read(se))
        return torch.from_numpy(codes.copy()).to(device), _bf16_tensor(torch, scales, device)

    def router_weights(self, layer, device):
        """``gate.weight`` ``[E, H]`` (stored BF16) and ``expert_bias`` ``[E]``
        (stored F32), as float32."""
        import torch

        m = self._moe()
        prefix = f"model.layers.{layer}.feed_forward."
        gs, ge = self.store.locate(prefix + "gate.weight", "BF16", (m.experts, m.hidden))
        bs, be = self.store.locate(prefix + "expert_bias", "F32", (m.experts,))
        gate = bf16_values(gs.read(ge))
        bias = np.array(bs.read(be), np.float32)
        return torch.from_numpy(gate).to(device), torch.from_numpy(bias).to(device)
