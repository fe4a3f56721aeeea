"""Block-FP8 safetensors checkpoints: header/extent validation, rejection of
unsupported semantics before any allocation, and bit-exact grouping of the
expert banks into the kernels' layout (the synthetic LFM2-MoE checkpoint of
tests/test_lfm_moe_native.py:16-70 and the rejections of :215-226)."""

import json
import struct

import numpy as np
import pytest

from oracle import fp8 as ofp8

E, H, F, TOP, LAYER = 4, 256, 256, 2, 1


def _config(**over):
    config = dict(
        model_type="lfm2_moe", hidden_size=H, moe_intermediate_size=F, num_experts=E,
        num_experts_per_tok=TOP, use_expert_bias=True, norm_topk_prob=True,
        routed_scaling_factor=1.5,
        quantization_config={
            "quant_method": "compressed-tensors", "format": "float-quantized",
            "config_groups": {"FP8_BLOCK": {
                "weights": dict(num_bits=8, type="float", strategy="block",
                                block_structure=[128, 128], dynamic=False, symmetric=True),
                "input_activations": dict(num_bits=8, type="float", strategy="group",
                                          group_size=128, dynamic=True, symmetric=True)}}})
    config.update(over)
    return config


def _tensors(seed=93):
    """name -> (safetensors dtype, storage array) of one LFM2-MoE layer plus
    a dense quantized linear; scales are rounded to bf16 before the codes are
    encoded, as a BF16-scale checkpoint is."""
    rng = np.random.default_rng(seed)
    out = {}
    base = f"model.layers.{LAYER}.feed_forward."
    for e in range(E):
        for w, (n, k) in (("w1", (F, H)), ("w3", (F, H)), ("w2", (H, F))):
            codes, scales = ofp8.quantize_weight_blocks(rng.normal(0, 0.03, (n, k)).astype(np.float32))
            out[f"{base}experts.{e}.{w}.weight"] = ("F8_E4M3", codes)
            out[f"{base}experts.{e}.{w}.weight_scale"] = ("BF16", ofp8.bf16_bits(scales))
    out[base + "gate.weight"] = ("BF16", ofp8.bf16_bits(rng.normal(0, 0.05, (E, H)).astype(np.float32)))
    out[base + "expert_bias"] = ("F32", rng.normal(0, 0.1, E).astype(np.float32))
    codes, scales = ofp8.quantize_weight_blocks(rng.normal(0, 0.03, (384, H)).astype(np.float32))
    out["model.layers.0.feed_forward.w1.weight"] = ("F8_E4M3", codes)
    out["model.layers.0.feed_forward.w1.weight_scale"] = ("BF16", ofp8.bf16_bits(scales))
    return out


def _write_shard(path, tensors, edit_header=None, truncate=0):
    payload, header = bytearray(), {}
    for name, (dtype, arr) in tensors.items():
        start = len(payload)
        payload.extend(np.ascontiguousarray(arr).tobytes())
        header[name] = dict(dtype=dtype, shape=list(arr.shape), data_offsets=[start, len(payload)])
    if edit_header is not None:
        edit_header(header)
    encoded = json.dumps(header).encode()
    blob = struct.pack("<Q", len(encoded)) + encoded + bytes(payload)
    path.write_bytes(blob[:len(blob) - truncate] if truncate else blob)


def write_checkpoint(directory, tensors=None, config=None, shards=1, edit_header=None, truncate=0):
    directory.mkdir(parents=True, exist_ok=True)
    tensors = _tensors() if tensors is None else tensors
    (directory / "config.json").write_text(json.dumps(config or _config()))
    if shards == 1:
        _write_shard(directory / "model.safetensors", tensors, edit_header, truncate)
    else:
        names = sorted(tensors)
        weight_map = {}
        for s in range(shards):
            part = {n: tensors[n] for n in names[s::shards]}
            fname = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
            _write_shard(directory / fname, part, edit_header if s == 0 else None)
            weight_map.update({n: fname for n in part})
        (directory / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    return directory


def _bits(t):
    import torch

    return t.cpu().view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.cpu().numpy()


@pytest.mark.parametrize("shards", [1, 3])
def test_expert_banks_grouped_bit_exact(tmp_path, shards):
    from akas_amd.checkpoint import BlockFP8Checkpoint

    tensors = _tensors()
    ck = BlockFP8Checkpoint(write_checkpoint(tmp_path / "ck", tensors, shards=shards))
    wts = ck.expert_weights(LAYER, "cpu")
    base = f"model.layers.{LAYER}.feed_forward.experts."
    for w, codes, scales in (("w1", wts.w1, wts.s1), ("w3", wts.w3, wts.s3), ("w2", wts.w2, wts.s2)):
        assert codes.dtype.itemsize == 1 and str(scales.dtype) == "torch.bfloat16"
        exp_c = np.stack([tensors[f"{base}{e}.{w}.weight"][1] for e in range(E)])
        exp_s = np.stack([tensors[f"{base}{e}.{w}.weight_scale"][1] for e in range(E)])
        np.testing.assert_array_equal(_bits(codes), exp_c)
        np.testing.assert_array_equal(_bits(scales), exp_s)
    assert wts.experts == E and wts.hidden == H and wts.width == F
    assert ck.moe_options() == dict(top=TOP, router="biased_router", scale=1.5, normalize=True)


def test_router_and_dense_linear(tmp_path):
    from akas_amd.checkpoint import BlockFP8Checkpoint, bf16_values

    tensors = _tensors()
    ck = BlockFP8Checkpoint(write_checkpoint(tmp_path / "ck", tensors))
    gate, bias = ck.router_weights(LAYER, "cpu")
    base = f"model.layers.{LAYER}.feed_forward."
    np.testing.assert_array_equal(gate.numpy(), bf16_values(tensors[base + "gate.weight"][1]))
    np.testing.assert_array_equal(bias.numpy(), tensors[base + "expert_bias"][1])
    codes, scales = ck.linear_weight("model.layers.0.feed_forward.w1", "cpu")
    np.testing.assert_array_equal(_bits(codes), tensors["model.layers.0.feed_forward.w1.weight"][1])
    np.testing.assert_array_equal(_bits(scales),
                                  tensors["model.layers.0.feed_forward.w1.weight_scale"][1])
    assert tuple(scales.shape) == (3, 2)  # ceil(384/128) x 256/128


def test_bf16_values_closed_form():
    from akas_amd.checkpoint import bf16_values

    bits = np.array([0x3F80, 0xBF80, 0x0000, 0x8000, 0x7F80, 0x4049, 0x0001], np.uint16)
    got = bf16_values(bits)
    assert got[0] == 1.0 and got[1] == -1.0 and got[2] == 0.0 and np.signbit(got[3])
    assert np.isinf(got[4]) and got[5] == np.float32(3.140625) and got[6] == np.float32(2.0 ** -133)


def test_unquantized_checkpoint_is_not_block_fp8(tmp_path):
    from akas_amd.checkpoint import BlockFP8Checkpoint, block_fp8_config

    assert block_fp8_config({"hidden_size": 256}) is False
    config = _config()
    del config["quantization_config"]
    with pytest.raises(ValueError):
        BlockFP8Checkpoint(write_checkpoint(tmp_path / "ck", config=config))


def _q(d):
    return d["quantization_config"]


@pytest.mark.parametrize("mutation", [
    lambda d: d.update(num_experts_per_tok=5),
    lambda d: d.update(num_experts_per_tok=0),
    lambda d: d.update(use_expert_bias=False),
    lambda d: d.update(moe_intermediate_size=200),
    lambda d: _q(d)["config_groups"]["FP8_BLOCK"]["weights"].update(block_structure=[64, 128]),
    lambda d: _q(d)["config_groups"]["FP8_BLOCK"]["weights"].update(dynamic=True),
    lambda d: _q(d)["config_groups"]["FP8_BLOCK"]["input_activations"].update(group_size=64),
    lambda d: _q(d).update(quant_method="fp8"),
    lambda d: _q(d).update(kv_cache_scheme={"num_bits": 8}),
    lambda d: _q(d)["config_groups"].update(OTHER={}),
])
def test_rejects_unsupported_semantics(tmp_path, mutation):
    from akas_amd.checkpoint import BlockFP8Checkpoint

    config = _config()
    mutation(config)
    with pytest.raises(ValueError):
        BlockFP8Checkpoint(write_checkpoint(tmp_path / "ck", config=config))


def _set(name, key, value):
    def edit(header):
        header[name][key] = value
    return edit


W1 = f"model.layers.{LAYER}.feed_forward.experts.0.w1.weight"


@pytest.mark.parametrize("edit,truncate", [
    (_set(W1 + "_scale", "dtype", "F32"), 0),          # declared dtype differs
    (_set(W1, "shape", [F, H // 2]), 0),                # shape differs from the contract
    (_set(W1 + "_scale", "data_offsets", [F * H - 4, F * H + 4]), 0),  # overlaps the codes
    (_set(W1, "data_offsets", [-1, F * H - 1]), 0),     # negative offset
    (None, 64),                                         # payload truncated
    (lambda h: h.pop(W1), 0),                           # tensor missing from the shard
])
def test_rejects_invalid_extents_before_reading(tmp_path, edit, truncate):
    from akas_amd.checkpoint import BlockFP8Checkpoint

    path = write_checkpoint(tmp_path / "ck", edit_header=edit, truncate=truncate)
    with pytest.raises(ValueError):
        ck = BlockFP8Checkpoint(path)
        ck.expert_weights(LAYER, "cpu")


@pytest.mark.parametrize("what", ["nonfinite_code", "zero_scale", "nan_scale", "negative_scale"])
def test_rejects_invalid_values(tmp_path, what):
    from akas_amd.checkpoint import BlockFP8Checkpoint

    tensors = _tensors()
    dtype, codes = tensors[W1]
    dtype_s, scales = tensors[W1 + "_scale"]
    codes, scales = codes.copy(), scales.copy()
    if what == "nonfinite_code":
        codes[3, 5] = 0xFF  # e4m3 NaN
    else:
        scales[0, 1] = {"zero_scale": 0x0000, "nan_scale": 0x7FC0, "negative_scale": 0xBF80}[what]
    tensors[W1], tensors[W1 + "_scale"] = (dtype, codes), (dtype_s, scales)
    ck = BlockFP8Checkpoint(write_checkpoint(tmp_path / "ck", tensors))
    with pytest.raises(ValueError):
        ck.expert_weights(LAYER, "cpu")


def test_rejects_shard_outside_directory(tmp_path):
    from akas_amd.checkpoint import BlockFP8Checkpoint

    path = write_checkpoint(tmp_path / "ck", shards=2)
    (tmp_path / "outside.safetensors").write_bytes((path / "model-00001-of-00002.safetensors").read_bytes())
    index = json.loads((path / "model.safetensors.index.json").read_text())
    index["weight_map"] = {n: ("../outside.safetensors" if f.startswith("model-00001") else f)
                           for n, f in index["weight_map"].items()}
    (path / "model.safetensors.index.json").write_text(json.dumps(index))
    ck = BlockFP8Checkpoint(path)
    with pytest.raises(ValueError):
        ck.expert_weights(LAYER, "cpu")


def test_rejects_duplicate_json_keys(tmp_path):
    from akas_amd.checkpoint import json_document

    with pytest.raises(ValueError):
        json_document('{"a": 1, "a": 2}')


@pytest.mark.gpu
def test_checkpoint_moe_block_on_gpu(tmp_path, dev):
    """The loaded banks (bf16 block scales, grouped [E, N, K]) feed the MoE
    block with the checkpoint's router options; the result matches the layer
    equation on the same bits."""
    import torch
    from akas_amd import moe
    from akas_amd.checkpoint import BlockFP8Checkpoint, bf16_values
    from golden_inputs import bf16_normal, rel_fro
    from oracle import moe as omoe

    tensors = _tensors()
    ck = BlockFP8Checkpoint(write_checkpoint(tmp_path / "ck", tensors))
    wts = ck.expert_weights(LAYER, dev)
    gate, bias = ck.router_weights(LAYER, dev)
    rows = 64
    x = bf16_normal(np.random.default_rng(5), (rows, H))
    logits = (x.astype(np.float32) @ gate.cpu().numpy().T).astype(np.float32)
    out = moe.routed_moe(torch.from_numpy(x).to(dev).to(torch.bfloat16),
                         torch.from_numpy(logits).to(dev), bias, wts, **ck.moe_options())
    base = f"model.layers.{LAYER}.feed_forward.experts."
    host = []
    for w in ("w1", "w3", "w2"):
        host.append(np.stack([tensors[f"{base}{e}.{w}.weight"][1] for e in range(E)]))
        host.append(np.stack([bf16_values(tensors[f"{base}{e}.{w}.weight_scale"][1]) for e in range(E)]))
    opts = ck.moe_options()
    exp, _, _ = omoe.moe_layer(x, logits, bias.cpu().numpy(), *host, opts["top"], router="sigmoid",
                               scale=opts["scale"], normalize=opts["normalize"])
    torch.cuda.synchronize()
    assert rel_fro(out.cpu().numpy(), exp) < 1e-2
