"""The HIP path against the committed golden fixtures (tests/golden/*.npz).

Codes, scales, routing tables and tile maps must match bit for bit; GEMM
outputs within 1e-2 relative Frobenius of the fixture (the oracle's
float64-accumulated product) -- the measured agreement is ~1e-6 for f32
outputs.  Weight banks are regenerated from their seeds and quantized on the
GPU; their SHA-256 must equal the fixture's.
"""

import os

import numpy as np
import pytest

from golden import cases
from golden_inputs import rel_fro

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(HERE, name + ".npz"))


def _bf16(bits, dev):
    import torch

    return torch.from_numpy(np.asarray(bits, np.uint16).view(np.int16).copy()).to(dev).view(torch.bfloat16)


def _np(t):
    import torch

    t = t.detach().cpu()
    return t.float().numpy() if t.dtype in (torch.bfloat16, torch.float16) else t.numpy()


def test_config1_linear(dev):
    import torch
    from akas_amd import ops

    g = _load("config1")
    wf, _ = cases.config1_inputs()
    w, ws = ops.quantize_weight_blocks(torch.from_numpy(wf).to(dev))
    assert (cases.sha256(_np(w)) == g["w_sha256"]).all()
    np.testing.assert_array_equal(_np(ws), g["w_scales"])
    x = _bf16(g["x_bf16"], dev)
    xc, xs = ops.quantize(x)
    np.testing.assert_array_equal(_np(xc), g["x_codes"])
    np.testing.assert_array_equal(_np(xs), g["x_scales"])
    y = ops.fp8_linear(x, w, ws, out_dtype=torch.float32)
    assert rel_fro(_np(y), g["y"]) < 1e-4
    yb = ops.fp8_linear(x, w, ws, out_dtype=torch.bfloat16)
    assert rel_fro(_np(yb), g["y"]) < 1e-2


@pytest.mark.parametrize("bf16_scales", [False, True])
def test_dense_small(dev, bf16_scales):
    import torch
    from akas_amd import ops

    g = _load("dense_small")
    wf = torch.from_numpy(cases.dense_small_weights()).to(dev)
    sdt = torch.bfloat16 if bf16_scales else torch.float32
    w, ws = ops.quantize_weight_blocks(wf, scale_dtype=sdt)
    key = "_bf16s" if bf16_scales else ""
    np.testing.assert_array_equal(_np(w), g["w_codes" + key])
    np.testing.assert_array_equal(_np(ws), g["w_scales" + key])
    x = _bf16(g["x_bf16"], dev)
    xc, xs = ops.quantize(x)
    np.testing.assert_array_equal(_np(xc), g["x_codes"])
    np.testing.assert_array_equal(_np(xs), g["x_scales"])
    y = ops.fp8_linear(x, w, ws, out_dtype=torch.float32)
    assert rel_fro(_np(y), g["y" + ("_bf16s" if bf16_scales else "")]) < 1e-4


def test_routing_tables(dev):
    import torch
    from akas_amd import ops

    g = _load("routing")
    logits = torch.from_numpy(g["logits"]).to(dev)
    bias = torch.from_numpy(g["bias"]).to(dev)
    ids, w = ops.biased_softmax_router(logits, bias, top=4)
    np.testing.assert_array_equal(_np(ids), g["softmax_ids"])
    np.testing.assert_allclose(_np(w), g["softmax_weights"], rtol=2e-6)
    sids, sw = ops.biased_router(logits, bias, top=4, scale=2.5, normalize=True)
    np.testing.assert_array_equal(_np(sids), g["sigmoid_ids"])
    np.testing.assert_allclose(_np(sw), g["sigmoid_weights"], rtol=2e-6)
    active = torch.from_numpy(g["active"]).to(dev)
    counts, routes = ops.quantized_routes(ids, active, experts=16)
    np.testing.assert_array_equal(_np(counts), g["counts"])
    np.testing.assert_array_equal(_np(routes), g["routes"])
    for m in (64, 128):
        te, tr = ops.expert_tile_map(counts, r=64, top=4, max_block_m=m)
        np.testing.assert_array_equal(_np(te), g[f"tile_experts_{m}"])
        np.testing.assert_array_equal(_np(tr), g[f"tile_rows_{m}"])


@pytest.mark.parametrize("packed", [False, True])
def test_moe_small_layer(dev, packed):
    import torch
    from akas_amd import moe, ops

    g = _load("moe_small")
    x, logits, banks = cases.moe_small_inputs()
    q = {}
    for n in ("w1", "w3", "w2"):
        c, s = ops.quantize_weight_blocks(torch.from_numpy(banks[n]).to(dev))
        assert (cases.sha256(_np(c)) == g[n + "_sha256"]).all()
        np.testing.assert_array_equal(_np(s), g[n + "_scales"])
        q[n] = (c, s)
    wts = moe.ExpertWeights(*q["w1"], *q["w3"], *q["w2"])
    out, routing = moe.routed_moe(_bf16(g["x_bf16"], dev), torch.from_numpy(g["logits"]).to(dev), None,
                                  wts, top=2, packed=packed, return_routing=True)
    np.testing.assert_array_equal(_np(routing["ids"]), g["ids"])
    assert rel_fro(_np(out), g["out"]) < 1e-2
