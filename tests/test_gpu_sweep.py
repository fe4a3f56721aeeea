"""GPU parity on seeded random shapes and policies, beyond the fixed cases.

Each case draws its configuration from its own seeded generator, so a
failure names a reproducible case:
- the dense linear: random M (decode, mid and prefill sizes), K, N and x,
  output and weight-scale dtypes, checked against the oracle's float64
  equation (src/akas/ops/linear/validation.py:206-230); the quantizer is
  checked bit for bit on the same input, and the prequantized binding and the
  K-partitioned product with its merge against the same reference;
- the shared-expert block in one call: random token counts, widths, expert
  counts up to 511, top-k and dtypes, bit for bit against its kinds composed
  over a bank extended with the shared expert, and against the oracle's
  block equation;
- the routed MoE block: random token counts, hidden and expert widths,
  expert counts, top-k, routers (softmax or sigmoid + bias), packed or
  compact, fused or separate SwiGLU, intermediate policy, inactive rows and
  skewed routing, against the oracle's layer equation
  (tests/support/native_fp8_reference.py:116-144 of the reference).
"""

import numpy as np
import pytest

from golden_inputs import bf16_normal
from oracle import fp8 as ofp8
from oracle import moe as omoe

pytestmark = pytest.mark.gpu

_DT = ("float32", "float16", "bfloat16")


def _rel_fro(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


@pytest.mark.parametrize("case", range(40))
def test_linear_random_shapes(dev, case):
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(1000 + case)
    kind = rng.choice(["decode", "mid", "prefill"], p=[0.5, 0.35, 0.15])
    m = int({"decode": rng.integers(1, 33), "mid": rng.integers(17, 300),
             "prefill": rng.integers(257, 1500)}[kind])
    k = int(128 * rng.choice([1, 2, 3, 4, 8, 16, 24, 32, 48, 64]))
    n = int(16 * rng.integers(1, 400)) if rng.random() < 0.7 else int(128 * rng.integers(1, 64))
    xd, od = str(rng.choice(_DT)), str(rng.choice(_DT))
    sd = str(rng.choice(["float32", "bfloat16"]))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    if rng.random() < 0.5:
        x *= np.where(rng.random((m, k)) < 0.01, 20.0, 1.0).astype(np.float32)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    wc, ws = ops.quantize_weight_blocks(torch.from_numpy(w).to(dev), scale_dtype=getattr(torch, sd))
    xt = torch.from_numpy(x).to(dev).to(getattr(torch, xd))
    odt = getattr(torch, od)
    y = ops.fp8_linear(xt, wc, ws, out_dtype=odt)
    codes, scales = ops.quantize(xt)
    y_pre = ops.fp8_linear(codes, wc, ws, activation_scales=scales, out_dtype=odt)
    torch.cuda.synchronize()

    xin = xt.float().cpu().numpy()
    want = ofp8.fp8_linear(xin, wc.cpu().numpy(), ws.float().cpu().numpy(), out_dtype=od)
    tol = 1e-4 if od == "float32" else 4e-3
    label = (m, k, n, xd, od, sd)
    assert _rel_fro(y.float().cpu().numpy(), want) <= tol, label
    assert _rel_fro(y_pre.float().cpu().numpy(), want) <= tol, label
    ec, es = ofp8.quantize(xin)
    np.testing.assert_array_equal(codes.cpu().numpy(), ec)
    np.testing.assert_array_equal(scales.cpu().numpy(), es)
    parts = [p for p in (2, 3, 4, 8) if (k // 128) % p == 0]
    if parts:
        p = int(rng.choice(parts))
        partial = ops.projection_partial(codes, scales, wc, ws, partitions=p, out_dtype=torch.float32)
        merged = ops.projection_merge(partial, out_dtype=odt)
        assert _rel_fro(merged.float().cpu().numpy(), want) <= tol, label + (p,)


@pytest.mark.parametrize("case", range(20))
def test_routed_moe_random_configurations(dev, case):
    import torch
    from akas_amd import moe

    rng = np.random.default_rng(2000 + case)
    T = int(rng.choice([1, 2, 3, 7, 16, 33, 64, 100, 256, 513, 1000]))
    H = int(128 * rng.choice([2, 4, 8, 16]))
    F = int(128 * rng.choice([2, 3, 4, 6, 12]))
    E = int(rng.choice([4, 8, 16, 32, 64]))
    while E * F * H > 24_000_000 and E > 4:
        E //= 2
    top = int(rng.choice([t for t in (1, 2, 4, 8) if t <= E]))
    packed = bool(rng.random() < 0.3)
    fused = packed or bool(rng.random() < 0.7)
    max_block_m = int(rng.choice([64, 128]))
    sigmoid = bool(rng.random() < 0.5)
    policy = str(rng.choice(["float32", "bfloat16"]))
    use_active = bool(rng.random() < 0.3)
    x = bf16_normal(rng, (T, H))
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    if rng.random() < 0.3:  # skewed routing
        logits += (-1.1 * np.log1p(rng.permutation(E))).astype(np.float32)[None, :]
    bias = rng.normal(0, 0.5, E).astype(np.float32) if sigmoid else np.zeros(E, np.float32)
    active = (rng.random(T) > 0.15).astype(np.int32) if use_active else None
    bank = {}
    for name, shape in (("w1", (E, F, H)), ("w3", (E, F, H)), ("w2", (E, H, F))):
        bank[name] = ofp8.quantize_weight_blocks(rng.normal(0, 0.05, shape).astype(np.float32))

    def dev_t(a, dtype=None):
        t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        return t.to(dtype) if dtype is not None else t

    wts = moe.ExpertWeights(*(dev_t(a) for n in ("w1", "w3", "w2") for a in bank[n]))
    dt = getattr(torch, policy)
    scale = 2.5 if sigmoid else 1.0
    out = moe.routed_moe(dev_t(x, torch.bfloat16), dev_t(logits), dev_t(bias) if sigmoid else None,
                         wts, top=top, active=dev_t(active) if use_active else None,
                         router="biased_router" if sigmoid else "biased_softmax_router",
                         scale=scale, normalize=True, packed=packed, fused_swiglu=fused,
                         max_block_m=max_block_m, product_dtype=dt, activation_dtype=dt,
                         contribution_dtype=dt)
    exp, _, _ = omoe.moe_layer(x, logits, bias, *bank["w1"], *bank["w3"], *bank["w2"], top,
                               router="sigmoid" if sigmoid else "softmax", scale=scale,
                               normalize=True, active=active, activation_dtype=policy,
                               contribution_dtype=policy)
    got = out.cpu().numpy()
    label = (T, H, F, E, top, packed, fused, max_block_m, sigmoid, policy, use_active)
    assert np.isfinite(got).all(), label
    if use_active:
        assert np.all(got[active == 0] == 0), label
    assert _rel_fro(got, exp) < 1e-2, label


@pytest.mark.parametrize("case", range(12))
def test_shared_expert_block_random(dev, case):
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(3000 + case)
    T = int(rng.choice([1, 2, 5, 16, 64, 100, 300, 700]))
    H = int(128 * rng.choice([1, 2, 4, 8]))
    F = int(128 * rng.choice([1, 2, 3, 4]))
    E = int(rng.choice([2, 8, 32, 64, 128, 256, 511]))
    while E * F * H > 32_000_000 and E > 2:
        E //= 2
    top = int(rng.integers(1, min(8, E) + 1))
    xd, gd = str(rng.choice(_DT)), str(rng.choice(_DT))
    sd = str(rng.choice(["float32", "bfloat16"]))
    bank = {}
    for name, shape in (("w1", (E, F, H)), ("w3", (E, F, H)), ("w2", (E, H, F)),
                        ("sw1", (F, H)), ("sw3", (F, H)), ("sw2", (H, F))):
        bank[name] = ofp8.quantize_weight_blocks(rng.normal(0, 0.05, shape).astype(np.float32), sd)
    dbank = {n: (torch.from_numpy(c).to(dev), torch.from_numpy(s).to(dev).to(getattr(torch, sd)))
             for n, (c, s) in bank.items()}
    x = torch.from_numpy(bf16_normal(rng, (T, H))).to(dev).to(getattr(torch, xd))
    logits = torch.from_numpy(rng.normal(0, 1, (T, E)).astype(np.float32)).to(dev)
    gate = torch.from_numpy(rng.normal(0, 1.5, T).astype(np.float32)).to(dev).to(getattr(torch, gd))
    args = [t for n in ("w1", "w3", "w2", "sw1", "sw3", "sw2") for t in dbank[n]]
    out = ops.shared_expert_moe_block(x, logits, gate, *args, top=top)

    ids, prob = ops.router(logits, top=top)
    codes, scales = ops.quantize(x)
    ext = torch.cat([ids, torch.full((T, 1), E, dtype=torch.int32, device=dev)], 1).contiguous()
    counts, routes = ops.quantized_routes(ext, torch.ones(T, dtype=torch.int32, device=dev),
                                          experts=E + 1)
    full = {n: tuple(torch.cat([dbank[n][i], dbank["s" + n][i].unsqueeze(0)]).contiguous()
                     for i in range(2)) for n in ("w1", "w3", "w2")}
    act, act_scales = ops.fp8_expert_swiglu(codes, scales, *full["w1"], *full["w3"], counts, routes,
                                            r=T, top=top + 1)
    contrib = ops.expert_partial(act, act_scales, *full["w2"], counts, routes, r=T, top=top + 1,
                                 routed_input=True, output_dtype=torch.bfloat16)
    want = ops.moe_combine(contrib[:, :top].contiguous(), prob, contrib[:, top].contiguous(), gate)
    torch.cuda.synchronize()
    label = (T, H, F, E, top, xd, gd, sd)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got, want.cpu().numpy(), err_msg=str(label))
    host = {n: (c, s.astype(np.float32)) for n, (c, s) in bank.items()}
    exp = omoe.shared_expert_moe_layer(x.float().cpu().numpy(), logits.cpu().numpy(),
                                       gate.float().cpu().numpy(),
                                       *(a for n in ("w1", "w3", "w2", "sw1", "sw3", "sw2")
                                         for a in host[n]), top)
    assert np.isfinite(got).all(), label
    assert _rel_fro(got, exp) < 1e-2, label
