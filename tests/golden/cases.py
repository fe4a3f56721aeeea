"""Seeded golden cases: inputs (fixed draw order) and oracle outputs.

Test infrastructure (imports the oracle).  Each builder returns the arrays
stored in ``<name>.npz``; the CPU golden test calls the same builders and
requires identical arrays.
"""

import hashlib

import numpy as np

from golden_inputs import bf16_normal, stress_rows
from oracle import fp8 as ofp8
from oracle import moe as omoe


def sha256(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), np.uint8)


def dense_weights(rng, n, k):
    return rng.normal(0, 0.02, (n, k)).astype(np.float32)


def config1_inputs():
    """The single-linear workload: rng(0); W f32 [2048, 2048] ~ N(0, 0.02)
    (drawn first), x [16, 2048] ~ N(0, 1) rounded to bf16."""
    rng = np.random.default_rng(0)
    wf = dense_weights(rng, 2048, 2048)
    x = bf16_normal(rng, (16, 2048))
    return wf, x


def config1():
    wf, x = config1_inputs()
    w, ws = ofp8.quantize_weight_blocks(wf)
    xc, xs = ofp8.quantize(x)
    y = ofp8.fp8_linear(x, w, ws)
    return dict(x_bf16=ofp8.bf16_bits(x), w_sha256=sha256(w), w_scales=ws, x_codes=xc,
                x_scales=xs, y=y, y_bf16=ofp8.bf16_bits(y))


def dense_small_weights():
    """rng(1), first draw: W [256, 512] f32 ~ N(0, 0.02)."""
    return dense_weights(np.random.default_rng(1), 256, 512)


def dense_small():
    """rng(1): W [256, 512] f32 (f32 and bf16 block scales); x [16, 512] bf16
    with 1% x20 outliers plus two quantizer stress rows."""
    rng = np.random.default_rng(1)
    wf = dense_weights(rng, 256, 512)
    x = ofp8.bf16_round(np.concatenate([bf16_normal(rng, (14, 512), outliers=0.01),
                                        stress_rows(512, 2, rng)]))
    w, ws = ofp8.quantize_weight_blocks(wf)
    wb, wsb = ofp8.quantize_weight_blocks(wf, "bfloat16")
    xc, xs = ofp8.quantize(x)
    return dict(x_bf16=ofp8.bf16_bits(x), w_codes=w, w_scales=ws, w_codes_bf16s=wb,
                w_scales_bf16s=wsb, x_codes=xc, x_scales=xs, y=ofp8.fp8_linear(x, w, ws),
                y_bf16s=ofp8.fp8_linear(x, wb, wsb))


def routing():
    """rng(2): T=64 tokens, 16 experts, top-4; logits with an all-tie row and
    a tie at the top; last token inactive."""
    rng = np.random.default_rng(2)
    T, E, top = 64, 16, 4
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    logits[0] = 0.0
    logits[1, 3] = logits[1, 7] = np.float32(logits[1].max() + 1)
    bias = rng.normal(0, 0.3, E).astype(np.float32)
    active = np.ones(T, np.int32)
    active[-1] = 0
    ids, w = omoe.biased_softmax_router(logits, bias, top, scale=1.0)
    sids, sw = omoe.biased_router(logits, bias, top, scale=2.5, normalize=True)
    counts, routes = omoe.quantized_routes(ids, active, E)
    te64, tr64 = omoe.expert_tile_map(counts, T, top, 64)
    te128, tr128 = omoe.expert_tile_map(counts, T, top, 128)
    return dict(logits=logits, bias=bias, active=active, softmax_ids=ids, softmax_weights=w,
                sigmoid_ids=sids, sigmoid_weights=sw, counts=counts, routes=routes,
                tile_experts_64=te64, tile_rows_64=tr64, tile_experts_128=te128,
                tile_rows_128=tr128, offsets_64=omoe.expert_offsets(counts, 64))


def moe_small_inputs():
    """rng(3): T=48, H=256, F=256, E=8, top=2; x bf16, logits, then banks
    w1, w3, w2 ~ N(0, 0.05) drawn expert by expert."""
    rng = np.random.default_rng(3)
    T, H, F, E = 48, 256, 256, 8
    x = bf16_normal(rng, (T, H))
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    banks = {n: [] for n in ("w1", "w3", "w2")}
    for _ in range(E):
        for n, shape in (("w1", (F, H)), ("w3", (F, H)), ("w2", (H, F))):
            banks[n].append(rng.normal(0, 0.05, shape).astype(np.float32))
    return x, logits, {n: np.stack(v) for n, v in banks.items()}


def moe_small():
    x, logits, banks = moe_small_inputs()
    top = 2
    q = {n: ofp8.quantize_weight_blocks(v) for n, v in banks.items()}
    out, ids, prob = omoe.moe_layer(x, logits, np.zeros(logits.shape[1], np.float32),
                                    *q["w1"], *q["w3"], *q["w2"], top)
    data = dict(x_bf16=ofp8.bf16_bits(x), logits=logits, ids=ids, weights=prob, out=out)
    for n, (c, s) in q.items():
        data[n + "_sha256"] = sha256(c)
        data[n + "_scales"] = s
    return data


FIXTURES = dict(config1=config1, dense_small=dense_small, routing=routing, moe_small=moe_small)
