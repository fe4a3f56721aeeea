"""GPU parity: routing, permutation, tile maps, packing, grouped expert GEMMs,
fused SwiGLU re-quantization and the weighted combine."""

import numpy as np
import pytest

from oracle import fp8 as ofp8
from oracle import moe as omoe
from golden_inputs import bf16_normal, exact_codes, random_codes, rel_fro

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(dev)


def _np(t):
    import torch

    torch.cuda.synchronize()
    return t.float().cpu().numpy() if t.dtype in (torch.bfloat16, torch.float16) else t.cpu().numpy()


def pattern_routes(rows, top, experts, mult=1, inactive_last=True):
    ids = ((np.arange(rows)[:, None] * mult + np.arange(top)[None, :]) % experts).astype(np.int32)
    active = np.ones(rows, np.int32)
    if rows > 1 and inactive_last:
        active[-1] = 0
    return ids, active


# ---------------------------------------------------------------------------
# routers
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("rows,experts,top", [(1, 64, 4), (257, 64, 4), (64, 256, 8), (9, 7, 3),
                                              (1000, 64, 8), (33, 32, 6), (17, 64, 1),
                                              (20, 1000, 6), (5, 1024, 32), (7, 64, 9)])
def test_softmax_router(dev, rows, experts, top):
    """Up to 64 experts and top 8 take the sixteen-lanes-per-row kernel, the
    rest the one-wave-per-row kernel (4 expert slots per lane up to 256
    experts, 16 above); ties within a lane's experts (0, 1) and across lanes
    (20, 40) resolve to the lower id."""
    from akas_amd import ops

    rng = np.random.default_rng(17)
    logits = rng.normal(0, 1, (rows, experts)).astype(np.float32)
    bias = rng.normal(0, 0.1, experts).astype(np.float32)
    logits[0, 1] = logits[0, 0]  # forced tie resolved to the lower id
    bias[1] = bias[0]
    if experts > 40:
        logits[0, 20] = logits[0, 40] = 5.0
        bias[40] = bias[20]
    ids, w = ops.biased_softmax_router(_t(logits, dev), _t(bias, dev), top=top, scale=1.5)
    eids, ew = omoe.biased_softmax_router(logits, bias, top, scale=1.5)
    np.testing.assert_array_equal(_np(ids), eids)
    np.testing.assert_allclose(_np(w), ew, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("rows,experts,top", [(64, 256, 8), (257, 64, 4), (3, 300, 5), (9, 7, 3),
                                              (1, 64, 8), (5, 1024, 32)])
def test_decode_router(dev, rows, experts, top):
    """The block-fp8 router kind: selection on the bf16-rounded logits.  Row 0
    holds 1 and 1 + 2^-10 (one bf16 value) as its two largest logits, the
    larger f32 value at the higher index: the tie goes to the lower index.
    Covers the sixteen-lanes-per-row kernel (<= 64 experts) and the
    one-wave-per-row kernel with 4 (<= 256) and 16 expert slots per lane."""
    from akas_amd import ops

    rng = np.random.default_rng(19)
    logits = rng.normal(0, 1, (rows, experts)).astype(np.float32)
    logits[0] = np.minimum(logits[0], 0.5)
    logits[0, 1] = 1.0
    logits[0, min(5, experts - 1)] = np.float32(1.0 + 2.0 ** -10)
    ids, w = ops.router(_t(logits, dev), top=top)
    eids, ew = omoe.router(logits, top)
    np.testing.assert_array_equal(_np(ids), eids)
    assert _np(ids)[0, 0] == 1
    np.testing.assert_allclose(_np(w), ew, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("normalize", [True, False])
@pytest.mark.parametrize("rows,experts,top", [(65, 64, 4), (33, 256, 8), (5, 1024, 32), (9, 7, 3)])
def test_sigmoid_router(dev, normalize, rows, experts, top):
    """The sigmoid + bias router up to its limits (1024 experts, top 32)."""
    from akas_amd import ops

    rng = np.random.default_rng(18 + experts)
    logits = rng.normal(0, 1, (rows, experts)).astype(np.float32)
    logits[0] = 0  # exact ties: bias decides, then the lowest id
    bias = (np.arange(experts)[::-1] % 3 * 0.1).astype(np.float32)
    ids, w = ops.biased_router(_t(logits, dev), _t(bias, dev), top=top, scale=2.0,
                               normalize=normalize)
    eids, ew = omoe.biased_router(logits, bias, top, 2.0, normalize)
    np.testing.assert_array_equal(_np(ids), eids)
    np.testing.assert_allclose(_np(w), ew, rtol=2e-6, atol=1e-7)


def test_sigmoid_router_score_every_float32(dev):
    """The device's 1 / (1 + e^-l) equals the oracle's for every float32
    logit on which it depends on the exponential's last bit: all l in
    [-88.75, 17] with |l| >= 2^-26 (about 524 million values), plus the
    tails and a sample of tinier ones.  Read through the router itself: one
    expert, top 1, unnormalized, scale 1 makes the weight the score term."""
    import torch
    from akas_amd import ops

    def check(bits):
        logits = torch.from_numpy(bits.view(np.float32).reshape(-1, 1)).to(dev)
        _, w = ops.biased_router(logits, None, top=1, normalize=False)
        got = w.cpu().numpy().ravel()
        exp = omoe.router_sigmoid(bits.view(np.float32))
        bad = np.flatnonzero(got.view(np.uint32) != exp.view(np.uint32))
        assert bad.size == 0, (bits[bad[:8]], got[bad[:8]], exp[bad[:8]])

    step = 1 << 25
    for sign, hi in ((0x80000000, 0x42B18000), (0, 0x41880000)):  # l < 0, then l > 0
        for a in range(0x32800000, hi + 1, step):
            check(np.arange(a, min(a + step, hi + 1), dtype=np.uint32) | np.uint32(sign))
    rng = np.random.default_rng(9)
    tails = np.concatenate([rng.integers(0, 0x32800000, 1 << 20),        # |l| < 2^-26
                            rng.integers(0x42B18000, 0x7F800000, 1 << 20),  # l < -88.75
                            rng.integers(0x41880000, 0x7F800000, 1 << 20)]).astype(np.uint32)
    signs = np.array([0, 0x80000000, 0], np.uint32).repeat(1 << 20)
    signs[: 1 << 20] = rng.integers(0, 2, 1 << 20).astype(np.uint32) << 31
    check(tails | signs)


def _logit_for_score(target, lo=0.0, hi=16.0):
    """Smallest float32 l in [lo, hi] with router_sigmoid(l) >= target (the
    score term is monotone in l), by bisection on the float32 patterns."""
    a = np.full(target.shape, np.float32(lo)).view(np.uint32).astype(np.int64)
    b = np.full(target.shape, np.float32(hi)).view(np.uint32).astype(np.int64)
    while np.any(a < b):
        m = (a + b) // 2
        ok = omoe.router_sigmoid(m.astype(np.uint32).view(np.float32)) >= target
        b = np.where(ok, m, b)
        a = np.where(ok, a, m + 1)
    return a.astype(np.uint32).view(np.float32)


def test_sigmoid_router_near_ties(dev):
    """Scores that tie exactly or differ in the last bit: logits one float32
    step apart (whose score terms often round to the same value), and pairs
    whose biases differ by 0.25 with the logit of the biased expert chosen
    so that sigmoid + bias lands exactly on the other expert's score.  Ties
    go to the lower expert index, so one wrong bit anywhere in the score
    changes the ids."""
    from akas_amd import ops

    rng = np.random.default_rng(31)
    rows, experts, top = 4096, 64, 4
    bias = np.zeros(experts, np.float32)
    bias[32:] = 0.25
    logits = (rng.normal(0, 1, (rows, experts)) - 4).astype(np.float32)  # low background
    r = np.arange(rows)
    # pair A: two unbiased experts, logits one float32 step apart, either order
    i, j = rng.integers(0, 16, rows), rng.integers(16, 32, rows)
    u = rng.uniform(1.0, 3.0, rows).astype(np.float32)
    up = np.nextafter(u, np.float32(np.inf))
    swap = rng.random(rows) < 0.5
    logits[r, i] = np.where(swap, up, u)
    logits[r, j] = np.where(swap, u, up)
    # pair B: an unbiased expert with score s and a biased one whose
    # sigmoid + 0.25 rounds to s; the biased expert sits at the higher index
    lo_e, hi_e = rng.integers(0, 16, rows), rng.integers(32, 64, rows)
    lo_e = np.where(lo_e == i, (lo_e + 1) % 16, lo_e)
    lb = rng.uniform(2.0, 3.0, rows).astype(np.float32)
    s = omoe.router_sigmoid(lb)
    lh = _logit_for_score(s - np.float32(0.25))
    hit = (omoe.router_sigmoid(lh) + np.float32(0.25)).astype(np.float32) == s
    assert hit.mean() > 0.9
    logits[r, lo_e] = lb
    logits[r, hi_e] = lh
    ids, w = ops.biased_router(_t(logits, dev), _t(bias, dev), top=top, scale=1.0, normalize=True)
    eids, ew = omoe.biased_router(logits, bias, top, 1.0, True)
    np.testing.assert_array_equal(_np(ids), eids)
    np.testing.assert_allclose(_np(w), ew, rtol=2e-6, atol=1e-7)
    # the ties are real: equal scores among the chosen experts in most rows
    score = (omoe.router_sigmoid(logits) + bias).astype(np.float32)
    top_scores = np.take_along_axis(score, eids, axis=1)
    assert (np.diff(top_scores, axis=1) == 0).any(axis=1).mean() > 0.5


# ---------------------------------------------------------------------------
# routes / tile map / pack
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("rows,top,experts,mult", [(1, 4, 64, 1), (33, 2, 4, 1), (1025, 4, 64, 3),
                                                   (16384, 4, 64, 7), (257, 3, 7, 1),
                                                   (4100, 4, 64, 5), (12, 4, 5, 1),
                                                   (300, 8, 1024, 7), (64, 32, 256, 3)])
def test_quantized_routes_patterns(dev, rows, top, experts, mult):
    from akas_amd import ops

    ids, active = pattern_routes(rows, top, experts, mult)
    counts, routes = ops.quantized_routes(_t(ids, dev), _t(active, dev), experts=experts)
    ec, er = omoe.quantized_routes(ids, active, experts)
    np.testing.assert_array_equal(_np(counts), ec)
    np.testing.assert_array_equal(_np(routes), er)


def test_quantized_routes_from_router_zipf(dev):
    """Skewed top-4 routing of 16384 tokens over 64 experts."""
    from akas_amd import ops

    rng = np.random.default_rng(0)
    rows, experts, top = 16384, 64, 4
    logits = rng.normal(0, 1, (rows, experts)).astype(np.float32)
    logits += (-1.1 * np.log1p(rng.permutation(experts))).astype(np.float32)[None, :]
    ids, _ = ops.biased_softmax_router(_t(logits, dev), None, top=top)
    active = np.ones(rows, np.int32)
    active[rng.random(rows) < 0.05] = 0
    counts, routes = ops.quantized_routes(ids, _t(active, dev), experts=experts)
    ec, er = omoe.quantized_routes(_np(ids), active, experts)
    np.testing.assert_array_equal(_np(counts), ec)
    np.testing.assert_array_equal(_np(routes), er)
    assert ec.max() > 3 * ec.mean()  # the skew is real


def test_quantized_routes_empty_batch(dev):
    from akas_amd import ops

    ids, _ = pattern_routes(8, 2, 5)
    active = np.zeros(8, np.int32)
    counts, routes = ops.quantized_routes(_t(ids, dev), _t(active, dev), experts=5)
    assert not _np(counts).any()
    assert (_np(routes) == -1).all()


@pytest.mark.parametrize("top", [4, 2])
def test_quantized_routes_zero_rows(dev, top):
    """A batch of no rows (zero-element tensors, whose device pointers are
    null): every count is 0 and nothing else is touched
    (``tests/test_lfm_moe.py:204-214``).  top == 4 is the four-rows-per-thread
    kernel's shape, which must not run on an empty batch."""
    import torch
    from akas_amd import ops

    ids = torch.empty((0, top), dtype=torch.int32, device=dev)
    active = torch.empty((0,), dtype=torch.int32, device=dev)
    counts = torch.full((64,), 7, dtype=torch.int32, device=dev)
    counts, routes = ops.quantized_routes(ids, active, experts=64, counts=counts)
    assert tuple(routes.shape) == (64, 0)
    assert not _np(counts).any()


def test_routed_moe_zero_rows(dev):
    """The routed MoE block on an empty batch returns an empty f32 output."""
    import torch
    from akas_amd import moe

    rng = np.random.default_rng(2)
    H, F, E = 256, 128, 8
    bank = {}
    for name, shape in (("w1", (E, F, H)), ("w3", (E, F, H)), ("w2", (E, H, F))):
        bank[name] = ofp8.quantize_weight_blocks(rng.normal(0, 0.05, shape).astype(np.float32))
    wts = moe.ExpertWeights(*(_t(a, dev) for n in ("w1", "w3", "w2") for a in bank[n]))
    x = torch.empty((0, H), dtype=torch.bfloat16, device=dev)
    logits = torch.empty((0, E), dtype=torch.float32, device=dev)
    for fused in (True, False):
        out = moe.routed_moe(x, logits, None, wts, top=4, fused_swiglu=fused)
        torch.cuda.synchronize()
        assert tuple(out.shape) == (0, H) and out.dtype == torch.float32


@pytest.mark.parametrize("rows,top,experts,maxm", [(33, 3, 7, 64), (257, 3, 7, 128), (1, 4, 64, 64),
                                                   (16384, 4, 64, 128)])
def test_expert_tile_map(dev, rows, top, experts, maxm):
    from akas_amd import ops

    ids, active = pattern_routes(rows, top, experts, 3)
    ec, _ = omoe.quantized_routes(ids, active, experts)
    te, tr = ops.expert_tile_map(_t(ec, dev), r=rows, top=top, max_block_m=maxm)
    ete, etr = omoe.expert_tile_map(ec, rows, top, maxm)
    np.testing.assert_array_equal(_np(te), ete)
    np.testing.assert_array_equal(_np(tr), etr)


@pytest.mark.parametrize("rows,maximum,routed", [(1, 16, False), (33, 64, False), (129, 128, True)])
def test_expert_pack(dev, rows, maximum, routed):
    """(src/akas/ops/moe/validation.py:595-618 geometry: k=256, top=3, experts=7)"""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(rows)
    top, experts, k = 3, 7, 256
    ids, active = pattern_routes(rows, top, experts, 3)
    counts, routes = omoe.quantized_routes(ids, active, experts)
    shape = (rows, top, k) if routed else (rows, k)
    x = random_codes(rng, shape)
    xs = rng.uniform(0.0625, 0.25, (*shape[:-1], k // 128)).astype(np.float32)
    te, tr = omoe.expert_tile_map(counts, rows, top, maximum)
    cap = omoe.tile_capacity(rows, top, experts, maximum) * maximum
    packed = torch.zeros((cap, k), dtype=torch.uint8, device=dev)
    pscales = torch.ones((cap, k // 128), dtype=torch.float32, device=dev)
    offs = torch.zeros((experts,), dtype=torch.int32, device=dev)
    ops.expert_pack(_t(x, dev), _t(xs, dev), _t(counts, dev), _t(routes, dev), _t(te, dev),
                    _t(tr, dev), top=top, max_block_m=maximum, routed_input=routed,
                    packed=packed, packed_scales=pscales, expert_offsets=offs)
    ep, es, eo = omoe.expert_pack(x, xs, counts, routes, top, experts, maximum, routed)
    np.testing.assert_array_equal(_np(packed), ep)
    np.testing.assert_array_equal(_np(pscales), es)
    np.testing.assert_array_equal(_np(offs), eo)


# ---------------------------------------------------------------------------
# grouped expert GEMMs
# ---------------------------------------------------------------------------

def _expert_case(rng, rows, top, experts, o, k, routed, exact=True, mult=1):
    ids, active = pattern_routes(rows, top, experts, mult)
    counts, routes = omoe.quantized_routes(ids, active, experts)
    shape = (rows, top, k) if routed else (rows, k)
    gen = exact_codes if exact else random_codes
    x = gen(rng, shape)
    w = gen(rng, (experts, o, k))
    if exact:
        xs = (2.0 ** rng.integers(-4, 1, (*shape[:-1], k // 128))).astype(np.float32)
        ws = (2.0 ** rng.integers(-4, 1, (experts, o // 128, k // 128))).astype(np.float32)
    else:
        xs = rng.uniform(0.0625, 0.25, (*shape[:-1], k // 128)).astype(np.float32)
        ws = ofp8.bf16_round(rng.uniform(0.0625, 0.25, (experts, o // 128, k // 128)).astype(np.float32))
    return ids, active, counts, routes, x, xs, w, ws


@pytest.mark.parametrize("rows,top,experts,o,k,routed", [
    (3, 2, 4, 128, 256, False), (1, 4, 64, 128, 256, False), (33, 2, 4, 128, 256, False),
    (33, 2, 4, 128, 384, True), (257, 3, 7, 256, 384, True), (256, 4, 64, 256, 512, False),
    (2048, 4, 8, 256, 256, False),
    # 32-row tiles with 256 columns (N % 256 == 0), routed input, N = 768
    (200, 4, 32, 768, 256, True),
    # >= 128 rows per expert: 256-row DMA tiles (ragged last tiles, gathered
    # and routed rows, N = 256 and 512, and N = 384 on the 128-row fallback)
    (1500, 2, 6, 512, 384, True), (700, 4, 16, 256, 512, False), (600, 3, 5, 384, 256, False),
    # the most experts the entry points take (tile lookup over 16 count chunks)
    (300, 8, 1024, 128, 256, False)])
def test_expert_partial_exact(dev, rows, top, experts, o, k, routed):
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(37)
    ids, active, counts, routes, x, xs, w, ws = _expert_case(rng, rows, top, experts, o, k, routed)
    exp = omoe.expert_partial(x, xs, w, ws, counts, routes, top, routed_input=routed)
    for sdt in (torch.float32, torch.bfloat16):  # binary scales are exact in bf16
        out = ops.expert_partial(_t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev, sdt),
                                 _t(counts, dev), _t(routes, dev), r=rows, top=top,
                                 routed_input=routed)
        np.testing.assert_array_equal(_np(out), exp)


def test_expert_partial_dma_deepest_k(dev):
    """The expert prefill kernel (256-row tiles) at the deepest k range it
    takes: K = 16384, a full 128-entry weight-scale table.  Scales 2^-2 or
    2^-1 keep every partial sum exact in float32 while a wrong k-block or
    scale index still changes the result; the whole output is compared."""
    from akas_amd import ops

    rng = np.random.default_rng(16385)
    rows, top, experts, o, k = 600, 1, 2, 256, 16384
    ids, active = pattern_routes(rows, top, experts, 1)
    counts, routes = omoe.quantized_routes(ids, active, experts)
    x = exact_codes(rng, (rows, k))
    w = exact_codes(rng, (experts, o, k))
    xs = (2.0 ** rng.integers(-2, 0, (rows, k // 128))).astype(np.float32)
    ws = (2.0 ** rng.integers(-2, 0, (experts, o // 128, k // 128))).astype(np.float32)
    out = ops.expert_partial(_t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev), _t(counts, dev),
                             _t(routes, dev), r=rows, top=top)
    exp = omoe.expert_partial(x, xs, w, ws, counts, routes, top)
    np.testing.assert_array_equal(_np(out), exp)


@pytest.mark.parametrize("rows", [257, 1200])
@pytest.mark.parametrize("out_dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("scale_dtype", ["float32", "bfloat16"])
def test_expert_partial_random_dtypes(dev, rows, out_dtype, scale_dtype):
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(41)
    top, experts, o, k = 3, 7, 256, 384
    ids, active, counts, routes, x, xs, w, ws = _expert_case(rng, rows, top, experts, o, k, False,
                                                             exact=False, mult=3)
    sdt = getattr(torch, scale_dtype)
    out = ops.expert_partial(_t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev, sdt),
                             _t(counts, dev), _t(routes, dev), r=rows, top=top,
                             output_dtype=getattr(torch, out_dtype))
    exp = omoe.expert_partial(x, xs, w, ws, counts, routes, top)
    assert rel_fro(_np(out), exp) < (1e-4 if out_dtype == "float32" else 4e-3)


@pytest.mark.parametrize("rows,o", [(33, 128), (600, 256)])
def test_expert_partial_partitions_and_merge(dev, rows, o):
    from akas_amd import ops

    rng = np.random.default_rng(43)
    top, experts, k = 2, 4, 512
    ids, active, counts, routes, x, xs, w, ws = _expert_case(rng, rows, top, experts, o, k, False)
    out = ops.expert_partial(_t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev), _t(counts, dev),
                             _t(routes, dev), r=rows, top=top, partitions=2)
    exp = omoe.expert_partial(x, xs, w, ws, counts, routes, top, partitions=2)
    np.testing.assert_array_equal(_np(out), exp)
    merged = ops.expert_merge(out)
    np.testing.assert_array_equal(_np(merged), omoe.expert_merge(exp))


@pytest.mark.parametrize("rows,maxm", [(33, 64), (600, 128)])
@pytest.mark.parametrize("routed", [False, True])
def test_expert_partial_packed_input(dev, routed, rows, maxm):
    from akas_amd import ops

    rng = np.random.default_rng(47)
    top, experts, o, k = 3, 7, 256, 384
    ids, active, counts, routes, x, xs, w, ws = _expert_case(rng, rows, top, experts, o, k, routed)
    te, tr = omoe.expert_tile_map(counts, rows, top, maxm)
    px, pxs, offs = omoe.expert_pack(x, xs, counts, routes, top, experts, maxm, routed)
    out = ops.expert_partial(_t(px, dev), _t(pxs, dev), _t(w, dev), _t(ws, dev), _t(counts, dev),
                             _t(routes, dev), _t(te, dev), _t(tr, dev), _t(offs, dev), r=rows,
                             top=top, packed_input=True, max_block_m=maxm)
    exp = omoe.expert_partial(x, xs, w, ws, counts, routes, top, routed_input=routed)
    np.testing.assert_array_equal(_np(out), exp)


SWIGLU_CASES = [(1, 3, 7, 128, 256, "float32", "float32"),
                (33, 3, 7, 256, 384, "float32", "float32"),
                (33, 3, 7, 256, 384, "bfloat16", "bfloat16"),
                (33, 3, 7, 256, 384, "float16", "float16"),
                (257, 3, 7, 256, 384, "bfloat16", "bfloat16"),
                (256, 4, 64, 256, 512, "bfloat16", "bfloat16"),
                (2048, 4, 8, 256, 256, "float32", "bfloat16"),
                # >= 128 rows per expert: 256-row DMA tiles
                (1200, 3, 7, 256, 384, "bfloat16", "bfloat16"),
                (900, 2, 5, 384, 256, "float32", "float32")]


@pytest.mark.parametrize("rows,top,experts,o,k,pd,ad", SWIGLU_CASES)
def test_fused_swiglu_matches_separate_chain_bitwise(dev, rows, top, experts, o, k, pd, ad):
    """Fused gate/up/SwiGLU/re-quantization equals expert_partial x2 ->
    swiglu_experts -> quantize bit for bit, on signed codes 32..80 and varying
    scales (the reference's device equivalence recipe, seed 903,
    tests/test_lfm_moe_native.py:295-347)."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(903)
    ids, active = pattern_routes(rows, top, experts, 1)
    counts, routes = omoe.quantized_routes(ids, active, experts)
    x = random_codes(rng, (rows, k))
    w = random_codes(rng, (experts, o, k))
    w2 = random_codes(rng, (experts, o, k))
    xs = rng.uniform(0.0625, 0.25, (rows, k // 128)).astype(np.float32)
    ws = ofp8.bf16_round(rng.uniform(0.0625, 0.25, (experts, o // 128, k // 128)).astype(np.float32))
    ws2 = ofp8.bf16_round(rng.uniform(0.0625, 0.25, (experts, o // 128, k // 128)).astype(np.float32))
    P, A = getattr(torch, pd), getattr(torch, ad)
    args = [_t(x, dev), _t(xs, dev)]
    cnt, rts = _t(counts, dev), _t(routes, dev)
    codes, scales = ops.fp8_expert_swiglu(*args, _t(w, dev), _t(ws, dev), _t(w2, dev), _t(ws2, dev),
                                          cnt, rts, r=rows, top=top, product_dtype=P,
                                          activation_dtype=A)
    gate = ops.expert_partial(*args, _t(w, dev), _t(ws, dev), cnt, rts, r=rows, top=top,
                              output_dtype=P)
    up = ops.expert_partial(*args, _t(w2, dev), _t(ws2, dev), cnt, rts, r=rows, top=top,
                            output_dtype=P)
    act = ops.swiglu_experts(gate, up, output_dtype=A)
    ecodes, escales = ops.quantize(act, top=top)
    live = np.zeros((rows, top), bool)
    for e in range(experts):
        for route in routes[e, :counts[e]]:
            live[route // top, route % top] = True
    np.testing.assert_array_equal(_np(codes)[live], _np(ecodes)[live])
    np.testing.assert_array_equal(_np(scales)[live], _np(escales)[live])
    # and against the CPU oracle: dequantized activations within 1e-2
    oc, osc, _ = omoe.fp8_expert_swiglu(x, xs, w, ws, w2, ws2, counts, routes, top, pd, ad)
    got = ofp8.dequantize_activation(_np(codes), _np(scales))[live]
    exp = ofp8.dequantize_activation(oc, osc)[live]
    assert rel_fro(got, exp) < 1e-2


def _distinct_ids(rng, rows, top, experts):
    """Each row's top ids: distinct experts in random order."""
    return np.argsort(rng.random((rows, experts)), axis=1)[:, :top].astype(np.int32)


# (rows, top, experts, o, k, active, scale dtype): one launch (16-row tiles at
# up to 8 routes per expert, the one-round and the two-stage 32-row tiles,
# rows past a 16-entry boundary, inactive rows, ids outside the bank, one
# expert taking every row, more than 64 and more than 256 experts) and the
# two-launch shapes (4096 routes at 64 per expert, 8192 routes)
ROUTED_SWIGLU_CASES = [(256, 4, 64, 256, 512, "ones", "float32"),
                       (8, 4, 64, 256, 256, "ones", "bfloat16"),
                       (3, 2, 8, 128, 256, None, "float32"),
                       (100, 3, 32, 256, 384, "random", "bfloat16"),
                       (37, 3, 16, 128, 256, "holes", "float32"),
                       (256, 4, 64, 2048, 256, "skew", "float32"),
                       (768, 4, 64, 256, 256, "random", "float32"),
                       (1, 4, 64, 128, 128, None, "float32"),
                       (20, 40, 64, 128, 128, "random", "float32"),
                       (300, 1, 16, 128, 256, None, "bfloat16"),
                       (1024, 4, 64, 256, 256, "ones", "float32"),
                       (64, 8, 128, 256, 256, "random", "bfloat16"),
                       (40, 8, 300, 128, 256, "holes", "bfloat16"),
                       (1024, 8, 256, 128, 128, "random", "float32")]


@pytest.mark.parametrize("rows,top,experts,o,k,act,sdt", ROUTED_SWIGLU_CASES)
def test_routed_fp8_expert_swiglu_is_its_kinds(dev, rows, top, experts, o, k, act, sdt):
    """routed_fp8_expert_swiglu (the route scan inside the gate/up launch)
    equals quantized_routes -> fp8_expert_swiglu: counts and the whole route
    table (-1 padding included) exactly, the codes and scales of every routed
    entry bit for bit.  Run twice into the same buffers."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(rows * 131 + experts)
    ids = _distinct_ids(rng, rows, top, experts)
    active = np.ones(rows, np.int32)
    if act == "random":
        active = (rng.random(rows) < 0.7).astype(np.int32)
    elif act == "holes":
        ids[rng.random((rows, top)) < 0.2] = -1
        ids[0, 0] = experts  # outside the bank: never routed
    elif act == "skew":
        ids = np.stack([np.argsort(rng.random(experts - 1))[: top - 1] + 1 for _ in range(rows)])
        ids = np.concatenate([np.zeros((rows, 1), np.int64), ids], axis=1).astype(np.int32)
    x = random_codes(rng, (rows, k))
    w = random_codes(rng, (experts, o, k))
    w2 = random_codes(rng, (experts, o, k))
    xs = rng.uniform(0.0625, 0.25, (rows, k // 128)).astype(np.float32)
    ws = ofp8.bf16_round(rng.uniform(0.0625, 0.25, (experts, o // 128, k // 128)).astype(np.float32))
    ws2 = ofp8.bf16_round(rng.uniform(0.0625, 0.25, (experts, o // 128, k // 128)).astype(np.float32))
    S = getattr(torch, sdt)
    dids, dact = _t(ids, dev), _t(active, dev)
    data = [_t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev, S), _t(w2, dev), _t(ws2, dev, S)]
    bf = torch.bfloat16
    counts, routes = ops.quantized_routes(dids, dact, experts=experts)
    ecodes, escales = ops.fp8_expert_swiglu(*data, counts, routes, r=rows, top=top,
                                            product_dtype=bf, activation_dtype=bf)
    live = np.zeros((rows, top), bool)
    hc, hr = _np(counts), _np(routes)
    for e in range(experts):
        for route in hr[e, :hc[e]]:
            live[route // top, route % top] = True
    outs = None
    for _ in range(2):
        outs = ops.routed_fp8_expert_swiglu(dids, None if act is None else dact, data[0], data[1],
                                            *data[2:], product_dtype=bf, activation_dtype=bf,
                                            **({} if outs is None else dict(
                                                counts=outs[0], routes=outs[1], out=outs[2],
                                                output_scales=outs[3])))
        np.testing.assert_array_equal(_np(outs[0]), hc)
        np.testing.assert_array_equal(_np(outs[1]), hr)
        np.testing.assert_array_equal(_np(outs[2])[live], _np(ecodes)[live])
        np.testing.assert_array_equal(_np(outs[3])[live], _np(escales)[live])
    assert live.sum() == hc.sum() and hc.sum() > 0


def test_routed_fp8_expert_swiglu_zero_rows(dev):
    """An empty batch writes zero counts and launches no expert work."""
    import torch
    from akas_amd import ops

    E, o, k = 8, 128, 128
    w = torch.zeros((E, o, k), dtype=torch.uint8, device=dev)
    s = torch.ones((E, 1, 1), dtype=torch.float32, device=dev)
    counts = torch.full((E,), 7, dtype=torch.int32, device=dev)
    out = ops.routed_fp8_expert_swiglu(
        torch.zeros((0, 4), dtype=torch.int32, device=dev), None,
        torch.zeros((0, k), dtype=torch.uint8, device=dev),
        torch.zeros((0, 1), dtype=torch.float32, device=dev), w, s, w, s, counts=counts)
    assert out[2].shape == (0, 4, o)
    assert _np(counts).tolist() == [0] * E


def test_routed_fp8_expert_swiglu_lfm2_decode(dev, lfm2_bank):
    """The LFM2 decode layer's gate/up at its real size (T=256, 64 experts,
    top 4, 2048 -> 1536, 768 workgroups three to a CU) from router ids:
    the same tables and codes as the two kinds."""
    import torch
    from akas_amd import ops

    wts, _ = lfm2_bank
    rng = np.random.default_rng(5)
    rows, H = 256, 2048
    x = _t(bf16_normal(rng, (rows, H)), dev, torch.bfloat16)
    logits = _t(rng.normal(0, 1, (rows, 64)).astype(np.float32), dev)
    ids, _ = ops.biased_softmax_router(logits, torch.zeros(64, device=dev), top=4, scale=1.0)
    codes, scales = ops.quantize(x)
    active = torch.ones(rows, dtype=torch.int32, device=dev)
    bf = torch.bfloat16
    counts, routes = ops.quantized_routes(ids, active, experts=64)
    ecodes, escales = ops.fp8_expert_swiglu(codes, scales, wts.w1, wts.s1, wts.w3, wts.s3, counts,
                                            routes, r=rows, top=4, product_dtype=bf,
                                            activation_dtype=bf)
    c2, r2, codes2, scales2 = ops.routed_fp8_expert_swiglu(
        ids, active, codes, scales, wts.w1, wts.s1, wts.w3, wts.s3, product_dtype=bf,
        activation_dtype=bf)
    assert torch.equal(c2, counts) and torch.equal(r2, routes)
    assert torch.equal(codes2, ecodes) and torch.equal(scales2, escales)


@pytest.mark.parametrize("rows", [33, 1200])
def test_fused_swiglu_groups_holding_infinity(dev, rows):
    """Activations that overflow float16 (rows with large activation scales):
    the fused re-quantization still equals the separate chain bit for bit,
    scales inf included, and the finite activations of a group holding inf
    quantize to +-0 (x / inf under IEEE division).  1200 rows take the
    256-row DMA tiles' epilogue, 33 rows the 32-row tiles'."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(907)
    top, experts, o, k = 3, 7, 256, 384
    ids, active = pattern_routes(rows, top, experts, 1)
    counts, routes = omoe.quantized_routes(ids, active, experts)
    x = random_codes(rng, (rows, k))
    w = random_codes(rng, (experts, o, k))
    w2 = random_codes(rng, (experts, o, k))
    xs = rng.uniform(0.0625, 0.25, (rows, k // 128)).astype(np.float32)
    xs[::2] = 8.0  # products of these rows stay finite in float16, their SwiGLU does not
    ws = ofp8.bf16_round(rng.uniform(0.0625, 0.25, (experts, o // 128, k // 128)).astype(np.float32))
    ws2 = ofp8.bf16_round(rng.uniform(0.0625, 0.25, (experts, o // 128, k // 128)).astype(np.float32))
    H = torch.float16
    args = [_t(x, dev), _t(xs, dev)]
    cnt, rts = _t(counts, dev), _t(routes, dev)
    codes, scales = ops.fp8_expert_swiglu(*args, _t(w, dev), _t(ws, dev), _t(w2, dev), _t(ws2, dev),
                                          cnt, rts, r=rows, top=top, product_dtype=H,
                                          activation_dtype=H)
    gate = ops.expert_partial(*args, _t(w, dev), _t(ws, dev), cnt, rts, r=rows, top=top,
                              output_dtype=H)
    up = ops.expert_partial(*args, _t(w2, dev), _t(ws2, dev), cnt, rts, r=rows, top=top,
                            output_dtype=H)
    act = ops.swiglu_experts(gate, up, output_dtype=H)
    ecodes, escales = ops.quantize(act, top=top)
    live = np.zeros((rows, top), bool)
    for e in range(experts):
        for route in routes[e, :counts[e]]:
            live[route // top, route % top] = True
    assert np.isfinite(_np(gate)[live]).all() and np.isfinite(_np(up)[live]).all()
    c, s = _np(codes), _np(scales)
    np.testing.assert_array_equal(c[live], _np(ecodes)[live])
    np.testing.assert_array_equal(s[live], _np(escales)[live])
    a = _np(act)
    in_inf = np.isinf(a).reshape(rows, top, o // 128, 128).any(-1) & live[..., None]
    assert in_inf.sum() >= 4
    assert np.isinf(s[in_inf]).all()
    spread = np.repeat(in_inf, 128, axis=-1) & np.isfinite(a)
    assert spread.sum() >= 64
    assert (c[spread] & 0x7F == 0).all()
    assert (c[np.isinf(a) & live[..., None]] & 0x7F == 126).all()


@pytest.mark.parametrize("rows,top,experts,o,k,pd,ad", SWIGLU_CASES)
def test_fused_swiglu_exact_products_midpoint_band(dev, rows, top, experts, o, k, pd, ad):
    """Exact-product operands (codes {56,64} with sign, scales 0.125; seed 831):
    codes equal the oracle except where the f32 activation interval straddles
    an e4m3 midpoint; scales within 2e-6 (src/akas/ops/moe/validation.py:327-440)."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(831)
    ids, active = pattern_routes(rows, top, experts, 1)
    counts, routes = omoe.quantized_routes(ids, active, experts)
    x, w, w2 = (exact_codes(rng, s) for s in ((rows, k), (experts, o, k), (experts, o, k)))
    xs = np.full((rows, k // 128), 0.125, np.float32)
    ws = np.full((experts, o // 128, k // 128), 0.125, np.float32)
    codes, scales = ops.fp8_expert_swiglu(
        _t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev), _t(w2, dev), _t(ws, dev),
        _t(counts, dev), _t(routes, dev), r=rows, top=top, product_dtype=getattr(torch, pd),
        activation_dtype=getattr(torch, ad))
    oc, osc, norm = omoe.fp8_expert_swiglu(x, xs, w, ws, w2, ws, counts, routes, top, pd, ad)
    live = np.zeros((rows, top), bool)
    for e in range(experts):
        for route in routes[e, :counts[e]]:
            live[route // top, route % top] = True
    ok = omoe.codes_within_midpoint_band(_np(codes), oc, norm)
    assert ok[live].all()
    np.testing.assert_allclose(_np(scales)[live], osc[live], rtol=2e-6, atol=1e-12)


@pytest.mark.parametrize("rows,maxm", [(33, 64), (700, 128)])
@pytest.mark.parametrize("pd,ad", [("float32", "float32"), ("bfloat16", "bfloat16")])
def test_fused_swiglu_packed_in_out(dev, pd, ad, rows, maxm):
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(1035)
    top, experts, o, k = 3, 7, 256, 384
    ids, active = pattern_routes(rows, top, experts, 3)
    counts, routes = omoe.quantized_routes(ids, active, experts)
    x = random_codes(rng, (rows, k))
    w = random_codes(rng, (experts, o, k))
    w2 = random_codes(rng, (experts, o, k))
    xs = rng.uniform(0.0625, 0.25, (rows, k // 128)).astype(np.float32)
    ws = rng.uniform(0.0625, 0.25, (experts, o // 128, k // 128)).astype(np.float32)
    ws2 = rng.uniform(0.0625, 0.25, (experts, o // 128, k // 128)).astype(np.float32)
    te, tr = omoe.expert_tile_map(counts, rows, top, maxm)
    px, pxs, offs = omoe.expert_pack(x, xs, counts, routes, top, experts, maxm)
    P, A = getattr(torch, pd), getattr(torch, ad)
    weights = [_t(w, dev), _t(ws, dev), _t(w2, dev), _t(ws2, dev)]
    cnt, rts, tte, ttr = _t(counts, dev), _t(routes, dev), _t(te, dev), _t(tr, dev)
    pc, psc = ops.fp8_expert_swiglu(_t(px, dev), _t(pxs, dev), *weights, cnt, rts, tte, ttr,
                                    _t(offs, dev), r=rows, top=top, product_dtype=P,
                                    activation_dtype=A, packed_input=True, packed_output=True,
                                    max_block_m=maxm)
    uc, usc = ops.fp8_expert_swiglu(_t(x, dev), _t(xs, dev), *weights, cnt, rts, r=rows, top=top,
                                    product_dtype=P, activation_dtype=A)
    pc, psc, uc, usc = _np(pc), _np(psc), _np(uc), _np(usc)
    for e in range(experts):
        for local, route in enumerate(routes[e, :counts[e]]):
            row, rank = divmod(int(route), top)
            np.testing.assert_array_equal(pc[offs[e] + local], uc[row, rank])
            np.testing.assert_array_equal(psc[offs[e] + local], usc[row, rank])


# ---------------------------------------------------------------------------
# the FP8 paired kinds without re-quantization: expert_swiglu and
# expert_pair_partial (the partitions policy's gate/up producer)
# ---------------------------------------------------------------------------

def _paired_case(rng, rows, top, experts, o, k, mult=1):
    ids, active = pattern_routes(rows, top, experts, mult)
    counts, routes = omoe.quantized_routes(ids, active, experts)
    x = random_codes(rng, (rows, k))
    w = random_codes(rng, (experts, o, k))
    w2 = random_codes(rng, (experts, o, k))
    xs = rng.uniform(0.0625, 0.25, (rows, k // 128)).astype(np.float32)
    ws = ofp8.bf16_round(rng.uniform(0.0625, 0.25, (experts, o // 128, k // 128)).astype(np.float32))
    ws2 = ofp8.bf16_round(rng.uniform(0.0625, 0.25, (experts, o // 128, k // 128)).astype(np.float32))
    live = np.zeros((rows, top), bool)
    for e in range(experts):
        for route in routes[e, :counts[e]]:
            live[route // top, route % top] = True
    return counts, routes, x, xs, w, ws, w2, ws2, live


# (rows, top, experts, o, k, product, activation, output dtype): 32-row,
# 128-row and DMA-fed 256-row tiles
EXPERT_SWIGLU_CASES = [(1, 3, 7, 128, 256, "float32", "float32", "float32"),
                       (33, 3, 7, 256, 384, "bfloat16", "bfloat16", "bfloat16"),
                       (257, 3, 7, 256, 384, "float16", "float32", "float16"),
                       (256, 4, 64, 256, 512, "bfloat16", "bfloat16", "float32"),
                       (1200, 3, 7, 256, 384, "bfloat16", "bfloat16", "bfloat16"),
                       (900, 2, 5, 384, 256, "float32", "float32", "float16")]


@pytest.mark.parametrize("rows,top,experts,o,k,pd,ad,od", EXPERT_SWIGLU_CASES)
def test_expert_swiglu_matches_separate_chain_bitwise(dev, rows, top, experts, o, k, pd, ad, od):
    """The FP8 paired expert_swiglu equals expert_partial x2 ->
    swiglu_experts with the same dtypes, bit for bit, is within 1e-2 of the
    oracle, and (f32 activations and output) quantizes to exactly the fused
    fp8_expert_swiglu codes and scales."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(904)
    counts, routes, x, xs, w, ws, w2, ws2, live = _paired_case(rng, rows, top, experts, o, k)
    P, A, O = (getattr(torch, d) for d in (pd, ad, od))
    args = [_t(x, dev), _t(xs, dev)]
    weights = [_t(w, dev), _t(ws, dev), _t(w2, dev), _t(ws2, dev)]
    cnt, rts = _t(counts, dev), _t(routes, dev)
    out = ops.expert_swiglu(*args, *weights, cnt, rts, r=rows, top=top, product_dtype=P,
                            activation_dtype=A, output_dtype=O)
    gate = ops.expert_partial(*args, weights[0], weights[1], cnt, rts, r=rows, top=top,
                              output_dtype=P)
    up = ops.expert_partial(*args, weights[2], weights[3], cnt, rts, r=rows, top=top,
                            output_dtype=P)
    if ad == od:
        sep = ops.swiglu_experts(gate, up, output_dtype=O)
    else:  # round to the activation dtype, then to the output dtype
        sep = ops.swiglu_experts(gate, up, output_dtype=A).to(O)
    np.testing.assert_array_equal(_np(out)[live], _np(sep)[live])
    exp = omoe.expert_swiglu(x, xs, w, ws, w2, ws2, counts, routes, top, pd, ad, od)
    assert rel_fro(_np(out)[live], exp[live]) < 1e-2
    if ad == od == "float32":
        codes, scales = ops.fp8_expert_swiglu(*args, *weights, cnt, rts, r=rows, top=top,
                                              product_dtype=P, activation_dtype=A)
        qc, qs = ops.quantize(out, top=top)
        np.testing.assert_array_equal(_np(qc)[live], _np(codes)[live])
        np.testing.assert_array_equal(_np(qs)[live], _np(scales)[live])


@pytest.mark.parametrize("rows,maxm", [(33, 64), (700, 128)])
def test_expert_swiglu_packed_in_out(dev, rows, maxm):
    """Packed input and output: each packed row holds the unpacked result of
    its (row, rank)."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(1036)
    top, experts, o, k = 3, 7, 256, 384
    counts, routes, x, xs, w, ws, w2, ws2, live = _paired_case(rng, rows, top, experts, o, k, 3)
    te, tr = omoe.expert_tile_map(counts, rows, top, maxm)
    px, pxs, offs = omoe.expert_pack(x, xs, counts, routes, top, experts, maxm)
    bf = torch.bfloat16
    weights = [_t(w, dev), _t(ws, dev), _t(w2, dev), _t(ws2, dev)]
    cnt, rts = _t(counts, dev), _t(routes, dev)
    packed = ops.expert_swiglu(_t(px, dev), _t(pxs, dev), *weights, cnt, rts, _t(te, dev),
                               _t(tr, dev), _t(offs, dev), r=rows, top=top, product_dtype=bf,
                               activation_dtype=bf, output_dtype=bf, packed_input=True,
                               packed_output=True, max_block_m=maxm)
    flat = ops.expert_swiglu(_t(x, dev), _t(xs, dev), *weights, cnt, rts, r=rows, top=top,
                             product_dtype=bf, activation_dtype=bf, output_dtype=bf)
    packed, flat = _np(packed), _np(flat)
    for e in range(experts):
        for local, route in enumerate(routes[e, :counts[e]]):
            row, rank = divmod(int(route), top)
            np.testing.assert_array_equal(packed[offs[e] + local], flat[row, rank])


# (rows, top, experts, o, k, partitions): r = 1 with two partitions (the
# reference's seed policy for one-row decode), 32-row, 128-row and DMA tiles
PAIR_PARTIAL_CASES = [(1, 4, 64, 256, 2048, 2), (1, 2, 5, 128, 512, 4), (33, 3, 7, 256, 384, 3),
                      (257, 3, 7, 256, 512, 2), (1200, 3, 7, 256, 512, 2),
                      (900, 2, 5, 384, 256, 1)]


@pytest.mark.parametrize("rows,top,experts,o,k,parts", PAIR_PARTIAL_CASES)
def test_expert_pair_partial_exact(dev, rows, top, experts, o, k, parts):
    """Exact products (codes {56, 64} with sign, binary scales; the up
    weights are the flipped gate weights, as in the reference's
    paired_partial_validation): gate and up partials equal the oracle bit
    for bit with float32 and with bfloat16 weight scales; unrouted entries
    are untouched."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(905)
    ids, active = pattern_routes(rows, top, experts, 1)
    counts, routes = omoe.quantized_routes(ids, active, experts)
    x, w = exact_codes(rng, (rows, k)), exact_codes(rng, (experts, o, k))
    xs = (2.0 ** rng.integers(-4, 2, (rows, k // 128))).astype(np.float32)
    ws = (2.0 ** rng.integers(-4, 2, (experts, o // 128, k // 128))).astype(np.float32)
    w2, ws2 = np.flip(w, axis=-2).copy(), np.flip(ws, axis=-1).copy()
    eg, eu = omoe.expert_pair_partial(x, xs, w, ws, w2, ws2, counts, routes, top, parts)
    for sdt in (torch.float32, torch.bfloat16):  # binary scales are exact in bf16
        gate, up = ops.expert_pair_partial(_t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev, sdt),
                                           _t(w2, dev), _t(ws2, dev, sdt), _t(counts, dev),
                                           _t(routes, dev), r=rows, top=top, partitions=parts)
        np.testing.assert_array_equal(_np(gate), eg)
        np.testing.assert_array_equal(_np(up), eu)


@pytest.mark.parametrize("rows,parts", [(1, 2), (40, 3), (1200, 2)])
def test_expert_pair_partial_then_swiglu_policy(dev, rows, parts):
    """The reference's partitions policy for fp8_expert_swiglu
    (src/akas/ops/moe/definition.py:796-948): expert_pair_partial ->
    swiglu_experts (partitions summed in f32) -> quantize.  Gate and up are
    each bit-identical to expert_partial with the same partitions, and the
    chain's codes match the oracle's fused kind within the midpoint band."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(906)
    top, experts, o, k = 4, 8, 256, 768
    counts, routes, x, xs, w, ws, w2, ws2, live = _paired_case(rng, rows, top, experts, o, k)
    args = [_t(x, dev), _t(xs, dev)]
    cnt, rts = _t(counts, dev), _t(routes, dev)
    gate, up = ops.expert_pair_partial(*args, _t(w, dev), _t(ws, dev), _t(w2, dev), _t(ws2, dev),
                                       cnt, rts, r=rows, top=top, partitions=parts)
    g1 = ops.expert_partial(*args, _t(w, dev), _t(ws, dev), cnt, rts, r=rows, top=top,
                            partitions=parts)
    u1 = ops.expert_partial(*args, _t(w2, dev), _t(ws2, dev), cnt, rts, r=rows, top=top,
                            partitions=parts)
    g_np, u_np = _np(gate), _np(up)
    if parts == 1:
        g_np, u_np = g_np[:, :, 0], u_np[:, :, 0]
    np.testing.assert_array_equal(g_np[live], _np(g1)[live])
    np.testing.assert_array_equal(u_np[live], _np(u1)[live])
    act = ops.swiglu_experts(gate, up, output_dtype=torch.float32)
    codes, scales = ops.quantize(act, top=top)
    oc, osc, norm = omoe.fp8_expert_swiglu(x, xs, w, ws, w2, ws2, counts, routes, top)
    got = ofp8.dequantize_activation(_np(codes), _np(scales))[live]
    assert rel_fro(got, ofp8.dequantize_activation(oc, osc)[live]) < 1e-2


# ---------------------------------------------------------------------------
# elementwise: swiglu, combine
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("parts", [1, 2])
def test_swiglu_experts(dev, parts):
    from akas_amd import ops

    rng = np.random.default_rng(5)
    shape = (9, 3, parts, 256) if parts > 1 else (9, 3, 256)
    g = rng.normal(0, 3, shape).astype(np.float32)
    u = rng.normal(0, 3, shape).astype(np.float32)
    out = ops.swiglu_experts(_t(g, dev), _t(u, dev), round_inputs=True, round_dtype="bfloat16")
    exp = omoe.swiglu_experts(g, u, round_inputs=True, round_dtype="bfloat16")
    np.testing.assert_allclose(_np(out), exp, rtol=2e-6, atol=1e-7)


def test_swiglu_wide_range_accuracy(dev):
    """g / (1 + exp(-g)) * u against a float64 evaluation over g in
    [-104, 88] (exp(-g) from far above overflow to far below underflow),
    within the reference's 2e-6 relative code band."""
    from akas_amd import ops

    rng = np.random.default_rng(11)
    g = np.concatenate([np.linspace(-104, 88, 96 * 256), rng.normal(0, 8, 32 * 256)]).astype(np.float32)
    u = rng.uniform(0.5, 2.0, g.size).astype(np.float32) * rng.choice([-1, 1], g.size).astype(np.float32)
    shape = (g.size // 256, 1, 256)
    out = _np(ops.swiglu_experts(_t(g.reshape(shape), dev), _t(u.reshape(shape), dev))).ravel()
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    with np.errstate(over="ignore"):
        exact = g64 / (1.0 + np.exp(-g64)) * u64
    np.testing.assert_allclose(out, exact, rtol=2e-6, atol=1e-30)


@pytest.mark.parametrize("in_dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("top,c", [(4, 2048), (6, 2048), (1, 24), (3, 2040)])
def test_routed_combine(dev, in_dtype, top, c):
    """Eight-column vector kernel (c % 8 == 0; top 6 leaves a partial batch
    of ranks) and the generic kernel (c = 2040), inactive rows zero."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(6 + top)
    rows = 33
    e = rng.normal(0, 1, (rows, top, c)).astype(np.float32)
    if in_dtype != "float32":
        e = ofp8.round_to(e, in_dtype)
    w = rng.uniform(0, 1, (rows, top)).astype(np.float32)
    active = np.ones(rows, np.int32)
    active[-1] = 0
    out = ops.routed_combine(_t(e, dev, getattr(torch, in_dtype)), _t(w, dev), _t(active, dev))
    np.testing.assert_allclose(_np(out), omoe.routed_combine(e, w, active), rtol=1e-5, atol=1e-6)


COMBINE_CASES = [
    # rows, top, experts, o, k, routed, packed, max_block_m, contribution dtype
    (256, 4, 64, 512, 256, True, False, 64, "bfloat16"),   # 32-row tiles (decode)
    (256, 4, 64, 512, 256, True, False, 64, "float32"),
    (1, 4, 64, 256, 256, True, False, 64, "float32"),
    (700, 4, 16, 384, 256, True, False, 64, "float16"),    # 128-row tiles
    (1500, 2, 6, 512, 384, True, False, 64, "bfloat16"),   # 256-row DMA tiles
    (1024, 4, 8, 512, 256, False, True, 128, "bfloat16"),  # packed input, DMA tiles
    (1024, 4, 8, 512, 256, True, True, 128, "float32"),    # packed routed input
    (600, 3, 5, 256, 256, False, True, 128, "float32")]


def _combine_inputs(dev, rng, rows, top, experts, o, k, routed, packed, maxm):
    import torch
    from akas_amd import ops

    ids, active, counts, routes, x, xs, w, ws = _expert_case(rng, rows, top, experts, o, k, routed,
                                                             exact=False, mult=3)
    cw = rng.uniform(0, 1, (rows, top)).astype(np.float32)
    d = dict(ids=_t(ids, dev), active=_t(active, dev), counts=_t(counts, dev),
             routes=_t(routes, dev), w=_t(w, dev), ws=_t(ws, dev, torch.bfloat16), cw=_t(cw, dev),
             offsets=None, x=_t(x, dev), xs=_t(xs, dev))
    if packed:
        d["x"], d["xs"], d["offsets"] = ops.expert_pack(d["x"], d["xs"], d["counts"], d["routes"],
                                                        None, None, top=top, max_block_m=maxm,
                                                        routed_input=routed)
    return d, (ids, active, counts, routes, x, xs, w, ws, cw)


def _routed_mask(ids, active, experts):
    return (active[:, None] != 0) & (ids >= 0) & (ids < experts)


@pytest.mark.parametrize("rows,top,experts,o,k,routed,packed,maxm,cdt", COMBINE_CASES)
def test_expert_combine_matches_partial_then_combine(dev, rows, top, experts, o, k, routed, packed,
                                                     maxm, cdt):
    """expert_combine (down projection with the combine folded into its
    epilogue) against expert_partial -> routed_combine on the device: the
    combined rows and every routed contribution bit for bit, on every tile
    shape (32-row, 128-row, DMA-fed 256-row; packed input); the arrival
    counters are zero again after each of two calls."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(53 + rows)
    d, host = _combine_inputs(dev, rng, rows, top, experts, o, k, routed, packed, maxm)
    ct = getattr(torch, cdt)
    common = dict(r=rows, top=top, max_block_m=maxm, routed_input=routed and not packed,
                  packed_input=packed)
    ref_c = ops.expert_partial(d["x"], d["xs"], d["w"], d["ws"], d["counts"], d["routes"], None,
                               None, d["offsets"], output_dtype=ct, **common)
    ref = ops.routed_combine(ref_c, d["cw"], d["active"])
    arrivals = torch.zeros(rows * (o // 128), dtype=torch.int32, device=dev)
    for _ in range(2):
        out, contrib = ops.expert_combine(d["x"], d["xs"], d["w"], d["ws"], d["counts"], d["routes"],
                                          d["ids"], d["cw"], d["active"], d["offsets"],
                                          contribution_dtype=ct, arrivals=arrivals, **common)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        mask = torch.from_numpy(_routed_mask(host[0], host[1], experts)).to(dev)
        assert torch.equal(contrib[mask], ref_c[mask])
        assert not arrivals.any()


def test_expert_combine_dead_ranks_and_inactive_rows(dev):
    """Rows whose ids leave [0, experts) keep only their live ranks, a row
    with no live rank and an inactive row are zero; exact products, so the
    contributions equal the oracle's and the fold is within an f32 rounding
    per rank of its float32 loop."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(59)
    rows, top, experts, o, k = 300, 4, 16, 256, 256
    ids, active = pattern_routes(rows, top, experts, 3)
    ids[3, 2] = 99
    ids[10, :] = -1
    active[20] = 0
    x = exact_codes(rng, (rows, k))
    xs = (2.0 ** rng.integers(-4, 1, (rows, k // 128))).astype(np.float32)
    w = exact_codes(rng, (experts, o, k))
    ws = (2.0 ** rng.integers(-4, 1, (experts, o // 128, k // 128))).astype(np.float32)
    cw = rng.uniform(0, 1, (rows, top)).astype(np.float32)
    counts, routes = ops.quantized_routes(_t(ids, dev), _t(active, dev), experts=experts)
    out, contrib = ops.expert_combine(_t(x, dev), _t(xs, dev), _t(w, dev), _t(ws, dev), counts,
                                      routes, _t(ids, dev), _t(cw, dev), _t(active, dev), r=rows,
                                      top=top, contribution_dtype=torch.float32)
    hc, hr = omoe.quantized_routes(ids, active, experts)
    exp, exp_c = omoe.expert_combine(x, xs, w, ws, hc, hr, ids, cw, active, top)
    mask = _routed_mask(ids, active, experts)
    np.testing.assert_array_equal(_np(contrib)[mask], exp_c[mask])
    got = _np(out)
    # per rank the device rounds once (fma) and the oracle twice: at most
    # 2 * top half-ulps of the running magnitude sum|c * w|
    live = np.where(mask[:, :, None], np.abs(exp_c.astype(np.float64)), 0.0)
    bound = 2 * top * 2.0 ** -24 * (live * cw[:, :, None]).sum(1)
    assert (np.abs(got.astype(np.float64) - exp) <= bound).all()
    assert not got[10].any() and not got[20].any()


def test_expert_combine_graph_replays(dev):
    """expert_combine captured in a HIP graph: three replays, each after eager
    calls that change the output buffer, equal the eager result."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(61)
    rows, top, experts, o, k = 256, 4, 64, 512, 256
    d, _ = _combine_inputs(dev, rng, rows, top, experts, o, k, True, False, 64)
    args = (d["x"], d["xs"], d["w"], d["ws"], d["counts"], d["routes"], d["ids"], d["cw"],
            d["active"])
    kw = dict(r=rows, top=top, routed_input=True, contribution_dtype=torch.bfloat16)
    eager, _ = ops.expert_combine(*args, **kw)
    out = torch.empty_like(eager)
    ops.expert_combine(*args, out=out, **kw)  # warm the stream's arrival buffer
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.expert_combine(*args, out=out, **kw)
    for _ in range(3):
        out.fill_(7.0)
        ops.expert_combine(*args, **kw)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


# ---------------------------------------------------------------------------
# the whole layer
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("rows,packed,fused", [(256, False, True), (256, False, False),
                                               (1000, True, True), (1, False, True)])
def test_routed_moe_layer(dev, rows, packed, fused):
    import torch
    from akas_amd import moe

    rng = np.random.default_rng(0)
    H, F, E, top = 512, 256, 16, 4
    x = bf16_normal(rng, (rows, H))
    logits = rng.normal(0, 1, (rows, E)).astype(np.float32)
    bank = {}
    for name, shape in (("w1", (E, F, H)), ("w3", (E, F, H)), ("w2", (E, H, F))):
        bank[name] = ofp8.quantize_weight_blocks(rng.normal(0, 0.05, shape).astype(np.float32))
    wts = moe.ExpertWeights(*(_t(a, dev) for n in ("w1", "w3", "w2") for a in bank[n]))
    out = moe.routed_moe(_t(x, dev, torch.bfloat16), _t(logits, dev), None, wts, top=top,
                         packed=packed, fused_swiglu=fused)
    exp, _, _ = omoe.moe_layer(x, logits, np.zeros(E, np.float32), *bank["w1"], *bank["w3"],
                               *bank["w2"], top)
    assert rel_fro(_np(out), exp) < 1e-2


@pytest.mark.parametrize("rows,parts", [(1, 2), (64, 2), (200, 4)])
def test_routed_moe_layer_partitions_policy(dev, rows, parts):
    """The block under the reference's partitions policy (gate/up through
    expert_pair_partial -> swiglu_experts -> quantize, down through
    expert_partial(partitions) -> expert_merge) against the layer equation;
    with partition_maximum_rows below the batch the policy is off and the
    result is the plain block's, bit for bit."""
    import torch
    from akas_amd import moe

    rng = np.random.default_rng(12)
    H, F, E, top = 512, 512, 16, 4  # both depths split into 4 partitions
    x = bf16_normal(rng, (rows, H))
    logits = rng.normal(0, 1, (rows, E)).astype(np.float32)
    bank = {}
    for name, shape in (("w1", (E, F, H)), ("w3", (E, F, H)), ("w2", (E, H, F))):
        bank[name] = ofp8.quantize_weight_blocks(rng.normal(0, 0.05, shape).astype(np.float32))
    wts = moe.ExpertWeights(*(_t(a, dev) for n in ("w1", "w3", "w2") for a in bank[n]))
    xt, lt = _t(x, dev, torch.bfloat16), _t(logits, dev)
    out = moe.routed_moe(xt, lt, None, wts, top=top, partitions=parts)
    exp, _, _ = omoe.moe_layer(x, logits, np.zeros(E, np.float32), *bank["w1"], *bank["w3"],
                               *bank["w2"], top)
    assert rel_fro(_np(out), exp) < 1e-2
    off = moe.routed_moe(xt, lt, None, wts, top=top, partitions=parts,
                         partition_maximum_rows=rows - 1)
    plain = moe.routed_moe(xt, lt, None, wts, top=top)
    np.testing.assert_array_equal(_np(off), _np(plain))
    # Packed expert calls are not partitioned (the rewrite splits compact
    # calls only, src/akas/ops/moe/definition.py:796-815): a plan combining
    # both, as the reference's sm_90a seed does, runs the packed block.
    packed = moe.routed_moe(xt, lt, None, wts, top=top, partitions=parts, packed=True)
    np.testing.assert_array_equal(
        _np(packed), _np(moe.routed_moe(xt, lt, None, wts, top=top, packed=True)))
    # The seed packs from packed_minimum_rows rows on (definition.py:951-965):
    # a smaller batch runs the compact block, with its partitions.
    seed = moe.routed_moe(xt, lt, None, wts, top=top, partitions=parts, packed=True,
                          packed_minimum_rows=rows + 1)
    np.testing.assert_array_equal(_np(seed), _np(out))
    with pytest.raises(ValueError):
        moe.routed_moe(xt, lt, None, wts, top=top, packed=True, packed_minimum_rows=0)


@pytest.mark.parametrize("rows,packed,policy", [(8, False, "float32"), (200, False, "bfloat16"),
                                                (300, True, "bfloat16")])
def test_routed_moe_separate_activation_quantize(dev, rows, packed, policy):
    """The separate-quantize rewrite (expert_swiglu stores the activations
    unquantized, quantize follows; src/akas/ops/moe/definition.py:1056-1120),
    and the fused quantize's minimum rows below which that form runs
    (:1194-1200), give the fused block's result bit for bit."""
    import torch
    from akas_amd import moe

    rng = np.random.default_rng(rows + 5)
    H, F, E, top = 256, 384, 16, 4
    x = bf16_normal(rng, (rows, H))
    logits = rng.normal(0, 1, (rows, E)).astype(np.float32)
    bank = {}
    for name, shape in (("w1", (E, F, H)), ("w3", (E, F, H)), ("w2", (E, H, F))):
        bank[name] = ofp8.quantize_weight_blocks(rng.normal(0, 0.05, shape).astype(np.float32))
    wts = moe.ExpertWeights(*(_t(a, dev) for n in ("w1", "w3", "w2") for a in bank[n]))
    xt, lt = _t(x, dev, torch.bfloat16), _t(logits, dev)
    dt = getattr(torch, policy)
    kw = dict(top=top, packed=packed, max_block_m=128 if packed else 64, product_dtype=dt,
              activation_dtype=dt, contribution_dtype=dt)
    fused = _np(moe.routed_moe(xt, lt, None, wts, **kw))
    separate = _np(moe.routed_moe(xt, lt, None, wts, separate_activation_quantize=True, **kw))
    below = _np(moe.routed_moe(xt, lt, None, wts, fused_quantize_minimum_rows=rows + 1, **kw))
    above = _np(moe.routed_moe(xt, lt, None, wts, fused_quantize_minimum_rows=rows, **kw))
    np.testing.assert_array_equal(separate, fused)
    np.testing.assert_array_equal(below, fused)
    np.testing.assert_array_equal(above, fused)
    with pytest.raises(ValueError):
        moe.routed_moe(xt, lt, None, wts, top=top, fused_quantize_minimum_rows=0)
    with pytest.raises(ValueError):
        moe.routed_moe(xt, lt, None, wts, top=top, fused_swiglu=False,
                       fused_quantize_minimum_rows=4)
    # the rewrite's row tile: checked as the reference checks it, no effect
    tiled = _np(moe.routed_moe(xt, lt, None, wts, block_m=32, **kw))
    np.testing.assert_array_equal(tiled, fused)
    with pytest.raises(ValueError):
        moe.routed_moe(xt, lt, None, wts, top=top, block_m=48)
    with pytest.raises(ValueError):
        moe.routed_moe(xt, lt, None, wts, top=top, block_m=128, max_block_m=64)


@pytest.mark.parametrize("rows,packed,fused,policy", [
    (256, False, True, "bfloat16"), (256, False, False, "bfloat16"),
    (1000, True, True, "bfloat16"), (300, False, True, "float32")])
def test_routed_moe_layer_sigmoid_router_policies(dev, rows, packed, fused, policy):
    """The LFM2 block's sigmoid+bias router (``src/akas/ops/moe/kernel.py:154-203``)
    with a nonzero bias and route scale, bf16 intermediate policies
    (``src/akas/ops/moe/definition.py:677-793``) and inactive rows, against
    the layer equation of ``tests/support/native_fp8_reference.py:116-144``."""
    import torch
    from akas_amd import moe

    rng = np.random.default_rng(7)
    H, F, E, top = 512, 384, 32, 4
    x = bf16_normal(rng, (rows, H))
    logits = rng.normal(0, 1, (rows, E)).astype(np.float32)
    bias = rng.normal(0, 0.5, E).astype(np.float32)
    active = (rng.random(rows) > 0.1).astype(np.int32)
    bank = {}
    for name, shape in (("w1", (E, F, H)), ("w3", (E, F, H)), ("w2", (E, H, F))):
        bank[name] = ofp8.quantize_weight_blocks(rng.normal(0, 0.05, shape).astype(np.float32))
    wts = moe.ExpertWeights(*(_t(a, dev) for n in ("w1", "w3", "w2") for a in bank[n]))
    dt = getattr(torch, policy)
    out = moe.routed_moe(_t(x, dev, torch.bfloat16), _t(logits, dev), _t(bias, dev), wts,
                         top=top, active=_t(active, dev), router="biased_router", scale=2.5,
                         normalize=True, packed=packed, fused_swiglu=fused,
                         product_dtype=dt, activation_dtype=dt, contribution_dtype=dt)
    exp, ids, _ = omoe.moe_layer(x, logits, bias, *bank["w1"], *bank["w3"], *bank["w2"], top,
                                 router="sigmoid", scale=2.5, normalize=True, active=active,
                                 activation_dtype=policy, contribution_dtype=policy)
    got = _np(out)
    assert np.all(got[active == 0] == 0)
    assert rel_fro(got, exp) < 1e-2


# ---------------------------------------------------------------------------
# the layer at the LFM2-MoE dimensions (H=2048, F=1536, E=64, top 4)
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def lfm2_bank(dev):
    """Expert banks at the benchmark's dimensions, block-quantized on the GPU
    (N(0, 0.02) weights) with host copies of the codes and scales for the
    oracle."""
    import torch
    from akas_amd import moe, ops

    E, H, F = 64, 2048, 1536
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    dev_bank, host_bank = [], []
    for n, k in ((F, H), (F, H), (H, F)):
        codes, scales = [], []
        for _ in range(E):
            w = torch.randn((n, k), generator=g, device=dev, dtype=torch.float32) * 0.02
            c, s = ops.quantize_weight_blocks(w)
            codes.append(c)
            scales.append(s)
        c, s = torch.stack(codes), torch.stack(scales)
        dev_bank += [c, s]
        host_bank += [_np(c), _np(s)]
    return moe.ExpertWeights(*dev_bank), host_bank


@pytest.mark.parametrize("rows,packed,zipf", [(256, False, False), (2048, True, True)])
def test_routed_moe_layer_lfm2_dims(dev, lfm2_bank, rows, packed, zipf):
    """Decode (32-row expert tiles) and prefill (packed, DMA-fed 256-row
    tiles, Zipf-skewed routing) at the real layer size with the benchmark's
    bf16 intermediate policies, against the layer equation."""
    import torch
    from akas_amd import moe

    wts, host = lfm2_bank
    E, H = 64, 2048
    rng = np.random.default_rng(3)
    x = bf16_normal(rng, (rows, H))
    logits = rng.normal(0, 1, (rows, E)).astype(np.float32)
    if zipf:
        logits += (-1.1 * np.log1p(rng.permutation(E))).astype(np.float32)[None, :]
    bf = torch.bfloat16
    out = moe.routed_moe(_t(x, dev, bf), _t(logits, dev), None, wts, top=4, packed=packed,
                         max_block_m=128 if packed else 64, product_dtype=bf,
                         activation_dtype=bf, contribution_dtype=bf)
    exp, _, _ = omoe.moe_layer(x, logits, np.zeros(E, np.float32), *host, 4,
                               activation_dtype="bfloat16", contribution_dtype="bfloat16")
    assert rel_fro(_np(out), exp) < 1e-2
    # the combine folded into the down epilogue equals the separate combine
    fused = moe.routed_moe(_t(x, dev, bf), _t(logits, dev), None, wts, top=4, packed=packed,
                           max_block_m=128 if packed else 64, product_dtype=bf,
                           activation_dtype=bf, contribution_dtype=bf, fused_combine=True)
    assert torch.equal(out, fused)


def test_routed_moe_layer_zipf_prefill_full_size(dev, lfm2_bank):
    """The skewed prefill batch of the benchmark: T = 16384 tokens, Zipf(1.1)
    per-expert logit offsets, packed 128-aligned experts on the DMA-fed
    256-row tiles (the top expert holds about 14.6k routed rows, 57 tiles),
    and the unpacked policy bit-identical to it.
    The whole batch runs on the device; the routes are compared in full and
    the layer output on a token sample holding, for every live expert, its
    first two and last two routed tokens, plus every token of the largest
    expert's last 256-row tile.  Tokens are independent in the layer
    equation, so the oracle runs on the sample alone."""
    import torch
    from akas_amd import moe

    wts, host = lfm2_bank
    E, H, T, top = 64, 2048, 16384, 4
    rng = np.random.default_rng(0)
    x = bf16_normal(rng, (T, H))
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    logits += (-1.1 * np.log1p(rng.permutation(E))).astype(np.float32)[None, :]
    bf = torch.bfloat16
    out, routing = moe.routed_moe(_t(x, dev, bf), _t(logits, dev), None, wts, top=top,
                                  packed=True, max_block_m=128, product_dtype=bf,
                                  activation_dtype=bf, contribution_dtype=bf,
                                  return_routing=True)
    got = _np(out)
    ids, _ = omoe.biased_softmax_router(logits, np.zeros(E, np.float32), top)
    np.testing.assert_array_equal(_np(routing["ids"]), ids)
    counts, routes = omoe.quantized_routes(ids, np.ones(T, np.int32), E)
    np.testing.assert_array_equal(_np(routing["counts"]), counts)
    np.testing.assert_array_equal(_np(routing["routes"]), routes)
    big = int(np.argmax(counts))
    assert counts[big] > 50 * 256  # the skew puts many tiles on one expert
    sample = []
    for e in np.nonzero(counts)[0]:
        owners = routes[e, :counts[e]] // top
        sample += [owners[:2], owners[-2:]]
    owners = routes[big, :counts[big]] // top
    sample.append(owners[256 * ((counts[big] - 1) // 256):])
    rows = np.unique(np.concatenate(sample))
    exp, _, _ = omoe.moe_layer(x[rows], logits[rows], np.zeros(E, np.float32), *host, top,
                               activation_dtype="bfloat16", contribution_dtype="bfloat16")
    assert rel_fro(got[rows], exp) < 1e-2
    # the rows outside the sample are finite and as large as the sampled ones
    assert np.isfinite(got).all()
    norms = np.linalg.norm(got, axis=1)
    assert 0.5 < np.median(norms) / np.median(np.linalg.norm(exp, axis=1)) < 2.0
    # unpacked (the benchmark's policy: rows gathered through the route
    # table by the grouped kernels) gives the same bits on every token
    flat = moe.routed_moe(_t(x, dev, bf), _t(logits, dev), None, wts, top=top, packed=False,
                          max_block_m=64, product_dtype=bf, activation_dtype=bf,
                          contribution_dtype=bf)
    np.testing.assert_array_equal(_np(flat), got)


# ---------------------------------------------------------------------------
# the Qwen3.5 block-fp8 variant: moe_combine and the shared-expert block
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("in_dtype,shared_dtype", [("float32", "float32"), ("bfloat16", "float32"),
                                                    ("float16", "bfloat16")])
@pytest.mark.parametrize("rows,top,c", [(5, 8, 2048), (300, 8, 512), (1, 2, 8)])
def test_moe_combine(dev, in_dtype, shared_dtype, rows, top, c):
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(rows + top + c)
    e = rng.normal(0, 1, (rows, top, c)).astype(np.float32)
    w = np.abs(rng.normal(0, 1, (rows, top))).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    sh = rng.normal(0, 1, (rows, c)).astype(np.float32)
    g = rng.normal(0, 2, (rows, 1)).astype(np.float32)
    et = _t(e, dev, getattr(torch, in_dtype))
    st = _t(sh, dev, getattr(torch, shared_dtype))
    out = ops.moe_combine(et, _t(w, dev), st, _t(g, dev))
    exp = omoe.moe_combine(_np(et), w, _np(st), g)
    np.testing.assert_allclose(_np(out), exp, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("shared_dtype,gate_dtype", [("float32", "bfloat16"), ("bfloat16", "float32"),
                                                      ("float16", "float16")])
def test_moe_combine_shared_row_alignment(dev, shared_dtype, gate_dtype):
    """The shared row is read as 16-byte loads where it is 16-byte aligned and
    element by element where it is not (a contiguous view one element into
    its storage): both give the oracle's result, bit for bit the same."""
    import torch
    from akas_amd import ops

    rows, top, c = 37, 8, 512
    rng = np.random.default_rng(61)
    e = _t(rng.normal(0, 1, (rows, top, c)).astype(np.float32), dev, torch.bfloat16)
    w = np.abs(rng.normal(0, 1, (rows, top))).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    sh = rng.normal(0, 1, (rows, c)).astype(np.float32)
    g = _t(rng.normal(0, 2, rows).astype(np.float32), dev, getattr(torch, gate_dtype))
    sdt = getattr(torch, shared_dtype)
    aligned = _t(sh, dev, sdt)
    store = torch.empty(rows * c + 1, dtype=sdt, device=dev)
    store[1:] = aligned.reshape(-1)
    unaligned = store[1:].view(rows, c)
    assert unaligned.data_ptr() % 16 != 0 and unaligned.is_contiguous()
    a = ops.moe_combine(e, _t(w, dev), aligned, g)
    b = ops.moe_combine(e, _t(w, dev), unaligned, g)
    exp = omoe.moe_combine(_np(e), w, _np(aligned), _np(g.float()))
    np.testing.assert_array_equal(_np(a), _np(b))
    np.testing.assert_allclose(_np(a), exp, rtol=1e-5, atol=1e-6)


def _device_bank(dev, seed, shapes, std):
    """Block-quantized N(0, std) weights generated on the GPU: device codes
    and scales plus host copies for the oracle."""
    import torch
    from akas_amd import ops

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    dev_bank, host_bank = {}, {}
    for name, shape in shapes.items():
        w = torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * std
        c, s = ops.quantize_weight_blocks(w)
        del w
        dev_bank[name] = (c, s)
        host_bank[name] = (_np(c), _np(s))
    return dev_bank, host_bank


@pytest.mark.parametrize("rows,E,H,F,packed", [(6, 32, 256, 128, False), (300, 32, 256, 128, False),
                                              (1024, 16, 512, 256, True),
                                              (4, 256, 2048, 512, False)])
def test_shared_expert_moe_block(dev, rows, E, H, F, packed):
    """The Qwen3.5 block (256 experts, top 8, o=512 at its real size for a
    decode batch) against the block equation."""
    import torch
    from akas_amd import moe

    rng = np.random.default_rng(rows + E)
    top = 8
    dbank, bank = _device_bank(dev, rows + E, {
        "w1": (E, F, H), "w3": (E, F, H), "w2": (E, H, F),
        "sw1": (F, H), "sw3": (F, H), "sw2": (H, F)}, 0.02 if H == 2048 else 0.05)
    x = bf16_normal(rng, (rows, H))
    logits = rng.normal(0, 1, (rows, E)).astype(np.float32)
    gate = rng.normal(0, 1.5, rows).astype(np.float32)
    wts = moe.ExpertWeights(*(a for n in ("w1", "w3", "w2") for a in dbank[n]))
    shared = moe.SharedExpert(*(a for n in ("sw1", "sw3", "sw2") for a in dbank[n]))
    out = moe.shared_expert_moe(_t(x, dev, torch.bfloat16), _t(logits, dev), _t(gate, dev), wts,
                                shared, top=top, packed=packed, max_block_m=128 if packed else 64)
    exp = omoe.shared_expert_moe_layer(x, logits, gate, *bank["w1"], *bank["w3"], *bank["w2"],
                                       *bank["sw1"], *bank["sw3"], *bank["sw2"], top)
    assert rel_fro(_np(out), exp) < 1e-2


# ---------------------------------------------------------------------------
# block-fp8 decode variant kinds: moe_groups / fp8_experts
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case", ["router64x8", "duplicates", "single", "wide"])
def test_moe_groups(dev, case):
    """Bit-exact group tables: distinct top-8 ids over 256 experts, repeated
    ids inside and across rows (the last rank wins), one id, and 1100 rows
    (route rows longer than a workgroup's stride)."""
    from akas_amd import ops

    rng = np.random.default_rng(71)
    if case == "router64x8":
        ids = np.argsort(-rng.normal(0, 1, (64, 256)), axis=1, kind="stable")[:, :8]
    elif case == "duplicates":
        ids = rng.integers(0, 6, (33, 4))
        ids[0] = [3, 3, 1, 3]
    elif case == "single":
        ids = np.array([[5]])
    else:
        ids = rng.integers(0, 40, (1100, 2))
    ids = ids.astype(np.int32)
    experts, routes = ops.moe_groups(_t(ids, dev))
    eexp, eroutes = omoe.moe_groups(ids)
    np.testing.assert_array_equal(_np(experts), eexp)
    np.testing.assert_array_equal(_np(routes), eroutes)


@pytest.mark.parametrize("r,top,E,o,k,routed,scale_dtype", [
    (64, 8, 256, 512, 2048, False, "bfloat16"),
    (64, 8, 256, 2048, 512, True, "bfloat16"),
    (5, 3, 7, 256, 384, False, "float32"),
    (300, 4, 16, 128, 256, True, "float32")])
def test_fp8_experts(dev, r, top, E, o, k, routed, scale_dtype):
    """The decode variant's expert products over moe_groups' tables: the
    Qwen3.5 shapes (gate/up o=512 k=2048, down o=2048 k=512 on routed
    activations) and small ones; rows no group routes keep out's values."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(72 + r)
    ids = np.stack([rng.permutation(E)[:top] for _ in range(r)]).astype(np.int32)
    x = bf16_normal(rng, (r, top, k) if routed else (r, k))
    w = random_codes(rng, (E, o, k))
    ws = (2.0 ** rng.integers(-8, -4, (E, o // 128, k // 128))).astype(np.float32)
    if scale_dtype == "bfloat16":
        ws = ofp8.bf16_round(ws)
    experts, routes = omoe.moe_groups(ids)
    experts[experts == ids[0, 0]] = -1  # row 0's first pick routed by no group
    out = torch.full((r, top, o), 7.0, dtype=torch.float32, device=dev)
    ops.fp8_experts(_t(x, dev, torch.bfloat16), _t(w, dev), _t(ws, dev, getattr(torch, scale_dtype)),
                    _t(experts, dev), _t(routes, dev), top=top, routed_input=routed, out=out)
    exp = omoe.fp8_experts(x, w, ws, experts, routes, top, routed,
                           out=np.full((r, top, o), 7.0, np.float32))
    got = _np(out)
    assert (got[0, 0] == 7.0).all()
    assert rel_fro(got, exp) < 1e-4  # f32 accumulation, as the grouped products' bar


@pytest.mark.parametrize("rows,E,H,F", [(6, 32, 256, 128), (4, 256, 2048, 512)])
def test_shared_expert_moe_block_group_kinds(dev, rows, E, H, F):
    """The Qwen3.5 block with its routed experts through the decode program's
    own kinds (moe_groups, fp8_experts, swiglu_experts) against the block
    equation and against the routes/grouped-GEMM path."""
    import torch
    from akas_amd import moe

    rng = np.random.default_rng(rows * 3 + E)
    top = 8
    dbank, bank = _device_bank(dev, rows * 3 + E, {
        "w1": (E, F, H), "w3": (E, F, H), "w2": (E, H, F),
        "sw1": (F, H), "sw3": (F, H), "sw2": (H, F)}, 0.02 if H == 2048 else 0.05)
    x = bf16_normal(rng, (rows, H))
    logits = rng.normal(0, 1, (rows, E)).astype(np.float32)
    gate = rng.normal(0, 1.5, rows).astype(np.float32)
    wts = moe.ExpertWeights(*(a for n in ("w1", "w3", "w2") for a in dbank[n]))
    shared = moe.SharedExpert(*(a for n in ("sw1", "sw3", "sw2") for a in dbank[n]))
    args = (_t(x, dev, torch.bfloat16), _t(logits, dev), _t(gate, dev), wts, shared)
    out = _np(moe.shared_expert_moe(*args, top=top, routed_kinds="groups"))
    ref_path = _np(moe.shared_expert_moe(*args, top=top))
    exp = omoe.shared_expert_moe_layer(x, logits, gate, *bank["w1"], *bank["w3"], *bank["w2"],
                                       *bank["sw1"], *bank["sw3"], *bank["sw2"], top)
    assert rel_fro(out, exp) < 1e-2
    assert rel_fro(out, ref_path) < 1e-3


@pytest.mark.parametrize("rows,E,H,F,top,x_dtype,scale_dtype,gate_dtype", [
    (6, 32, 256, 128, 8, "bfloat16", "float32", "float32"),     # 32-row decode tiles
    (64, 256, 2048, 512, 8, "bfloat16", "bfloat16", "float32"),  # the Qwen3.5 decode batch
    (1, 8, 256, 128, 1, "float32", "float32", "bfloat16"),      # one row, top 1
    (300, 32, 256, 256, 8, "float16", "float32", "float32"),    # 128-row tiles
    (1024, 16, 512, 256, 8, "bfloat16", "float32", "bfloat16"),  # DMA-fed 256-row tiles
    (97, 64, 384, 384, 4, "bfloat16", "bfloat16", "float16")])
def test_shared_expert_block_is_its_kinds(dev, rows, E, H, F, top, x_dtype, scale_dtype,
                                          gate_dtype):
    """The one-call block equals, bit for bit, the kinds it fuses run one by
    one over a bank extended with the shared expert as expert E: router ->
    quantize -> quantized_routes over ids with rank `top` = E on every row ->
    fp8_expert_swiglu -> expert_partial (bf16) -> moe_combine with rank
    `top` as the shared expert.  The row tiles of the grouped kernels differ
    with the rows per expert (decode, 128-row, DMA-fed)."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(rows * 7 + E)
    sdt = getattr(torch, scale_dtype)
    g = torch.Generator(device=dev)
    g.manual_seed(rows + E)
    bank = {}
    for name, shape in (("w1", (E, F, H)), ("w3", (E, F, H)), ("w2", (E, H, F)),
                        ("sw1", (F, H)), ("sw3", (F, H)), ("sw2", (H, F))):
        w = torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * 0.05
        bank[name] = ops.quantize_weight_blocks(w, scale_dtype=sdt)
    x = _t(bf16_normal(rng, (rows, H)), dev, getattr(torch, x_dtype))
    logits = _t(rng.normal(0, 1, (rows, E)).astype(np.float32), dev)
    gate = _t(rng.normal(0, 1.5, rows).astype(np.float32), dev, getattr(torch, gate_dtype))
    args = [t for n in ("w1", "w3", "w2", "sw1", "sw3", "sw2") for t in bank[n]]
    out = ops.shared_expert_moe_block(x, logits, gate, *args, top=top)

    ids, prob = ops.router(logits, top=top)
    codes, scales = ops.quantize(x)
    ext = torch.cat([ids, torch.full((rows, 1), E, dtype=torch.int32, device=dev)], 1).contiguous()
    counts, routes = ops.quantized_routes(ext, torch.ones(rows, dtype=torch.int32, device=dev),
                                          experts=E + 1)
    full = {n: tuple(torch.cat([bank[n][i], bank["s" + n][i].unsqueeze(0)]).contiguous()
                     for i in range(2)) for n in ("w1", "w3", "w2")}
    act, act_scales = ops.fp8_expert_swiglu(codes, scales, *full["w1"], *full["w3"], counts, routes,
                                            r=rows, top=top + 1)
    contrib = ops.expert_partial(act, act_scales, *full["w2"], counts, routes, r=rows, top=top + 1,
                                 routed_input=True, output_dtype=torch.bfloat16)
    want = ops.moe_combine(contrib[:, :top].contiguous(), prob, contrib[:, top].contiguous(), gate)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_np(out), _np(want))
    assert np.isfinite(_np(out)).all()


def test_shared_expert_block_paths_agree(dev):
    """The shared expert on a second stream (dense FP8 linears) and as an
    expert of the routed launches give the same block within the products'
    summation-order tolerance, at the Qwen3.5 decode size."""
    import torch
    from akas_amd import moe

    rows, E, H, F, top = 64, 256, 2048, 512, 8
    rng = np.random.default_rng(123)
    dbank, _ = _device_bank(dev, 123, {
        "w1": (E, F, H), "w3": (E, F, H), "w2": (E, H, F),
        "sw1": (F, H), "sw3": (F, H), "sw2": (H, F)}, 0.02)
    wts = moe.ExpertWeights(*(a for n in ("w1", "w3", "w2") for a in dbank[n]))
    shared = moe.SharedExpert(*(a for n in ("sw1", "sw3", "sw2") for a in dbank[n]))
    args = (_t(bf16_normal(rng, (rows, H)), dev, torch.bfloat16),
            _t(rng.normal(0, 1, (rows, E)).astype(np.float32), dev),
            _t(rng.normal(0, 1.5, rows).astype(np.float32), dev), wts, shared)
    one_call = _np(moe.shared_expert_moe(*args, top=top))
    two_streams = _np(moe.shared_expert_moe(*args, top=top, shared_as_expert=False))
    assert rel_fro(one_call, two_streams) < 1e-4


@pytest.mark.parametrize("shared_as_expert", [True, False])
def test_shared_expert_moe_block_graph_replays(dev, shared_as_expert):
    """The block captured in a HIP graph, either as one call or with the
    shared expert forked onto a second stream and joined before the combine:
    every replay (with eager work and synchronizations between them) equals
    the eager result."""
    import torch
    from akas_amd import moe

    rows, E, H, F, top = 6, 32, 256, 128, 8
    rng = np.random.default_rng(97)
    dbank, _ = _device_bank(dev, 97, {
        "w1": (E, F, H), "w3": (E, F, H), "w2": (E, H, F),
        "sw1": (F, H), "sw3": (F, H), "sw2": (H, F)}, 0.05)
    wts = moe.ExpertWeights(*(a for n in ("w1", "w3", "w2") for a in dbank[n]))
    shared = moe.SharedExpert(*(a for n in ("sw1", "sw3", "sw2") for a in dbank[n]))
    x = _t(bf16_normal(rng, (rows, H)), dev, torch.bfloat16)
    logits = _t(rng.normal(0, 1, (rows, E)).astype(np.float32), dev)
    gate = _t(rng.normal(0, 1.5, rows).astype(np.float32), dev)
    kw = dict(top=top, shared_as_expert=shared_as_expert)
    eager = moe.shared_expert_moe(x, logits, gate, wts, shared, **kw).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        moe.shared_expert_moe(x, logits, gate, wts, shared, **kw)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = moe.shared_expert_moe(x, logits, gate, wts, shared, **kw)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(out), _np(eager))
        moe.shared_expert_moe(x, logits, gate, wts, shared, **kw)  # eager work between
        torch.cuda.synchronize()


@pytest.mark.parametrize("rows", [64, 300])
@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("fused_combine", [False, True])
def test_routed_moe_layer_graph_replays(dev, packed, fused_combine, rows):
    """The routed block captured in a HIP graph: every replay (with eager work
    and synchronizations between them) equals the eager result.  Unpacked, 64
    rows take the route scan inside the gate/up launch (16 routes per expert),
    300 rows its own launch (75 per expert)."""
    import torch
    from akas_amd import moe

    H, F, E, top = 512, 256, 16, 4
    rng = np.random.default_rng(98)
    bank = {}
    for name, shape in (("w1", (E, F, H)), ("w3", (E, F, H)), ("w2", (E, H, F))):
        bank[name] = ofp8.quantize_weight_blocks(rng.normal(0, 0.05, shape).astype(np.float32))
    wts = moe.ExpertWeights(*(_t(a, dev) for n in ("w1", "w3", "w2") for a in bank[n]))
    x = _t(bf16_normal(rng, (rows, H)), dev, torch.bfloat16)
    logits = _t(rng.normal(0, 1, (rows, E)).astype(np.float32), dev)
    kw = dict(top=top, packed=packed, max_block_m=128 if packed else 64, fused_combine=fused_combine)
    eager = moe.routed_moe(x, logits, None, wts, **kw).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        moe.routed_moe(x, logits, None, wts, **kw)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = moe.routed_moe(x, logits, None, wts, **kw)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(out), _np(eager))
        moe.routed_moe(x, logits, None, wts, **kw)  # eager work between
        torch.cuda.synchronize()


@pytest.mark.parametrize("fused_combine", [False, True])
def test_routed_moe_two_streams(dev, fused_combine):
    """The routed block called on two streams at once, on different inputs,
    repeatedly: the per-stream caches (workspaces, the fused combine's
    arrival counters) keep the calls apart, and every result equals the
    one-stream result bit for bit."""
    import torch
    from akas_amd import moe

    rows, H, F, E, top = 300, 512, 256, 16, 4
    rng = np.random.default_rng(99)
    bank = {}
    for name, shape in (("w1", (E, F, H)), ("w3", (E, F, H)), ("w2", (E, H, F))):
        bank[name] = ofp8.quantize_weight_blocks(rng.normal(0, 0.05, shape).astype(np.float32))
    wts = moe.ExpertWeights(*(_t(a, dev) for n in ("w1", "w3", "w2") for a in bank[n]))
    xs = [_t(bf16_normal(rng, (rows, H)), dev, torch.bfloat16) for _ in range(2)]
    logits = [_t(rng.normal(0, 1, (rows, E)).astype(np.float32), dev) for _ in range(2)]
    kw = dict(top=top, fused_combine=fused_combine)
    ref = [moe.routed_moe(x, lg, None, wts, **kw).clone() for x, lg in zip(xs, logits)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    outs = [[] for _ in streams]
    for rep in range(10):
        for j, st in enumerate(streams):
            with torch.cuda.stream(st):
                outs[j].append(moe.routed_moe(xs[j], logits[j], None, wts, **kw))
    torch.cuda.synchronize()
    for j in range(len(streams)):
        for out in outs[j]:
            np.testing.assert_array_equal(_np(out), _np(ref[j]))


@pytest.mark.parametrize("rows,experts,top,k,x_dtype,softmax,with_bias", [
    (1, 64, 4, 2048, "bfloat16", True, False), (257, 64, 4, 2048, "float32", False, True),
    (16384, 64, 4, 2048, "bfloat16", True, True), (33, 32, 6, 512, "float16", False, False),
    (5, 7, 3, 256, "bfloat16", True, True)])
def test_router_quantize_matches_separate_kinds(dev, rows, experts, top, k, x_dtype, softmax,
                                                with_bias):
    """The block's one-launch router + quantizer: ids, weights, codes and
    scales bit-identical to the router kind and the quantize kind run apart."""
    import torch
    from akas_amd import ops

    rng = np.random.default_rng(rows + experts)
    logits = _t(rng.normal(0, 1, (rows, experts)).astype(np.float32), dev)
    bias = _t(rng.normal(0, 0.1, experts).astype(np.float32), dev) if with_bias else None
    x = _t(bf16_normal(rng, (rows, k), outliers=0.01), dev, getattr(torch, x_dtype))
    ids, w, codes, scales = ops.router_quantize(logits, bias, x, top=top, softmax=softmax,
                                                scale=1.5, normalize=True)
    if softmax:
        eids, ew = ops.biased_softmax_router(logits, bias, top=top, scale=1.5)
    else:
        eids, ew = ops.biased_router(logits, bias, top=top, scale=1.5, normalize=True)
    ec, es = ops.quantize(x)
    torch.cuda.synchronize()
    assert torch.equal(ids, eids) and torch.equal(w.view(torch.int32), ew.view(torch.int32))
    assert torch.equal(codes, ec) and torch.equal(scales.view(torch.int32), es.view(torch.int32))
