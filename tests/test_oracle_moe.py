"""Pins the oracle's routing, tile maps, packing, expert products and combine.

Independent formulations only: stable argsort and scipy's softmax / expit
for the routers, vectorised constructions for routes, tile maps and packing,
integer brute force on exact-product inputs for the expert GEMMs, a float64
SwiGLU for the fused re-quantization, explicit loops for the combine, plus
the reference's own known answers (tile_capacity(1, 4, 64, 16) == 4, empty
batches, deterministic route patterns).  CPU only.
"""

import numpy as np
import pytest
from scipy.special import expit, softmax

from golden_inputs import bf16_normal, exact_codes, random_codes, rel_fro
from oracle import fp8 as ofp8
from oracle import moe as omoe


def _pattern(rows, top, experts, mult=1):
    """src/akas/ops/moe/validation.py:82-99 / :606-611: ids (row*mult + rank) %
    experts, last row inactive."""
    ids = ((np.arange(rows)[:, None] * mult + np.arange(top)[None, :]) % experts).astype(np.int32)
    active = np.ones(rows, np.int32)
    if rows > 1:
        active[-1] = 0
    return ids, active


# ---------------------------------------------------------------------------
# routers
# ---------------------------------------------------------------------------

def _logits_with_ties(rng, rows, experts):
    logits = rng.normal(0, 1, (rows, experts)).astype(np.float32)
    logits[0] = 0.0                     # all-tie row
    logits[1, 3] = logits[1, 5] = logits[1].max() + 1  # tie at the top
    return logits


@pytest.mark.parametrize("rows,experts,top", [(40, 64, 4), (9, 7, 3), (5, 256, 8)])
def test_softmax_router(rows, experts, top):
    rng = np.random.default_rng(21)
    logits = _logits_with_ties(rng, rows, experts)
    bias = rng.normal(0, 0.5, experts).astype(np.float32)
    ids, w = omoe.biased_softmax_router(logits, bias, top, scale=1.5)
    exp_ids = np.argsort(-(logits + bias), axis=1, kind="stable")[:, :top]
    np.testing.assert_array_equal(ids, exp_ids)
    sel = np.take_along_axis(logits.astype(np.float64), exp_ids, axis=1)
    np.testing.assert_allclose(w, 1.5 * softmax(sel, axis=1), rtol=1e-6)
    zero_ids, _ = omoe.biased_softmax_router(np.zeros((1, experts), np.float32), np.zeros(experts, np.float32), top)
    np.testing.assert_array_equal(zero_ids[0], np.arange(top))


def _bf16_tie_logits(rng, rows, experts):
    """Random logits with, in row 0, two distinct f32 values that round to the
    same bf16 value (1 and 1 + 2^-10), the larger one at the higher index, as
    the row's two largest logits."""
    logits = rng.normal(0, 1, (rows, experts)).astype(np.float32)
    logits[0] = np.minimum(logits[0], 0.5)
    lo, hi = 1, min(5, experts - 1)
    logits[0, lo] = 1.0
    logits[0, hi] = np.float32(1.0 + 2.0 ** -10)
    return logits


@pytest.mark.parametrize("rows,experts,top", [(40, 64, 4), (9, 7, 3), (5, 256, 8)])
def test_decode_router(rows, experts, top):
    """Closed forms: stable argsort of the bf16-rounded logits (rounded by
    torch, not the oracle's own rounding) and scipy's softmax over the
    selected ones; the bf16 tie in row 0 goes to the lower index although the
    f32 logit at the higher index is larger."""
    import torch

    rng = np.random.default_rng(23)
    logits = _bf16_tie_logits(rng, rows, experts)
    ids, w = omoe.router(logits, top)
    rounded = torch.from_numpy(logits).to(torch.bfloat16).float().numpy()
    exp_ids = np.argsort(-rounded, axis=1, kind="stable")[:, :top]
    np.testing.assert_array_equal(ids, exp_ids)
    assert ids[0, 0] == 1 and (top < 2 or ids[0, 1] == min(5, experts - 1))
    sel = np.take_along_axis(rounded.astype(np.float64), exp_ids, axis=1)
    np.testing.assert_allclose(w, softmax(sel, axis=1), rtol=1e-6)


@pytest.mark.parametrize("normalize", [True, False])
def test_sigmoid_router(normalize):
    rng = np.random.default_rng(22)
    logits = _logits_with_ties(rng, 33, 64)
    bias = rng.normal(0, 0.1, 64).astype(np.float32)
    ids, w = omoe.biased_router(logits, bias, 4, scale=2.0, normalize=normalize)
    sig = expit(logits.astype(np.float64))
    score = (sig.astype(np.float32) + bias).astype(np.float32)
    exp_ids = np.argsort(-score, axis=1, kind="stable")[:, :4]
    np.testing.assert_array_equal(ids, exp_ids)
    chosen = np.take_along_axis(sig, exp_ids, axis=1)
    exp_w = 2.0 * chosen / (chosen.sum(1, keepdims=True) + 1e-6) if normalize else 2.0 * chosen
    np.testing.assert_allclose(w, exp_w, rtol=1e-6)


# ---------------------------------------------------------------------------
# the sigmoid router's float32 exponential
# ---------------------------------------------------------------------------

F32_MAX_MIDPOINT = 2.0 ** 128 - 2.0 ** 103  # IEEE round-to-nearest overflows from here


def _rn32_exp_decimal(x):
    """RN32(e^x) of one float32 ``x`` from Python's ``decimal`` exponential
    (correctly rounded at 60 significant digits): the nearer float32
    neighbour of the 60-digit value, ties to the even pattern.  Independent
    of numpy's and mpmath's exponentials."""
    from decimal import Decimal, localcontext

    with localcontext() as ctx:
        ctx.prec = 60
        t = Decimal(float(x)).exp()
        if t >= Decimal(F32_MAX_MIDPOINT):
            return np.float32(np.inf)
        c = np.float32(min(float(t), float(np.finfo(np.float32).max)))
        best = None
        for f in (np.nextafter(c, np.float32(0)), c, np.nextafter(c, np.float32(np.inf))):
            if not np.isfinite(f):
                continue
            key = (abs(Decimal(float(f)) - t), int(np.array(f, np.float32).view(np.uint32)) & 1)
            if best is None or key < best[0]:
                best = (key, f)
        return best[1]


def _midpoint_hazards(margin=64):
    """Every float32 x with 2^-26 <= |x|, x in [-17, 88.75] (the inputs on
    which 1 / (1 + e^-l) depends on the exponential's last bit) whose float64
    e^x lies within ``margin`` double ulps of a float32 rounding midpoint."""
    found = []
    for sign, hi in ((0, 0x42B18000), (0x80000000, 0x41880000)):
        for a in range(0x32800000, hi + 1, 1 << 24):
            bits = np.arange(a, min(a + (1 << 24), hi + 1), dtype=np.uint32) | np.uint32(sign)
            y = np.exp(bits.view(np.float32).astype(np.float64))
            low = (y.view(np.uint64) & np.uint64((1 << 29) - 1)).astype(np.int64)
            found.append(bits[np.abs(low - (1 << 28)) <= margin])
    return np.concatenate(found).view(np.float32)


def test_exp_rn32_is_correctly_rounded():
    """Where float64 e^x sits near a float32 midpoint (all of them, found by
    an exhaustive scan of the sigmoid's input range), the oracle's exp_rn32
    equals the decimal-derived correctly rounded value; elsewhere numpy's
    float64 exp, within an ulp of double on a random sample and at the range
    ends, is 64 double ulps clear of every midpoint, so its float32 rounding
    is correct."""
    from decimal import Decimal, localcontext

    hazards = _midpoint_hazards()
    assert 0 < hazards.size < 500
    got = omoe.exp_rn32(hazards)
    exp = np.array([_rn32_exp_decimal(v) for v in hazards], np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))
    # numpy's float64 exp is within 1 ulp of double on a sample of the range
    rng = np.random.default_rng(3)
    sample = np.concatenate([rng.uniform(-17, 88.75, 3000), rng.uniform(-1e-3, 1e-3, 1000),
                             [88.72283, 88.72284, -17.0, 88.75]]).astype(np.float32)
    y = np.exp(sample.astype(np.float64))
    with localcontext() as ctx:
        ctx.prec = 60
        for v, yv in zip(sample, y):
            t = Decimal(float(v)).exp()
            assert abs(Decimal(float(yv)) - t) <= Decimal(float(np.spacing(yv)))
    np.testing.assert_array_equal(omoe.exp_rn32(sample).view(np.uint32),
                                  np.array([_rn32_exp_decimal(v) for v in sample],
                                           np.float32).view(np.uint32))


def test_exp_rn32_overflow_threshold():
    """The largest float32 x with a finite RN32(e^x), and the next one up."""
    x = np.float32(88.72283)
    while np.isfinite(_rn32_exp_decimal(np.nextafter(x, np.float32(np.inf)))):
        x = np.nextafter(x, np.float32(np.inf))
    while not np.isfinite(_rn32_exp_decimal(x)):
        x = np.nextafter(x, np.float32(0))
    up = np.nextafter(x, np.float32(np.inf))
    got = omoe.exp_rn32(np.array([x, up], np.float32))
    assert np.isfinite(got[0]) and np.isinf(got[1])


def test_router_sigmoid_closed_forms():
    """1 / (1 + e^-l) with each step rounded once: exact values at 0 and in
    the saturated tails, monotone over a dense sweep, within three float32
    ulps of the exact logistic (scipy's float64 expit: three roundings of at
    most half an ulp each, relative to a result that may sit at the bottom
    of its binade), and the reflection sigma(l) + sigma(-l) = 1 to two ulps."""
    s = omoe.router_sigmoid
    assert s(np.float32(0.0)) == np.float32(0.5)
    assert np.all(s(np.array([17.0, 30.0, 1e30], np.float32)) == 1.0)
    assert np.all(s(np.array([-89.0, -1e30], np.float32)) == 0.0)
    sweep = np.sort(np.random.default_rng(4).uniform(-40, 40, 200001).astype(np.float32))
    sig = s(sweep)
    assert np.all(np.diff(sig) >= 0)
    ref = expit(sweep.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    tiny = ref > 1e-30
    assert np.all(np.abs(sig - ref)[tiny] <= 3 * ulp[tiny])
    mid = np.abs(sweep) < 15
    assert np.all(np.abs(sig[mid] + s(-sweep[mid]) - 1.0) <= 2 * np.spacing(np.float32(1.0)))


# ---------------------------------------------------------------------------
# routes, tile maps, packing
# ---------------------------------------------------------------------------

def _routes_vectorised(ids, active, experts):
    rows, top = ids.shape
    flat = np.where(np.repeat(active[:, None] != 0, top, 1), ids, -1).ravel()
    counts = np.zeros(experts, np.int32)
    routes = np.full((experts, rows), -1, np.int32)
    for e in range(experts):
        pos = np.flatnonzero(flat == e)       # position = row*top + rank, ascending
        counts[e] = pos.size
        routes[e, :pos.size] = pos
    return counts, routes


@pytest.mark.parametrize("rows,top,experts,mult", [(1, 4, 64, 1), (33, 2, 4, 1), (257, 4, 64, 3),
                                                   (600, 3, 7, 5), (16, 8, 256, 7)])
def test_quantized_routes(rows, top, experts, mult):
    ids, active = _pattern(rows, top, experts, mult)
    counts, routes = omoe.quantized_routes(ids, active, experts)
    ec, er = _routes_vectorised(ids, active, experts)
    np.testing.assert_array_equal(counts, ec)
    np.testing.assert_array_equal(routes, er)


def test_quantized_routes_random_and_empty():
    rng = np.random.default_rng(23)
    ids = rng.integers(0, 64, (500, 4)).astype(np.int32)
    active = (rng.random(500) < 0.8).astype(np.int32)
    counts, routes = omoe.quantized_routes(ids, active, 64)
    ec, er = _routes_vectorised(ids, active, 64)
    np.testing.assert_array_equal(counts, ec)
    np.testing.assert_array_equal(routes, er)
    # every routed (row, rank) exactly once; tests/test_lfm_moe.py:204-214 empty batch
    assert sorted(routes[routes >= 0].tolist()) == sorted(
        (r * 4 + k) for r in range(500) if active[r] for k in range(4))
    counts, routes = omoe.quantized_routes(ids, np.zeros(500, np.int32), 64)
    assert (counts == 0).all() and (routes == -1).all()


def test_tile_capacity_and_layouts():
    """tests/test_lfm_moe_native.py:476-488 and src/akas/ops/moe/definition.py:19-26."""
    assert omoe.tile_capacity(1, 4, 64, 16) == 4
    rng = np.random.default_rng(29)
    for _ in range(200):
        rows, experts, block_m = (int(rng.integers(1, 65)) for _ in range(3))
        top = int(rng.integers(1, experts + 1))
        counts = np.zeros(experts, np.int64)
        for _ in range(rows):
            counts[rng.choice(experts, top, replace=False)] += 1
        cap = omoe.tile_capacity(rows, top, experts, block_m)
        assert int(((counts + block_m - 1) // block_m).sum()) <= cap <= rows * top
    assert [omoe.tile_layouts(m) for m in (4, 8, 16, 32, 64, 128)] == [1, 2, 3, 4, 5, 6]
    for bad in (2, 48, 256):
        with pytest.raises(ValueError):
            omoe.tile_layouts(bad)
    with pytest.raises(ValueError):
        omoe.tile_capacity(0, 4, 64, 16)


@pytest.mark.parametrize("max_block_m", [64, 128])
def test_expert_tile_map(max_block_m):
    rng = np.random.default_rng(31)
    rows, top, experts = 300, 4, 16
    counts = np.bincount(rng.integers(0, experts, rows * top), minlength=experts).astype(np.int32)
    counts[3] = 0
    te, tr = omoe.expert_tile_map(counts, rows, top, max_block_m)
    assert te.shape == (omoe.tile_layouts(max_block_m), (rows * top + 3) // 4 + experts)
    for layout in range(te.shape[0]):
        block = 4 << layout
        n = (counts + block - 1) // block
        exp_e = np.repeat(np.arange(experts), n)
        exp_t = np.concatenate([np.arange(v) for v in n])
        np.testing.assert_array_equal(te[layout, :exp_e.size], exp_e)
        np.testing.assert_array_equal(tr[layout, :exp_e.size], exp_t)
        assert (te[layout, exp_e.size:] == -1).all() and (tr[layout, exp_e.size:] == 0).all()
    # tests/test_lfm_moe.py:215-225: zero counts -> an all-padding map
    te, tr = omoe.expert_tile_map(np.zeros(experts, np.int32), rows, top, max_block_m)
    assert (te == -1).all() and (tr == 0).all()


@pytest.mark.parametrize("routed", [False, True])
def test_expert_pack(routed):
    rng = np.random.default_rng(33)
    rows, top, experts, k, align = 129, 3, 7, 256, 64
    ids = np.array([[(r * 3 + j) % experts for j in range(top)] for r in range(rows)], np.int32)
    active = np.ones(rows, np.int32)
    active[-1] = 0
    counts, routes = omoe.quantized_routes(ids, active, experts)
    shape = (rows, top, k) if routed else (rows, k)
    x = rng.integers(0, 255, shape, dtype=np.uint8)
    xs = rng.uniform(0.1, 2, (*shape[:-1], k // 128)).astype(np.float32)
    packed, pscales, offs = omoe.expert_pack(x, xs, counts, routes, top, experts, align, routed)
    padded = (counts + align - 1) // align * align
    exp_offs = np.concatenate([[0], np.cumsum(padded)[:-1]])
    np.testing.assert_array_equal(offs[counts > 0], exp_offs[counts > 0])
    assert packed.shape[0] == omoe.tile_capacity(rows, top, experts, align) * align
    for e in range(experts):
        seg = slice(exp_offs[e], exp_offs[e] + counts[e])
        owner, rank = np.divmod(routes[e, :counts[e]], top)
        src = x[owner, rank] if routed else x[owner]
        srcs = xs[owner, rank] if routed else xs[owner]
        np.testing.assert_array_equal(packed[seg], src)
        np.testing.assert_array_equal(pscales[seg], srcs)
        pad = slice(exp_offs[e] + counts[e], exp_offs[e] + padded[e])
        assert (packed[pad] == 0).all() and (pscales[pad] == 1).all()


# ---------------------------------------------------------------------------
# expert products
# ---------------------------------------------------------------------------

def _exact_expert_case(rng, rows, top, experts, o, k, routed):
    ids, active = _pattern(rows, top, experts, 1)
    counts, routes = omoe.quantized_routes(ids, active, experts)
    shape = (rows, top, k) if routed else (rows, k)
    x = exact_codes(rng, shape)
    xs = (2.0 ** rng.integers(-4, 2, (*shape[:-1], k // 128))).astype(np.float32)
    w = exact_codes(rng, (experts, o, k))
    ws = (2.0 ** rng.integers(-4, 2, (experts, o // 128, k // 128))).astype(np.float32)
    return counts, routes, x, xs, w, ws


def _int_products(x, xs, w, ws):
    """Per-row products from integer codes: value = (+-1|+-2) * 2^e exactly."""
    dx = ofp8.decode_e4m3(x).astype(np.float64) * np.repeat(xs.astype(np.float64), 128, -1)
    dw = ofp8.decode_e4m3(w).astype(np.float64) * np.repeat(np.repeat(ws.astype(np.float64), 128, -2), 128, -1)
    return dx @ dw.T


@pytest.mark.parametrize("routed", [False, True])
def test_expert_partial_exact(routed):
    rng = np.random.default_rng(37)
    rows, top, experts, o, k = 40, 3, 5, 256, 384
    counts, routes, x, xs, w, ws = _exact_expert_case(rng, rows, top, experts, o, k, routed)
    prior = np.full((rows, top, o), 7.0, np.float32)
    out = omoe.expert_partial(x, xs, w, ws, counts, routes, top, routed_input=routed, out=prior)
    seen = np.zeros((rows, top), bool)
    for e in range(experts):
        for route in routes[e, :counts[e]]:
            row, rank = divmod(int(route), top)
            seen[row, rank] = True
            src = (x[row, rank], xs[row, rank]) if routed else (x[row], xs[row])
            exp = _int_products(src[0][None], src[1][None], w[e], ws[e])[0]
            np.testing.assert_array_equal(out[row, rank], exp.astype(np.float32))
    assert (out[~seen] == 7.0).all()  # rows not routed keep the prior contents
    parts = omoe.expert_partial(x, xs, w, ws, counts, routes, top, routed_input=routed, partitions=3)
    np.testing.assert_array_equal(omoe.expert_merge(parts)[seen], out[seen])


@pytest.mark.parametrize("pd,ad", [("float32", "float32"), ("bfloat16", "bfloat16"), ("float16", "float16")])
def test_fused_swiglu_against_float64_and_composition(pd, ad):
    """Exact gate/up products, SwiGLU evaluated in float64 from the rounded
    products, then the activation rounding and the 1x128 quantizer: the fused
    oracle's codes sit in the reference's midpoint band of that float64
    chain (src/akas/ops/moe/validation.py:327-432), and equal the separate
    chain expert_partial x2 -> swiglu_experts -> quantize bit for bit."""
    rng = np.random.default_rng(831)
    rows, top, experts, o, k = 33, 3, 7, 256, 384
    counts, routes, x, xs, w, ws = _exact_expert_case(rng, rows, top, experts, o, k, False)
    w2 = exact_codes(rng, (experts, o, k))
    codes, scales, norm = omoe.fp8_expert_swiglu(x, xs, w, ws, w2, ws, counts, routes, top, pd, ad)
    live = np.zeros((rows, top), bool)
    for e in range(experts):
        for route in routes[e, :counts[e]]:
            row, rank = divmod(int(route), top)
            live[row, rank] = True
            g = ofp8.round_to(_int_products(x[row][None], xs[row][None], w[e], ws[e]).astype(np.float32), pd)
            u = ofp8.round_to(_int_products(x[row][None], xs[row][None], w2[e], ws[e]).astype(np.float32), pd)
            a = ofp8.round_to((g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u).astype(np.float32), ad)
            s = (np.maximum(np.abs(a.reshape(-1, 128)).max(-1), 1e-12) / 448).astype(np.float32)
            with np.errstate(invalid="ignore"):  # inf / inf in a group holding inf
                q = (a.reshape(-1, 128).astype(np.float64) / s[:, None]).astype(np.float32).reshape(-1)
            ok = omoe.codes_within_midpoint_band(codes[row, rank], ofp8.encode_e4m3(q), q)
            assert ok.all()
            np.testing.assert_allclose(scales[row, rank], s, rtol=2e-6)
    gate = omoe.expert_partial(x, xs, w, ws, counts, routes, top, output_dtype=pd)
    up = omoe.expert_partial(x, xs, w2, ws, counts, routes, top, output_dtype=pd)
    sep_codes, sep_scales = ofp8.quantize(omoe.swiglu_experts(gate, up, output_dtype=ad))
    np.testing.assert_array_equal(codes[live], sep_codes[live])
    np.testing.assert_array_equal(scales[live], sep_scales[live])


@pytest.mark.parametrize("pd,ad,od", [("float32", "float32", "float32"),
                                      ("bfloat16", "bfloat16", "bfloat16"),
                                      ("float16", "float32", "float16")])
def test_expert_swiglu_against_float64(pd, ad, od):
    """The unquantized paired SwiGLU: on exact products, each routed entry is
    the float64 SwiGLU of the rounded products, rounded to the activation and
    then the output dtype (``src/akas/ops/moe/validation.py:385-410``);
    unrouted entries stay 0; quantizing the float32 result reproduces the
    fused kind's codes bit for bit."""
    rng = np.random.default_rng(832)
    rows, top, experts, o, k = 21, 2, 5, 256, 256
    counts, routes, x, xs, w, ws = _exact_expert_case(rng, rows, top, experts, o, k, False)
    w2 = exact_codes(rng, (experts, o, k))
    out = omoe.expert_swiglu(x, xs, w, ws, w2, ws, counts, routes, top, pd, ad, od)
    live = np.zeros((rows, top), bool)
    for e in range(experts):
        for route in routes[e, :counts[e]]:
            row, rank = divmod(int(route), top)
            live[row, rank] = True
            g = ofp8.round_to(_int_products(x[row][None], xs[row][None], w[e], ws[e]).astype(np.float32), pd)
            u = ofp8.round_to(_int_products(x[row][None], xs[row][None], w2[e], ws[e]).astype(np.float32), pd)
            a = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u).astype(np.float32)
            exp = ofp8.round_to(ofp8.round_to(a, ad), od)[0]
            np.testing.assert_allclose(out[row, rank], exp, rtol=8e-3 if od != "float32" else 2e-6,
                                       atol=1e-30)
    assert not out[~live].any()
    if od == "float32":
        codes, scales, _ = omoe.fp8_expert_swiglu(x, xs, w, ws, w2, ws, counts, routes, top, pd, ad)
        qc, qs = ofp8.quantize(out)
        np.testing.assert_array_equal(qc[live], codes[live])
        np.testing.assert_array_equal(qs[live], scales[live])


@pytest.mark.parametrize("parts", [1, 3])
def test_expert_pair_partial_exact(parts):
    """Paired partials on exact products: gate and up of every routed entry
    equal the integer brute force over each partition's k-range, the two
    outputs differ (distinct weights), and unrouted entries stay 0."""
    rng = np.random.default_rng(833)
    rows, top, experts, o, k = 17, 3, 4, 128, 384
    counts, routes, x, xs, w, ws = _exact_expert_case(rng, rows, top, experts, o, k, False)
    w2 = np.flip(w, axis=-2).copy()
    ws2 = np.flip(ws, axis=-1).copy()
    gate, up = omoe.expert_pair_partial(x, xs, w, ws, w2, ws2, counts, routes, top, parts)
    assert gate.shape == up.shape == (rows, top, parts, o)
    span = k // parts
    live = np.zeros((rows, top), bool)
    for e in range(experts):
        for route in routes[e, :counts[e]]:
            row, rank = divmod(int(route), top)
            live[row, rank] = True
            for p in range(parts):
                seg = slice(p * span, (p + 1) * span)
                bseg = slice(p * span // 128, (p + 1) * span // 128)
                for got, ww, ss in ((gate, w, ws), (up, w2, ws2)):
                    exp = _int_products(x[row][None, seg], xs[row][None, bseg], ww[e][:, seg],
                                        ss[e][:, bseg])[0]
                    np.testing.assert_array_equal(got[row, rank, p], exp.astype(np.float32))
    assert not gate[~live].any() and not up[~live].any()
    assert not np.array_equal(gate[live], up[live])


def test_swiglu_float64():
    rng = np.random.default_rng(9)
    g = rng.normal(0, 6, 5000).astype(np.float32)
    u = rng.normal(0, 2, 5000).astype(np.float32)
    exact = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(omoe.swiglu(g, u), exact, rtol=2e-6, atol=1e-30)


def test_routed_combine_loop():
    rng = np.random.default_rng(41)
    T, top, c = 7, 4, 256
    e = rng.normal(0, 1, (T, top, c)).astype(np.float32)
    w = rng.uniform(0, 1, (T, top)).astype(np.float32)
    active = np.array([1, 1, 0, 1, 1, 1, 0], np.int32)
    out = omoe.routed_combine(e, w, active)
    for t in range(T):
        for col in range(0, c, 17):
            acc = np.float32(0)
            for rank in range(top):
                acc = np.float32(acc + np.float32(e[t, rank, col] * w[t, rank]))
            assert out[t, col] == (acc if active[t] else 0)


@pytest.mark.parametrize("routed", [False, True])
def test_expert_combine_exact(routed):
    """expert_combine against exact products and a per-rank float32 fold:
    an out-of-range id drops its rank (quantized_routes routes no entry for
    it), a row whose ids are all out of range and an inactive row are zero."""
    rng = np.random.default_rng(43)
    rows, top, experts, o, k = 24, 3, 5, 256, 256
    ids, active = _pattern(rows, top, experts, 1)
    ids[2, 1] = experts      # one dead rank
    ids[5, :] = -1           # no live rank
    active[7] = 0
    counts, routes = omoe.quantized_routes(ids, active, experts)
    shape = (rows, top, k) if routed else (rows, k)
    x = exact_codes(rng, shape)
    xs = (2.0 ** rng.integers(-4, 2, (*shape[:-1], k // 128))).astype(np.float32)
    w = exact_codes(rng, (experts, o, k))
    ws = (2.0 ** rng.integers(-4, 2, (experts, o // 128, k // 128))).astype(np.float32)
    cw = rng.uniform(0, 1, (rows, top)).astype(np.float32)
    out, contributions = omoe.expert_combine(x, xs, w, ws, counts, routes, ids, cw, active, top,
                                             routed_input=routed, contribution_dtype="bfloat16")
    for t in range(rows):
        for col in range(0, o, 37):
            acc = np.float32(0)
            for rank in range(top):
                e = int(ids[t, rank])
                if not (active[t] and 0 <= e < experts):
                    continue
                src = x[t, rank] if routed else x[t]
                srcs = xs[t, rank] if routed else xs[t]
                prod = _int_products(src[None], srcs[None], w[e][col:col + 1], ws[e][col // 128:col // 128 + 1])
                c = ofp8.bf16_round(np.float32(prod[0, 0]))
                assert contributions[t, rank, col] == c
                acc = np.float32(acc + np.float32(c * cw[t, rank]))
            assert out[t, col] == acc
    assert not out[5].any() and not out[7].any()


def test_moe_layer_against_per_token_loop():
    """The composed layer equals a per-token loop over its selected experts
    built from the pinned pieces (quantize, dequantize, SwiGLU, combine)."""
    rng = np.random.default_rng(43)
    T, H, F, E, top = 6, 256, 128, 4, 2
    x = bf16_normal(rng, (T, H))
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    bank = [ofp8.quantize_weight_blocks(rng.normal(0, 0.05, s).astype(np.float32))
            for s in ((E, F, H), (E, F, H), (E, H, F))]
    (w1, s1), (w3, s3), (w2, s2) = bank
    out, ids, prob = omoe.moe_layer(x, logits, np.zeros(E, np.float32), w1, s1, w3, s3, w2, s2, top)
    xq = ofp8.fake_quantize(x).astype(np.float64)
    for t in range(T):
        acc = np.zeros(H, np.float32)
        sel = np.argsort(-logits[t], kind="stable")[:top]
        p = softmax(logits[t, sel].astype(np.float64))
        for rank, e in enumerate(sel):
            g = (xq[t] @ ofp8.dequantize_weight(w1[e], s1[e]).T).astype(np.float32)
            u = (xq[t] @ ofp8.dequantize_weight(w3[e], s3[e]).T).astype(np.float32)
            a = ofp8.fake_quantize((g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u).astype(np.float32)[None])[0]
            d = (a.astype(np.float64) @ ofp8.dequantize_weight(w2[e], s2[e]).T).astype(np.float32)
            acc = (acc + d * np.float32(p[rank])).astype(np.float32)
        assert rel_fro(out[t], acc) < 1e-5


def test_c_oracle_moe_layer():
    from oracle import native

    lib = native.load()
    rng = np.random.default_rng(44)
    T, H, F, E, top = 24, 256, 256, 8, 4
    x = bf16_normal(rng, (T, H))
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    bank = [ofp8.quantize_weight_blocks(rng.normal(0, 0.05, s).astype(np.float32))
            for s in ((E, F, H), (E, F, H), (E, H, F))]
    (w1, s1), (w3, s3), (w2, s2) = bank
    exp, _, _ = omoe.moe_layer(x, logits, np.zeros(E, np.float32), w1, s1, w3, s3, w2, s2, top)
    out = np.zeros((T, H), np.float32)
    p = native.ptr
    assert lib.ref_moe_layer_bf16(p(ofp8.bf16_bits(x)), p(logits), p(w1), p(s1), p(w3), p(s3), p(w2),
                                  p(s2), p(out), T, H, F, E, top, 2) == 0
    assert rel_fro(out, exp) < 1e-4


def test_moe_combine_closed_forms():
    """moe_combine: a saturated gate adds bf16(shared) itself, a zero gate
    half of it, one-hot weights pick a rank, inputs are bf16-rounded first."""
    rng = np.random.default_rng(4)
    r, top, c = 3, 8, 16
    experts = rng.normal(0, 1, (r, top, c)).astype(np.float32)
    shared = rng.normal(0, 1, (r, c)).astype(np.float32)
    onehot = np.zeros((r, top), np.float32)
    onehot[np.arange(r), [0, 3, 7]] = 1.0
    bf = lambda v: (np.asarray(v, np.float32).view(np.uint32) + 0x7FFF
                    + ((np.asarray(v, np.float32).view(np.uint32) >> 16) & 1) & 0xFFFF0000).view(np.float32)
    pick = experts[np.arange(r), [0, 3, 7]]
    out = omoe.moe_combine(experts, onehot, shared, np.full(r, 100.0, np.float32))
    np.testing.assert_allclose(out, bf(pick) + bf(shared), rtol=1e-6)
    out0 = omoe.moe_combine(experts, onehot, shared, np.zeros(r, np.float32))
    np.testing.assert_allclose(out0, bf(pick) + bf(shared) / 2, rtol=1e-6)
    # a value between two bf16 neighbours rounds before it is weighted
    e = np.full((1, 1, 8), 1.0 + 2.0 ** -10, np.float32)
    got = omoe.moe_combine(e, np.ones((1, 1), np.float32), np.zeros((1, 8), np.float32),
                           np.zeros(1, np.float32))
    assert np.all(got == 1.0)


# ---------------------------------------------------------------------------
# block-fp8 decode variant: moe_groups / fp8_experts
# ---------------------------------------------------------------------------

def _groups_independent(ids):
    """moe_groups by a different formulation: owners from np.unique's first
    indices, ranks from the last matching column of each row."""
    r, top = ids.shape
    flat = ids.reshape(-1)
    _, first = np.unique(flat, return_index=True)
    experts = np.full(r * top, -1, np.int32)
    experts[first] = flat[first]
    routes = np.full((r * top, r), -1, np.int32)
    for g in first:
        hit = ids == flat[g]
        last = top - 1 - np.argmax(hit[:, ::-1], axis=1)
        routes[g] = np.where(hit.any(axis=1), last, -1)
    return experts, routes


@pytest.mark.parametrize("case", ["router", "duplicates", "single"])
def test_moe_groups(case):
    rng = np.random.default_rng(31)
    if case == "router":
        ids = np.argsort(-rng.normal(0, 1, (24, 16)), axis=1, kind="stable")[:, :4].astype(np.int32)
    elif case == "duplicates":
        ids = rng.integers(0, 5, (9, 3)).astype(np.int32)
        ids[0] = [2, 2, 2]  # one row selecting an expert three times: the last rank wins
    else:
        ids = np.array([[7]], np.int32)
    experts, routes = omoe.moe_groups(ids)
    eexp, eroutes = _groups_independent(ids)
    np.testing.assert_array_equal(experts, eexp)
    np.testing.assert_array_equal(routes, eroutes)
    if case == "router":
        # distinct ids per row: every (row, rank) pair is routed by exactly one owner
        covered = np.zeros(ids.shape, int)
        for g in np.nonzero(experts >= 0)[0]:
            for b in np.nonzero(routes[g] >= 0)[0]:
                covered[b, routes[g, b]] += 1
        assert (covered == 1).all()
    if case == "duplicates":
        g = int(np.nonzero(experts == 2)[0][0])
        assert routes[g, 0] == 2


@pytest.mark.parametrize("routed_input", [False, True])
def test_fp8_experts_matches_grouped_products(routed_input):
    """fp8_experts over moe_groups' tables equals the grouped expert products
    (pinned separately by exact-product inputs) over quantized_routes' tables
    for the same ids; entries no group routes keep out's values."""
    rng = np.random.default_rng(32)
    r, top, E, o, k = 6, 3, 5, 128, 256
    ids = np.stack([rng.permutation(E)[:top] for _ in range(r)]).astype(np.int32)
    x = rng.normal(0, 1, (r, top, k) if routed_input else (r, k)).astype(np.float32)
    w = random_codes(rng, (E, o, k))
    ws = (2.0 ** rng.integers(-8, -4, (E, 1, k // 128))).astype(np.float32)
    experts, routes = omoe.moe_groups(ids)
    sentinel = np.full((r, top, o), 7.0, np.float32)
    out = omoe.fp8_experts(x, w, ws, experts, routes, top, routed_input, out=sentinel)
    counts, proutes = omoe.quantized_routes(ids, np.ones(r, np.int32), E)
    codes, scales = ofp8.quantize(x.reshape(-1, k))
    codes = codes.reshape(*x.shape[:-1], k)
    scales = scales.reshape(*x.shape[:-1], k // 128)
    exp = omoe.expert_partial(codes, scales, w, ws, counts, proutes, top, routed_input=routed_input,
                              out=sentinel)
    np.testing.assert_array_equal(out, exp)
    # a row that no group routes keeps the sentinel
    experts2 = experts.copy()
    experts2[experts2 == ids[0, 0]] = -1
    out2 = omoe.fp8_experts(x, w, ws, experts2, routes, top, routed_input, out=sentinel)
    assert (out2[0, 0] == 7.0).all()
