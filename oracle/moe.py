"""Routing, permutation, tile maps, packing, expert products and combine (oracle).

Test infrastructure only; see ``oracle/__init__.py``.
"""

import numpy as np

from .fp8 import (
    BLOCK, bf16_round, decode_e4m3, dequantize_activation, dequantize_weight, encode_e4m3,
    fake_quantize, group_scales, quantize, round_to,
)


# --------------------------------------------------------------------------
# routers
# --------------------------------------------------------------------------

def _iterative_topk(scores, top):
    """Top-k by repeated maximum; ties go to the lowest expert index.

    Follows ``src/akas/ops/moe/kernel.py:176-193`` (and ``:467-483``), which is
    the same selection as ``argsort(-scores, kind='stable')[:, :top]``
    (``src/akas/ops/moe/validation.py:142``).
    """
    s = np.array(scores, dtype=np.float32, copy=True)
    rows, experts = s.shape
    ids = np.zeros((rows, top), np.int32)
    for rank in range(top):
        m = s.max(axis=1, keepdims=True)
        first = np.argmax(s == m, axis=1)  # lowest index among the maxima
        ids[:, rank] = first
        s[np.arange(rows), first] = -np.inf
    return ids


_MIDPOINT_MARGIN = 64  # double ulps around a float32 rounding midpoint


def _exp_rn32_exact(v):
    """RN32(e^v) from the exact exponential (mpmath, 200 bits): the nearer of
    the float32 neighbours of e^v, ties to the even one; +inf from the
    overflow threshold 2^128 - 2^103 up (IEEE round-to-nearest)."""
    import mpmath

    with mpmath.workprec(200):
        t = mpmath.exp(mpmath.mpf(float(v)))
        if t >= mpmath.mpf(2) ** 128 - mpmath.mpf(2) ** 103:
            return np.float32(np.inf)
        c = np.float32(float(t))
        if not np.isfinite(c):
            c = np.float32(np.finfo(np.float32).max)
        cands = (np.nextafter(c, np.float32(0)), c, np.nextafter(c, np.float32(np.inf)))
        cands = [f for f in cands if np.isfinite(f)]
        return min(cands, key=lambda f: (abs(mpmath.mpf(float(f)) - t),
                                         int(np.array(f, np.float32).view(np.uint32)) & 1))


def exp_rn32(x):
    """Correctly rounded float32 exponential: the float32 nearest to e^x
    (ties to even) for float32 ``x`` whose result is a normal float32 or
    overflows.

    e^x in float64 rounded once to float32 is that value unless e^x lies
    within a few double ulps of a float32 rounding midpoint (the pattern
    2^28 in the 29 fraction bits below float32 precision).  Results within
    64 double ulps of one (a few dozen of all float32 inputs) are recomputed
    from the exact exponential.  This is the exponential of the reference
    router's float32 expression ``1 / (1 + T.exp(-l))``
    (``src/akas/ops/moe/kernel.py:171``) rounded once, which the device's
    sigmoid router computes as well.
    """
    x = np.asarray(x, np.float32)
    flat = x.ravel()
    with np.errstate(over="ignore"):
        y = np.exp(flat.astype(np.float64))
        out = y.astype(np.float32)
    low = (y.view(np.uint64) & np.uint64((1 << 29) - 1)).astype(np.int64)
    near = (np.abs(low - (1 << 28)) <= _MIDPOINT_MARGIN) & np.isfinite(y) & (y >= 2.0 ** -126)
    for i in np.flatnonzero(near):
        out[i] = _exp_rn32_exact(flat[i])
    return out.reshape(x.shape)


def router_sigmoid(logits):
    """``1 / (1 + exp(-l))`` in float32: correctly rounded exponential, IEEE
    float32 addition and division (``src/akas/ops/moe/kernel.py:171``)."""
    logits = np.asarray(logits, np.float32)
    return (np.float32(1) / (np.float32(1) + exp_rn32(-logits))).astype(np.float32)


def biased_router(logits, bias, top, scale=1.0, normalize=True):
    """Sigmoid scores plus bias select; unbiased sigmoid weights combine.

    ``score = 1/(1+exp(-l)) + b``; weights ``sigmoid(l_sel) * scale / (sum + 1e-6)``
    (``normalize``) or ``sigmoid(l_sel) * scale``.  Follows
    ``src/akas/ops/moe/kernel.py:154-203`` and ``validation.py:138-150``.
    Selection is on the float32 score, every operation rounded once
    (:func:`router_sigmoid`, then an IEEE float32 addition of the bias).
    """
    logits = np.asarray(logits, np.float32)
    sig = router_sigmoid(logits)
    scores = (sig + np.asarray(bias, np.float32)[None, :]).astype(np.float32)
    ids = _iterative_topk(scores, top)
    chosen = np.take_along_axis(sig.astype(np.float64), ids, axis=1)
    if normalize:
        weights = chosen * scale / (chosen.sum(axis=1, keepdims=True) + 1e-6)
    else:
        weights = chosen * scale
    return ids, weights.astype(np.float32)


def biased_softmax_router(logits, bias, top, scale=1.0):
    """Select on ``logits + bias``; softmax over the selected unbiased logits.

    Follows ``src/akas/ops/moe/kernel.py:444-499`` and ``validation.py:708-728``.
    With zero bias this is softmax -> top-k -> renormalise.
    """
    logits = np.asarray(logits, np.float32)
    scores = (logits + np.asarray(bias, np.float32)[None, :]).astype(np.float32)
    ids = _iterative_topk(scores, top)
    selected = np.take_along_axis(logits.astype(np.float64), ids, axis=1)
    p = np.exp(selected - selected.max(axis=1, keepdims=True))
    p *= scale / p.sum(axis=1, keepdims=True)
    return ids, p.astype(np.float32)


def router(logits, top):
    """The block-fp8 decode variant's router (``src/akas/ops/moe/cuda.py:2011-2050``):
    the f32 logits are rounded to bf16, selected by repeated maximum (ties ->
    lowest index) and weighted ``exp(l_j - l_0) / sum_rank exp(l_rank - l_0)``
    over the selected rounded logits, ``l_0`` the first (largest) one."""
    values = bf16_round(np.asarray(logits, np.float32))
    ids = _iterative_topk(values, top)
    selected = np.take_along_axis(values.astype(np.float64), ids, axis=1)
    p = np.exp(selected - selected[:, :1])
    return ids, (p / p.sum(axis=1, keepdims=True)).astype(np.float32)


# --------------------------------------------------------------------------
# routes, tile maps, packing
# --------------------------------------------------------------------------

def quantized_routes(ids, active, experts):
    """Stable expert compaction in (row, rank) order over active rows.

    ``routes[e, i] = row*top + rank`` for the i-th active occurrence of expert
    ``e``; ``counts[e]`` occurrences; the remainder is ``-1``.  Follows
    ``src/akas/ops/moe/kernel.py:121-151`` and ``validation.py:85-99``.
    """
    ids = np.asarray(ids, np.int32)
    active = np.asarray(active, np.int32)
    rows, top = ids.shape
    counts = np.zeros(experts, np.int32)
    routes = np.full((experts, rows), -1, np.int32)
    for row in range(rows):
        if active[row] == 0:
            continue
        for rank in range(top):
            e = int(ids[row, rank])
            if 0 <= e < experts:
                routes[e, counts[e]] = row * top + rank
                counts[e] += 1
    return counts, routes


def moe_groups(ids):
    """The block-fp8 decode variant's route tables
    (``src/akas/ops/moe/cuda.py:1978-2008``).

    Over the flattened ``(row, rank)`` groups ``g`` of ``ids [r, top]``:
    ``experts[g] = ids[g]`` when no earlier group holds that expert, else -1;
    ``routes[g, b]`` = the last rank ``j`` with ``ids[b, j] == experts[g]`` for
    an owning group (-1 when row ``b`` did not select it), all -1 otherwise.
    """
    ids = np.asarray(ids, np.int32)
    r, top = ids.shape
    flat = ids.reshape(-1)
    experts = np.full(r * top, -1, np.int32)
    routes = np.full((r * top, r), -1, np.int32)
    seen = set()
    for g, e in enumerate(flat.tolist()):
        if e in seen:
            continue
        seen.add(e)
        experts[g] = e
        for b in range(r):
            for j in range(top):
                if ids[b, j] == e:
                    routes[g, b] = j
    return experts, routes


def fp8_experts(x, w, scales, experts, routes, top, routed_input=False, out=None):
    """The block-fp8 decode variant's expert products over moe_groups' tables
    (``src/akas/ops/moe/cuda.py:439-531``): each routed row of ``x`` (float,
    ``[r, k]`` or ``[r, top, k]``) is quantized per 1x128 group and
    multiplied by the dequantized ``w[e]`` in float64;
    ``out[b, rank] = x_row . w[e]^T`` for group ``g`` of expert ``e`` and
    ``rank = routes[g, b] >= 0``.  Other entries keep ``out``'s values."""
    x = np.asarray(x, np.float32)
    r, k = x.shape[0], x.shape[-1]
    E, o, _ = w.shape
    out = np.zeros((r, top, o), np.float32) if out is None else np.array(out, np.float32)
    source = fake_quantize(x.reshape(-1, k)).reshape(x.shape).astype(np.float64)
    for g in range(r * top):
        e = int(experts[g])
        if e < 0 or e >= E:
            continue
        weight = dequantize_weight(w[e], scales[e])
        for b in range(r):
            rank = int(routes[g, b])
            if rank < 0 or rank >= top:
                continue
            row = source[b, rank] if routed_input else source[b]
            out[b, rank] = (row @ weight.T).astype(np.float32)
    return out


def tile_capacity(rows, top, experts, block_m):
    """Upper bound of non-empty expert tiles (``src/akas/ops/moe/definition.py:9-16``)."""
    if any(type(v) is not int or v < 1 for v in (rows, top, experts, block_m)):
        raise ValueError("expert tile geometry must contain positive integers")
    routes = rows * top
    return min(routes, (routes + block_m - 1) // block_m + experts - 1)


def tile_layouts(max_block_m=64):
    """Number of power-of-two row layouts 4..max_block_m (``definition.py:19-26``)."""
    if type(max_block_m) is not int or max_block_m not in (4, 8, 16, 32, 64, 128):
        raise ValueError(
            "expert maximum row tile must be a supported power of two from 4 through 128")
    return max_block_m.bit_length() - 2


def map_capacity(rows, top, experts):
    """Columns of the shared tile map: ``(rows*top + 3)//4 + experts``
    (``src/akas/ops/moe/kernel.py:86``)."""
    return (rows * top + 3) // 4 + experts


def expert_tile_map(counts, rows, top, max_block_m=64):
    """Per layout L (row tile ``4 << L``), the ``(expert, tile)`` list.

    Follows ``src/akas/ops/moe/kernel.py:79-118`` and ``validation.py:41-53``.
    Returns ``(tile_experts, tile_rows)`` int32 ``[layouts, capacity]``, padded
    with ``(-1, 0)``.
    """
    counts = np.asarray(counts, np.int32)
    layouts = tile_layouts(max_block_m)
    capacity = map_capacity(rows, top, len(counts))
    experts = np.full((layouts, capacity), -1, np.int32)
    tile_rows = np.zeros((layouts, capacity), np.int32)
    for layout in range(layouts):
        block = 4 << layout
        cursor = 0
        for e, c in enumerate(counts):
            for t in range((int(c) + block - 1) // block):
                experts[layout, cursor] = e
                tile_rows[layout, cursor] = t
                cursor += 1
    return experts, tile_rows


def expert_offsets(counts, alignment):
    """``off[e] = sum_{e'<e} ceil(c_e'/A)*A`` (``src/akas/ops/moe/cuda.py:2461-2469``)."""
    counts = np.asarray(counts, np.int64)
    padded = (counts + alignment - 1) // alignment * alignment
    return np.concatenate([[0], np.cumsum(padded)[:-1]]).astype(np.int32)


def expert_pack(x, activation_scales, counts, routes, top, experts, max_block_m=64,
                routed_input=False, out=None):
    """Copy routed codes/scales into expert-contiguous, A-aligned segments.

    Padding rows hold codes 0 and scale 1; ``expert_offsets`` is written only
    for non-empty experts (untouched entries keep ``out``'s prior value, zero
    by default).  Follows ``src/akas/ops/moe/validation.py:621-642`` and the
    kernel ``src/akas/ops/moe/cuda.py:2423-2502``.
    """
    x = np.asarray(x, np.uint8)
    sc = np.asarray(activation_scales, np.float32)
    rows = x.shape[0]
    depth = x.shape[-1]
    cap = tile_capacity(rows, top, experts, max_block_m) * max_block_m
    if out is None:
        packed = np.zeros((cap, depth), np.uint8)
        packed_scales = np.ones((cap, depth // BLOCK), np.float32)
        offsets = np.zeros(experts, np.int32)
    else:
        packed, packed_scales, offsets = (a.copy() for a in out)
    off = 0
    for e, c in enumerate(np.asarray(counts)):
        c = int(c)
        if not c:
            continue
        offsets[e] = off
        padded = (c + max_block_m - 1) // max_block_m * max_block_m
        packed[off:off + padded] = 0
        packed_scales[off:off + padded] = 1
        for local, route in enumerate(routes[e, :c]):
            row, rank = divmod(int(route), top)
            index = (row, rank) if routed_input else row
            packed[off + local] = x[index]
            packed_scales[off + local] = sc[index]
        off += padded
    return packed, packed_scales, offsets


# --------------------------------------------------------------------------
# expert products
# --------------------------------------------------------------------------

def expert_partial(x, activation_scales, w, scales, counts, routes, top,
                   routed_input=False, partitions=1, output_dtype="float32", out=None):
    """Grouped FP8 expert projection scattered to ``out[row, rank]``.

    ``x``: codes ``[r, k]`` (or ``[r, top, k]`` when ``routed_input``) with
    1x128 scales; ``w``: ``[E, o, k]`` codes with block scales
    ``[E, ceil(o/128), k/128]``.  Rows not routed keep ``out``'s prior values.
    Follows ``src/akas/ops/moe/validation.py:516-583`` (``fp8_experts``) and,
    for ``partitions > 1``, ``validation.py:254-296``.
    """
    x = np.asarray(x, np.uint8)
    r = x.shape[0]
    k = x.shape[-1]
    E, o, _ = w.shape
    activation = dequantize_activation(x, activation_scales).astype(np.float64)
    if out is None:
        shape = (r, top, partitions, o) if partitions > 1 else (r, top, o)
        out = np.zeros(shape, np.float32)
    else:
        out = out.copy()
    span = k // partitions
    for e in range(E):
        c = int(counts[e])
        if not c:
            continue
        weight = dequantize_weight(w[e], scales[e])
        owners, ranks = np.divmod(routes[e, :c].astype(np.int64), top)
        source = activation[owners, ranks] if routed_input else activation[owners]
        if partitions == 1:
            out[owners, ranks] = round_to((source @ weight.T).astype(np.float32), output_dtype)
        else:
            for part in range(partitions):
                seg = slice(part * span, (part + 1) * span)
                out[owners, ranks, part] = source[:, seg] @ weight[:, seg].T
    return out


def swiglu(gate, up, round_dtype=None):
    """``g / (1 + exp(-g)) * u`` in float32 with optional operand rounding.

    Follows ``src/akas/ops/activation/kernel.py:83-88``.
    """
    g = np.asarray(gate, np.float32)
    u = np.asarray(up, np.float32)
    if round_dtype is not None:
        g, u = round_to(g, round_dtype), round_to(u, round_dtype)
    with np.errstate(over="ignore"):  # exp(-g) = inf for g < -88: the quotient is -0
        return (g / (np.float32(1) + np.exp(-g)) * u).astype(np.float32)


def swiglu_experts(gate, up, round_inputs=False, round_dtype="float32", output_dtype="float32"):
    """Expert-row SwiGLU; partitioned inputs ``[r, top, parts, c]`` are summed first.

    Follows ``src/akas/ops/activation/kernel.py:28-88``.
    """
    g = np.asarray(gate, np.float32)
    u = np.asarray(up, np.float32)
    if g.ndim == 4:
        gs = np.zeros(g.shape[:2] + g.shape[3:], np.float32)
        us = np.zeros_like(gs)
        for part in range(g.shape[2]):
            gs += g[:, :, part]
            us += u[:, :, part]
        g, u = gs, us
    out = swiglu(g, u, round_dtype if round_inputs else None)
    return round_to(out, output_dtype)


def _paired_activations(x, activation_scales, w, scales, w2, scales2, counts, routes, top,
                        product_dtype, activation_dtype):
    """Per live expert: ``(owners, ranks, a)`` with ``g, u`` the float32
    products (float64 accumulation) rounded to ``product_dtype`` and
    ``a = silu(g) * u`` rounded to ``activation_dtype``
    (``src/akas/ops/moe/validation.py:385-404``)."""
    x = np.asarray(x, np.uint8)
    source = dequantize_activation(x, activation_scales).astype(np.float64)
    for e in range(w.shape[0]):
        c = int(counts[e])
        if not c:
            continue
        owners, ranks = np.divmod(routes[e, :c].astype(np.int64), top)
        products = [(source[owners] @ dequantize_weight(ww[e], ss[e]).T).astype(np.float32)
                    for ww, ss in ((w, scales), (w2, scales2))]
        g, u = (round_to(v, product_dtype) for v in products)
        yield owners, ranks, round_to(swiglu(g, u), activation_dtype)


def expert_swiglu(x, activation_scales, w, scales, w2, scales2, counts, routes, top,
                  product_dtype="float32", activation_dtype="float32", output_dtype="float32"):
    """The FP8 paired ``expert_swiglu``: gate/up products, SwiGLU, no
    re-quantization -- ``out [r, top, o]`` holds the activation rounded to
    ``output_dtype`` for routed entries, 0 elsewhere.  Follows
    ``src/akas/ops/moe/validation.py:327-410`` with ``quantized_output``
    false (``cuda.py:1531-1534``)."""
    r = np.asarray(x).shape[0]
    out = np.zeros((r, top, w.shape[1]), np.float32)
    for owners, ranks, act in _paired_activations(x, activation_scales, w, scales, w2, scales2,
                                                  counts, routes, top, product_dtype,
                                                  activation_dtype):
        out[owners, ranks] = round_to(act, output_dtype)
    return out


def expert_pair_partial(x, activation_scales, w, scales, w2, scales2, counts, routes, top,
                        partitions=1):
    """``(gate, up)``, each float32 ``[r, top, partitions, o]``: the
    K-partition products of the gate weights ``w`` and the up weights ``w2``
    for every routed (row, rank), 0 elsewhere.  Follows
    ``src/akas/ops/moe/validation.py:299-324`` (both products evaluated
    independently by ``_partial_products``, ``:254-296``)."""
    r = np.asarray(x).shape[0]
    shape = (r, top, partitions, w.shape[1])
    pair = []
    for ww, ss in ((w, scales), (w2, scales2)):
        part = expert_partial(x, activation_scales, ww, ss, counts, routes, top,
                              partitions=partitions)
        pair.append(part.reshape(shape))
    return tuple(pair)


def fp8_expert_swiglu(x, activation_scales, w, scales, w2, scales2, counts, routes, top,
                      product_dtype="float32", activation_dtype="float32"):
    """Fused gate/up products, SwiGLU and per-128-group FP8 re-quantization.

    For each routed (row, rank): ``g, u`` (float32 from float64 products) are
    rounded to ``product_dtype``, ``a = silu(g)*u`` rounded to
    ``activation_dtype``, then ``s = max(max|a|, 1e-12)/448`` per 128 columns and
    ``codes = enc(a/s)``.  Returns ``(codes [r, top, o], scales [r, top, o/128],
    normalized)``; ``normalized`` is ``a/s`` for the reference's midpoint
    tolerance (``src/akas/ops/moe/validation.py:423-432``).  Follows
    ``src/akas/ops/moe/validation.py:327-421``.
    """
    r = np.asarray(x).shape[0]
    o = w.shape[1]
    codes = np.zeros((r, top, o), np.uint8)
    out_scales = np.zeros((r, top, o // BLOCK), np.float32)
    normalized = np.zeros((r, top, o), np.float32)
    for owners, ranks, act in _paired_activations(x, activation_scales, w, scales, w2, scales2,
                                                  counts, routes, top, product_dtype,
                                                  activation_dtype):
        c = owners.size
        blocks = act.reshape(c, o // BLOCK, BLOCK)
        s = group_scales(blocks)
        with np.errstate(invalid="ignore"):  # inf / inf for a group holding inf
            q = (blocks / s[..., None]).astype(np.float32)
        normalized[owners, ranks] = q.reshape(c, o)
        codes[owners, ranks] = encode_e4m3(q).reshape(c, o)
        out_scales[owners, ranks] = s
    return codes, out_scales, normalized


def codes_within_midpoint_band(actual, expected, normalized):
    """Reference tolerance for fused SwiGLU codes: a different code is allowed
    only where ``normalized +- (2e-6|v| + 1e-8)`` straddles a rounding midpoint
    (``src/akas/ops/moe/validation.py:423-432``)."""
    tol = np.abs(normalized) * np.float32(2e-6) + np.float32(1e-8)
    lower = encode_e4m3(normalized - tol)
    upper = encode_e4m3(normalized + tol)
    return (actual == expected) | (actual == lower) | (actual == upper)


def expert_merge(partial, output_dtype="float32"):
    """Serial float32 sum over expert K-partitions ``[r, top, parts, o]``
    (``src/akas/ops/moe/validation.py:196-210``)."""
    p = np.asarray(partial, np.float32)
    total = np.zeros(p.shape[:2] + p.shape[3:], np.float32)
    for part in range(p.shape[2]):
        total += p[:, :, part]
    return round_to(total, output_dtype)


def routed_combine(experts, weights, active):
    """``out[r, c] = sum_rank experts[r, rank, c] * w[r, rank]`` in float32,
    serial rank order; inactive rows are 0.  Follows
    ``src/akas/ops/moe/kernel.py:248-265`` and ``validation.py:152-159``."""
    e = np.asarray(experts, np.float32)
    w = np.asarray(weights, np.float32)
    out = np.zeros((e.shape[0], e.shape[2]), np.float32)
    for rank in range(e.shape[1]):
        out += e[:, rank] * w[:, rank, None]
    out[np.asarray(active) == 0] = 0
    return out


def expert_combine(x, activation_scales, w, scales, counts, routes, ids, weights, active, top,
                   routed_input=False, contribution_dtype="float32"):
    """The down projection with the weighted combine folded in: the
    ``expert_partial`` contributions (``partitions`` 1, rounded to
    ``contribution_dtype``) and ``routed_combine`` over each row's live ranks
    (ids inside ``[0, E)``, the ranks ``quantized_routes`` routes); rows
    without a live rank, and inactive rows, are 0.  Composes
    ``expert_partial`` (``src/akas/ops/moe/cuda.py:541-1354``, scatter
    ``:956-966``) and ``routed_combine`` (``src/akas/ops/moe/kernel.py:206-267``).
    Returns ``(out float32 [r, o], contributions [r, top, o])``."""
    ids = np.asarray(ids, np.int64)
    E = w.shape[0]
    contributions = expert_partial(x, activation_scales, w, scales, counts, routes, top,
                                   routed_input=routed_input, output_dtype=contribution_dtype)
    live = (ids >= 0) & (ids < E)
    out = routed_combine(np.where(live[:, :, None], contributions, 0.0), weights, active)
    return out, contributions


def moe_combine(experts, weights, shared, gate):
    """Weighted top-k combine plus a sigmoid-gated shared expert:
    ``sum_rank bf16(e) * w + bf16(shared) / (1 + exp(-bf16(gate)))``.
    Follows ``src/akas/ops/moe/validation.py:506-515`` (kind ``moe_combine``,
    ``cuda.py:392-422``); the rank sum is float32 in rank order."""
    e = bf16_round(np.asarray(experts, np.float32))
    w = np.asarray(weights, np.float32)
    out = np.zeros((e.shape[0], e.shape[2]), np.float32)
    for rank in range(e.shape[1]):
        out += e[:, rank] * w[:, rank, None]
    g = bf16_round(np.asarray(gate, np.float32).reshape(-1, 1)).astype(np.float64)
    sh = bf16_round(np.asarray(shared, np.float32)).astype(np.float64)
    return (out.astype(np.float64) + sh / (1.0 + np.exp(-g))).astype(np.float32)


# --------------------------------------------------------------------------
# the whole routed MoE layer
# --------------------------------------------------------------------------

def moe_layer(x, logits, bias, w1, s1, w3, s3, w2, s2, top, router="softmax",
              scale=1.0, normalize=True, active=None, activation_dtype="float32",
              contribution_dtype="float32"):
    """One LFM2-style routed MoE feed-forward on block-FP8 experts.

    Router (softmax-top-k or sigmoid+bias), FP8 quantization of ``x``,
    per-expert gate/up products, SwiGLU, FP8 re-quantization of the
    activation, down product and weighted top-k combine.  Follows
    ``tests/support/native_fp8_reference.py:116-144`` with the router of
    ``src/akas/ops/moe/kernel.py:444-499`` for ``router='softmax'``.
    Returns ``(out float32 [T, H], ids, weights)``.
    """
    x = np.asarray(x, np.float32)
    T = x.shape[0]
    if active is None:
        active = np.ones(T, np.int32)
    if router == "softmax":
        ids, prob = biased_softmax_router(logits, bias, top, scale)
    else:
        ids, prob = biased_router(logits, bias, top, scale, normalize)
    source = fake_quantize(x).astype(np.float64)
    E = w1.shape[0]
    contributions = np.zeros((T, top, w2.shape[1]), np.float32)
    for e in range(E):
        owners, ranks = np.nonzero((ids == e) & (np.asarray(active)[:, None] != 0))
        if owners.size == 0:
            continue
        sel = source[owners]
        g = (sel @ dequantize_weight(w1[e], s1[e]).T).astype(np.float32)
        u = (sel @ dequantize_weight(w3[e], s3[e]).T).astype(np.float32)
        g, u = round_to(g, activation_dtype), round_to(u, activation_dtype)
        act = fake_quantize(round_to(swiglu(g, u), activation_dtype)).astype(np.float64)
        prod = (act @ dequantize_weight(w2[e], s2[e]).T).astype(np.float32)
        contributions[owners, ranks] = round_to(prod, contribution_dtype)
    out = routed_combine(contributions, prob, active)
    return out, ids, prob


def shared_expert_moe_layer(x, logits, shared_gate, w1, s1, w3, s3, w2, s2,
                            sw1, ss1, sw3, ss3, sw2, ss2, top):
    """The Qwen3.5 block-fp8 MoE block: routed experts selected by the
    softmax router on bf16-rounded logits (``decode_router``,
    ``src/akas/ops/moe/cuda.py:2011-2050``), a shared expert (FP8 gate/up,
    SwiGLU, FP8 down; ``ops/moe/definition.py:293-373``) and ``moe_combine``
    with the shared expert's sigmoid gate.  Returns float32 ``[T, H]``."""
    x = np.asarray(x, np.float32)
    T = x.shape[0]
    ids, prob = router(logits, top)
    source = fake_quantize(x).astype(np.float64)
    contributions = np.zeros((T, top, w2.shape[1]), np.float32)
    for e in range(w1.shape[0]):
        owners, ranks = np.nonzero(ids == e)
        if owners.size == 0:
            continue
        sel = source[owners]
        g = (sel @ dequantize_weight(w1[e], s1[e]).T).astype(np.float32)
        u = (sel @ dequantize_weight(w3[e], s3[e]).T).astype(np.float32)
        act = fake_quantize(swiglu(g, u)).astype(np.float64)
        contributions[owners, ranks] = (act @ dequantize_weight(w2[e], s2[e]).T).astype(np.float32)
    g = (source @ dequantize_weight(sw1, ss1).T).astype(np.float32)
    u = (source @ dequantize_weight(sw3, ss3).T).astype(np.float32)
    act = fake_quantize(swiglu(g, u)).astype(np.float64)
    shared = (act @ dequantize_weight(sw2, ss2).T).astype(np.float32)
    return moe_combine(contributions, prob, shared, shared_gate)
