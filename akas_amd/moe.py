"""The routed MoE block over block-FP8 experts, composed from the operator kinds.

Mirrors ``routed_moe`` (src/akas/ops/moe/definition.py:29-201) and the
policy rewrites that the LFM2-MoE decode/prefill programs use
(``fused_swiglu``, ``packed``, bf16 intermediate dtypes;
src/akas/ops/moe/definition.py:442-540, 677-793, 951-1053):

    router + quantize(x) (one launch up to 64 experts and top 8)
      -> quantized_routes [-> expert_pack] -> fp8_expert_swiglu (or expert_partial x2 ->
      swiglu_experts -> quantize) -> expert_partial(down, routed_input)
      -> routed_combine (or expert_combine: the down projection with
      routed_combine folded into its epilogue)

The reference program also builds ``expert_tile_map`` between the routes and
the products, because its grouped kernels read their (expert, row tile) from
it.  Here every grouped kernel locates its tile from ``counts`` on the
device, so the block passes no tile map and skips that launch;
``ops.expert_tile_map`` stays available, bit-exact, for callers that want the
table itself.
"""

from dataclasses import dataclass

import torch

from . import ops


@dataclass
class ExpertWeights:
    """Block-FP8 expert banks: gate ``w1``/up ``w3`` ``[E, F, H]`` and down
    ``w2`` ``[E, H, F]`` with 128x128 block scales (f32 or bf16)."""

    w1: torch.Tensor
    s1: torch.Tensor
    w3: torch.Tensor
    s3: torch.Tensor
    w2: torch.Tensor
    s2: torch.Tensor

    @property
    def experts(self):
        return self.w1.shape[0]

    @property
    def hidden(self):
        return self.w1.shape[2]

    @property
    def width(self):
        return self.w1.shape[1]


_ACTIVE = {}


def _all_active(rows, device):
    """Cached all-ones activity mask (filled once per size and device)."""
    key = (rows, str(device))
    if key not in _ACTIVE:
        _ACTIVE[key] = torch.ones(rows, dtype=torch.int32, device=device)
    return _ACTIVE[key]


_SIDE = {}


def _side_stream(device):
    """A second stream per device (default priority) for work that is
    independent of the routed experts."""
    key = str(device)
    if key not in _SIDE:
        _SIDE[key] = torch.cuda.Stream(device=device)
    return _SIDE[key]


@dataclass
class SharedExpert:
    """Dense block-FP8 shared expert: gate ``w1``/up ``w3`` ``[F, H]`` and down
    ``w2`` ``[H, F]`` with 128x128 block scales (f32 or bf16)."""

    w1: torch.Tensor
    s1: torch.Tensor
    w3: torch.Tensor
    s3: torch.Tensor
    w2: torch.Tensor
    s2: torch.Tensor


def _expert_contributions(x, ids, active, weights, *, top, fused_swiglu, packed, max_block_m,
                          product_dtype, activation_dtype, contribution_dtype, quantized=None,
                          partitions=1, combine_weights=None, separate_quantize=False,
                          every_row_active=False):
    """Routes, FP8 activations and the grouped expert products:
    ``[T, top, H]`` contributions in ``contribution_dtype``.  ``quantized``:
    x's codes and scales when the caller made them already.  ``partitions``
    > 1 splits every expert product over K as the reference's partitions
    policy does (src/akas/ops/moe/definition.py:796-948): gate/up through
    expert_pair_partial -> swiglu_experts -> quantize, the down projection
    through expert_partial(partitions) -> expert_merge.

    Returns ``(contributions, counts, routes, combined)``: with
    ``combine_weights`` (and ``partitions`` 1) the down projection is
    ``expert_combine``, which also folds the weighted combine, and
    ``combined`` is its f32 ``[T, H]``; otherwise ``combined`` is None."""
    rows, hidden = x.shape
    experts = weights.experts
    codes, scales = ops.quantize(x) if quantized is None else quantized
    # Unpacked fused SwiGLU: the route scan rides in the gate/up launch
    # (one launch fewer per decode layer, the same tables and codes).
    routed_gate_up = fused_swiglu and not packed and not separate_quantize and partitions == 1
    if routed_gate_up:
        # every_row_active: active is the all-ones mask, which the scan then
        # need not read
        counts, routes, act, act_scales = ops.routed_fp8_expert_swiglu(
            ids, None if every_row_active else active, codes, scales, weights.w1, weights.s1, weights.w3, weights.s3,
            product_dtype=product_dtype, activation_dtype=activation_dtype)
    else:
        counts, routes = ops.quantized_routes(ids, active, experts=experts)
    tile_experts = tile_rows = None  # the kernels locate tiles from counts
    common = dict(r=rows, top=top, max_block_m=max_block_m)
    offsets = None
    if packed:
        codes, scales, offsets = ops.expert_pack(codes, scales, counts, routes, tile_experts,
                                                 tile_rows, top=top, max_block_m=max_block_m)
    # Intermediates are left unfilled: every entry a consumer reads is
    # written -- active rows route all `top` ranks, the expert products read
    # only routed entries and the combine skips inactive rows.
    width = weights.width
    if partitions > 1:
        gate, up = ops.expert_pair_partial(codes, scales, weights.w1, weights.s1, weights.w3,
                                           weights.s3, counts, routes, tile_experts, tile_rows,
                                           partitions=partitions, **common)
        activated = ops.swiglu_experts(gate, up, round_inputs=True, round_dtype=product_dtype,
                                       output_dtype=activation_dtype)
        act, act_scales = ops.quantize(activated, top=top)
        partial = ops.expert_partial(act, act_scales, weights.w2, weights.s2, counts, routes,
                                     tile_experts, tile_rows, routed_input=True,
                                     partitions=partitions, **common)
        return ops.expert_merge(partial, output_dtype=contribution_dtype), counts, routes, None
    if routed_gate_up:
        pass
    elif fused_swiglu and separate_quantize:
        # the paired kernel stores the activations unquantized and quantize
        # follows (_separate_expert_quantize, src/akas/ops/moe/definition.py:
        # 1056-1120): the same codes as the fused epilogue
        activated = ops.expert_swiglu(
            codes, scales, weights.w1, weights.s1, weights.w3, weights.s3, counts, routes,
            tile_experts, tile_rows, offsets, product_dtype=product_dtype,
            activation_dtype=activation_dtype, output_dtype=activation_dtype,
            packed_input=packed, packed_output=packed, **common)
        act, act_scales = ops.quantize(activated) if packed else ops.quantize(activated, top=top)
    elif fused_swiglu:
        act_rows = ((ops.tile_capacity(rows, top, experts, max_block_m) * max_block_m,) if packed
                    else (rows, top))
        act, act_scales = ops.fp8_expert_swiglu(
            codes, scales, weights.w1, weights.s1, weights.w3, weights.s3, counts, routes,
            tile_experts, tile_rows, offsets, product_dtype=product_dtype,
            activation_dtype=activation_dtype, packed_input=packed, packed_output=packed,
            out=torch.empty((*act_rows, width), dtype=torch.uint8, device=x.device),
            output_scales=torch.empty((*act_rows, width // ops.BLOCK), dtype=torch.float32,
                                      device=x.device),
            **common)
    else:
        gate = ops.expert_partial(codes, scales, weights.w1, weights.s1, counts, routes,
                                  tile_experts, tile_rows, output_dtype=product_dtype, **common)
        up = ops.expert_partial(codes, scales, weights.w3, weights.s3, counts, routes,
                                tile_experts, tile_rows, output_dtype=product_dtype, **common)
        activated = ops.swiglu_experts(gate, up, output_dtype=activation_dtype)
        act, act_scales = ops.quantize(activated, top=top)
    contributions = torch.empty((rows, top, hidden), dtype=ops._torch_dtype(contribution_dtype),
                                device=x.device)
    if combine_weights is not None:
        combined, contributions = ops.expert_combine(
            act, act_scales, weights.w2, weights.s2, counts, routes, ids, combine_weights,
            active, offsets, routed_input=not packed, packed_input=packed,
            contribution_dtype=contribution_dtype, contributions=contributions, **common)
        return contributions, counts, routes, combined
    contributions = ops.expert_partial(
        act, act_scales, weights.w2, weights.s2, counts, routes, tile_experts, tile_rows,
        offsets, routed_input=not packed, packed_input=packed, output_dtype=contribution_dtype,
        out=contributions, **common)
    return contributions, counts, routes, None


def routed_moe(x, logits, bias, weights: ExpertWeights, *, top, active=None,
               router="biased_softmax_router", scale=1.0, normalize=True, fused_swiglu=True,
               packed=False, max_block_m=64, product_dtype=torch.float32,
               activation_dtype=torch.float32, contribution_dtype=torch.float32,
               partitions=1, partition_maximum_rows=None, packed_minimum_rows=1,
               fused_quantize_minimum_rows=None, separate_activation_quantize=False,
               block_m=None, fused_combine=False, return_routing=False):
    """One routed MoE feed-forward: ``x [T, H]`` (f32/f16/bf16) -> f32 ``[T, H]``.

    ``partitions`` > 1 applies the reference's K-partition policy to batches
    of at most ``partition_maximum_rows`` rows (all batches when None), as
    its one-row decode seed does (``partitions: 2, partition_maximum_rows:
    1``, src/akas/ops/moe/definition.py:637-652).  ``packed`` packs batches
    of at least ``packed_minimum_rows`` rows, as the packing rewrite does
    (``_pack_experts``, definition.py:951-965; the same seed packs from 2048
    rows, so its decode batches run unpacked).  With ``fused_swiglu``, the
    activations' FP8 quantization is fused into the gate/up launch for
    batches of at least ``fused_quantize_minimum_rows`` rows; smaller
    batches, or all with ``separate_activation_quantize``, store the
    activations unquantized and run quantize after (definition.py:442-540,
    :1056-1120, :1194-1200); the codes are the same.  ``block_m``, the
    rewrite's row tile (16, 32, 64 or 128, at most ``max_block_m``;
    definition.py:1499-1560), is checked as the reference checks it and
    changes nothing else: the grouped kernels pick their row tiles on the
    device, and no row tile changes a result.  ``fused_combine`` folds
    ``routed_combine`` into the down projection's epilogue
    (``expert_combine``, the same result bit for bit).  It is off by default:
    handing every workgroup's contributions to another XCD inside the launch
    costs a device-scope release (an L2 write-back) per workgroup, which on
    MI355X outweighs the combine launch it saves.  With partitions the down
    projection keeps expert_partial -> expert_merge -> routed_combine.
    """
    if router not in ("biased_router", "biased_softmax_router"):
        raise ValueError("unknown routed expert scoring")
    if packed and not fused_swiglu:
        raise ValueError("packing requires the fused SwiGLU pair kernel")
    if fused_quantize_minimum_rows is not None:
        if type(fused_quantize_minimum_rows) is not int or fused_quantize_minimum_rows < 1:
            raise ValueError("expert quantization minimum rows must be a positive integer")
        if not fused_swiglu:
            raise ValueError("expert quantization minimum rows requires SwiGLU fusion")
    if block_m is not None:
        if type(block_m) is not int or block_m not in (16, 32, 64, 128):
            raise ValueError("compact expert block_m must be 16, 32, 64 or 128")
        if block_m > max_block_m:
            raise ValueError("expert row tile exceeds its shared map's maximum")
    rows = x.shape[0]
    separate_quantize = bool(separate_activation_quantize) or (
        fused_quantize_minimum_rows is not None and rows < fused_quantize_minimum_rows)
    if type(packed_minimum_rows) is not int or packed_minimum_rows < 1:
        raise ValueError("expert packing minimum rows must be positive")
    if packed and rows < packed_minimum_rows:
        packed = False
    if partition_maximum_rows is not None and rows > partition_maximum_rows:
        partitions = 1
    if packed:
        # The partitions rewrite splits compact expert calls only; packed
        # calls keep one partition (src/akas/ops/moe/definition.py:796-815),
        # as the reference's seed combining "partitions: 2" with "packed:
        # True" runs (:637-652).
        partitions = 1
    every_row_active = active is None
    if every_row_active:
        active = _all_active(rows, x.device)
    quantized = None
    if weights.experts <= 64 and top <= 8 and x.shape[1] % ops.BLOCK == 0:
        # router and x's quantizer share one launch (they share no data)
        ids, probability, codes, scales = ops.router_quantize(
            logits, bias, x, top=top, softmax=router == "biased_softmax_router", scale=scale,
            normalize=normalize)
        quantized = (codes, scales)
    elif router == "biased_router":
        ids, probability = ops.biased_router(logits, bias, top=top, scale=scale,
                                             normalize=normalize)
    else:
        ids, probability = ops.biased_softmax_router(logits, bias, top=top, scale=scale)
    contributions, counts, routes, out = _expert_contributions(
        x, ids, active, weights, top=top, fused_swiglu=fused_swiglu, packed=packed,
        max_block_m=max_block_m, product_dtype=product_dtype,
        activation_dtype=activation_dtype, contribution_dtype=contribution_dtype,
        quantized=quantized, partitions=partitions,
        combine_weights=probability if fused_combine and partitions == 1 else None,
        separate_quantize=separate_quantize, every_row_active=every_row_active)
    if out is None:
        out = ops.routed_combine(contributions, probability, active)
    if return_routing:
        return out, dict(ids=ids, weights=probability, counts=counts, routes=routes)
    return out


def _group_contributions(x, ids, weights: ExpertWeights, *, top):
    """The routed experts exactly as the block-fp8 decode program emits them
    (src/akas/ops/moe/definition.py:306-343): ``moe_groups`` tables,
    ``fp8_experts`` for gate and up, ``swiglu_experts`` and ``fp8_experts``
    for the down projection on the routed activations -> f32 ``[T, top, H]``."""
    rows = x.shape[0]
    experts, routes = ops.moe_groups(ids)
    shape = (rows, top, weights.width)
    g = ops.fp8_experts(x, weights.w1, weights.s1, experts, routes, top=top,
                        out=torch.empty(shape, dtype=torch.float32, device=x.device))
    u = ops.fp8_experts(x, weights.w3, weights.s3, experts, routes, top=top,
                        out=torch.empty(shape, dtype=torch.float32, device=x.device))
    activated = ops.swiglu_experts(g, u)
    return ops.fp8_experts(activated, weights.w2, weights.s2, experts, routes, top=top,
                           routed_input=True,
                           out=torch.empty((rows, top, x.shape[1]), dtype=torch.float32,
                                           device=x.device))


def shared_expert_moe(x, logits, shared_gate, weights: ExpertWeights, shared: SharedExpert, *,
                      top, fused_swiglu=True, packed=False, max_block_m=64,
                      contribution_dtype=torch.bfloat16, routed_kinds="routes",
                      shared_as_expert=True):
    """The Qwen3.5 block-fp8 MoE block: ``x [T, H]``, router ``logits [T, E]``
    and the shared expert's gate logit ``shared_gate [T]`` (both from the
    caller's bf16 projections) -> f32 ``[T, H]``.

    Router: iterative top-k on the bf16-rounded logits, softmax over the
    selected ones (``decode_router``, src/akas/ops/moe/cuda.py:2011-2050).
    Routed experts as in :func:`routed_moe` (f32 products and activations);
    the shared expert is FP8 gate/up -> SwiGLU -> FP8 down
    (src/akas/ops/moe/definition.py:293-373 decode, :375-418 prefill); the
    combine adds it under its sigmoid gate (``moe_combine``,
    src/akas/ops/moe/cuda.py:392-422).  ``contribution_dtype`` bf16 loses
    nothing: the combine rounds each contribution to bf16 first.

    ``routed_kinds="groups"`` runs the routed experts through the decode
    program's own kinds (``moe_groups`` -> ``fp8_experts`` x2 ->
    ``swiglu_experts`` -> ``fp8_experts``); the default ``"routes"`` uses
    ``quantized_routes`` and the grouped GEMMs above (one fused gate/up
    launch).

    ``shared_as_expert``: with the default routes, fused SwiGLU, unpacked
    rows, a shared expert as wide as the routed ones and one scale dtype, the
    block is ``ops.shared_expert_moe_block``: the shared expert is one more
    expert of the routed launches (rank ``top`` of every row), four launches
    in all for decode batches.  Otherwise, or with ``shared_as_expert=False``, the shared expert
    runs as dense FP8 linears on a second stream beside the routed experts.
    (64 tokens, 256 experts, top 8, H 2048, F 512: 180-181 us with the
    second stream; 168 us without any shared expert.)
    """
    if routed_kinds not in ("routes", "groups"):
        raise ValueError(f"unknown routed_kinds {routed_kinds!r}")
    rows = x.shape[0]
    if (shared_as_expert and routed_kinds == "routes" and fused_swiglu and not packed
            and ops._torch_dtype(contribution_dtype) in (torch.bfloat16, torch.float32)
            and tuple(shared.w1.shape) == tuple(weights.w1.shape[1:])
            and len({t.dtype for t in (weights.s1, weights.s3, weights.s2, shared.s1,
                                       shared.s3, shared.s2)}) == 1):
        # bf16 and f32 contributions give the same result: the combine rounds
        # each one to bf16 before its fold.
        return ops.shared_expert_moe_block(
            x, logits, shared_gate, weights.w1, weights.s1, weights.w3, weights.s3, weights.w2,
            weights.s2, shared.w1, shared.s1, shared.w3, shared.s3, shared.w2, shared.s2, top=top)
    # The shared expert depends only on x: it runs on a second stream while
    # the routed experts stream their weights, and the combine waits for it.
    main = torch.cuda.current_stream(x.device)
    side = _side_stream(x.device)
    width = shared.w1.shape[0]
    side.wait_stream(main)
    x.record_stream(side)  # read on the side stream: not reused before that work ends
    with torch.cuda.stream(side):  # fp8_linear takes the side stream's own workspace
        g = ops.fp8_linear(x, shared.w1, shared.s1)
        u = ops.fp8_linear(x, shared.w3, shared.s3)
        activated = ops.swiglu_experts(g.view(rows, 1, width), u.view(rows, 1, width))
        shared_out = ops.fp8_linear(activated.view(rows, width), shared.w2, shared.s2)
    ids, probability = ops.router(logits, top=top)
    if routed_kinds == "groups":
        contributions = _group_contributions(x, ids, weights, top=top)
    else:
        contributions, _, _, _ = _expert_contributions(
            x, ids, _all_active(rows, x.device), weights, top=top, fused_swiglu=fused_swiglu,
            packed=packed, max_block_m=max_block_m, product_dtype=torch.float32,
            activation_dtype=torch.float32, contribution_dtype=contribution_dtype,
            every_row_active=True)
    main.wait_stream(side)
    shared_out.record_stream(main)  # made on the side stream, read on this one
    return ops.moe_combine(contributions, probability, shared_out, shared_gate)
