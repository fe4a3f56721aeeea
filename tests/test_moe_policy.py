"""Host-side checks of the MoE blocks' policy settings (CPU only).

``moe.routed_moe`` and ``moe.shared_expert_moe`` check their settings as the
reference's expert-policy lowering does (src/akas/ops/moe/definition.py:
1185-1230, :1499-1560) before they touch a tensor, so an invalid plan fails
on the host with ValueError; these tests need no GPU and call no kernel.
"""

import pytest


def _blocks():
    import torch
    from akas_amd import moe

    x = torch.zeros((4, 256))
    logits = torch.zeros((4, 8))
    w = torch.zeros((8, 128, 256), dtype=torch.uint8)
    s = torch.ones((8, 1, 2))
    w2 = torch.zeros((8, 256, 128), dtype=torch.uint8)
    s2 = torch.ones((8, 2, 1))
    return moe, x, logits, moe.ExpertWeights(w, s, w, s, w2, s2)


@pytest.mark.parametrize("kw,message", [
    (dict(router="topk"), "scoring"),
    (dict(packed=True, fused_swiglu=False), "packing requires"),
    (dict(fused_quantize_minimum_rows=0), "minimum rows"),
    (dict(fused_quantize_minimum_rows=2.5), "minimum rows"),
    (dict(fused_quantize_minimum_rows=4, fused_swiglu=False), "requires SwiGLU fusion"),
    (dict(block_m=48), "block_m"),
    (dict(block_m=128, max_block_m=64), "exceeds"),
    (dict(packed_minimum_rows=0), "packing minimum rows"),
])
def test_routed_moe_rejects_invalid_policies(kw, message):
    moe, x, logits, wts = _blocks()
    with pytest.raises(ValueError, match=message):
        moe.routed_moe(x, logits, None, wts, top=2, **kw)


def test_shared_expert_moe_rejects_unknown_routed_kinds():
    import torch

    moe, x, logits, wts = _blocks()
    shared = moe.SharedExpert(*(torch.zeros(1) for _ in range(6)))
    with pytest.raises(ValueError, match="routed_kinds"):
        moe.shared_expert_moe(x, logits, torch.zeros(4), wts, shared, top=2,
                              routed_kinds="dense", shared_as_expert=False)
