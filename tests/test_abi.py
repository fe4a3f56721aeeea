"""CPU: the C-ABI library loads and exports every entry point of the header."""

import ctypes
import os
import re

from akas_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "akas_fp8.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(akas_\w+)\s*\(", text)))


def test_header_and_binding_table_agree():
    assert header_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(_lib.LIBRARY)  # dlopen only; nothing touches a GPU
    for name in header_functions():
        assert hasattr(lib, name), name
    lib.akas_abi_count.restype = ctypes.c_int
    assert lib.akas_abi_count() == len(header_functions())
    lib.akas_status_string.restype = ctypes.c_char_p
    assert lib.akas_status_string(0) == b"ok"
    assert lib.akas_status_string(-1) == b"invalid geometry"


def test_host_validation_rejects_before_launch():
    """Invalid geometry returns an error code without touching the device."""
    lib = _lib.load()
    # k not a multiple of 128
    assert lib.akas_quantize(1, 2, 1, 1, 4, 200, None) == -1
    # bad dtype code
    assert lib.akas_quantize(1, 7, 1, 1, 4, 256, None) == -3
    # null pointers with real work
    assert lib.akas_quantize(None, 2, None, None, 4, 256, None) == -2
    # zero rows is a no-op
    assert lib.akas_quantize(None, 2, None, None, 0, 256, None) == 0
    # fused RMSNorm-quantize: channels, dtype, eps, nulls, alignment
    assert lib.akas_rms_quantize(16, 2, 16, 0, 1e-5, 0, None, 2, 16, 16, 4, 200, None) == -1
    assert lib.akas_rms_quantize(16, 2, 16, 0, 1e-5, 0, None, 2, 16, 16, 4, 8320, None) == -1
    assert lib.akas_rms_quantize(16, 2, 16, 1, 1e-5, 0, None, 2, 16, 16, 4, 256, None) == -3
    assert lib.akas_rms_quantize(16, 2, 16, 0, -1.0, 0, None, 2, 16, 16, 4, 256, None) == -1
    assert lib.akas_rms_quantize(None, 2, 16, 0, 1e-5, 0, None, 2, 16, 16, 4, 256, None) == -2
    assert lib.akas_rms_quantize(18, 2, 16, 0, 1e-5, 0, None, 2, 16, 16, 4, 256, None) == -1
    assert lib.akas_rms_quantize(None, 2, None, 0, 1e-5, 0, None, 2, None, None, 0, 256, None) == 0
    # linear: o not a multiple of 16, workspace too small
    assert lib.akas_fp8_linear(1, 2, 1, 1, 0, 1, 0, 1, 1 << 30, 4, 256, 100, None) == -1
    assert lib.akas_fp8_linear(1, 2, 1, 1, 0, 1, 0, 1, 16, 4, 256, 128, None) == -5
    # no-allocation linear: a workspace beyond the static scratch is refused
    # on the host (-6), before the device is touched; no rows is a no-op
    assert lib.akas_fp8_linear_noalloc(1, 2, 1, 1, 0, 1, 0, 16384, 4096, 2048, None) == -6
    assert lib.akas_fp8_linear_noalloc(1, 2, 1, 1, 0, 1, 0, 4, 256, 100, None) == -1
    assert lib.akas_fp8_linear_noalloc(None, 2, None, None, 0, None, 0, 0, 256, 128, None) == 0
    # partitions must divide k/128
    assert lib.akas_projection_partial(1, 1, 1, 1, 0, 1, 0, 4, 384, 128, 2, None) == -1
    # tile map: unsupported maximum row tile
    assert lib.akas_expert_tile_map(1, 1, 1, 4, 8, 2, 48, None) == -1
    # router: top larger than experts
    assert lib.akas_biased_router(1, 1, 1, 1, 4, 8, 9, 1.0, 1, None) == -1
    # block-fp8 router: top above 32 or experts, experts above 1024, nulls, no rows
    assert lib.akas_router(1, 1, 1, 4, 64, 33, None) == -1
    assert lib.akas_router(1, 1, 1, 4, 8, 9, None) == -1
    assert lib.akas_router(1, 1, 1, 4, 1025, 4, None) == -1
    assert lib.akas_router(None, 1, 1, 4, 64, 4, None) == -2
    assert lib.akas_router(None, None, None, 0, 64, 4, None) == 0
    # moe_groups: negative rows, nulls, no rows
    assert lib.akas_moe_groups(1, 1, 1, -1, 4, None) == -1
    assert lib.akas_moe_groups(None, 1, 1, 4, 4, None) == -2
    assert lib.akas_moe_groups(None, None, None, 0, 4, None) == 0
    # fp8_experts: o not a multiple of 128, x dtype code, nulls, workspace
    big = 1 << 30
    assert lib.akas_fp8_experts(1, 2, 1, 1, 0, 1, 1, 1, 0, 1, big, 4, 2, 8, 100, 256, 0, None) == -1
    assert lib.akas_fp8_experts(1, 7, 1, 1, 0, 1, 1, 1, 0, 1, big, 4, 2, 8, 128, 256, 0, None) == -3
    assert lib.akas_fp8_experts(1, 2, 1, 1, 0, None, 1, 1, 0, 1, big, 4, 2, 8, 128, 256, 0, None) == -2
    assert lib.akas_fp8_experts(1, 2, 1, 1, 0, 1, 1, 1, 0, 1, 16, 4, 2, 8, 128, 256, 0, None) == -5
    assert lib.akas_fp8_experts_workspace_size(4, 2, 8, 256, 1) == 8 * 256 + 256 + 256 + 8 * 4 * 4
    # expert partial: o not a multiple of 128
    assert lib.akas_expert_partial(1, 1, 1, 1, 0, 1, 1, 1, 1, None, 1, 0, 4, 2, 4, 100, 256,
                                   0, 1, 64, 0, None) == -1
    # fused swiglu: packed output without packed input
    assert lib.akas_fp8_expert_swiglu(1, 1, 1, 1, 1, 1, 0, 1, 1, 1, 1, 1, 1, 1, 4, 2, 4, 128,
                                      256, 0, 0, 64, 0, 1, None) == -1
    # routes + fused swiglu: o not a multiple of 128, product dtype code,
    # scale dtype code, null x, null counts
    rsw = lambda x, counts, sdt, o, pd: lib.akas_routed_fp8_expert_swiglu(
        1, None, counts, 1, x, 1, 1, 1, 1, 1, sdt, 1, 1, 4, 2, 8, o, 256, pd, 0, None)
    assert rsw(1, 1, 0, 100, 0) == -1
    assert rsw(1, 1, 0, 128, 7) == -3
    assert rsw(1, 1, 1, 128, 0) == -3
    assert rsw(None, 1, 0, 128, 0) == -2
    assert rsw(1, None, 0, 128, 0) == -2
    # shared-expert block: 1024 experts leave no index for the shared one, h
    # not a multiple of 128, gate dtype code, nulls, workspace, no rows
    blk = lambda x, gdt, ws, wsb, r, e, top, h, f: lib.akas_shared_expert_moe(
        x, 2, 1, 1, gdt, *([1] * 12), 0, 16, ws, wsb, r, e, top, h, f, None)
    assert blk(1, 0, 16, big, 4, 1024, 8, 256, 128) == -1
    assert blk(1, 0, 16, big, 4, 32, 8, 200, 128) == -1
    assert blk(1, 0, 16, big, 4, 32, 33, 256, 128) == -1
    assert blk(1, 9, 16, big, 4, 32, 8, 256, 128) == -3
    assert blk(None, 0, 16, big, 4, 32, 8, 256, 128) == -2
    assert blk(1, 0, 16, 64, 4, 32, 8, 256, 128) == -5
    assert blk(1, 0, None, big, 4, 32, 8, 256, 128) == -5
    assert blk(None, 0, None, 0, 0, 32, 8, 256, 128) == 0


def test_workspace_size_formula():
    lib = _lib.load()
    # shared-expert block, 4 rows, 8 experts, top 2, h 256, f 128: ids and
    # weights, x's codes and scales, counts, routes, then 12 ranks' activation
    # codes, scales and bf16 contributions, each 256-byte aligned
    assert lib.akas_shared_expert_moe_workspace_size(4, 8, 2, 256, 128) == (
        256 + 256 + 1024 + 256 + 256 + 256 + 1536 + 256 + 6144)
    assert lib.akas_shared_expert_moe_workspace_size(0, 8, 2, 256, 128) == 0
    assert lib.akas_fp8_linear_workspace_size(16, 2048, 6144) == 16 * 2048 + 16 * 16 * 4
    assert lib.akas_fp8_linear_workspace_size(0, 2048, 6144) == 0
    # codes take whole 16-row tiles (the decode GEMM's fragment-major layout)
    assert lib.akas_fp8_linear_workspace_size(17, 2048, 6144) == 32 * 2048 + 17 * 16 * 4 + 192
    # deeper than 2048 at 17-256 rows: f32 partials of the 2048-deep partitions
    assert lib.akas_fp8_linear_workspace_size(64, 8192, 2048) == 64 * 8192 + 64 * 64 * 4 + 64 * 4 * 2048 * 4
    assert lib.akas_fp8_linear_workspace_size(16, 8192, 2048) == 16 * 8192 + 16 * 64 * 4


def test_ops_refuse_tensors_on_two_devices():
    """The Python kinds run on their tensors' device; device tensors on two
    different devices raise ValueError before the library is called.  (Stand-in
    tensors report a device, so this runs without a GPU.)"""
    import pytest
    import torch

    from akas_amd import ops

    class OnDevice(torch.Tensor):
        @staticmethod
        def __new__(cls, t, index):
            r = torch.Tensor._make_subclass(cls, t)
            r._index = index
            return r

        @property
        def is_cuda(self):
            return True

        @property
        def device(self):
            return torch.device("cuda", self._index)

    x0 = OnDevice(torch.zeros(2, 128), 0)
    codes1 = OnDevice(torch.zeros(2, 128, dtype=torch.uint8), 1)
    w1 = OnDevice(torch.zeros(128, 128, dtype=torch.uint8), 1)
    s1 = OnDevice(torch.zeros(1, 1), 1)
    with pytest.raises(ValueError, match="tensors on cuda:0 and cuda:1"):
        ops.quantize(x0, out=codes1)
    with pytest.raises(ValueError, match="tensors on cuda:0 and cuda:1"):
        ops.fp8_linear(x0, w1, s1)
    with pytest.raises(ValueError, match="tensors on cuda:0 and cuda:1"):
        ops.routed_combine(x0, s1, None)
