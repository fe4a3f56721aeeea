"""GPU: akas_fp8_linear_noalloc, the fp8_linear entry point whose workspace is
the library's static device scratch, called through the C ABI and compared
bit for bit with akas_fp8_linear on a caller workspace (the same kernels).

Calls come in pairs on one stream, the second smaller than the first, so
that the second runs on a scratch array still holding the first call's
codes, scales and partials.
"""

import ctypes

import numpy as np
import pytest

from golden_inputs import bf16_normal, block_weights

pytestmark = pytest.mark.gpu

BF16, F32 = 2, 0

# (r, k, o) pairs: every fp8_linear path -- the fused-quantize wide kernel
# (r <= 16), the fragment-major split kernel (17..256 rows), 2048-deep
# partitions with the serial merge (k > 2048), the prefill DMA kernel --
# each followed by a smaller call.
PAIRS = [((256, 2048, 6144), (64, 2048, 6144)),
         ((128, 8192, 2048), (40, 4096, 1040)),
         ((8192, 2048, 6144), (300, 2048, 512)),
         ((16, 2048, 2048), (1, 2048, 2048))]


def _linear(lib, x, w, s, out, ws, r, k, o, stream):
    return lib.akas_fp8_linear(x.data_ptr(), BF16, w.data_ptr(), s.data_ptr(), F32,
                               out.data_ptr(), F32, ws.data_ptr(), ws.numel(), r, k, o, stream)


def _noalloc(lib, x, w, s, out, r, k, o, stream):
    return lib.akas_fp8_linear_noalloc(x.data_ptr(), BF16, w.data_ptr(), s.data_ptr(), F32,
                                       out.data_ptr(), F32, r, k, o, stream)


def _case(dev, r, k, o, seed):
    import torch

    rng = np.random.default_rng(seed)
    codes, scales = block_weights(rng, (o, k))
    x = bf16_normal(rng, (r, k), outliers=0.01)
    return (torch.from_numpy(x).to(torch.bfloat16).to(dev), torch.from_numpy(codes).to(dev),
            torch.from_numpy(scales).to(dev))


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_workspace_entry_point(dev, first, second):
    import torch
    from akas_amd import _lib

    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    for i, (r, k, o) in enumerate((first, second)):
        x, w, s = _case(dev, r, k, o, seed=r + k + o + i)
        need = lib.akas_fp8_linear_workspace_size(r, k, o)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        ref = torch.empty((r, o), dtype=torch.float32, device=dev)
        got = torch.full((r, o), float("nan"), dtype=torch.float32, device=dev)
        assert _linear(lib, x, w, s, ref, ws, r, k, o, stream) == 0
        assert _noalloc(lib, x, w, s, got, r, k, o, stream) == 0
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy())


def test_noalloc_rejects_problems_beyond_the_scratch(dev):
    """A problem whose workspace exceeds the static scratch is refused on
    the host with AKAS_ERR_SCRATCH (the output is left untouched); an empty
    batch is a no-op."""
    import torch
    from akas_amd import _lib

    lib = _lib.load()
    cap = 64 << 20
    r, k, o = 16384, 4096, 2048  # 64 MiB of codes alone
    assert lib.akas_fp8_linear_workspace_size(r, k, o) > cap
    out = torch.zeros((4,), dtype=torch.float32, device=dev)
    p = out.data_ptr()
    assert lib.akas_fp8_linear_noalloc(p, BF16, p, p, F32, p, F32, r, k, o, None) == -6
    assert lib.akas_fp8_linear_noalloc(None, BF16, None, None, F32, None, F32, 0, k, o, None) == 0
    torch.cuda.synchronize()
    assert not out.cpu().numpy().any()
    assert b"static scratch" in lib.akas_status_string(-6)


def test_noalloc_allocates_nothing(dev):
    """torch's allocator sees no new device memory across the calls (the
    static array is part of the loaded code object, not an allocation)."""
    import torch
    from akas_amd import _lib

    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    r, k, o = 256, 2048, 6144
    x, w, s = _case(dev, r, k, o, seed=5)
    out = torch.empty((r, o), dtype=torch.float32, device=dev)
    assert _noalloc(lib, x, w, s, out, r, k, o, stream) == 0
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(dev)
    free_before = torch.cuda.mem_get_info(dev)[0]
    for _ in range(3):
        assert _noalloc(lib, x, w, s, out, r, k, o, stream) == 0
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(dev) == before
    assert torch.cuda.mem_get_info(dev)[0] >= free_before - (2 << 20)
