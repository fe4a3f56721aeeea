"""ctypes binding of ``libakas_fp8.so`` (the C ABI in ``include/akas_fp8.h``).

The library is loaded after ``torch`` so that its ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch already loaded (same SONAME):
device pointers and streams are then shared between torch and the kernels.
There is no fallback: if the library is missing, every operation raises.
"""

import ctypes
import os

LIBRARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libakas_fp8.so")

F32, F16, BF16 = 0, 1, 2
OK = 0

_p, _i, _i64, _f, _sz = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float,
                         ctypes.c_size_t)

# name -> (restype, argtypes); mirrors include/akas_fp8.h
SIGNATURES = {
    "akas_version": (_i, []),
    "akas_status_string": (ctypes.c_char_p, [_i]),
    "akas_abi_count": (_i, []),
    "akas_quantize": (_i, [_p, _i, _p, _p, _i64, _i64, _p]),
    "akas_rms_quantize": (_i, [_p, _i, _p, _i, _f, _i, _p, _i, _p, _p, _i64, _i64, _p]),
    "akas_dequantize_fp8": (_i, [_p, _p, _p, _i, _i64, _i64, _p]),
    "akas_quantize_weight_blocks": (_i, [_p, _p, _p, _i, _i64, _i64, _i64, _p]),
    "akas_fp8_linear_workspace_size": (_sz, [_i64, _i64, _i64]),
    "akas_fp8_linear": (_i, [_p, _i, _p, _p, _i, _p, _i, _p, _sz, _i64, _i64, _i64, _p]),
    "akas_fp8_linear_noalloc": (_i, [_p, _i, _p, _p, _i, _p, _i, _i64, _i64, _i64, _p]),
    "akas_projection_partial": (_i, [_p, _p, _p, _p, _i, _p, _i, _i64, _i64, _i64, _i, _p]),
    "akas_projection_merge": (_i, [_p, _p, _i, _i64, _i64, _i, _p]),
    "akas_biased_router": (_i, [_p, _p, _p, _p, _i64, _i, _i, _f, _i, _p]),
    "akas_biased_softmax_router": (_i, [_p, _p, _p, _p, _i64, _i, _i, _f, _p]),
    "akas_router": (_i, [_p, _p, _p, _i64, _i, _i, _p]),
    "akas_moe_groups": (_i, [_p, _p, _p, _i64, _i, _p]),
    "akas_router_quantize": (_i, [_p, _p, _p, _p, _i64, _i, _i, _f, _i, _i, _p, _i, _p, _p,
                                  _i64, _p]),
    "akas_fp8_experts_workspace_size": (_sz, [_i64, _i, _i, _i64, _i]),
    "akas_fp8_experts": (_i, [_p, _i, _p, _p, _i, _p, _p, _p, _i, _p, _sz, _i64, _i, _i,
                              _i64, _i64, _i, _p]),
    "akas_quantized_routes": (_i, [_p, _p, _p, _p, _i64, _i, _i, _p]),
    "akas_expert_tile_map": (_i, [_p, _p, _p, _i64, _i, _i, _i, _p]),
    "akas_expert_pack": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i, _i, _i64, _i, _i,
                              _p]),
    "akas_expert_partial": (_i, [_p, _p, _p, _p, _i, _p, _p, _p, _p, _p, _p, _i, _i64, _i, _i,
                                 _i64, _i64, _i, _i, _i, _i, _p]),
    "akas_expert_combine": (_i, [_p, _p, _p, _p, _i, _p, _p, _p, _p, _p, _p, _p, _i, _p, _p, _i64,
                                 _i, _i, _i64, _i64, _i, _i, _i, _p]),
    "akas_fp8_expert_swiglu": (_i, [_p, _p, _p, _p, _p, _p, _i, _p, _p, _p, _p, _p, _p, _p,
                                    _i64, _i, _i, _i64, _i64, _i, _i, _i, _i, _i, _p]),
    "akas_routed_fp8_expert_swiglu": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _p, _p,
                                           _i64, _i, _i, _i64, _i64, _i, _i, _p]),
    "akas_expert_swiglu": (_i, [_p, _p, _p, _p, _p, _p, _i, _p, _p, _p, _p, _p, _p, _i, _i64, _i,
                                _i, _i64, _i64, _i, _i, _i, _i, _i, _p]),
    "akas_expert_pair_partial": (_i, [_p, _p, _p, _p, _p, _p, _i, _p, _p, _p, _p, _p, _p, _i64,
                                      _i, _i, _i64, _i64, _i, _i, _p]),
    "akas_swiglu_experts": (_i, [_p, _p, _i, _p, _i, _i64, _i, _i64, _i, _i, _i, _p]),
    "akas_moe_combine": (_i, [_p, _i, _p, _p, _i, _p, _i, _p, _i64, _i, _i64, _p]),
    "akas_routed_combine": (_i, [_p, _i, _p, _p, _p, _i64, _i, _i64, _p]),
    "akas_shared_expert_moe_workspace_size": (_sz, [_i64, _i, _i, _i64, _i64]),
    "akas_shared_expert_moe": (_i, [_p, _i, _p, _p, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                                    _p, _p, _i, _p, _p, _sz, _i64, _i, _i, _i64, _i64, _p]),
}

_LIB = None


class AkasError(RuntimeError):
    """A C-ABI call returned a launch/runtime failure."""


def load(path=LIBRARY):
    """Load the HIP extension (once) and declare every entry point."""
    global _LIB
    if _LIB is not None:
        return _LIB
    import torch  # noqa: F401  -- load torch's HIP runtime first

    if not os.path.exists(path):
        raise RuntimeError(
            f"HIP extension not built: {path} is missing (run `python -m akas_amd.build`)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def check(status, what):
    """Map a C-ABI status to the reference's exception types."""
    if status == OK:
        return
    text = load().akas_status_string(status).decode()
    if status in (-1, -2, -3, -5, -6):
        raise ValueError(f"{what}: {text}")
    raise AkasError(f"{what}: {text}")
