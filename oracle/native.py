"""Build and load the oracle's C restatement ``oracle/cpu_ref.c``.

Test infrastructure only (see ``oracle/__init__.py``).  The shared library is
written to ``oracle/lib/liboracle_ref.so`` (ignored by git, shipped with the
tree) with gcc -O3 -fopenmp.
"""

import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCE = os.path.join(HERE, "cpu_ref.c")
LIBRARY = os.path.join(HERE, "lib", "liboracle_ref.so")

_LIB = None


def build():
    os.makedirs(os.path.dirname(LIBRARY), exist_ok=True)
    tmp = LIBRARY + ".tmp"
    cmd = ["gcc", "-O3", "-march=x86-64-v2", "-fopenmp", "-fPIC", "-shared", "-std=c11",
           "-ffp-contract=off", SOURCE, "-o", tmp, "-lm"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    os.replace(tmp, LIBRARY)
    return LIBRARY


def load():
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIBRARY) or os.path.getmtime(LIBRARY) < os.path.getmtime(SOURCE):
        build()
    lib = ctypes.CDLL(LIBRARY)
    p, i64, i = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.ref_quantize_bf16.argtypes = [p, p, p, i64, i64, i]
    lib.ref_quantize_bf16.restype = i
    lib.ref_fp8_linear_bf16.argtypes = [p, p, p, p, i, i64, i64, i64, i]
    lib.ref_fp8_linear_bf16.restype = i
    lib.ref_moe_layer_bf16.argtypes = [p, p, p, p, p, p, p, p, p, i64, i64, i64, i, i, i]
    lib.ref_moe_layer_bf16.restype = i
    lib.ref_check_exact_quotient.argtypes = [i64, ctypes.c_uint64, ctypes.POINTER(i64)]
    lib.ref_check_exact_quotient.restype = i64
    lib.ref_encode_e4m3.argtypes = [ctypes.c_float]
    lib.ref_encode_e4m3.restype = ctypes.c_uint8
    lib.ref_decode_e4m3.argtypes = [ctypes.c_uint8]
    lib.ref_decode_e4m3.restype = ctypes.c_float
    _LIB = lib
    return lib


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)
