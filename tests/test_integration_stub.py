"""CPU: the reference-side registry stub in INTEGRATION.md binds as the
reference's runtime binds a call.

The runtime resolves a call's kernel and passes the call's buffers in the
order of ``kernel.manifest["arguments"]``, looked up by name
(src/akas/execution/plan.py:66-69).  So each launcher of the stub must name
exactly the buffers its kind binds: for ``fp8_linear``, ``x, w, scales, out``
plus ``activation_scales`` in the prequantized (prefill) registration
(src/akas/ops/linear/definition.py:558-568, :942-963).  The stub is run here
against stand-ins for the registry record, the two shared libraries and the
runtime's buffers; the workspace size comes from the real library (a host
function).
"""

import ctypes
import os
import re
import sys
import types

import pytest

from akas_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# The kind's bindings, as the reference's emitter builds them
# (src/akas/ops/linear/definition.py:558-568).
FP8_LINEAR_BINDINGS = {"x", "w", "scales", "out"}
FP8_PREQUANTIZED_BINDINGS = FP8_LINEAR_BINDINGS | {"activation_scales"}


def stub_source():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    found = [b for b in blocks if '"""MI355X (gfx950) provider' in b]
    assert len(found) == 1, "INTEGRATION.md holds one provider stub"
    return found[0]


class _Fn:
    """A library function stand-in: records its calls, returns ``result(args)``."""

    def __init__(self, name, calls, result):
        self.name, self.calls, self.result = name, calls, result

    def __call__(self, *args):
        self.calls.append((self.name, args))
        return self.result(args)


class _Library:
    def __init__(self, calls, results):
        self._calls, self._results = calls, results

    def __getattr__(self, name):
        fn = _Fn(name, self._calls, self._results.get(name, lambda args: 0))
        setattr(self, name, fn)
        return fn


class _Buffer:
    def __init__(self, ptr, dtype):
        self.ptr, self.dtype = ptr, dtype


@pytest.fixture
def stub(monkeypatch):
    calls = []
    real = ctypes.CDLL(_lib.LIBRARY)  # dlopen only; host functions only
    real.akas_fp8_linear_workspace_size.restype = ctypes.c_size_t
    real.akas_fp8_linear_workspace_size.argtypes = [ctypes.c_int64] * 3

    def malloc(args):
        args[0]._obj.value = 0xA000
        return 0

    libs = {
        "hip": _Library(calls, {"hipMalloc": malloc}),
        "akas": _Library(calls, {"akas_fp8_linear_workspace_size":
                                 lambda a: real.akas_fp8_linear_workspace_size(*a)}),
    }
    monkeypatch.setattr(ctypes, "CDLL",
                        lambda name, *a, **k: libs["hip" if "amdhip" in name else "akas"])

    registered = []

    class Implementation:
        def __init__(self, kind, module, contract, **fields):
            registered.append(dict(kind=kind, module=module, contract=contract, **fields))

    pkg = {name: types.ModuleType(name) for name in ("akas", "akas.kernels", "akas.kernels.contracts")}
    pkg["akas.kernels.contracts"].Implementation = Implementation
    for name, mod in pkg.items():
        monkeypatch.setitem(sys.modules, name, mod)
    ns = {"__name__": "akas.ops.mi355x"}
    exec(compile(stub_source(), "INTEGRATION.md:mi355x.py", "exec"), ns)
    return types.SimpleNamespace(ns=ns, calls=calls, registered=registered)


def _spec(**params):
    return types.SimpleNamespace(parameters=params)


def _bind(kernel, buffers, stream):
    """What the runtime does: buffers by the manifest's names, in its order."""
    args = tuple(buffers[item["name"]] for item in kernel.manifest["arguments"])
    kernel(*args, stream=stream)


def test_registrations_cover_both_fp8_linear_factories(stub):
    regs = [r for r in stub.registered if r["kind"] == "fp8_linear"]
    assert {r["phase"] for r in regs} == {"decode", "prefill"}
    for r in regs:
        assert r["provider"] == "rocm"
        assert callable(stub.ns[r["factory"]])


def test_decode_launcher_binds_the_kinds_buffers_on_the_static_scratch(stub):
    kernel = stub.ns["fp8_linear"](_spec(r=16, k=2048, o=6144, input_dtype="bfloat16"), {})
    names = [a["name"] for a in kernel.manifest["arguments"]]
    assert set(names) == FP8_LINEAR_BINDINGS and len(names) == len(FP8_LINEAR_BINDINGS)
    bufs = dict(x=_Buffer(0x100, "bfloat16"), w=_Buffer(0x200, "uint8"),
                scales=_Buffer(0x300, "bfloat16"), out=_Buffer(0x400, "float32"))
    del stub.calls[:]
    _bind(kernel, bufs, stream=77)
    assert stub.calls == [("akas_fp8_linear_noalloc",
                           (0x100, 2, 0x200, 0x300, 2, 0x400, 0, 16, 2048, 6144, 77))]


def test_decode_launcher_beyond_the_scratch_allocates_once_in_the_factory(stub):
    # 8192 x 8192 codes alone are 64 MiB: past the static scratch
    kernel = stub.ns["fp8_linear"](_spec(r=8192, k=8192, o=2048), {})
    mallocs = [c for c in stub.calls if c[0] == "hipMalloc"]
    assert len(mallocs) == 1
    bufs = dict(x=_Buffer(1, "bfloat16"), w=_Buffer(2, "uint8"), scales=_Buffer(3, "float32"),
                out=_Buffer(4, "bfloat16"))
    del stub.calls[:]
    for _ in range(3):
        _bind(kernel, bufs, stream=5)
    assert [c[0] for c in stub.calls] == ["akas_fp8_linear"] * 3
    name, args = stub.calls[0]
    assert args[:7] == (1, 2, 2, 3, 0, 4, 2)
    assert args[7].value == 0xA000 and args[8] > 64 << 20 and args[9:] == (8192, 8192, 2048, 5)


def test_prefill_launcher_binds_codes_and_activation_scales(stub):
    kernel = stub.ns["fp8_linear_prequantized"](_spec(r=8192, k=2048, o=6144), {})
    names = [a["name"] for a in kernel.manifest["arguments"]]
    assert set(names) == FP8_PREQUANTIZED_BINDINGS and len(names) == len(FP8_PREQUANTIZED_BINDINGS)
    bufs = dict(x=_Buffer(0x10, "uint8"), w=_Buffer(0x20, "uint8"), scales=_Buffer(0x30, "bfloat16"),
                activation_scales=_Buffer(0x40, "float32"), out=_Buffer(0x50, "float32"))
    del stub.calls[:]
    _bind(kernel, bufs, stream=9)
    assert stub.calls == [("akas_projection_partial",
                           (0x10, 0x40, 0x20, 0x30, 2, 0x50, 0, 8192, 2048, 6144, 1, 9))]
    assert not any(c[0] == "hipMalloc" for c in stub.calls)


def test_stub_argtypes_match_the_binding_table(stub):
    """The stub's ctypes declarations agree with akas_amd/_lib.py (which
    test_abi checks against the header)."""
    lib = stub.ns["_LIB"]
    for name in ("akas_fp8_linear", "akas_fp8_linear_noalloc", "akas_projection_partial",
                 "akas_fp8_linear_workspace_size"):
        res, args = _lib.SIGNATURES[name]
        assert getattr(lib, name).argtypes == args, name
        assert getattr(lib, name).restype == res, name
