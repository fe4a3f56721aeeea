"""Build the gfx950 HIP extension ``akas_amd/lib/libakas_fp8.so`` with hipcc.

Every ``csrc/*.hip`` file is compiled for gfx950 only and linked into one
shared library exposing the C ABI of ``include/akas_fp8.h``.  Object files go
to ``_build/`` at the repository root (ignored by git); the library is built
in-tree so that it travels with the repository snapshot.
"""

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "akas_amd", "csrc")
LIBDIR = os.path.join(ROOT, "akas_amd", "lib")
LIBRARY = os.path.join(LIBDIR, "libakas_fp8.so")
# Probes in a library of their own, not part of the path: the roofline
# ceilings the benchmark reports (HBM streaming read, FP8 MFMA peak, the split
# GEMM's loads) and an exhaustive numerics check the tests run.
PROBE_DIR = os.path.join(CSRC, "probe")
PROBE_LIBRARY = os.path.join(LIBDIR, "libakas_probe.so")
OBJDIR = os.path.join(ROOT, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Only the C ABI (declared with default visibility in include/akas_fp8.h)
    # is exported; kernels and C++ helpers stay internal to the library.
    "-fvisibility=hidden",
    # No packed FP32 instructions anywhere in this library.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the per-block scale FMA reads them directly.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-command-line-argument",
]


def sources(csrc=CSRC):
    return sorted(os.path.join(csrc, f) for f in os.listdir(csrc) if f.endswith(".hip"))


def _compile(src, objdir=OBJDIR):
    sub = "probe_" if os.path.dirname(src) == PROBE_DIR else ""
    obj = os.path.join(objdir, sub + os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose=False, jobs=None):
    """Compile all HIP sources for gfx950 and link the shared library."""
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(OBJDIR, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sources()
    probes = sorted(os.path.join(PROBE_DIR, f) for f in os.listdir(PROBE_DIR) if f.endswith(".hip"))
    jobs = jobs or min(len(srcs) + len(probes), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, srcs + probes))
    for lib, parts in ((LIBRARY, objs[:len(srcs)]), (PROBE_LIBRARY, objs[len(srcs):])):
        tmp = lib + ".tmp"
        # -Bsymbolic-functions: calls inside the library bind to its own definitions.
        cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,-Bsymbolic-functions",
               *parts, "-o", tmp]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
        os.replace(tmp, lib)
    if verbose:
        print(f"built {LIBRARY} from {len(srcs)} sources and {PROBE_LIBRARY}", file=sys.stderr)
    return LIBRARY


def build_tree(csrc, library):
    """Build the path's library from another source tree (for instance an
    earlier commit's ``akas_amd/csrc``, from ``git archive``) into
    ``library``, with this build's flags; for timing builds side by side."""
    objdir = os.path.join(os.path.dirname(os.path.abspath(library)), "_obj")
    os.makedirs(objdir, exist_ok=True)
    srcs = sources(csrc)
    with ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 2)) as pool:
        objs = list(pool.map(lambda s: _compile(s, objdir), srcs))
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,-Bsymbolic-functions", *objs,
           "-o", library]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    shutil.rmtree(objdir)
    return library


if __name__ == "__main__":
    if len(sys.argv) == 4 and sys.argv[1] == "--tree":
        print(build_tree(sys.argv[2], sys.argv[3]))
    else:
        build(verbose=True)
