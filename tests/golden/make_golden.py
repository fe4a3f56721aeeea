"""Write the golden fixtures in this directory from the oracle.

    python tests/golden/make_golden.py

Inputs come from ``cases.py`` (seeded NumPy, fixed draw order); expected
outputs from the oracle (``oracle/``), which ``tests/test_oracle_*.py`` pin
independently.  Large weight banks are regenerated from their seeds, so the
fixtures hold their SHA-256 instead of the bytes.  ``tests/test_golden.py``
recomputes everything on the CPU and ``tests/test_gpu_golden.py`` checks the
HIP path against these files.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import cases  # noqa: E402


def main():
    for name, build in cases.FIXTURES.items():
        data = build()
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **data)
        print(f"{path}: {os.path.getsize(path)} bytes, {len(data)} arrays")


if __name__ == "__main__":
    main()
