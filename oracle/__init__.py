"""CPU oracle for the block-scaled FP8 matrix-product path.

TEST INFRASTRUCTURE ONLY.  This package restates, in plain NumPy (and in the
C file ``cpu_ref.c`` next to it), the reference's CPU equations for the FP8
codec, the 1x128 activation quantizer, the 128x128 block-scaled linear,
expert routing/permutation/tile maps/packing, the grouped expert products,
the fused SwiGLU re-quantization and the weighted top-k combine.  Every
function cites the reference file:line it follows (paths are relative to the
reference repository root, ``src/akas/...`` or ``tests/...``).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import, call, link or execute anything in this directory, and
there only as the reference the results are compared with, or as the timed
CPU baseline.  The product path
(``akas_amd``) never imports it and has no CPU fallback.

Pinning (what each function is checked against, in ``tests/test_oracle_*.py``):

* ``encode_e4m3`` / ``decode_e4m3``: brute force over every code, an
  independent nearest-even search over the 253 finite magnitudes, torch's
  ``float8_e4m3fn`` cast on finite values, and the quantizer stress row of
  ``src/akas/quantization/activations/fp8/validation.py:24``.
* ``bf16_round``: torch's ``bfloat16`` cast (round-to-nearest-even).
* ``quantize``: the stress row known answers and the zero-row scale
  ``1e-12/448``; closed-form round trip bounds.
* ``fp8_linear`` and the expert products: exact-product inputs (integer
  codes with binary scales, ``src/akas/ops/moe/validation.py:327-360``) whose
  float64 result is exact, linearity in the weight scales, and a per-element
  brute-force triple loop on tiny shapes.
* routing, tile maps and packing: brute-force enumerations written
  independently in the tests (stable argsort, explicit loops; the block-fp8
  ``router`` against stable argsort of torch-rounded bf16 logits), the
  deterministic route patterns of ``src/akas/ops/moe/validation.py:82-99`` and
  ``:606-611``, and the empty-batch invariants of ``tests/test_lfm_moe.py``.
* ``moe_groups``: an independent construction (first occurrences from
  ``np.unique``, ranks from the last matching column) and full coverage of
  every (row, rank) pair for distinct ids; ``fp8_experts``: equality with
  the grouped expert products over ``quantized_routes``' tables for the same
  ids, and untouched entries where no group routes.
* ``routed_combine``: explicit per-element loop.
* ``rms_norm`` (``norm.py``): closed forms -- a constant row maps to
  ``sign(c) * w`` as eps -> 0 and to ``c / sqrt(c^2 + eps) * w`` exactly, the
  mean square of the output is 1 for ``w = 1, eps = 0``, invariance under
  scaling of a row when ``eps = 0``, ``zero_centered`` as ``w + 1``, and a
  zero row maps to zero for ``eps > 0``.

No function here is "parity unpinned".
"""
