"""CPU oracle for the DAWN-SRW Select-Read-Write forward.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (the ``dawn-srw_amd``
package, its C-ABI library or its kernels) imports, links or calls this
package.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and there only as the
checker (or, for ``cpu_baseline``, as the timed CPU restatement).

The reference (madst0614/DAWN-SRW) is JAX/Flax; JAX is not installable in
this image, so the reference cannot be imported.  ``srw_ref`` restates its
SRW functions line by line in PyTorch-CPU (fp64 / fp32 / bf16-emulated),
citing ``models/dawn_spatial_v41_exp.py`` (v4.1, the registered model) and
``models/legacy/dawn_spatial_v401_exp.py`` (v4.0.1, the GELU gate).

Pinning status (how each function is checked, see ``tests/test_oracle_*``):

* gate scalar functions: closed forms evaluated in fp64 on a margin grid,
  special cases (intensity == eps below the cutoff, cap at eps+max, GELU
  zero for z <= 0, Phi via the library erf);
* moments / tau: textbook mean / variance in fp64; one-pass vs two-pass
  bound; Gram identity;
* whole layer: brute-force fp64 per-unit loops on tiny inputs (an
  independent formulation, not the matrix form), plus invariants: token
  row independence, unit-permutation equivariance, paired == two singles,
  leave-one-out additivity, den closed form, den floor;
* bf16 emulation: rounding points checked against explicit RNE rounding of
  fp64 results, and the bf16 layer against the fp64 layer within the bf16
  error budget;
* the v4.0.1 fused function (``fused_gate_srw_gelu_v401``): its exact
  (float64) form against the brute-force loop (R / W rows of non-unit norm,
  two chunks), against the pinned ``srw_inference_gelu_v401`` and its
  16-tuple against numpy / scipy closed forms; its bf16 form within the bf16
  budget of the exact form; planted mistakes (den from sum z+, rows not
  normalised, a gate below z = 0, Phi without 1/sqrt 2) are caught;
* ``gate_norm`` of ``srw_inference_with_gates``: against gate / max(sum
  gate, 1e-8) of the brute-force gates, rows summing to one, the 1e-8
  floor, and three plausible wrong normalisers rejected.

Every function of ``srw_ref`` has such a pin (``tests/test_oracle_pins.py``);
``srw_vjp`` is pinned in ``tests/test_backward_oracle.py`` and ``dawn_ref``
in ``tests/test_model_oracle.py``.

The reference ships no tests, golden vectors or fixtures for this path
(its ``tests/`` holds one docstring), and the arithmetic of its bf16 dots
lives in XLA (third-party, version unpinned: ``jax[tpu]>=0.4.1`` in
``requirements_tpu.txt:1-2``).  Bit-level agreement with XLA's bf16 dot
accumulation order and ``jax.nn.sigmoid`` ulps is therefore parity
unpinned; agreement is to tolerance, with a tie band for the passing set.
"""

from .srw_ref import *  # noqa: F401,F403
