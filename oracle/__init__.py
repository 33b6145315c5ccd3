"""CPU oracle for the Gated DeltaNet hot paths — TEST INFRASTRUCTURE ONLY.

This package is a clean-room CPU restatement of the reference project's PyTorch
implementations (diacccc/GDN_18646 ``reference/*.py`` and the baseline layer in
``gdn_layer.py``).  It is the checker, never the product:

* only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
  ``bench.py`` may import it;
* nothing in ``gdn_18646_amd/`` imports it, and the product path raises when
  its HIP library is missing instead of falling back to anything here.

Modules and the reference code each one restates:

==========================  ==================================================
``oracle.prefill_ref``      ``reference/prefill_ref.py:11-132`` (``ref_prefill``)
                            plus ``ref_prefill_varlen`` (per-sequence loop; the
                            reference has no varlen path)
``oracle.decode_ref``       ``reference/decode_ref.py:10-61`` (``ref_decode``)
``oracle.rmsnorm_ref``      ``reference/rmsnorm_ref.py:8-28`` (``ref_rmsnorm``)
``oracle.proj_ref``         ``reference/fused_proj_conv_silu_ref.py:9-66``
``oracle.recurrence_f64``   the per-token recurrence of the docstring at
                            ``reference/prefill_ref.py:18-23``, in float64 numpy
``oracle.layer_ref``        ``gdn_layer.py:31-200`` (``GDNLayerBaseline``)
==========================  ==================================================

Parity pins (see ``tests/test_oracle_*.py``): every function here is checked
against closed forms, invariants, a float64 brute-force recurrence, library
routines (``torch.linalg.solve_triangular``, ``torch.nn.RMSNorm``,
``F.conv1d``) and brute-force loops on tiny inputs.  The reference ships no
golden vectors or fixtures for this path, so there are none to check against;
the bit-level fp32 operation order of the reference (einsum / cumsum order) is
not reproduced and is "parity unpinned" at the bit level only, well inside the
tolerances the product is held to.
"""
