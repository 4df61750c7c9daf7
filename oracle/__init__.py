"""CPU oracle for the hclsm_amd hot path.  TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference algorithms of RightNow-AI/hclsm's
``hclsm/kernels`` hot path (and the in-model code that owns it) so that the HIP
kernels in ``hclsm_amd`` can be checked against them.  Each function cites the
reference file:line it follows.

Rules that keep it honest:
  * Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
    ``cpu_baseline`` leg may import anything from here, and only as the checker
    (or as the timed CPU baseline).  The product package ``hclsm_amd`` never
    imports it and has no CPU fallback.
  * Every function is pinned by tests in ``tests/test_oracle_*.py`` against
    closed forms, invariants, library routines (torch CPU ops with identical
    weights) or brute force on tiny inputs -- not by re-typing its own formula.

Modules:
  ssm_scan         selective SSM scan forward/backward (raw and model clamp modes)
  slot_attention   slot-attention core and the fused slot-attention iteration
  events           event index / offsets / gather / scatter, varlen event attention
"""
