"""CPU restatement (oracle) of the reference's merged global-attention path.

TEST INFRASTRUCTURE ONLY.  This package is the checker for the gfx950 HIP
kernels: only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import it.  The product package (`4d_ttt_merging_amd`) never
imports it and has no CPU fallback.

Each function restates, in plain PyTorch-CPU / numpy arithmetic, the algorithm
of one reference function (file:line in its docstring, paths relative to the
reference root `vggt_omega/...`).  How each one is pinned (golden fixtures made
from the real reference, closed forms, library routines, invariants):

* attention.mass_bias_attention   — pinned: torch SDPA with a float mask (the
  reference's own fallback, attention.py:400), key-duplication identity for
  integer masses, bias-shift invariance, fp64 brute force.
* projection.top4_project         — pinned: one-hot = gather, uniform = mean,
  fp64 closed form, golden restore fixtures.
* merging.*                       — pinned: golden fixtures written by
  tests/golden/make_fixtures.py from the real reference, plus invariants
  (conservation of mass, keep/removed partition, protected tokens).
"""
