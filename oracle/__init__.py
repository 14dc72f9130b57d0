"""CPU oracle of WarpGBM's hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference's four native operators
(warpgbm/cuda/*.cu) and the reference estimator's tree growth
(warpgbm/core.py).  It is the checker for the HIP implementation in
``warpgbm_amd``: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and never as the thing
that is measured or shipped.

Modules
  ops  -- numpy restatements of the operators (each cites the reference line
          it follows) and of the exact-sum arithmetic the HIP kernels use
  gbm  -- the reference's recursive depth-first tree growth (core.py:597-658)
          and forest loops, on top of ``ops``
  clib -- ctypes loader of ``csrc/oracle.c`` (gcc): exact histograms for
          large inputs and the fma-based exp used by the softmax residuals

How each function is pinned (checked against something other than itself:
brute force, the torch routine the reference calls, closed forms,
invariants) is listed in the header of tests/test_oracle_pins.py, which
covers every function here, including the start values of the fit
(base_score, class_prior_logits, uniform_prior_logits) against torch's own
float32 / float64 evaluation of the reference's expressions.  The literal
float32 growth mode (gbm.Forest(..., literal_f32=True)) is the one part not
held to bit equality: the reference's float32 atomics have no fixed order,
so it is compared tree for tree with the exact mode, every difference
required to be a near-tie.
"""
