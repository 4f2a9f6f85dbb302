"""CPU oracle of minispeed's gradient-accumulation boundary step.

TEST INFRASTRUCTURE ONLY.  Nothing in ``minispeed_amd`` imports this
package; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it: as the expected result the GPU
path is compared with (and, for ``bench.py``, as the timed CPU baseline),
never as the thing measured.

Modules
  boundary   torch-CPU restatement of the reference op sequence
             (engine.py:268-322 and everything it calls).  Run on the same
             torch CPU build it reproduces minispeed's bits; pinned by the
             golden vectors under tests/golden/ (made by running minispeed
             itself) and by the reference's known-answer tests.
  recipe     numpy restatement of the per-element arithmetic the HIP kernels
             implement: the same rounding points, an exact fp32 fma and a
             correctly rounded sqrt.  It differs from ``boundary`` only where
             torch's CPU sqrt (MKL) is not correctly rounded.
  (recipe.adamw_f64 is the float64 yardstick for ulp-error bounds.)
"""
