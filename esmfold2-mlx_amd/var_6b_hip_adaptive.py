"""Variant (6B release model): adaptive recycling for the parcae loop on the HIP kernels
(the reference's var_6b_adaptive, var_6b_adaptive.py:1-30).

``var_6b_hip_loop`` with the early exit on: after step k >= 2, stop once the 95th
percentile over pairs of |change| in the distogram's expected distance (on the real output
path, readout -> coda -> head) is below 0.5 A; the exit step's coda output is handed on to
forward, and the skipped steps' dropout masks are still drawn.
"""

from . import var_6b_hip_loop

THRESHOLD = 0.5  # var_6b_adaptive.py:22 (calibrated by the reference on its own set)
SOURCE = "coda"
MIN_STEPS = 2


def apply(model, **kw):
    cfg = dict(adaptive=True, threshold=THRESHOLD, source=SOURCE, min_steps=MIN_STEPS, burn_rng=True)
    cfg.update(kw)
    return var_6b_hip_loop.apply(model, **cfg)
