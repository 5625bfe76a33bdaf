"""Variant (6B release model): the parcae loop of ``var_6b_hip_loop`` with the reference's early
exit switched on (var_6b_adaptive.py:1-30).

The exit is judged on the real output path (readout -> coda -> distogram head): from step 2 on,
the loop stops once the 95th percentile over pairs of the change of the expected distance is
below 0.5 A, hands the exit step's coda output to forward and still draws the skipped steps'
dropout masks. Keyword arguments override single fields of that policy.
"""

from . import var_6b_hip_loop
from .var_6b_hip_loop import ExitPolicy

# The reference's calibrated values (var_6b_adaptive.py:22-24): data, not code.
POLICY = ExitPolicy(adaptive=True, threshold=0.5, source="coda", min_steps=2, burn_rng=True)


def apply(model, **overrides):
    return var_6b_hip_loop.install(model, var_6b_hip_loop.with_policy(POLICY, **overrides))
