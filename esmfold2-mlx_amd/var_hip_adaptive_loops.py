"""Variant: adaptive recycling of the folding trunk (the reference's var_adaptive_loops,
var_adaptive_loops.py:1-23, :79-156), with its exit signal on the HIP kernels.

Wraps whatever ``model.folding_trunk`` is (apply it last, e.g. after ``var_hip_trunk``).
Per fold it compares each trunk output with the previous one; once the change is below the
threshold it returns that output for every remaining call without running the trunk, which
makes the fold identical to one run with fewer loops. ``model.forward`` is wrapped (an
instance attribute) to reset the state and learn the scheduled number of passes.

Signal ("disto_p95", the default): the 95th percentile over pairs of |change| of the
distogram head's expected distance (128 bins over 2-52 A), one ``distogram_expected_distance``
and one ``abs_diff_quantile`` launch per pass; "z_rel" is |out - prev| / |out|.

Extra passes (``max_extra``, off by default as in the reference): forward's loop is
``z = trunk(z_init + pair_loop_proj(z))``; the first call's input is
``z_init + pair_loop_proj(0)``, so z_init is recovered exactly and extra passes inside the
last scheduled call repeat the same recurrence.
"""

from __future__ import annotations

import torch
from torch import nn

from .recycle import DistogramSignal, centers_experimental

METRIC = "disto_p95"
THRESHOLD = 0.6   # var_adaptive_loops.py:32 (the reference's calibration)
MIN_PASSES = 2    # a comparison needs two passes
MAX_EXTRA = 0
METRICS = ("disto_p95", "z_rel")


class AdaptiveTrunk(nn.Module):
    def __init__(self, trunk, model, metric: str = METRIC, threshold: float = THRESHOLD,
                 min_passes: int = MIN_PASSES, max_extra: int = MAX_EXTRA, extra_threshold=None):
        super().__init__()
        if metric not in METRICS:
            raise ValueError(f"metric {metric!r}: one of {METRICS}")
        self.trunk = trunk
        # plain attributes (not submodules), so the model's state dict is unchanged
        self.__dict__["_proj"] = model.pair_loop_proj
        head = model.distogram_head
        self.__dict__["_signal"] = None if metric != "disto_p95" else DistogramSignal(
            head.weight, head.bias, centers_experimental(), device=head.weight.device if head.weight.is_cuda else None)
        self.metric, self.threshold, self.min_passes = metric, threshold, min_passes
        self.max_extra = max_extra
        self.extra_threshold = threshold if extra_threshold is None else extra_threshold
        self.reset(None)

    def set_chunk_size(self, chunk_size):
        if hasattr(self.trunk, "set_chunk_size"):
            self.trunk.set_chunk_size(chunk_size)

    def set_kernel_backend(self, backend):
        if hasattr(self.trunk, "set_kernel_backend"):
            self.trunk.set_kernel_backend(backend)

    def reset(self, scheduled_passes):
        self.scheduled = scheduled_passes
        self.calls = 0
        self.passes = 0     # trunk passes actually run
        self.prev = self.prev_ed = None
        self.z_init = None
        self.converged = False
        self.history = []   # the metric after each pass from the second on

    def _pass(self, pair, mask):
        out = self.trunk(pair, pair_attention_mask=mask)
        self.passes += 1
        if self.metric == "disto_p95":
            ed = self._signal.expected_distance(out)
            if self.prev_ed is not None:
                self.history.append({"disto_p95": DistogramSignal.p95_change(ed, self.prev_ed)})
            self.prev_ed = ed
        elif self.prev is not None:
            o, p = out.float(), self.prev.float()
            self.history.append({"z_rel": float((o - p).norm() / o.norm())})
        self.prev = out
        return out

    def forward(self, pair, pair_attention_mask=None):
        self.calls += 1
        if self.converged:
            return self.prev  # the same as a fold with fewer loops
        if self.calls == 1 and self.max_extra:
            self.z_init = pair - self._proj(torch.zeros_like(pair))
        out = self._pass(pair, pair_attention_mask)
        if self.passes >= self.min_passes and self.history[-1][self.metric] < self.threshold:
            self.converged = True
            return out
        if self.scheduled is not None and self.calls == self.scheduled and self.max_extra:
            for _ in range(self.max_extra):
                out = self._pass(self.z_init + self._proj(out), pair_attention_mask)
                if self.history[-1][self.metric] < self.extra_threshold:
                    break
        return out


def apply(model, **kw) -> AdaptiveTrunk:
    trunk = AdaptiveTrunk(model.folding_trunk, model, **kw)
    model.folding_trunk = trunk
    forward = model.forward

    def adaptive_forward(*a, num_loops=None, **k):
        n = num_loops if num_loops is not None else model.config.num_loops
        trunk.reset(n + 1)
        return forward(*a, num_loops=num_loops, **k)

    model.forward = adaptive_forward  # nn.Module.__call__ dispatches to the instance attribute
    return trunk
