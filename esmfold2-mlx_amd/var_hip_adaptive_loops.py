"""Variant: adaptive recycling of the folding trunk, with its exit signal on the HIP kernels (the
reference's var_adaptive_loops; behaviour of var_adaptive_loops.py:79-156, calibrated constants
:31-37).

Upstream's forward recycles ``z = folding_trunk(z_init + pair_loop_proj(z))`` num_loops + 1
times from z = 0. ``apply(model)`` puts an ``AdaptiveTrunk`` where ``model.folding_trunk`` was
and a forward pre-hook on the model that opens a new ``FoldRecord`` per call, holding the number
of trunk calls the fold will make. Within a fold:

* each trunk pass feeds a ``ChangeMeter``, which measures the change from the previous pass:
  "disto_p95" (the default) is the 95th percentile over pairs of |change| of the distogram
  head's expected distance (128 bins over 2-52 A; one expected-distance and one quantile kernel
  per pass), "z_rel" is |out - prev| / |out|;
* from pass ``min_passes`` on, a change below ``threshold`` settles the fold: that output is
  returned for every later call without running the trunk, which is the fold with fewer loops;
* with ``max_extra`` > 0 (off by default, as upstream), a fold not settled by its last
  scheduled call runs up to that many more passes inside it, continuing the same recurrence
  from ``z_init``. The first call's input is ``z_init + pair_loop_proj(0)``, so ``z_init`` is
  that input minus ``pair_loop_proj(0)``, exactly.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
from torch import nn

from .recycle import DistogramSignal, centers_experimental
from .trunk import relay_trunk_setting

METRICS = ("disto_p95", "z_rel")
# The reference's calibration (var_adaptive_loops.py:31-37): data, not code.
METRIC = "disto_p95"
THRESHOLD = 0.6
MIN_PASSES = 2
MAX_EXTRA = 0


class ChangeMeter:
    """The change of the trunk's output from one pass to the next, within one fold."""

    def __init__(self, metric: str, distogram_head: nn.Module):
        if metric not in METRICS:
            raise ValueError(f"metric {metric!r}: one of {METRICS}")
        self.metric = metric
        self.signal = None
        if metric == "disto_p95":
            w = distogram_head.weight
            self.signal = DistogramSignal(w, distogram_head.bias, centers_experimental(),
                                          device=w.device if w.is_cuda else None)
        self.last = None  # the previous pass's expected distances (or output, for z_rel)

    def restart(self) -> None:
        self.last = None

    def __call__(self, out: torch.Tensor) -> float | None:
        """The change since the previous pass; None on a fold's first pass."""
        cur = out if self.signal is None else self.signal.expected_distance(out)
        prev, self.last = self.last, cur
        if prev is None:
            return None
        if self.signal is not None:
            return DistogramSignal.p95_change(cur, prev)
        o = cur.detach().float()
        return float((o - prev.detach().float()).norm() / o.norm())


@dataclass
class FoldRecord:
    """One fold's progress through the trunk."""

    scheduled: int | None          # trunk calls the fold makes (num_loops + 1); None: not known
    calls: int = 0
    passes: int = 0                # trunk passes actually run
    settled: bool = False
    last: torch.Tensor | None = None
    first_input: torch.Tensor | None = None  # kept only when extra passes may run
    history: list = field(default_factory=list)  # {metric: change} from the second pass on


class AdaptiveTrunk(nn.Module):
    def __init__(self, trunk, model, metric: str = METRIC, threshold: float = THRESHOLD,
                 min_passes: int = MIN_PASSES, max_extra: int = MAX_EXTRA, extra_threshold=None):
        super().__init__()
        self.trunk = trunk
        self.threshold, self.min_passes = threshold, min_passes
        self.max_extra, self.extra_threshold = max_extra, extra_threshold
        self.meter = ChangeMeter(metric, model.distogram_head)
        self.__dict__["loop_proj"] = model.pair_loop_proj  # not a submodule: the state dict is unchanged
        self.new_fold(None)

    metric = property(lambda self: self.meter.metric)
    calls = property(lambda self: self.record.calls)
    passes = property(lambda self: self.record.passes)
    converged = property(lambda self: self.record.settled)
    history = property(lambda self: self.record.history)

    def new_fold(self, scheduled: int | None) -> None:
        self.record = FoldRecord(scheduled)
        self.meter.restart()

    def set_chunk_size(self, chunk_size):
        relay_trunk_setting(self.trunk, "set_chunk_size", chunk_size)

    def set_kernel_backend(self, backend):
        relay_trunk_setting(self.trunk, "set_kernel_backend", backend)

    def _run_trunk(self, pair, mask) -> torch.Tensor:
        out = self.trunk(pair, pair_attention_mask=mask)
        rec = self.record
        rec.passes += 1
        change = self.meter(out)
        if change is not None:
            rec.history.append({self.metric: change})
        rec.last = out
        return out

    def _last_change_below(self, limit: float) -> bool:
        h = self.record.history
        return bool(h) and h[-1][self.metric] < limit

    def _extra_passes(self, out, mask) -> torch.Tensor:
        first = self.record.first_input
        z_init = first - self.loop_proj(torch.zeros_like(first))
        limit = self.threshold if self.extra_threshold is None else self.extra_threshold
        for _ in range(self.max_extra):
            out = self._run_trunk(z_init + self.loop_proj(out), mask)
            if self._last_change_below(limit):
                break
        return out

    def forward(self, pair, pair_attention_mask=None):
        rec = self.record
        rec.calls += 1
        if rec.settled:
            return rec.last
        if rec.calls == 1 and self.max_extra:
            rec.first_input = pair
        out = self._run_trunk(pair, pair_attention_mask)
        if rec.passes >= self.min_passes and self._last_change_below(self.threshold):
            rec.settled = True
        elif self.max_extra and rec.calls == rec.scheduled:
            out = self._extra_passes(out, pair_attention_mask)
        return out


def apply(model, **options) -> AdaptiveTrunk:
    inner = model.folding_trunk
    if isinstance(inner, AdaptiveTrunk):  # applied again: replace the wrapper, not stack a second
        inner = inner.trunk
    trunk = AdaptiveTrunk(inner, model, **options)
    model.folding_trunk = trunk

    def open_fold(module, args, kwargs):
        n = kwargs.get("num_loops")
        trunk.new_fold((module.config.num_loops if n is None else n) + 1)

    old = model.__dict__.get("_hip_fold_hook")
    if old is not None:
        old.remove()
    model.__dict__["_hip_fold_hook"] = model.register_forward_pre_hook(open_fold, with_kwargs=True)
    return trunk
