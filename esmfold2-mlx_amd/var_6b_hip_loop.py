"""Variant (6B release model): the parcae recycling loop on the HIP kernels, with an optional
early exit (the reference's var_6b_mlx_loop; behaviour of var_6b_mlx_loop.py:157-207, plugin
contract of :225-236).

What ``apply(model, **policy)`` installs:

* ``model._run_one_loop`` -- the name upstream's forward calls, with upstream's arguments
  ``(z, z_init, lm_z, msa_inputs, pair_mask, a, b_mat, tok_mask, total_steps)`` -- bound to a
  ``HipLoop``, which runs ``recycle.ParcaeLoop`` over ``PairTrunk`` stacks (stacks that
  ``var_6b_hip_trunks`` already swapped are used as they are). The dropout is drawn by torch in
  upstream's order; the LM encoder, the recurrence and the trunk are HIP kernels.
* With an exit on the coda path (``ExitPolicy.adaptive`` and ``source == "coda"``) the loop has
  already computed ``coda(readout(z))`` for the step it stops at. One ``ExitHandoff`` object owns
  that result until forward consumes it: a forward hook on ``parcae_readout`` swaps the readout
  of the returned ``z`` for the stored coda output, and ``parcae_coda`` is an ``ExitCache`` that
  passes that tensor through instead of running the coda again. Any other input takes the
  ordinary path, and the hand-off is dropped once used.
"""

from __future__ import annotations

import dataclasses
from dataclasses import dataclass

import torch
from torch import nn

from .recycle import ParcaeLoop
from .trunk import relay_trunk_setting

SOURCES = ("coda", "readout")


@dataclass(frozen=True)
class ExitPolicy:
    """When the loop may stop early. ``adaptive=False`` runs every scheduled step. Otherwise,
    after step k >= ``min_steps`` and before the last, the loop stops once the 95th percentile of
    the change of the distogram's expected distance (on ``source``: "coda" = readout -> coda ->
    head, the path forward takes; "readout" = readout -> head) is below ``threshold`` (A).
    ``burn_rng`` still draws the skipped steps' dropout masks, so later random draws match the
    full-length fold (var_6b_mlx_loop.py:46-50)."""

    adaptive: bool = False
    threshold: float | None = None
    source: str = "coda"
    min_steps: int = 2
    burn_rng: bool = True

    def __post_init__(self):
        if self.source not in SOURCES:
            raise ValueError(f"source {self.source!r}: one of {SOURCES}")
        if self.adaptive and self.threshold is None:
            raise ValueError("an adaptive loop needs a threshold")

    @property
    def hands_off_coda(self) -> bool:
        return self.adaptive and self.source == "coda"


class ExitHandoff:
    """The exit step's ``(z, coda output)`` pair, held from the loop's return until forward's
    readout -> coda sequence has consumed it (one use)."""

    def __init__(self):
        self.z = self.out = None

    def arm(self, z: torch.Tensor, out: torch.Tensor) -> None:
        self.z, self.out = z, out

    def clear(self) -> None:
        self.z = self.out = None

    def readout_hook(self, module, args, output):
        """Forward hook of ``parcae_readout``: the readout of the exit ``z`` becomes the coda
        output the loop already computed (returning None keeps the module's own output)."""
        if self.z is not None and args and args[0] is self.z:
            return self.out
        return None

    def pass_through(self, x) -> torch.Tensor | None:
        """For the coda: ``x`` itself if it is the stored output (and the hand-off ends), else None."""
        if self.out is not None and x is self.out:
            self.clear()
            return x
        return None


class ExitCache(nn.Module):
    """``parcae_coda`` under an exit hand-off: the stored coda output passes straight through;
    every other input runs the wrapped coda (``inner``)."""

    def __init__(self, inner: nn.Module, handoff: ExitHandoff):
        super().__init__()
        self.inner = inner
        self.__dict__["handoff"] = handoff  # plain attribute: the state dict keeps the coda's keys only

    def set_chunk_size(self, chunk_size):
        relay_trunk_setting(self.inner, "set_chunk_size", chunk_size)

    def set_kernel_backend(self, backend):
        relay_trunk_setting(self.inner, "set_kernel_backend", backend)

    def forward(self, x, *args, **kwargs):
        done = self.handoff.pass_through(x)
        return self.inner(x, *args, **kwargs) if done is None else done


def _bare_coda(model) -> nn.Module:
    coda = model.parcae_coda
    return coda.inner if isinstance(coda, ExitCache) else coda


class HipLoop:
    """The installed loop: ``run`` has upstream's ``_run_one_loop`` signature."""

    def __init__(self, model, policy: ExitPolicy = ExitPolicy()):
        self.model, self.policy = model, policy
        self.handoff = ExitHandoff()
        self.loop = ParcaeLoop.from_model(
            model, coda=_bare_coda(model), threshold=policy.threshold if policy.adaptive else None,
            source=policy.source, min_steps=policy.min_steps, burn_rng=policy.burn_rng)

    # what a caller inspects after a fold
    steps_run = property(lambda self: self.loop.steps_run)
    history = property(lambda self: self.loop.history)
    exit_z = property(lambda self: self.handoff.z)
    exit_out = property(lambda self: self.handoff.out)

    def _check_inputs(self, msa_inputs, lm_z):
        m = self.model
        if msa_inputs is not None or getattr(m, "msa_encoder", None) is not None:
            raise NotImplementedError("MSA input is not supported (var_6b_mlx_loop.py:159)")
        if lm_z is None or m.lm_encoder is None:
            raise ValueError("the parcae loop needs lm_z and an lm_encoder")
        if not getattr(m.config.lm_encoder, "per_loop_lm_dropout", False):
            raise ValueError("the loop draws a fresh LM dropout per step (config.lm_encoder.per_loop_lm_dropout)")

    def run(self, z, z_init, lm_z, msa_inputs, pair_mask, a, b_mat, tok_mask, total_steps):
        self._check_inputs(msa_inputs, lm_z)
        self.handoff.clear()
        z_out = self.loop.run(z, z_init, lm_z, pair_mask, a, b_mat, total_steps)
        if self.loop.exit_out is not None and self.policy.hands_off_coda:
            self.handoff.arm(z_out, self.loop.exit_out)
        return z_out


def _install_handoff(model, loop: HipLoop) -> None:
    """Wrap the coda once and point it, and a single readout hook, at this loop's hand-off."""
    if not isinstance(model.parcae_coda, ExitCache):
        model.parcae_coda = ExitCache(model.parcae_coda, loop.handoff)
    else:
        model.parcae_coda.__dict__["handoff"] = loop.handoff
    old = model.__dict__.get("_hip_readout_hook")
    if old is not None:
        old.remove()
    model.__dict__["_hip_readout_hook"] = model.parcae_readout.register_forward_hook(loop.handoff.readout_hook)


def install(model, policy: ExitPolicy) -> HipLoop:
    loop = HipLoop(model, policy)
    model._run_one_loop = loop.run  # the instance attribute shadows the class's method
    if policy.hands_off_coda or isinstance(model.parcae_coda, ExitCache):
        _install_handoff(model, loop)  # a re-install also retargets an earlier wrapper
    model._hip_loop = loop
    return loop


def apply(model, **policy) -> HipLoop:
    """Install the loop with ``ExitPolicy(**policy)`` (no early exit by default)."""
    return install(model, ExitPolicy(**policy))


def with_policy(base: ExitPolicy, **overrides) -> ExitPolicy:
    return dataclasses.replace(base, **overrides)
