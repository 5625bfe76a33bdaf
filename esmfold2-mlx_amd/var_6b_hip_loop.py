"""Variant (6B release model): the parcae recycling loop on the HIP kernels, with an optional
early exit once the predicted distances stop changing (the reference's var_6b_mlx_loop,
var_6b_mlx_loop.py:1-35, :116-236).

``apply(model)`` installs ``model._run_one_loop`` as an instance attribute (upstream's
forward calls it by name, var_6b_mlx_loop.py:231) with upstream's signature
``(z, z_init, lm_z, msa_inputs, pair_mask, a, b_mat, tok_mask, total_steps)``. Per step the
dropout stays in PyTorch (upstream's draws in upstream's order); the LM encoder, the parcae
recurrence and the trunk run on the HIP kernels (``recycle.ParcaeLoop`` over ``PairTrunk``s:
stacks already swapped by ``var_6b_hip_trunks`` are used as they are, others are converted).

Early exit (``adaptive=True``): after step k >= min_steps and before the last, the 95th
percentile of |change| of the distogram's expected distance (source "coda": readout ->
coda -> head, the real output path; "readout": readout -> head) below ``threshold`` returns z.
With source "coda" the exit step's coda output is handed on to forward: ``parcae_readout``
and ``parcae_coda`` are wrapped so that forward's readout of the returned z gives that output
and the coda passes it through (var_6b_mlx_loop.py:88-113, :232-234). ``burn_rng`` draws the
skipped steps' dropout masks so later random draws match the full-length fold.
"""

from __future__ import annotations

from torch import nn

from .recycle import ParcaeLoop

# Early-exit policy (off here; var_6b_hip_adaptive sets it), var_6b_mlx_loop.py:46-54.
SOURCE = "coda"
THRESHOLD = None
MIN_STEPS = 2
BURN_RNG = True


class ExitCache(nn.Module):
    """A stand-in for ``parcae_readout`` or ``parcae_coda`` that reuses the loop's exit-step
    coda output: readout(z_exit) returns it, and the coda returns that same tensor unchanged
    (clearing the cache); any other input goes to the wrapped module."""

    def __init__(self, inner: nn.Module, loop: "HipLoop", role: str):
        super().__init__()
        if role not in ("readout", "coda"):
            raise ValueError("role is 'readout' or 'coda'")
        self.inner = inner
        self.__dict__["_loop"] = loop  # not a submodule: the model's state dict is unchanged
        self.role = role

    def set_chunk_size(self, chunk_size):
        if hasattr(self.inner, "set_chunk_size"):
            self.inner.set_chunk_size(chunk_size)

    def set_kernel_backend(self, backend):
        if hasattr(self.inner, "set_kernel_backend"):
            self.inner.set_kernel_backend(backend)

    def forward(self, x, *a, **k):
        loop = self._loop
        if self.role == "readout" and loop.exit_z is not None and x is loop.exit_z:
            return loop.exit_out
        if self.role == "coda" and loop.exit_out is not None and x is loop.exit_out:
            loop.exit_z = loop.exit_out = None
            return x
        return self.inner(x, *a, **k)


def _unwrapped(m):
    return m.inner if isinstance(m, ExitCache) else m


class HipLoop:
    """The loop object ``apply`` installs: ``run`` is upstream's ``_run_one_loop``."""

    def __init__(self, model, adaptive: bool = False, threshold=None, source=None, min_steps=None, burn_rng=None):
        self.model = model
        self.adaptive = bool(adaptive)
        self.threshold = THRESHOLD if threshold is None else threshold
        self.source = source or SOURCE
        self.min_steps = MIN_STEPS if min_steps is None else min_steps
        self.burn_rng = BURN_RNG if burn_rng is None else burn_rng
        if self.adaptive and self.threshold is None:
            raise ValueError("adaptive recycling needs a threshold")

        class _View:  # the model with its readout / coda unwrapped, for ParcaeLoop.from_model
            pass

        view = _View()
        for name in ("lm_encoder", "folding_trunk", "parcae_input_norm", "distogram_head", "config"):
            setattr(view, name, getattr(model, name))
        view.parcae_readout = _unwrapped(model.parcae_readout)
        view.parcae_coda = _unwrapped(model.parcae_coda)
        self.loop = ParcaeLoop.from_model(view, threshold=self.threshold if self.adaptive else None,
                                          source=self.source, min_steps=self.min_steps, burn_rng=self.burn_rng)
        self.exit_z = self.exit_out = None

    @property
    def steps_run(self) -> int:
        return self.loop.steps_run

    @property
    def history(self):
        return self.loop.history

    def run(self, z, z_init, lm_z, msa_inputs, pair_mask, a, b_mat, tok_mask, total_steps):
        m = self.model
        if msa_inputs is not None or getattr(m, "msa_encoder", None) is not None:
            raise NotImplementedError("MSA input is not supported (var_6b_mlx_loop.py:159)")
        if lm_z is None or m.lm_encoder is None:
            raise ValueError("the parcae loop needs lm_z and an lm_encoder")
        if not getattr(m.config.lm_encoder, "per_loop_lm_dropout", False):
            raise ValueError("the loop draws a fresh LM dropout per step (config.lm_encoder.per_loop_lm_dropout)")
        self.exit_z = self.exit_out = None
        z_out = self.loop.run(z, z_init, lm_z, pair_mask, a, b_mat, total_steps)
        if self.loop.exit_out is not None:  # forward's readout -> coda will return this
            self.exit_z, self.exit_out = z_out, self.loop.exit_out
        return z_out


def apply(model, **kw) -> HipLoop:
    loop = HipLoop(model, **kw)
    model._run_one_loop = loop.run  # instance attribute: forward's self._run_one_loop(...) finds it
    if loop.adaptive and loop.source == "coda" and not isinstance(model.parcae_readout, ExitCache):
        model.parcae_readout = ExitCache(model.parcae_readout, loop, "readout")
        model.parcae_coda = ExitCache(model.parcae_coda, loop, "coda")
    elif isinstance(model.parcae_readout, ExitCache):  # re-applied: point the caches at this loop
        model.parcae_readout.__dict__["_loop"] = loop
        model.parcae_coda.__dict__["_loop"] = loop
    model._hip_loop = loop
    return loop
