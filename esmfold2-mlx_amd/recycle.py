"""The recycling step around the trunk on the HIP path: the 6B model's parcae loop with
its early exit (var_6b_mlx_loop.py: MLXLoop), and the distogram exit signal it and
var_adaptive_loops use.

Per step (var_6b_mlx_loop.py:4-11, :67-71, :172-207):

    lm_z_i = dropout(lm_z, p)                # torch's RNG, upstream's draw order
    u      = z_init + lm_encoder(lm_z_i)     # a short FoldingTrunk (PairTrunk here)
    z      = a * z + LN(u) @ B^T             # parcae_step kernel, fp32 state
    z      = folding_trunk(z)                # PairTrunk

Exit (adaptive): after step k >= min_steps (and before the last), the expected distance
per pair (distogram_expected_distance kernel, on the coda output or the readout) is
compared with the previous step's; when the 95th percentile of |change|
(abs_diff_quantile kernel) is below the threshold, z is returned. On an exit, the
skipped steps' dropout masks are still drawn when ``burn_rng`` (var_6b_mlx_loop.py:46-50),
so later random draws match the full-length fold.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import kernels

F16 = torch.float16


def centers_6b(device=None) -> torch.Tensor:
    """The 6B distogram's 64 bins over 2-22 A (var_6b_mlx_loop.py:53-54)."""
    e = torch.linspace(2.0, 22.0, 65, dtype=torch.float64)
    return ((e[:-1] + e[1:]) / 2).float().to(device)


def centers_experimental(device=None) -> torch.Tensor:
    """The experimental head's 128 bins, 127 edges over 2-52 A (var_adaptive_loops.py:41-42)."""
    e = torch.linspace(2.0, 52.0, 127, dtype=torch.float64)
    return torch.cat([e[:1] - 0.2, (e[1:] + e[:-1]) / 2, e[-1:] + 0.2]).float().to(device)


class DistogramSignal:
    """Expected distance per pair from a distogram head (weight [nbins, C], bias [nbins]),
    and the p95 of its change between consecutive calls."""

    def __init__(self, weight, bias, centers, device=None):
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.w = weight.detach().to(device=dev, dtype=F16).contiguous()
        self.b = bias.detach().to(device=dev, dtype=torch.float32).contiguous()
        self.c = centers.detach().to(device=dev, dtype=torch.float32).contiguous()

    def expected_distance(self, r: torch.Tensor) -> torch.Tensor:
        return kernels.expected_distance(r.float().contiguous(), self.w, self.b, self.c)

    @staticmethod
    def p95_change(ed: torch.Tensor, prev: torch.Tensor) -> float:
        return float(kernels.abs_diff_quantile(ed, prev, 0.95).item())


class ParcaeLoop:
    """The parcae recycling loop (MLXLoop.run, var_6b_mlx_loop.py:157-207) on PairTrunks."""

    def __init__(self, lm_encoder, folding_trunk, ln_w, ln_b, readout_w, signal: DistogramSignal, coda=None,
                 lm_dropout: float = 0.25, threshold: float | None = None, source: str = "coda", min_steps: int = 2,
                 burn_rng: bool = True, eps: float = 1e-5, device=None):
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        if source not in ("coda", "readout") or (source == "coda" and coda is None):
            raise ValueError("source is 'coda' (with a coda trunk) or 'readout'")
        self.lm_encoder, self.trunk, self.coda = lm_encoder, folding_trunk, coda
        f = lambda t: t.detach().to(device=dev, dtype=torch.float32).contiguous()  # noqa: E731
        self.ln_w, self.ln_b, self.eps = f(ln_w), f(ln_b), float(eps)
        self.readout_w = f(readout_w)
        self.signal = signal
        self.p, self.threshold, self.source = lm_dropout, threshold, source
        self.min_steps, self.burn_rng = min_steps, burn_rng
        self.steps_run, self.history = 0, []
        self.exit_out = None  # on an early exit with source "coda": coda(readout(z)) of the exit step

    @classmethod
    def from_model(cls, model, coda=None, **kw) -> "ParcaeLoop":
        """From a 6B-shaped model: lm_encoder, folding_trunk and parcae_coda (FoldingTrunks or
        PairTrunks), parcae_input_norm, parcae_readout, distogram_head, config.lm_encoder.
        ``coda`` replaces ``model.parcae_coda`` (e.g. the module a wrapper holds)."""
        from .trunk import PairTrunk
        trunk = lambda m: m if isinstance(m, PairTrunk) else PairTrunk.from_folding_trunk(m)  # noqa: E731
        if abs(model.parcae_input_norm.eps - 1e-5) > 1e-12:
            raise ValueError("parcae_input_norm.eps must be 1e-5 (var_6b_mlx_loop.py:130)")
        sig = DistogramSignal(model.distogram_head.weight, model.distogram_head.bias,
                              centers_6b() if model.distogram_head.weight.shape[0] == 64 else centers_experimental())
        return cls(trunk(model.lm_encoder), trunk(model.folding_trunk), model.parcae_input_norm.weight,
                   model.parcae_input_norm.bias, model.parcae_readout.weight, sig,
                   coda=trunk(model.parcae_coda if coda is None else coda),
                   lm_dropout=model.config.lm_encoder.lm_dropout, **kw)

    def step(self, z, z_init, lm_z_i, a, b16, mask=None):
        """One recurrence step on fp32 device tensors; returns the trunk's output (fp32)."""
        refined = self.lm_encoder(lm_z_i, mask)
        z = kernels.parcae_step(z, z_init, refined, self.ln_w, self.ln_b, self.eps, a, b16)
        return self.trunk(z, mask)

    def readout(self, z):
        """z @ W_readout^T (a per-cell linear, fp32)."""
        return torch.matmul(z, self.readout_w.T)

    def exit_distance(self, z, mask=None):
        """(expected distance per pair, the coda output or None) if the loop stopped at z."""
        r = self.readout(z)
        if self.source == "coda":
            r = self.coda(r, mask)
            return self.signal.expected_distance(r), r
        return self.signal.expected_distance(r), None

    def run(self, z, z_init, lm_z, pair_mask, a, b_mat, total_steps: int, dropout=None):
        """The loop; ``dropout(lm_z, p)`` defaults to torch's F.dropout(training=True)."""
        drop = dropout or (lambda t, p: F.dropout(t, p=p, training=True))
        mask = None
        if pair_mask is not None and not bool(pair_mask.all()):
            mask = pair_mask
        z, z_init = z.float().contiguous(), z_init.float().contiguous()
        a = a.float().expand(z.shape[-1]).contiguous() if a.numel() == 1 else a.float().contiguous()
        b16 = b_mat.to(F16).contiguous()
        self.history, self.steps_run, prev = [], 0, None
        self.exit_out = None
        adaptive = self.threshold is not None
        for k in range(1, total_steps + 1):
            lm_z_i = drop(lm_z, self.p)
            z = self.step(z, z_init, lm_z_i.to(z_init.dtype).contiguous(), a, b16, mask)
            self.steps_run = k
            if not adaptive or k < self.min_steps - 1 or k == total_steps:
                continue
            ed, out = self.exit_distance(z, mask)
            if k >= self.min_steps and prev is not None:
                d = DistogramSignal.p95_change(ed, prev)
                self.history.append({f"{self.source}_p95": d})
                if d < self.threshold:
                    if self.burn_rng:
                        for _ in range(total_steps - k):
                            drop(lm_z, self.p)
                    self.exit_out = out
                    return z
            prev = ed
        return z
