"""Oracle: the recycling step around the trunk, restated in torch.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restated:
  var_6b_mlx_loop.py:67-71   the parcae step: u = z_init + refined (refined = the LM
                             encoder's output), inj = LN(u; w, b, 1e-5),
                             z <- a * z + inj @ B^T, fp32; then the trunk runs on z;
  var_6b_mlx_loop.py:74-76   expected distance per pair: logits = (r + r^T) @ W + b
                             (r^T swaps the two residue axes), softmax over bins, dot
                             the bin centres;
  var_6b_mlx_loop.py:53-54   the 6B head's 64 bins over 2-22 A: centres of 65 edges;
  var_adaptive_loops.py:41-46 the experimental head's 128 bins: 127 edges over 2-52 A,
                             the outer centres 0.2 A past the outer edges;
  var_6b_mlx_loop.py:79-85,  the exit signal: the 95th percentile, with linear
  var_adaptive_loops.py:116  interpolation (torch.quantile), of |change| of the expected
                             distance between consecutive passes.

Pinned by (tests/test_oracle_recycle.py): `quantile` against torch.quantile and
numpy.percentile and a sorted-list formula; `expected_distance` against a per-pair
Python loop and its symmetry (ed[i, j] = ed[j, i]); the parcae step against a
per-cell Python loop; the centres against the edges they come from.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

EPS = 1e-5


def centers_6b() -> torch.Tensor:
    e = torch.linspace(2.0, 22.0, 65, dtype=torch.float64)
    return (e[:-1] + e[1:]) / 2


def centers_experimental() -> torch.Tensor:
    e = torch.linspace(2.0, 52.0, 127, dtype=torch.float64)
    return torch.cat([e[:1] - 0.2, (e[1:] + e[:-1]) / 2, e[-1:] + 0.2])


def parcae_step(z, z_init, refined, ln_w, ln_b, a, b_mat, eps: float = EPS):
    """a * z + LN(z_init + refined) @ B^T on [B, L, L, C]; a [C] (or scalar), B [C, C]."""
    inj = F.layer_norm(z_init + refined, (z.shape[-1],), ln_w, ln_b, eps)
    return a * z + inj @ b_mat.T


def expected_distance(r, w, b, centers):
    """softmax((r + r^T) @ W^T + b) @ centres: r [B, L, L, C], W [NB, C] (a Linear's weight)."""
    logits = (r + r.transpose(1, 2)) @ w.T + b
    return torch.softmax(logits, dim=-1) @ centers


def quantile(x: torch.Tensor, q: float) -> torch.Tensor:
    """q-th quantile of all of x, linear interpolation between the two nearest ranks."""
    v = torch.sort(x.flatten()).values
    pos = q * (v.numel() - 1)
    lo = int(pos)
    hi = min(lo + 1, v.numel() - 1)
    return v[lo] + (pos - lo) * (v[hi] - v[lo])
