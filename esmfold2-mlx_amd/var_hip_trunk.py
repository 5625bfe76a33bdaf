"""Variant plugin: the whole pair trunk on the HIP kernels (the reference's
``var_mlx_trunk``, var_mlx_trunk.py:24-49).

``apply(model)`` replaces ``model.folding_trunk`` with a ``PairTrunk`` built from its
blocks' weights: forward(pair, pair_attention_mask=None) -> fp32 on pair.device, an
all-ones mask elided, set_chunk_size / set_kernel_backend accepted and ignored.
"""

from __future__ import annotations

from .trunk import PairTrunk


def apply(model) -> None:
    model.folding_trunk = PairTrunk.from_folding_trunk(model.folding_trunk)
