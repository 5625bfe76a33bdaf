"""Variant plugin for the 6B release model: every folding-trunk stack on the HIP kernels
(the reference's ``var_6b_mlx_trunks16k``, var_6b_mlx_trunks16k.py:19-32).

The release model has four FoldingTrunk stacks: the main trunk (24 blocks), ``lm_encoder``
(4, absent in some configurations), the parcae coda (2) and the confidence head's trunk (4).
``apply(model)`` replaces each with a ``PairTrunk`` built from its blocks' weights
(``PairTrunk.from_folding_trunk``); a stack that already is one is kept, so the plugin can
follow ``var_hip_trunk`` in a variant list.
"""

from __future__ import annotations

from .trunk import PairTrunk


def _wrap(trunk) -> PairTrunk:
    return trunk if isinstance(trunk, PairTrunk) else PairTrunk.from_folding_trunk(trunk)


def apply(model) -> None:
    model.folding_trunk = _wrap(model.folding_trunk)
    if model.lm_encoder is not None:
        model.lm_encoder = _wrap(model.lm_encoder)
    model.parcae_coda = _wrap(model.parcae_coda)
    model.confidence_head.folding_trunk = _wrap(model.confidence_head.folding_trunk)
