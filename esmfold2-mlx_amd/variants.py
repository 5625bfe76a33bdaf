"""Variants applied by name, in order (the reference's ``apply_variants``, variants.py:74-86).

Each name ``n`` is the module ``var_<n>`` of this package with ``apply(model)``: ``hip_trimul``
(the triangle updates), ``hip_trunk`` (the folding trunk), ``6b_hip_trunks`` (all four trunk
stacks of the 6B release model), ``6b_hip_loop`` (the 6B parcae recycling loop),
``6b_hip_adaptive`` (that loop with its early exit), ``hip_adaptive_loops`` (adaptive
recycling of the trunk). Empty names are skipped; a name with no module raises ValueError,
while an error raised while importing an existing variant propagates as is.
"""

from __future__ import annotations

import importlib

NAMES = ("hip_trimul", "hip_trunk", "6b_hip_trunks", "6b_hip_loop", "6b_hip_adaptive", "hip_adaptive_loops")


def apply_variants(model, names):
    for name in [n for n in names if n]:
        target = f"{__package__}.var_{name}"
        try:
            module = importlib.import_module(target)
        except ModuleNotFoundError as e:
            if e.name != target:
                raise
            raise ValueError(f"unknown variant {name!r}: this package has {', '.join(NAMES)}") from None
        module.apply(model)
    return model
