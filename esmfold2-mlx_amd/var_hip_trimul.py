"""Variant plugin: run every triangle multiplicative update of a model on the HIP path.

Same shape as the reference's variants (variants.py:74-86 imports ``var_<name>`` and
calls ``apply(model)``): ``apply`` patches, in place, the forward of every
triangle-update module it finds, as fast_trunk.apply does (fast_trunk.py:45-64),
with one that runs the three gfx950 kernels and keeps the per-module contract
``forward(pair_grid, visibility=None) -> update``.

Direction: a pair block holds its two updates as ``tri_mul_out`` and ``tri_mul_in``
(the attributes the reference reads, mlx_trunk.py:128), each either the
update module itself or a wrapper whose ``_engine`` is (mlx_trunk.py:41).
"""

from __future__ import annotations

from .trimul import TriMul


def _engine(wrapper):
    return getattr(wrapper, "_engine", wrapper)


def _patch(engine, outgoing: bool) -> None:
    hip = TriMul.from_block(engine, outgoing)
    engine._hip_trimul = hip

    def forward(pair_grid, visibility=None):
        return hip(pair_grid, visibility)

    engine.forward = forward


def apply(model) -> int:
    """Patch every triangle update under ``model``; returns how many were patched."""
    found = []
    for m in model.modules():
        for attr, outgoing in (("tri_mul_out", True), ("tri_mul_in", False)):
            w = getattr(m, attr, None)
            if w is not None and not hasattr(_engine(w), "_hip_trimul"):
                found.append((_engine(w), outgoing))
    for engine, outgoing in found:  # patched after the walk: patching registers a submodule
        _patch(engine, outgoing)
    n = len(found)
    if n == 0:
        raise ValueError("var_hip_trimul: no tri_mul_out / tri_mul_in modules found in the model")
    return n
