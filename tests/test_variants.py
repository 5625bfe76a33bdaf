"""The variant loader (the reference's apply_variants, variants.py:74-86) and the 6B
plugin's bookkeeping, on the CPU: no stack is built here."""

import pytest
import torch

from tests import ref_modules


def test_unknown_variant_raises_value_error(pkg):
    model = torch.nn.Module()
    with pytest.raises(ValueError, match="unknown variant 'fast_trunk'"):
        pkg.variants.apply_variants(model, ["fast_trunk"])
    assert pkg.variants.apply_variants(model, ["", ""]) is model  # empty names are skipped


def test_variants_apply_in_order(pkg, monkeypatch):
    seen = []
    for name in ("hip_trimul", "hip_trunk", "6b_hip_trunks"):
        mod = getattr(pkg, f"var_{name}")
        monkeypatch.setattr(mod, "apply", lambda model, name=name: seen.append(name))
    pkg.variants.apply_variants(torch.nn.Module(), ["hip_trunk", "hip_trimul", "6b_hip_trunks"])
    assert seen == ["hip_trunk", "hip_trimul", "6b_hip_trunks"]


def test_6b_plugin_keeps_replaced_stacks_and_a_missing_lm_encoder(pkg):
    model = ref_modules.Model6B([], None, [], [])
    T = pkg.trunk.PairTrunk
    model.folding_trunk, model.parcae_coda, model.confidence_head.folding_trunk = T([]), T([]), T([])
    before = (model.folding_trunk, model.parcae_coda, model.confidence_head.folding_trunk)
    pkg.var_6b_hip_trunks.apply(model)
    assert (model.folding_trunk, model.parcae_coda, model.confidence_head.folding_trunk) == before
    assert model.lm_encoder is None


def test_missing_dependency_inside_a_variant_propagates(pkg, monkeypatch):
    """Only a missing var_<name> module is an unknown variant; a module missing inside an
    existing variant's import is reported as itself (variants.py:79-83)."""
    import importlib

    real = importlib.import_module

    def fake(name, *a, **k):
        if name.endswith(".var_hip_trunk"):
            raise ModuleNotFoundError("No module named 'somedep'", name="somedep")
        return real(name, *a, **k)

    monkeypatch.setattr(importlib, "import_module", fake)
    with pytest.raises(ModuleNotFoundError, match="somedep"):
        pkg.variants.apply_variants(torch.nn.Module(), ["hip_trunk"])
