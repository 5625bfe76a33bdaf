"""The committed golden fixtures (tests/golden/) against the oracle and the seeded generators."""

import json
import os

import numpy as np
import pytest
import torch

from oracle import q8, tmu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
import importlib.util  # noqa: E402

_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLD, "make_golden.py"))
mg = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(mg)


@pytest.fixture(scope="module")
def tmu_gold():
    return np.load(os.path.join(GOLD, "tmu_small.npz"))


@pytest.mark.parametrize("L", mg.TMU_LS)
@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("masked", [False, True])
def test_tmu_fixture_inputs_and_oracle(tmu_gold, L, outgoing, masked):
    key = f"L{L}_{'out' if outgoing else 'in'}_{'mask' if masked else 'nomask'}"
    seed, z, mask, p = mg.tmu_case(L, outgoing, masked)
    assert int(tmu_gold[key + "_seed"]) == seed
    assert mg.sha(z.view(torch.int16)) == str(tmu_gold[key + "_zsha"]), "seeded z generator drifted"
    assert mg.sha(p.w_bundle) == str(tmu_gold[key + "_wsha"]), "seeded weight generator drifted"
    y = tmu.trimul(z.double(), None if mask is None else mask.double(), p.to(torch.float64), outgoing)
    np.testing.assert_allclose(y.float().numpy(), tmu_gold[key + "_y"], rtol=1e-5, atol=1e-6)


def test_L76_summary():
    s = json.load(open(os.path.join(GOLD, "tmu_L76.json")))
    z, _, po, _ = tmu.make_pair_inputs(76, 128, 128, seed=0, dtype=torch.float32)
    assert mg.sha(z) == s["z_sha256"] and mg.sha(po.w_bundle) == s["w_bundle_sha256"]
    y = tmu.trimul(z.double(), None, po.to(torch.float64), True).float()
    assert abs(float(y.double().pow(2).mean().sqrt()) - s["y_rms"]) < 1e-6
    np.testing.assert_allclose(y[0, 37, 11, 64:72].numpy(), s["y_37_11_64_72"], rtol=1e-5, atol=1e-6)


def test_q8_fixture():
    g = np.load(os.path.join(GOLD, "q8_small.npz"))
    x, qq, s, b = q8.make_q8_inputs(4, 128, 64, seed=7)
    assert np.array_equal(x, g["x"]) and np.array_equal(qq, g["q"]) and np.array_equal(s, g["s"])
    assert np.array_equal(q8.dequant_f16(qq, s, b).view(np.uint16), g["w16"])
    assert np.array_equal(q8.dequant_f32(qq, s, b).view(np.uint32), g["w32"])
    np.testing.assert_allclose(q8.q8_linear(x, qq, s, b), g["y"], rtol=1e-12)
