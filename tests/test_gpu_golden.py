"""The HIP path against the committed golden fixtures (tests/golden/), through the C ABI."""

import json
import os

import numpy as np
import pytest
import torch

from test_golden import GOLD, mg

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("L", mg.TMU_LS)
@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("masked", [False, True])
def test_trimul_matches_golden(gpu_lib, pkg, L, outgoing, masked):
    gold = np.load(os.path.join(GOLD, "tmu_small.npz"))
    key = f"L{L}_{'out' if outgoing else 'in'}_{'mask' if masked else 'nomask'}"
    _, z, mask, p = mg.tmu_case(L, outgoing, masked)
    m = pkg.trimul.TriMul.from_weights(p)
    got = m(z.to(DEV), None if mask is None else mask.to(DEV)).double().cpu().numpy()
    ref = gold[key + "_y"].astype(np.float64)
    assert np.abs(got - ref).max() <= 1e-2 * np.sqrt((ref ** 2).mean())


def test_L76_fp32_matches_golden(gpu_lib, pkg):
    s = json.load(open(os.path.join(GOLD, "tmu_L76.json")))
    from oracle import tmu
    z, _, po, _ = tmu.make_pair_inputs(76, 128, 128, seed=0, dtype=torch.float32)
    got = pkg.trimul.TriMul.from_weights(po)(z.to(DEV)).double().cpu()
    assert abs(float(got.pow(2).mean().sqrt()) - s["y_rms"]) <= 1e-2 * s["y_rms"]
    np.testing.assert_allclose(got[0, 37, 11, 64:72].numpy(), s["y_37_11_64_72"], atol=1e-2 * s["y_rms"])


def test_q8_matches_golden(gpu_lib, pkg):
    g = np.load(os.path.join(GOLD, "q8_small.npz"))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    w = pkg.kernels.q8_dequant(t(g["q"]), t(g["s"]), t(g["b"])).cpu().numpy()
    assert np.array_equal(w.view(np.uint16), g["w16"])
    y = pkg.kernels.q8_linear(t(g["x"]), t(g["q"]), t(g["s"]), t(g["b"])).cpu().numpy().astype(np.float64)
    assert np.linalg.norm(y - g["y"]) <= 1e-3 * np.linalg.norm(g["y"])
