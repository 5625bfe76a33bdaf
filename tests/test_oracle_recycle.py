"""Pins the recycling-step oracle (oracle/recycle.py)."""

import numpy as np
import torch
import torch.nn.functional as F

from oracle import recycle as rc

D64 = torch.float64


def test_quantile_matches_torch_and_numpy():
    g = torch.Generator().manual_seed(0)
    for n in (1, 2, 7, 1000, 56644):
        x = torch.rand(n, generator=g, dtype=D64) * 3
        for q in (0.0, 0.5, 0.95, 1.0):
            got = rc.quantile(x, q)
            assert torch.isclose(got, torch.quantile(x, q), rtol=0, atol=1e-12)
            assert abs(float(got) - float(np.percentile(x.numpy(), 100 * q))) < 1e-12
    x = torch.tensor([4.0, 1.0, 3.0, 2.0], dtype=D64)  # sorted 1 2 3 4; 0.95 * 3 = 2.85 -> 3 + 0.85
    assert abs(float(rc.quantile(x, 0.95)) - 3.85) < 1e-12


def test_expected_distance_loop_and_symmetry():
    g = torch.Generator().manual_seed(1)
    r = torch.randn(1, 5, 5, 8, generator=g, dtype=D64)
    w, b = torch.randn(64, 8, generator=g, dtype=D64), torch.randn(64, generator=g, dtype=D64)
    c = rc.centers_6b()
    ed = rc.expected_distance(r, w, b, c)
    for i, j in ((0, 0), (1, 3), (4, 2)):
        logit = [float((r[0, i, j] + r[0, j, i]) @ w[k]) + float(b[k]) for k in range(64)]
        m = max(logit)
        p = [np.exp(t - m) for t in logit]
        ref = sum(pk * float(ck) for pk, ck in zip(p, c)) / sum(p)
        assert abs(float(ed[0, i, j]) - ref) < 1e-10
    torch.testing.assert_close(ed, ed.transpose(1, 2), rtol=0, atol=1e-12)
    assert (ed >= c[0]).all() and (ed <= c[-1]).all()


def test_centers():
    c6 = rc.centers_6b()
    assert c6.numel() == 64 and abs(float(c6[0]) - (2 + 10 / 64)) < 1e-12 and abs(float(c6[-1]) - (22 - 10 / 64)) < 1e-12
    ce = rc.centers_experimental()
    assert ce.numel() == 128 and abs(float(ce[0]) - 1.8) < 1e-12 and abs(float(ce[-1]) - 52.2) < 1e-12
    assert (ce[1:] > ce[:-1]).all()


def test_parcae_step_loop():
    g = torch.Generator().manual_seed(2)
    z, zi, rf = (torch.randn(1, 3, 3, 8, generator=g, dtype=D64) for _ in range(3))
    w, bb, a = torch.randn(8, generator=g, dtype=D64), torch.randn(8, generator=g, dtype=D64), \
        torch.rand(8, generator=g, dtype=D64)
    bm = torch.randn(8, 8, generator=g, dtype=D64)
    out = rc.parcae_step(z, zi, rf, w, bb, a, bm)
    u = (zi + rf)[0, 2, 1]
    n = (u - u.mean()) / torch.sqrt(u.var(unbiased=False) + 1e-5) * w + bb
    for co in range(8):
        ref = float(a[co] * z[0, 2, 1, co]) + sum(float(n[ci] * bm[co, ci]) for ci in range(8))
        assert abs(float(out[0, 2, 1, co]) - ref) < 1e-10
