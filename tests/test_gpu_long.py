"""Pair grids whose tensors pass 2 GB (the old bound was B * L * L * C < 2^30): the triangle
update at ESMFold2's width C = 256 with L = 2100 (z alone is 2.26 GB) and at C = 128 with
L = 2900, both directions, random mask and LayerNorm parameters, and the pair transition at
the same sizes. The whole update cannot be checked on the CPU at this size, so the oracle
evaluates it at 64 sampled cells (oracle.tmu.trimul_cells, which needs only the pair lines
those cells read and is pinned against the full oracle in test_oracle_tmu.py), spread over
the grid's first, middle and last rows and columns. Bar: max|err| <= 1e-2 x RMS of the
update at the sampled cells, as for the other sizes.
"""

import pytest
import torch

from oracle import tmu, transition as otr

pytestmark = pytest.mark.gpu
DEV = "cuda"
F64 = torch.float64


class _Lines:
    """Index a device tensor on demand: the slices the sampled-cell oracle reads, in fp64."""

    def __init__(self, t):
        self.t = t

    def __getitem__(self, key):
        return self.t[key].to(F64).cpu()


def _weights(seed, C):
    g = torch.Generator().manual_seed(seed)
    p = tmu.draw_weights(g, C, C, True)
    p.ln_in_w = 1 + 0.2 * torch.randn(C, generator=g)
    p.ln_in_b = 0.2 * torch.randn(C, generator=g)
    p.ln_mix_w = 1 + 0.2 * torch.randn(C, generator=g)
    p.ln_mix_b = 0.2 * torch.randn(C, generator=g)
    return p


def _sample(L, seed):
    g = torch.Generator().manual_seed(seed)
    picks = [0, 1, L // 3, L // 2, (2 * L) // 3, L - 2, L - 1]
    rows = picks + [int(torch.randint(2, L - 2, (1,), generator=g))]
    cols = picks[::-1] + [int(torch.randint(2, L - 2, (1,), generator=g))]
    return [(0, i, j) for i in rows for j in cols]  # 64 cells


def _bar(got, ref):
    rms = float(ref.pow(2).mean().sqrt())
    err = float((got - ref).abs().max())
    assert torch.isfinite(got).all()
    assert err <= 1e-2 * rms, f"max|err| {err:.3e} > 1e-2 * RMS {rms:.3e}"


@pytest.mark.parametrize("C,L", [(256, 2100), (128, 2900)])
@pytest.mark.parametrize("outgoing", [True, False])
def test_tmu_past_2gb_sampled_cells(gpu_lib, pkg, C, L, outgoing):
    assert L * L * C * 2 > 2 ** 31  # the pair tensor alone passes 2 GB
    print(f"[long] TMU C={C} L={L} outgoing={outgoing}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(C + L + outgoing)
    z = torch.randn(1, L, L, C, generator=g, device=DEV, dtype=torch.float32).to(torch.float16)
    m = (torch.rand(1, L, L, generator=g, device=DEV) > 0.2).to(torch.float16)
    p = _weights(C + outgoing, C)
    p.outgoing = outgoing
    mod = pkg.trimul.TriMul.from_weights(p, device=DEV)
    upd = mod(z, m)
    torch.cuda.synchronize()
    cells = _sample(L, C + L)
    got = torch.stack([upd[0, i, j].to(F64).cpu() for _, i, j in cells])
    del upd
    ref = tmu.trimul_cells(_Lines(z), _Lines(m), p.to(F64), cells, outgoing)
    _bar(got, ref)


@pytest.mark.parametrize("C,L,H,swiglu", [(128, 2900, 512, False), (256, 2100, 512, True)])
def test_transition_past_2gb_sampled_cells(gpu_lib, pkg, C, L, H, swiglu):
    print(f"[long] transition C={C} L={L} H={H} swiglu={swiglu}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(C + H)
    z = torch.randn(1, L, L, C, generator=g, device=DEV, dtype=torch.float32).to(torch.float16)
    gc = torch.Generator().manual_seed(C + H)
    w1 = torch.randn(H, C, generator=gc) * C ** -0.5
    w2 = torch.randn(H, C, generator=gc) * C ** -0.5 if swiglu else None
    w3 = torch.randn(C, H, generator=gc) * H ** -0.5
    lw, lb = 1 + 0.1 * torch.randn(C, generator=gc), 0.1 * torch.randn(C, generator=gc)
    tr = pkg.trunk.PairTransition(lw, lb, w1, w3, w2=w2, device=DEV)
    out = tr(z)
    torch.cuda.synchronize()
    cells = _sample(L, C + H)
    zc = torch.stack([z[0, i, j].to(F64).cpu() for _, i, j in cells])
    got = torch.stack([out[0, i, j].to(F64).cpu() for _, i, j in cells])
    del out
    pw = otr.TransitionWeights(lw.double(), lb.double(), w1.half().double(), w3.half().double(),
                               None if w2 is None else w2.half().double())
    ref = otr.transition(zc, pw)
    _bar(got - zc, ref - zc)
