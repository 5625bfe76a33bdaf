"""GPU parity of the TMU pair entry point, tmu_pair_forward (TriMulPair): the outgoing
update with its residual, then the incoming one in place, in one C call.

Checked against the fp64 oracle at the module bar, max|err| <= 1e-2 * RMS(update), with
random LayerNorm parameters, masks and batches, and bit for bit against the two updates
run one after the other through tmu_forward (at C = 128 and in the 256-wide path).
"""

import pytest
import torch

from oracle import tmu

pytestmark = pytest.mark.gpu

DEV = "cuda"
F64 = torch.float64


def _bar(got, ref, frac=1e-2):
    got, ref = got.double().cpu(), ref.double().cpu()
    assert torch.isfinite(got).all(), "non-finite output"
    err = float((got - ref).abs().max())
    rms = float(ref.pow(2).mean().sqrt())
    assert err <= frac * rms, f"max|err| {err:.3e} > {frac} * RMS {rms:.3e}"
    return err / rms


def _weights(seed, outgoing, C=128):
    g = torch.Generator().manual_seed(seed)
    p = tmu.draw_weights(g, C, C, outgoing)
    p.ln_in_w = 1 + 0.2 * torch.randn(C, generator=g)
    p.ln_in_b = 0.2 * torch.randn(C, generator=g)
    p.ln_mix_w = 1 + 0.2 * torch.randn(C, generator=g)
    p.ln_mix_b = 0.2 * torch.randn(C, generator=g)
    return p


def _mask(seed, B, L, kind):
    if kind is None:
        return None
    if kind == "random":
        return (torch.rand(B, L, L, generator=torch.Generator().manual_seed(seed)) > 0.25).half()
    v = (torch.arange(L) < max(1, L - L // 5)).half()  # padded tail
    return (v[:, None] * v[None, :]).expand(B, L, L).contiguous()


def _pair(pkg, po, pi, out_mask=(False, False)):
    T = pkg.trimul
    return T.TriMulPair(T.TriMul.from_weights(po, out_mask=out_mask[0]),
                        T.TriMul.from_weights(pi, out_mask=out_mask[1]))


@pytest.mark.parametrize("L", [1, 5, 17, 40, 64])
@pytest.mark.parametrize("mask_kind", [None, "random", "padded"])
def test_pair_forward_matches_oracle(gpu_lib, pkg, L, mask_kind):
    B = 2
    po, pi = _weights(11 * L, True), _weights(11 * L + 1, False)
    z = torch.randn(B, L, L, 128, generator=torch.Generator().manual_seed(L + 50)).half()
    mask = _mask(L + 2, B, L, mask_kind)
    got = _pair(pkg, po, pi)(z.to(DEV), None if mask is None else mask.to(DEV)).double().cpu()
    torch.cuda.synchronize()
    ref = tmu.trimul_pair(z.double(), None if mask is None else mask.double(), po.to(F64), pi.to(F64))
    _bar(got - z.double(), ref - z.double())


@pytest.mark.parametrize("out_mask", [(True, False), (False, True), (True, True)])
def test_pair_forward_out_mask(gpu_lib, pkg, out_mask):
    L, B = 37, 2
    po, pi = _weights(400, True), _weights(401, False)
    z = torch.randn(B, L, L, 128, generator=torch.Generator().manual_seed(402)).half()
    mask = _mask(403, B, L, "random")
    got = _pair(pkg, po, pi, out_mask)(z.to(DEV), mask.to(DEV)).double().cpu()
    torch.cuda.synchronize()
    zd, md = z.double(), mask.double()
    z1 = zd + tmu.trimul(zd, md, po.to(F64), True, out_mask=out_mask[0])
    ref = z1 + tmu.trimul(z1, md, pi.to(F64), False, out_mask=out_mask[1])
    _bar(got - zd, ref - zd)
    if all(out_mask):
        assert torch.equal(got[mask == 0], zd[mask == 0])


@pytest.mark.parametrize("L,B,mask_kind", [(100, 1, None), (129, 2, "random"), (238, 1, None), (238, 1, "padded")])
def test_pair_forward_is_two_updates(gpu_lib, pkg, L, B, mask_kind):
    # the pair call against the two full updates, bit for bit; in place (out = z) too
    po, pi = _weights(7 * L + B, True), _weights(7 * L + B + 1, False)
    z = torch.randn(B, L, L, 128, generator=torch.Generator().manual_seed(L)).half().to(DEV)
    mask = _mask(L, B, L, mask_kind)
    md = None if mask is None else mask.to(DEV)
    pair = _pair(pkg, po, pi)
    got = pair(z, md)
    ref = torch.empty_like(z)
    pair.t_out.run(z, md, ref, residual=True)
    pair.t_in.run(ref, md, ref, residual=True)
    inplace = z.clone()
    pair(inplace, md, out=inplace)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(inplace.view(torch.int16), got.view(torch.int16))


def test_pair_forward_wide_is_two_updates(gpu_lib, pkg):
    # C = c = 256: tmu_pair_forward runs the two wide updates, bit for bit
    L, B = 40, 1
    po, pi = _weights(90, True, C=256), _weights(91, False, C=256)
    z = torch.randn(B, L, L, 256, generator=torch.Generator().manual_seed(92)).half().to(DEV)
    pair = _pair(pkg, po, pi)
    got = pair(z)
    ref = torch.empty_like(z)
    pair.t_out.run(z, None, ref, residual=True)
    pair.t_in.run(ref, None, ref, residual=True)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
