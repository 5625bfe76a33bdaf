"""GPU parity of the pair transition (kernel e) against the fp32/fp64 oracle.

Bar: max|err| of the update (out - z) within 1e-2 x RMS(update) of the oracle's, with
the kernel's fp16 weights given to the oracle (the kernel's arithmetic is what is
tested, not the weights' rounding); both activations; in place; padded cell tiles.
"""

import pytest
import torch

from oracle import transition as otr

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _weights(C, H, swiglu, seed):
    g = torch.Generator().manual_seed(seed)
    p = otr.draw_transition(g, C, H)
    if swiglu:
        p.w2 = torch.randn(H, C, generator=g) * C ** -0.5
    # LayerNorm affine away from the identity so its parameters are exercised
    p.ln_w = 1 + 0.1 * torch.randn(C, generator=g)
    p.ln_b = 0.1 * torch.randn(C, generator=g)
    # the kernel takes fp16 weights: give the oracle the same values
    for f in ("w1", "w2", "w3"):
        if getattr(p, f) is not None:
            setattr(p, f, getattr(p, f).half().float())
    return p


def _run(pkg, z16, p, out=None):
    dev = lambda t: t.to(DEV).contiguous()  # noqa: E731
    return pkg.kernels.transition(z16, dev(p.ln_w.float()), dev(p.ln_b.float()), p.eps, dev(p.w1.half()),
                                  dev(p.w3.half()), None if p.w2 is None else dev(p.w2.half()), out=out)


def _check(got16, z16, p):
    z = z16.double().cpu()
    ref = otr.transition(z, otr.TransitionWeights(**{k: (v.double() if isinstance(v, torch.Tensor) else v)
                                                     for k, v in vars(p).items()})) - z
    upd = got16.double().cpu() - z
    rms = ref.pow(2).mean().sqrt()
    err = (upd - ref).abs().max()
    assert torch.isfinite(upd).all()
    assert err <= 1e-2 * rms, f"max|err| {float(err):.3e} vs RMS {float(rms):.3e}"
    return float(err / rms)


@pytest.mark.parametrize("H,swiglu", [(512, False), (256, False), (256, True)])
@pytest.mark.parametrize("B,L", [(1, 1), (1, 5), (2, 33), (1, 64), (1, 100)])
def test_transition_matches_oracle(gpu_lib, pkg, H, swiglu, B, L):
    p = _weights(128, H, swiglu, seed=H + L)
    g = torch.Generator().manual_seed(L)
    z16 = torch.randn(B, L, L, 128, generator=g).half()
    out = _run(pkg, z16.to(DEV), p)
    _check(out.cpu(), z16, p)


def test_transition_in_place_and_large(gpu_lib, pkg):
    p = _weights(128, 512, False, seed=1)
    g = torch.Generator().manual_seed(7)
    z16 = (3 * torch.randn(1, 238, 238, 128, generator=g) + 0.5).half()  # non-zero mean per cell
    zd = z16.to(DEV)
    ref_out = _run(pkg, zd.clone(), p)
    _run(pkg, zd, p, out=zd)  # in place
    assert torch.equal(zd.view(torch.int16), ref_out.view(torch.int16))
    _check(zd.cpu(), z16, p)


def test_transition_other_hidden_widths_and_unsupported(gpu_lib, pkg):
    # hidden widths outside the register-resident kernel's run the wide path (LN, then a GEMM
    # with the activation fused, then one with the residual fused)
    for H, swiglu in ((384, False), (512, True)):
        p = _weights(128, H, swiglu, seed=H)
        z16 = torch.randn(1, 29, 29, 128, generator=torch.Generator().manual_seed(H)).half()
        _check(_run(pkg, z16.to(DEV), p).cpu(), z16, p)
    # a hidden width that is not a multiple of 32 is refused before any launch
    p = _weights(128, 100, False, seed=0)
    z16 = torch.zeros(1, 4, 4, 128, dtype=torch.float16, device=DEV)
    with pytest.raises(pkg.capi.EsmError) as e:
        _run(pkg, z16, p)
    assert e.value.code == -4
