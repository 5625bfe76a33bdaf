"""GPU parity of the fused TMU pair (tmu_pair_forward) and of its middle launch, tmu_bridge
(the outgoing update's epilogue fused with the incoming update's projection).

tmu_bridge is checked piece by piece: its z1 against kernel (c) on the same x and z (same
arithmetic, another accumulation and LayerNorm summation order: within 2 fp16 ulps) and
against the fp64 oracle; its incoming operands bit for bit against tmu_project_frag run on
its own z1 (the identical arithmetic). The whole pair is checked against the oracle at the
module bar, max|err| <= 1e-2 * RMS(update), and against the unfused six-launch path.
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


def _frag_to_rows(planes, L):
    """[n, rbn*kbn*512] fragment-layout planes -> ([n, L, L] values, [n, L, k >= L] padding)."""
    n = planes.shape[0]
    rbn, kbn = (L + 31) // 32, (L + 15) // 16
    rows = planes.view(n, rbn, kbn, 2, 32, 8).permute(0, 1, 4, 2, 3, 5).reshape(n, 32 * rbn, 16 * kbn)
    return rows[:, :L, :L], rows[:, :L, L:]


def _d(t, dtype=None):
    return t.to(DEV) if dtype is None else t.to(device=DEV, dtype=dtype).contiguous()


def _bridge(pkg, x, ldx, z, mask, po, pi, z1, a, b, out_mask=False):
    lib = pkg.capi.lib()
    B, L = z.shape[0], z.shape[1]
    f32 = torch.float32
    args = [_d(po.ln_in_w, f32), _d(po.ln_in_b, f32), _d(po.ln_mix_w, f32), _d(po.ln_mix_b, f32),
            _d(po.w_emit, torch.float16), _d(po.w_gate, torch.float16), _d(pi.ln_in_w, f32), _d(pi.ln_in_b, f32),
            _d(pi.w_bundle, torch.float16)]
    lw, lb, mw, mb, we, wg, iw, ib, wb = args
    pkg.capi.check(lib.tmu_bridge(x.data_ptr(), ldx, z.data_ptr(), None if mask is None else mask.data_ptr(),
                                  lw.data_ptr(), lb.data_ptr(), po.ln_in_eps, mw.data_ptr(), mb.data_ptr(),
                                  po.ln_mix_eps, we.data_ptr(), wg.data_ptr(), int(out_mask), z1.data_ptr(),
                                  iw.data_ptr(), ib.data_ptr(), pi.ln_in_eps, wb.data_ptr(), a.data_ptr(),
                                  b.data_ptr(), B, L, 128, 128, pkg.capi.stream_ptr()))
    return args


@pytest.mark.parametrize("L", [1, 7, 9, 33, 64, 100])
@pytest.mark.parametrize("mask_kind,out_mask", [(None, False), ("random", False), ("random", True)])
def test_bridge_matches_epilogue_then_projection(gpu_lib, pkg, L, mask_kind, out_mask):
    lib, K = pkg.capi.lib(), pkg.kernels
    B = 2
    po, pi = _weights(3 * L + 1, True), _weights(3 * L + 2, False)
    g = torch.Generator().manual_seed(L)
    z = torch.randn(B, L, L, 128, generator=g).half()
    mask = _mask(L + 9, B, L, mask_kind)
    ld = K.leading_dim(L)
    x = torch.zeros(B, 128, L, ld, dtype=torch.float16)
    x[..., :L] = (2 * torch.randn(B, 128, L, L, generator=g) + 0.5).half()
    zd, xd, md = z.to(DEV), x.to(DEV), None if mask is None else mask.to(DEV)
    fp = int(lib.tmu_frag_plane_elems(L))
    a = torch.full((B * 128, fp), float("nan"), dtype=torch.float16, device=DEV)
    b = a.clone()
    z1 = torch.empty_like(zd)
    lw, lb, mw, mb, we, wg, iw, ib, wb = _bridge(pkg, xd, ld, zd, md, po, pi, z1, a, b, out_mask)
    # the same update through kernel (c)
    ref = K.epilogue(xd, zd, md, lw, lb, po.ln_in_eps, mw, mb, po.ln_mix_eps, we, wg, residual=True,
                     out_mask=out_mask)
    # the incoming projection of the bridge's own z1 through kernel (a)
    a2 = torch.full_like(a, float("nan"))
    b2 = a2.clone()
    pkg.capi.check(lib.tmu_project_frag(z1.data_ptr(), None if md is None else md.data_ptr(), iw.data_ptr(),
                                        ib.data_ptr(), pi.ln_in_eps, wb.data_ptr(), a2.data_ptr(), b2.data_ptr(), B,
                                        L, 128, 128, 1, pkg.capi.stream_ptr()))
    # in place (z1 = z) gives the same bits
    zi = zd.clone()
    ai, bi = torch.full_like(a, float("nan")), torch.full_like(a, float("nan"))
    _bridge(pkg, xd, ld, zi, md, po, pi, zi, ai, bi, out_mask)
    torch.cuda.synchronize()

    got, r = z1.double().cpu(), ref.double().cpu()
    assert torch.isfinite(got).all()
    # two ulps of z1 (of the larger of the two values), plus room for an fp16 LayerNorm output
    # that rounds the other way in one
    # order (one term of a 128-term dot product: ~1e-4 here)
    slack = 1e-3 * float((r - z.double()).pow(2).mean().sqrt())
    assert torch.all((got - r).abs() <= torch.maximum(got.abs(), r.abs()) * 2.0 ** -9 + slack), \
        f"z1 vs kernel (c): max {float((got - r).abs().max()):.3e}"
    # against the oracle (fp16-rounded weights, fp64 arithmetic)
    pd = po.to(F64)
    pd.w_emit, pd.w_gate = pd.w_emit.half().double(), pd.w_gate.half().double()
    n = tmu.layer_norm(z.double(), pd.ln_in_w, pd.ln_in_b, pd.ln_in_eps)
    xm = x[..., :L].double().permute(0, 2, 3, 1)
    upd = torch.nn.functional.linear(tmu.layer_norm(xm, pd.ln_mix_w, pd.ln_mix_b, pd.ln_mix_eps), pd.w_emit)
    upd = upd * torch.sigmoid(torch.nn.functional.linear(n, pd.w_gate))
    if out_mask:
        upd = upd * mask.double()[..., None]
    _bar(got - z.double(), upd)
    if out_mask:
        assert torch.equal(got[mask == 0], z.double()[mask == 0])
    for p1, p2 in ((a, a2), (b, b2)):
        v1, pad1 = _frag_to_rows(p1.cpu(), L)
        v2, _ = _frag_to_rows(p2.cpu(), L)
        assert torch.equal(v1.view(torch.int16), v2.view(torch.int16)), "incoming operands differ from kernel (a)"
        kpad = min(16 * ((L + 15) // 16), 8 * ((L + 7) // 8)) - L  # k past L written by the 8 x 8 tiles
        assert torch.count_nonzero(pad1[..., :kpad]) == 0
    assert torch.equal(zi.view(torch.int16), z1.view(torch.int16))
    for p1, p2 in ((a, ai), (b, bi)):
        assert torch.equal(_frag_to_rows(p1.cpu(), L)[0].view(torch.int16),
                           _frag_to_rows(p2.cpu(), L)[0].view(torch.int16))


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
def test_pair_forward_matches_unfused(gpu_lib, pkg, L, B, mask_kind):
    # the fused five launches against the two full updates (six launches): the same
    # arithmetic up to accumulation and summation order in the outgoing epilogue
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
    zc, g, r = z.double().cpu(), got.double().cpu(), ref.double().cpu()
    _bar(g - zc, r - zc)
    # z1 differs by an ulp here and there (another summation order), which the incoming
    # update carries to the output, where the final sum may round the other way too: a few
    # ulps of the output at most, plus a small absolute room, and rarely more than one
    slack = 2e-3 * float((r - zc).pow(2).mean().sqrt())
    big = torch.maximum(g.abs(), r.abs())
    assert torch.all((g - r).abs() <= big * 2.0 ** -8 + slack), f"max {float((g - r).abs().max()):.3e}"
    assert float(((g - r).abs() > big * 2.0 ** -10 + slack).double().mean()) < 1e-3
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
