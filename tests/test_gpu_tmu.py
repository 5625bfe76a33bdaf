"""GPU parity of the triangle multiplicative update (kernels a, b, c and the whole
module) against the CPU oracle, through the C ABI.

Tolerance (the bar for the fp16-activation / fp32-accumulate path against the
fp32/fp64 reference): max|err| <= 1e-2 * RMS(reference output), per tensor.
"""

import numpy as np
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


def _weights(seed, outgoing, C=128, random_ln=False):
    g = torch.Generator().manual_seed(seed)
    p = tmu.draw_weights(g, C, C, outgoing)
    if random_ln:
        p.ln_in_w = 1 + 0.2 * torch.randn(C, generator=g)
        p.ln_in_b = 0.2 * torch.randn(C, generator=g)
        p.ln_mix_w = 1 + 0.2 * torch.randn(C, generator=g)
        p.ln_mix_b = 0.2 * torch.randn(C, generator=g)
    return p


def _z(seed, B, L, C=128):
    return torch.randn(B, L, L, C, generator=torch.Generator().manual_seed(seed)).half()


def _mask(seed, B, L, kind):
    if kind is None:
        return None
    if kind == "random":
        return (torch.rand(B, L, L, generator=torch.Generator().manual_seed(seed)) > 0.25).half()
    v = (torch.arange(L) < max(1, L - L // 5)).half()  # padded tail
    return (v[:, None] * v[None, :]).expand(B, L, L).contiguous()


def _f16_weights(p):
    """The same weights rounded to fp16: what the fp16 kernels multiply by. Kernel-level
    checks use these; the module-level checks use the fp32 master weights."""
    q = p.to(F64)
    q.w_bundle, q.w_emit, q.w_gate = (w.half().double() for w in (q.w_bundle, q.w_emit, q.w_gate))
    return q


def _oracle_project(z, mask, p, incoming):
    n, a, b = tmu.project(z.double(), None if mask is None else mask.double(), _f16_weights(p))
    if incoming:  # kernel (a) stores the incoming operands spatially transposed
        a, b = a.transpose(1, 2), b.transpose(1, 2)
    return a.permute(0, 3, 1, 2), b.permute(0, 3, 1, 2)  # [B, c, L, L]


@pytest.mark.parametrize("L", [1, 7, 64, 65, 76, 130])
@pytest.mark.parametrize("incoming", [False, True])
@pytest.mark.parametrize("mask_kind", [None, "random"])
def test_project_kernel(gpu_lib, pkg, L, incoming, mask_kind):
    K = pkg.kernels
    p = _weights(L, not incoming, random_ln=True)
    z, mask = _z(L, 2, L), _mask(L, 2, L, mask_kind)
    a, b = K.project(z.to(DEV), None if mask is None else mask.to(DEV), p.ln_in_w.to(DEV), p.ln_in_b.to(DEV),
                     p.ln_in_eps, p.w_bundle.half().to(DEV), incoming)
    torch.cuda.synchronize()
    ra, rb = _oracle_project(z, mask, p, incoming)
    _bar(a[..., :L], ra)
    _bar(b[..., :L], rb)
    assert torch.count_nonzero(a[..., L:]) == 0 and torch.count_nonzero(b[..., L:]) == 0, "pad columns not zero"


@pytest.mark.parametrize("incoming", [False, True])
def test_project_kernel_eps_zero_padding(gpu_lib, pkg, incoming):
    """eps = 0 is accepted: the padding cells past L (zero inputs, zero variance) must still give
    exact zeros in the pad columns, not 0 * rsqrt(0) = NaN, which the contraction would spread."""
    L = 65
    p = _weights(L, not incoming, random_ln=True)
    z = _z(L, 1, L)
    a, b = pkg.kernels.project(z.to(DEV), None, p.ln_in_w.to(DEV), p.ln_in_b.to(DEV), 0.0,
                               p.w_bundle.half().to(DEV), incoming)
    torch.cuda.synchronize()
    assert torch.count_nonzero(a[..., L:]) == 0 and torch.count_nonzero(b[..., L:]) == 0
    assert torch.isfinite(a).all() and torch.isfinite(b).all()
    p0 = p.to(F64)
    p0.ln_in_eps = 0.0
    ra, rb = _oracle_project(z, None, p0, incoming)
    _bar(a[..., :L], ra)
    _bar(b[..., :L], rb)


@pytest.mark.parametrize("L", [1, 8, 33, 128, 129, 238])
def test_contract_kernel(gpu_lib, pkg, L):
    g = torch.Generator().manual_seed(L)
    ld = pkg.kernels.leading_dim(L)
    a = torch.zeros(3, L, ld, dtype=torch.float16)
    b = torch.zeros_like(a)
    a[..., :L] = torch.randn(3, L, L, generator=g).half()
    b[..., :L] = torch.randn(3, L, L, generator=g).half()
    x = pkg.kernels.contract(a.to(DEV), b.to(DEV), L, scale=0.25)
    torch.cuda.synchronize()
    A, Bm = a[..., :L].double(), b[..., :L].double()
    ref = 0.25 * (A @ Bm.transpose(-1, -2))
    got = x[..., :L].double().cpu()
    # fp32 accumulation of L exact products (error <= L * 2^-24 * sum|a||b|, a bound relative
    # to the magnitudes summed, not to the result, so cancellation is covered), then one
    # rounding to fp16 (<= 2^-11 |v|, or half the subnormal spacing 2^-25)
    acc_bound = 0.25 * L * 2.0 ** -24 * (A.abs() @ Bm.abs().transpose(-1, -2))
    tol = ref.abs() * 2.0 ** -10 + acc_bound * 1.001 + 2.0 ** -24
    assert torch.all((got - ref).abs() <= tol), f"max err {float((got - ref).abs().max()):.3e}"
    # and the error is at the rounding level for all but cancellation-dominated entries
    assert float(((got - ref).abs() > ref.abs() * 2.0 ** -10 + 2.0 ** -24).double().mean()) < 1e-3


def _frag_to_rows(planes, L):
    """[n, rbn*kbn*512] fragment-layout planes -> [n, L, L] row-major (rows and k past L
    dropped): tile (rb, kb), lane l holds row 32 rb + l % 32, k = 16 kb + 8 (l // 32) .. +7."""
    n = planes.shape[0]
    rbn, kbn = (L + 31) // 32, (L + 15) // 16
    t = planes.view(n, rbn, kbn, 2, 32, 8)            # [n, rb, kb, l // 32, l % 32, e]
    rows = t.permute(0, 1, 4, 2, 3, 5).reshape(n, 32 * rbn, 16 * kbn)
    return rows[:, :L, :L], rows[:, :L, L:]


@pytest.mark.parametrize("L", [1, 17, 33, 100, 238])
@pytest.mark.parametrize("incoming", [False, True])
def test_fragment_layout_path_matches_row_major(gpu_lib, pkg, L, incoming):
    # tmu_project_frag + tmu_contract_frag (the launches tmu_forward makes at C = 128) against
    # tmu_project + tmu_contract: the same operand values in the other layout, zeros for k
    # past L, and the contraction bit for bit
    lib, K = pkg.capi.lib(), pkg.kernels
    p = _weights(L + 5, not incoming, random_ln=True)
    z, mask = _z(L, 2, L), _mask(L + 1, 2, L, "random")
    zd, md = z.to(DEV), mask.to(DEV)
    w = p.w_bundle.half().to(DEV)
    lw, lb = p.ln_in_w.to(DEV), p.ln_in_b.to(DEV)
    a, b = K.project(zd, md, lw, lb, p.ln_in_eps, w, incoming)
    fp = int(lib.tmu_frag_plane_elems(L))
    af = torch.full((2 * 128, fp), float("nan"), dtype=torch.float16, device=DEV)  # rows past L stay NaN
    bf = af.clone()
    pkg.capi.check(lib.tmu_project_frag(zd.data_ptr(), md.data_ptr(), lw.data_ptr(), lb.data_ptr(), p.ln_in_eps,
                                        w.data_ptr(), af.data_ptr(), bf.data_ptr(), 2, L, 128, 128, int(incoming),
                                        pkg.capi.stream_ptr()))
    ld = K.leading_dim(L)
    x = K.contract(a, b, L, scale=1 / 256)
    xf = torch.empty(2 * 128, L, ld, dtype=torch.float16, device=DEV)
    pkg.capi.check(lib.tmu_contract_frag(af.data_ptr(), bf.data_ptr(), xf.data_ptr(), 2 * 128, L, ld, 1 / 256,
                                         pkg.capi.stream_ptr()))
    torch.cuda.synchronize()
    for got, ref in ((af, a), (bf, b)):
        vals, pad_k = _frag_to_rows(got.cpu(), L)
        kpad = min(16 * ((L + 15) // 16), 8 * ((L + 7) // 8)) - L  # k past L written by the 8 x 8 tiles
        assert torch.equal(vals.view(torch.int16), ref.cpu().reshape(2 * 128, L, ld)[..., :L].view(torch.int16))
        assert torch.count_nonzero(pad_k[..., :kpad]) == 0
    assert torch.equal(xf.view(torch.int16), x.reshape(2 * 128, L, ld).view(torch.int16))
    assert torch.isfinite(xf).all()


@pytest.mark.parametrize("L", [5, 64, 100])
@pytest.mark.parametrize("residual", [False, True])
def test_epilogue_kernel(gpu_lib, pkg, L, residual):
    p = _weights(100 + L, True, random_ln=True)
    g = torch.Generator().manual_seed(L)
    z = _z(L, 1, L)
    ld = pkg.kernels.leading_dim(L)
    x = torch.zeros(1, 128, L, ld, dtype=torch.float16)
    x[..., :L] = (3 * torch.randn(1, 128, L, L, generator=g) + 1).half()
    out = pkg.kernels.epilogue(x.to(DEV), z.to(DEV), None, p.ln_in_w.to(DEV), p.ln_in_b.to(DEV), p.ln_in_eps,
                               p.ln_mix_w.to(DEV), p.ln_mix_b.to(DEV), p.ln_mix_eps, p.w_emit.half().to(DEV),
                               p.w_gate.half().to(DEV), residual=residual)
    torch.cuda.synchronize()
    pd = _f16_weights(p)
    n = tmu.layer_norm(z.double(), pd.ln_in_w, pd.ln_in_b, pd.ln_in_eps)
    xm = x[..., :L].double().permute(0, 2, 3, 1)
    upd = torch.nn.functional.linear(tmu.layer_norm(xm, pd.ln_mix_w, pd.ln_mix_b, pd.ln_mix_eps), pd.w_emit)
    upd = upd * torch.sigmoid(torch.nn.functional.linear(n, pd.w_gate))
    if residual:
        _bar(out.double().cpu() - z.double(), upd)
    else:
        _bar(out, upd)


@pytest.mark.parametrize("L", [3, 33, 70])
@pytest.mark.parametrize("residual", [False, True])
def test_epilogue_kernel_masked_batch(gpu_lib, pkg, L, residual):
    """The out_mask variants, two batch entries, rows that end in a partial 32-cell unit;
    the output may alias z when the residual is added."""
    B = 2
    p = _weights(200 + L, True, random_ln=True)
    g = torch.Generator().manual_seed(1000 + L)
    z = _z(L + 7, B, L)
    mask = _mask(L + 3, B, L, "random")
    ld = pkg.kernels.leading_dim(L)
    x = torch.zeros(B, 128, L, ld, dtype=torch.float16)
    x[..., :L] = (2 * torch.randn(B, 128, L, L, generator=g) - 0.5).half()
    zd = z.to(DEV)
    out = pkg.kernels.epilogue(x.to(DEV), zd, mask.to(DEV), p.ln_in_w.to(DEV), p.ln_in_b.to(DEV), p.ln_in_eps,
                               p.ln_mix_w.to(DEV), p.ln_mix_b.to(DEV), p.ln_mix_eps, p.w_emit.half().to(DEV),
                               p.w_gate.half().to(DEV), residual=residual, out_mask=True,
                               out=zd if residual else None)
    torch.cuda.synchronize()
    pd = _f16_weights(p)
    n = tmu.layer_norm(z.double(), pd.ln_in_w, pd.ln_in_b, pd.ln_in_eps)
    xm = x[..., :L].double().permute(0, 2, 3, 1)
    upd = torch.nn.functional.linear(tmu.layer_norm(xm, pd.ln_mix_w, pd.ln_mix_b, pd.ln_mix_eps), pd.w_emit)
    upd = upd * torch.sigmoid(torch.nn.functional.linear(n, pd.w_gate)) * mask.double()[..., None]
    got = out.double().cpu()
    if residual:
        got = got - z.double()
    _bar(got, upd)
    assert torch.count_nonzero(got[mask == 0]) == 0


@pytest.mark.parametrize("L", [1, 2, 5, 17, 64, 76, 127, 129])
@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("mask_kind", [None, "random", "padded"])
def test_trimul_module(gpu_lib, pkg, L, outgoing, mask_kind):
    p = _weights(7 * L + outgoing, outgoing, random_ln=True)
    z, mask = _z(L, 2, L), _mask(L, 2, L, mask_kind)
    m = pkg.trimul.TriMul.from_weights(p)
    got = m(z.to(DEV), None if mask is None else mask.to(DEV))
    torch.cuda.synchronize()
    assert got.dtype == torch.float16 and got.shape == z.shape
    ref = tmu.trimul(z.double(), None if mask is None else mask.double(), p.to(F64), outgoing)
    _bar(got, ref)


@pytest.mark.parametrize("L", [8, 31, 33, 96, 160, 255, 257, 300])
@pytest.mark.parametrize("outgoing", [True, False])
def test_trimul_tile_edges(gpu_lib, pkg, L, outgoing):
    # sizes either side of the tilings' edges: 8-cell and 16-k fragment tiles, 32-row MFMA blocks,
    # 64-cell units and 128-row contraction blocks; random mask, random LN parameters, B = 1;
    # the oracle in fp32 on the CPU (the larger sizes would take minutes in fp64)
    p = _weights(11 * L + outgoing, outgoing, random_ln=True)
    z, mask = _z(L + 1, 1, L), _mask(L + 2, 1, L, "random")
    m = pkg.trimul.TriMul.from_weights(p)
    got = m(z.to(DEV), mask.to(DEV))
    torch.cuda.synchronize()
    with torch.no_grad():
        ref = tmu.trimul(z.float(), mask.float(), p, outgoing)
    _bar(got, ref)


@pytest.mark.parametrize("outgoing", [True, False])
def test_trimul_permutation_equivariance_full_size(gpu_lib, pkg, outgoing):
    # a size-independent property at the workload's size: relabelling the residues (the same
    # permutation on i and j of z and of the mask) relabels the update, T(z_P) = T(z)_P. The two
    # runs differ only in the contraction's summation order over k, which can flip a rounding of
    # x: the oracle bar holds between them and most values are identical; a wrong index or a
    # transposed operand in any kernel breaks both by O(1)
    L = 238
    p = _weights(91 + outgoing, outgoing, random_ln=True)
    z, mask = _z(90, 1, L), _mask(92, 1, L, "random")
    perm = torch.randperm(L, generator=torch.Generator().manual_seed(93))
    zp = z[:, perm][:, :, perm].contiguous()
    mp = mask[:, perm][:, :, perm].contiguous()
    m = pkg.trimul.TriMul.from_weights(p)
    got = m(z.to(DEV), mask.to(DEV)).double().cpu()
    gotp = m(zp.to(DEV), mp.to(DEV)).double().cpu()
    torch.cuda.synchronize()
    expect = got[:, perm][:, :, perm]
    _bar(gotp, expect)
    same = float((gotp == expect).double().mean())
    assert same > 0.9, f"only {same:.4f} of the values identical"
    assert not torch.equal(gotp, got)  # the relabelling is not the identity


def test_trimul_fp32_plumbing_L76(gpu_lib, pkg):
    # config: outgoing only, z [1,76,76,128] fp32 N(0,1), seed 0, all-ones mask
    z, _, po, _ = tmu.make_pair_inputs(76, 128, 128, seed=0, dtype=torch.float32)
    m = pkg.trimul.TriMul.from_weights(po)
    got = m(z.to(DEV), torch.ones(1, 76, 76, device=DEV))
    torch.cuda.synchronize()
    assert got.dtype == torch.float32  # returned in the input's dtype
    ref = tmu.trimul(z.double(), None, po.to(F64), True)
    _bar(got, ref)


def test_visibility_none_equals_all_ones(gpu_lib, pkg):
    p = _weights(3, True)
    z = _z(3, 1, 50).to(DEV)
    m = pkg.trimul.TriMul.from_weights(p)
    a = m(z, None)
    b = m(z, torch.ones(1, 50, 50, device=DEV))
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_no_residual_and_mask_not_on_output(gpu_lib, pkg):
    # the module returns the update only; the pair mask gates a and b, not the output
    p = _weights(4, False, random_ln=True)  # beta_mix != 0: padded cells get a nonzero update
    L = 40
    z = _z(4, 1, L)
    mask = _mask(4, 1, L, "padded")
    m = pkg.trimul.TriMul.from_weights(p)
    got = m(z.to(DEV), mask.to(DEV)).double().cpu()
    ref = tmu.trimul(z.double(), mask.double(), p.to(F64), False)
    _bar(got, ref)
    pad = mask.double() == 0
    assert float(got[pad].abs().max()) > 0.01  # unmasked output, as the reference
    m.out_mask = True
    got_m = m(z.to(DEV), mask.to(DEV)).double().cpu()
    assert torch.count_nonzero(got_m[pad]) == 0


def test_pair_L238_fp16(gpu_lib, pkg):
    # headline workload: z [1,238,238,128] fp16, outgoing then incoming, residuals
    z, mask, po, pi = tmu.make_pair_inputs(238, 128, 128, seed=0, dtype=torch.float16)
    pair = pkg.trimul.TriMulPair(pkg.trimul.TriMul.from_weights(po), pkg.trimul.TriMul.from_weights(pi))
    got = pair(z.to(DEV)).double().cpu()
    torch.cuda.synchronize()
    ref = tmu.trimul_pair(z.double(), None, po.to(F64), pi.to(F64))
    _bar(got - z.double(), ref - z.double())


def test_pair_L512_two_chain_padded(gpu_lib, pkg):
    # 300 + 160 residues, 52 padding positions: mask zero on padded rows/columns
    z, mask, po, pi = tmu.make_pair_inputs(512, 128, 128, seed=0, dtype=torch.float16, pad_from=460)
    pair = pkg.trimul.TriMulPair(pkg.trimul.TriMul.from_weights(po), pkg.trimul.TriMul.from_weights(pi))
    got = pair(z.to(DEV), mask.to(DEV)).double().cpu()
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    # beta_mix = 0 in this workload: padded cells receive an exactly-zero update (z unchanged)
    v = torch.arange(512) >= 460
    pad = v[:, None] | v[None, :]
    assert torch.equal(got[0][pad], z[0][pad].double())
    # oracle in fp32 on the CPU (fp64 would take minutes here); the bar is 1e-2 * RMS
    with torch.no_grad():
        ref = tmu.trimul_pair(z.float(), mask.float(), po, pi).double()
    _bar(got - z.double(), ref - z.double())


def test_bad_input_raises(gpu_lib, pkg):
    p = _weights(5, True)
    m = pkg.trimul.TriMul.from_weights(p)
    with pytest.raises(ValueError):
        m(torch.zeros(1, 4, 5, 128, device=DEV, dtype=torch.float16))
    with pytest.raises(ValueError):
        m(torch.zeros(1, 4, 4, 128, device=DEV, dtype=torch.float16), torch.ones(1, 4, 3, device=DEV))


def test_nan_propagates_to_its_cells(gpu_lib, pkg):
    p = _weights(6, True)
    z = _z(6, 1, 20)
    z[0, 3, 4, 7] = float("nan")
    m = pkg.trimul.TriMul.from_weights(p)
    got = m(z.to(DEV)).cpu()
    # outgoing: cell (3,4) feeds a[3,4] and b[3,4] -> every x[3, j] and x[i, 3], and gate (3,4)
    assert torch.isnan(got[0, 3]).any()
    assert not torch.isnan(got[0, 10, 11]).any()
