"""GPU parity of the wide path: the triangle update, the pair transition and the recycling
kernels at ESMFold2's real pair width, C = c = 256 (mlx_trunk.py:3-5), and at 384, against
the fp64 oracle, through the C ABI; and the trunk plugin on a 256-wide model shaped like the
reference's.

Bars as for the 128-wide kernels: the update's max|err| <= 1e-2 x RMS(reference update);
the transition's against the oracle with the fp16 weights the kernels use.
"""

import pytest
import torch

from oracle import recycle as orc, tmu, transition as otr
from tests import ref_modules

pytestmark = pytest.mark.gpu
DEV = "cuda"
F64 = torch.float64
FIELDS = ("w_bundle", "w_emit", "w_gate", "ln_in_w", "ln_in_b", "ln_mix_w", "ln_mix_b", "ln_in_eps", "ln_mix_eps",
          "outgoing")


def _bar(got, ref, base, frac=1e-2):
    """max|got - ref| <= frac * RMS(ref - base) (the update's RMS when base is the input)."""
    got, ref = got.double().cpu(), ref.double().cpu()
    assert torch.isfinite(got).all(), "non-finite output"
    err = float((got - ref).abs().max())
    rms = float((ref - base.double().cpu()).pow(2).mean().sqrt())
    assert err <= frac * rms, f"max|err| {err:.3e} > {frac} * RMS {rms:.3e}"
    return err / rms


def _weights(seed, C, outgoing, random_ln=True):
    g = torch.Generator().manual_seed(seed)
    p = tmu.draw_weights(g, C, C, outgoing)
    if random_ln:
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
    v = (torch.arange(L) < max(1, L - L // 5)).half()
    return (v[:, None] * v[None, :]).expand(B, L, L).contiguous()


@pytest.mark.parametrize("L", [1, 65, 238])
@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("mask_kind", [None, "random", "padded"])
def test_tmu_256_matches_oracle(gpu_lib, pkg, L, outgoing, mask_kind):
    C = 256
    p = _weights(L + 3 * outgoing, C, outgoing)
    z = torch.randn(1, L, L, C, generator=torch.Generator().manual_seed(L)).half()
    m = _mask(L + 1, 1, L, mask_kind)
    mod = pkg.trimul.TriMul.from_weights(p)
    upd = mod(z.to(DEV), None if m is None else m.to(DEV))
    assert upd.shape == z.shape and upd.dtype == torch.float16
    ref = tmu.trimul(z.double(), None if m is None else m.double(), p.to(F64))
    _bar(upd, ref, torch.zeros_like(ref))


@pytest.mark.parametrize("L", [8, 31, 129, 257])
@pytest.mark.parametrize("outgoing", [True, False])
def test_tmu_256_tile_edges(gpu_lib, pkg, L, outgoing):
    # sizes either side of the wide path's tilings (8 x 8-cell fragment tiles, 64-cell line tiles,
    # 128-row contraction blocks); random mask, random LN parameters; the oracle in fp32
    C = 256
    p = _weights(5 * L + outgoing, C, outgoing)
    z = torch.randn(1, L, L, C, generator=torch.Generator().manual_seed(L + 9)).half()
    m = _mask(L + 4, 1, L, "random")
    mod = pkg.trimul.TriMul.from_weights(p)
    upd = mod(z.to(DEV), m.to(DEV))
    with torch.no_grad():
        ref = tmu.trimul(z.float(), m.float(), p, outgoing)
    _bar(upd, ref, torch.zeros_like(ref))


@pytest.mark.parametrize("C,L,B", [(256, 40, 2), (384, 33, 1)])
def test_tmu_wide_residual_out_mask_and_batch(gpu_lib, pkg, C, L, B):
    p = _weights(7, C, False)
    z = torch.randn(B, L, L, C, generator=torch.Generator().manual_seed(3)).half()
    m = _mask(5, B, L, "padded")
    zd, md = z.to(DEV), m.to(DEV)
    ref = tmu.trimul(z.double(), m.double(), p.to(F64))
    # residual fused, written in place
    mod = pkg.trimul.TriMul.from_weights(p)
    zz = zd.clone()
    mod.run(zz, md, zz, residual=True)
    _bar(zz, z.double() + ref, z)
    # the output mask multiplies the update (off by default: the reference never masks it)
    mo = pkg.trimul.TriMul.from_weights(p, out_mask=True)
    upd = mo(zd, md)
    refm = tmu.trimul(z.double(), m.double(), p.to(F64), out_mask=True)
    _bar(upd, refm, torch.zeros_like(refm))
    assert torch.all(upd.cpu()[m == 0] == 0)


def test_tmu_pair_256_full_size(gpu_lib, pkg):
    # the pair at L=238 at the real width: z1 = z + T_out(z), z2 = z1 + T_in(z1)
    L, C = 238, 256
    z, _, po, pi = pkg.workloads.pair_inputs(L, C, C, seed=2)
    T = pkg.trimul
    pair = T.TriMulPair(T.TriMul.from_weights(po), T.TriMul.from_weights(pi))
    got = pair(z.to(DEV))
    as_oracle = lambda q: tmu.TriMulWeights(**{f: getattr(q, f) for f in FIELDS}).to(F64)  # noqa: E731
    ref = tmu.trimul_pair(z.double(), None, as_oracle(po), as_oracle(pi))
    _bar(got, ref, z)


def test_tmu_pair_256_L512_two_chain_padded(gpu_lib, pkg):
    # the two-chain complex (300 + 160 residues, 52 padding positions) at the real width: tiles
    # past the first 256 rows and columns, and the mask's zero rows and columns
    L, C, valid = 512, 256, 460
    z, mask, po, pi = tmu.make_pair_inputs(L, C, C, seed=4, dtype=torch.float16, pad_from=valid)
    T = pkg.trimul
    pair = T.TriMulPair(T.TriMul.from_weights(po), T.TriMul.from_weights(pi))
    got = pair(z.to(DEV), mask.to(DEV)).double().cpu()
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    # beta_mix = 0 in this workload: padded cells receive an exactly-zero update (z unchanged)
    v = torch.arange(L) >= valid
    pad = v[:, None] | v[None, :]
    assert torch.equal(got[0][pad], z[0][pad].double())
    # the oracle in fp32 on the CPU (a few seconds here); the bar is 1e-2 * RMS of the update
    with torch.no_grad():
        ref = tmu.trimul_pair(z.float(), mask.float(), po, pi).double()
    _bar(got, ref, z)


@pytest.mark.parametrize("C,H,swiglu", [(256, 512, True), (256, 1024, True), (256, 1024, False), (128, 512, True),
                                        (384, 768, True), (256, 256, False), (256, 128, True), (512, 256, False)])
def test_transition_wide_matches_oracle(gpu_lib, pkg, C, H, swiglu):
    g = torch.Generator().manual_seed(C + H)
    L, B = 37, 2
    z = torch.randn(B, L, L, C, generator=g).half()
    w1 = torch.randn(H, C, generator=g) * C ** -0.5
    w2 = torch.randn(H, C, generator=g) * C ** -0.5 if swiglu else None
    w3 = torch.randn(C, H, generator=g) * H ** -0.5
    lw, lb = 1 + 0.1 * torch.randn(C, generator=g), 0.1 * torch.randn(C, generator=g)
    tr = pkg.trunk.PairTransition(lw, lb, w1, w3, w2=w2)
    assert pkg.kernels.capi.lib().pair_transition_workspace_bytes(B, L, C, H, int(swiglu)) > 0
    zd = z.to(DEV)
    out = tr(zd)
    p = otr.TransitionWeights(lw.double(), lb.double(), w1.half().double(), w3.half().double(),
                              None if w2 is None else w2.half().double())
    ref = otr.transition(z.double(), p)
    _bar(out, ref, z)
    # in place
    zz = zd.clone()
    tr.run(zz, zz)
    assert torch.equal(zz, out)


@pytest.mark.parametrize("L", [129, 238])
@pytest.mark.parametrize("swiglu", [True, False])
def test_transition_256_h1024_across_line_tiles(gpu_lib, pkg, L, swiglu):
    # the streaming wide GEMM (K = H = 1024 for the second GEMM) over several 128-cell line
    # tiles, with a partial last tile: ESMFold2's real transition width at the pair sizes
    C, H = 256, 1024
    g = torch.Generator().manual_seed(L + 11 * swiglu)
    z = torch.randn(1, L, L, C, generator=g).half()
    w1 = torch.randn(H, C, generator=g) * C ** -0.5
    w2 = torch.randn(H, C, generator=g) * C ** -0.5 if swiglu else None
    w3 = torch.randn(C, H, generator=g) * H ** -0.5
    lw, lb = 1 + 0.1 * torch.randn(C, generator=g), 0.1 * torch.randn(C, generator=g)
    tr = pkg.trunk.PairTransition(lw, lb, w1, w3, w2=w2)
    out = tr(z.to(DEV))
    p = otr.TransitionWeights(lw.float(), lb.float(), w1.half().float(), w3.half().float(),
                              None if w2 is None else w2.half().float())
    with torch.no_grad():
        ref = otr.transition(z.float(), p)
    _bar(out, ref, z)


@pytest.mark.parametrize("C,L", [(384, 129), (384, 257), (512, 65), (512, 129)])
@pytest.mark.parametrize("outgoing", [True, False])
def test_tmu_384_512_across_tiles(gpu_lib, pkg, C, L, outgoing):
    # C = 384 and 512 run the streaming wide GEMM (K > 256) for the projection and emit/gate,
    # and ln_cf_to_cl at its largest LDS footprint; random mask, random LN parameters, the
    # oracle in fp32
    p = _weights(C + L + outgoing, C, outgoing)
    z = torch.randn(1, L, L, C, generator=torch.Generator().manual_seed(C + L)).half()
    m = _mask(C + L + 2, 1, L, "random")
    mod = pkg.trimul.TriMul.from_weights(p)
    upd = mod(z.to(DEV), m.to(DEV))
    with torch.no_grad():
        ref = tmu.trimul(z.float(), m.float(), p, outgoing)
    _bar(upd, ref, torch.zeros_like(ref))


def test_transition_wide_needs_its_workspace(gpu_lib, pkg):
    lib = pkg.capi.lib()
    C, H, L = 256, 512, 8
    z = torch.zeros(1, L, L, C, dtype=torch.float16, device=DEV)
    w = torch.zeros(H, C, dtype=torch.float16, device=DEV)
    w3 = torch.zeros(C, H, dtype=torch.float16, device=DEV)
    lw = torch.ones(C, device=DEV)
    rc = lib.pair_transition(z.data_ptr(), z.data_ptr(), lw.data_ptr(), lw.data_ptr(), 1e-5, w.data_ptr(),
                             w.data_ptr(), w3.data_ptr(), 1, L, C, H, None)
    assert rc == -1 and "workspace" in lib.esm_last_error().decode()
    need = lib.pair_transition_workspace_bytes(1, L, C, H, 1)
    ws = torch.empty(need + 256, dtype=torch.uint8, device=DEV)
    base = (ws.data_ptr() + 255) // 256 * 256
    rc = lib.pair_transition_ws(z.data_ptr(), z.data_ptr(), lw.data_ptr(), lw.data_ptr(), 1e-5, w.data_ptr(),
                                w.data_ptr(), w3.data_ptr(), 1, L, C, H, base, need - 1, None)
    assert rc == -2
    assert lib.pair_transition_workspace_bytes(1, L, 128, 512, 0) == 0  # the register-resident kernel


def test_parcae_and_distogram_256(gpu_lib, pkg):
    C, L = 256, 30
    g = torch.Generator().manual_seed(4)
    z, zi, rf = (torch.randn(1, L, L, C, generator=g) for _ in range(3))
    lw, lb = 1 + 0.1 * torch.randn(C, generator=g), 0.1 * torch.randn(C, generator=g)
    a = torch.rand(C, generator=g)
    bm = (torch.randn(C, C, generator=g) * C ** -0.5).half()
    got = pkg.kernels.parcae_step(z.to(DEV), zi.to(DEV), rf.to(DEV), lw.to(DEV), lb.to(DEV), 1e-5, a.to(DEV),
                                  bm.to(DEV))
    ref = orc.parcae_step(z.double(), zi.double(), rf.double(), lw.double(), lb.double(), a.double(), bm.double())
    inj = ref - a.double() * z.double()
    assert float((got.double().cpu() - ref).abs().max()) <= 1e-2 * float(inj.pow(2).mean().sqrt())
    for nb, cen in ((64, orc.centers_6b()), (128, orc.centers_experimental())):
        w = (torch.randn(nb, C, generator=g) * 0.05).half()
        bias = torch.randn(nb, generator=g)
        ed = pkg.kernels.expected_distance(z.to(DEV), w.to(DEV), bias.to(DEV), cen.float().to(DEV))
        # the kernel rounds the pair sums to fp16 for the MFMA: the oracle takes the same sums
        s = (z + z.transpose(1, 2)).half().double()
        logits = s @ w.double().T + bias.double()
        ref = torch.softmax(logits, -1) @ cen
        assert float((ed.double().cpu() - ref).abs().max()) <= 1e-3


def test_var_hip_trunk_plugin_256(gpu_lib, pkg):
    # a 256-wide trunk shaped like the reference's (SwiGLU transitions, H = 512, wrapped TMUs)
    C, L = 256, 20
    z, blocks = pkg.workloads.block_stack(L, n_blocks=2, C=C, c=C, H=512, seed=6)
    g = torch.Generator().manual_seed(12)
    for _, _, pt in blocks:
        pt.w2 = torch.randn(512, C, generator=g) * C ** -0.5
    model = ref_modules.Model(blocks)
    pkg.var_hip_trunk.apply(model)
    out = model.folding_trunk(z.to(DEV).float())
    assert out.dtype == torch.float32 and out.shape == z.shape
    ob = [otr.BlockWeights(tmu.TriMulWeights(**{f: getattr(po, f) for f in FIELDS}).to(F64),
                           tmu.TriMulWeights(**{f: getattr(pi, f) for f in FIELDS}).to(F64),
                           otr.TransitionWeights(pt.ln_w.double(), pt.ln_b.double(), pt.w1.double(), pt.w3.double(),
                                                 pt.w2.double()))
          for po, pi, pt in blocks]
    ref = otr.stack_forward(z.double(), None, ob, 1, store=torch.float16)
    d = out.double().cpu() - ref
    rms = float((ref - z.double()).pow(2).mean().sqrt())
    assert float(d.abs().max()) <= 3e-2 * rms and float(d.pow(2).mean().sqrt()) <= 1e-2 * rms
