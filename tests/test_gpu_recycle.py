"""GPU parity of the recycling step: the parcae recurrence, the distogram expected
distance, the exact quantile of the exit signal, and the loop with its early exit.

Bars: parcae_step within 1e-2 x RMS of the injected term LN(u) @ B^T against the fp64
oracle with the fp16 B the kernel uses; expected distance within 1e-4 A of the oracle
given the same fp16-rounded pair sums the kernel multiplies, and within 1e-2 A of the
unrounded oracle; the quantile equal to torch.quantile of the same fp32 values up to the
fp32 interpolation (1e-6 relative); the loop as the block stack (3e-2 max, 1e-2 normwise
of RMS(z)) against the oracle loop with fp16 trunk streams.
"""

import pytest
import torch

from oracle import recycle as orc, tmu as otmu, transition as otr

pytestmark = pytest.mark.gpu
DEV = "cuda"
D64 = torch.float64


@pytest.mark.parametrize("L,inplace", [(1, False), (33, False), (100, True)])
def test_parcae_step(gpu_lib, pkg, L, inplace):
    g = torch.Generator().manual_seed(L)
    z, zi, rf = (torch.randn(1, L, L, 128, generator=g) for _ in range(3))
    w, b = 1 + 0.1 * torch.randn(128, generator=g), 0.1 * torch.randn(128, generator=g)
    a = torch.rand(128, generator=g)
    bm = (torch.randn(128, 128, generator=g) * 128 ** -0.5).half()
    zd = z.to(DEV)
    out = pkg.kernels.parcae_step(zd, zi.to(DEV), rf.to(DEV), w.to(DEV), b.to(DEV), 1e-5, a.to(DEV), bm.to(DEV),
                                  out=zd if inplace else None)
    ref = orc.parcae_step(z.double(), zi.double(), rf.double(), w.double(), b.double(), a.double(), bm.double())
    inj = ref - a.double() * z.double()
    assert float((out.double().cpu() - ref).abs().max()) <= 1e-2 * float(inj.pow(2).mean().sqrt())


@pytest.mark.parametrize("L,nbins", [(1, 64), (5, 64), (130, 64), (37, 128)])
def test_expected_distance(gpu_lib, pkg, L, nbins):
    g = torch.Generator().manual_seed(L + nbins)
    r = torch.randn(2, L, L, 128, generator=g)
    w = (torch.randn(nbins, 128, generator=g) * 0.1).half()
    b = torch.randn(nbins, generator=g)
    c = orc.centers_6b() if nbins == 64 else orc.centers_experimental()
    ed = pkg.kernels.expected_distance(r.to(DEV), w.to(DEV), b.to(DEV), c.float().to(DEV)).double().cpu()
    s16 = (r + r.transpose(1, 2)).half().double()
    logits = s16 @ w.double().T + b.double()
    ref16 = torch.softmax(logits, -1) @ c
    assert float((ed - ref16).abs().max()) <= 1e-4
    ref = orc.expected_distance(r.double(), w.double(), b.double(), c)
    assert float((ed - ref).abs().max()) <= 1e-2
    assert torch.equal(ed, ed.transpose(1, 2))


@pytest.mark.parametrize("B,L,C,nbins", [(2, 257, 128, 64), (2, 97, 256, 128), (1, 257, 256, 64), (3, 32, 128, 128)])
def test_expected_distance_tiles_and_batches(gpu_lib, pkg, B, L, C, nbins):
    """Pairs j >= i in 32-pair tiles: a partial last row block (L = 257, 97), several batches (the
    unit index crossing b), both widths and both bin counts (128 bins at C = 256 reads the weight
    rows from LDS). The result is exactly symmetric and matches the fp16-rounded pair sums."""
    g = torch.Generator().manual_seed(B * 1000 + L + C + nbins)
    r = torch.randn(B, L, L, C, generator=g)
    w = (torch.randn(nbins, C, generator=g) * 0.05).half()
    b = torch.randn(nbins, generator=g)
    c = orc.centers_6b() if nbins == 64 else orc.centers_experimental()
    ed = pkg.kernels.expected_distance(r.to(DEV), w.to(DEV), b.to(DEV), c.float().to(DEV)).double().cpu()
    assert torch.equal(ed, ed.transpose(1, 2))
    s16 = (r + r.transpose(1, 2)).half().double()
    ref16 = torch.softmax(s16 @ w.double().T + b.double(), -1) @ c
    assert float((ed - ref16).abs().max()) <= 1e-4


@pytest.mark.parametrize("n", [1, 2, 3, 1000, 1001, 56644, 57343, 57344, 57345, 65536, 65537, 300000])
@pytest.mark.parametrize("q", [0.0, 0.5, 0.95, 1.0])
def test_abs_diff_quantile(gpu_lib, pkg, n, q):
    """Against torch.quantile, with ties, at the endpoints, across the largest size held in
    registers (57,344; n % 4 != 0 takes the tail loads) and across 2^16 values."""
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, generator=g) * 3
    y = torch.randn(n, generator=g) * 3
    if n >= 1000:
        x[: n // 3] = torch.round(x[: n // 3])  # ties
        y[: n // 3] = 0
    got = float(pkg.kernels.abs_diff_quantile(x.to(DEV), y.to(DEV), q).item())
    ref = float(torch.quantile((x - y).abs().double(), q))  # fp32 differences, as the kernel forms them
    assert abs(got - ref) <= 1e-6 * max(1.0, abs(ref))
    got1 = float(pkg.kernels.abs_diff_quantile(x.to(DEV), None, q).item())
    assert abs(got1 - float(torch.quantile(x.abs().double(), q))) <= 1e-6 * max(1.0, float(x.abs().max()))


@pytest.mark.parametrize("n", [1000, 57344, 60000])
def test_abs_diff_quantile_ranks_in_two_bins(gpu_lib, pkg, n):
    """The two order statistics around the quantile in different histogram bins (1.00x and
    1.5x differ in their top 16 bits), so the lower is the largest of one bin and the upper the
    smallest of the next; interpolated halfway, at the largest size held in registers and past it."""
    g = torch.Generator().manual_seed(7)
    k = n - n // 20
    x = torch.empty(n)
    x[:k] = 1.0 + torch.rand(k, generator=g) * 0.007  # all in the bin of 1.0 (top 16 bits 0x3f80)
    x[k:] = 1.5 + torch.rand(n - k, generator=g) * 0.4
    x = x[torch.randperm(n, generator=g)]
    # pos = k - 1/2: between the k-th smallest (1.00x) and the next (1.5x); q as the kernel
    # receives it (fp32), since here the interpolation weight moves the result by ~0.5 per unit
    q = float(torch.tensor((k - 0.5) / (n - 1), dtype=torch.float32))
    got = float(pkg.kernels.abs_diff_quantile(x.to(DEV), None, q).item())
    ref = float(torch.quantile(x.double(), q))
    assert abs(got - ref) <= 1e-6 * abs(ref)
    y = torch.rand(n, generator=g) * 0.001
    got = float(pkg.kernels.abs_diff_quantile((x + y).to(DEV), y.to(DEV), q).item())
    ref = float(torch.quantile(((x + y) - y).abs().double(), q))
    assert abs(got - ref) <= 1e-6 * abs(ref)


@pytest.mark.parametrize("n", [4096, 65536, 70000])
def test_abs_diff_quantile_one_value(gpu_lib, pkg, n):
    """Every value but one in a single histogram bin."""
    x = torch.full((n,), 2.5)
    x[n // 2] = 7.0
    got = float(pkg.kernels.abs_diff_quantile(x.to(DEV), None, 0.95).item())
    assert got == float(torch.quantile(x.double(), 0.95))


def _oracle_trunk(blocks):
    f = ("w_bundle", "w_emit", "w_gate", "ln_in_w", "ln_in_b", "ln_mix_w", "ln_mix_b", "ln_in_eps", "ln_mix_eps",
         "outgoing")
    return [otr.BlockWeights(otmu.TriMulWeights(**{k: getattr(po, k) for k in f}).to(D64),
                             otmu.TriMulWeights(**{k: getattr(pi, k) for k in f}).to(D64),
                             otr.TransitionWeights(pt.ln_w.double(), pt.ln_b.double(), pt.w1.double(), pt.w3.double()))
            for po, pi, pt in blocks]


@pytest.mark.parametrize("threshold", [None, 1e9])
def test_parcae_loop(gpu_lib, pkg, threshold):
    L, steps = 24, 3
    W = pkg.workloads
    _, lm_blocks = W.block_stack(L, n_blocks=1, seed=1)
    _, tr_blocks = W.block_stack(L, n_blocks=1, seed=2)
    _, coda_blocks = W.block_stack(L, n_blocks=1, seed=3)
    T = pkg.trunk.PairTrunk
    g = torch.Generator().manual_seed(4)
    z0, zi, lm_z = (torch.randn(1, L, L, 128, generator=g) for _ in range(3))
    ln_w, ln_b = 1 + 0.1 * torch.randn(128, generator=g), 0.1 * torch.randn(128, generator=g)
    a = torch.rand(128, generator=g)
    bm = torch.randn(128, 128, generator=g) * 128 ** -0.5
    ro = torch.randn(128, 128, generator=g) * 128 ** -0.5
    dw, db = torch.randn(64, 128, generator=g) * 0.1, torch.randn(64, generator=g)
    masks = [(torch.rand(1, L, L, 128, generator=g) > 0.25).float() / 0.75 for _ in range(steps)]
    calls = []

    def drop(t, p):  # deterministic stand-in for torch's dropout: the same masks on both sides
        calls.append(p)
        return t * masks[(len(calls) - 1) % steps].to(t.device)

    sig = pkg.recycle.DistogramSignal(dw, db, pkg.recycle.centers_6b())
    loop = pkg.recycle.ParcaeLoop(T.from_weights(lm_blocks), T.from_weights(tr_blocks), ln_w, ln_b, ro, sig,
                                  coda=T.from_weights(coda_blocks), threshold=threshold)
    z = loop.run(z0.to(DEV), zi.to(DEV), lm_z.to(DEV), None, a.to(DEV), bm.to(DEV), steps, dropout=drop)
    if threshold is None:
        assert loop.steps_run == steps and len(calls) == steps
    else:  # signals from step min_steps - 1; the first comparison at step 2 exits; rng burnt for step 3
        assert loop.steps_run == 2 and len(calls) == steps and len(loop.history) == 1
    # the oracle loop (fp16 residual streams in the trunks, fp16 B as the kernel uses)
    zz = z0.double()
    for k in range(loop.steps_run):
        refined = otr.stack_forward((lm_z * masks[k]).double(), None, _oracle_trunk(lm_blocks), 1,
                                    store=torch.float16)
        zz = orc.parcae_step(zz, zi.double(), refined, ln_w.double(), ln_b.double(), a.double(),
                             bm.half().double())
        zz = otr.stack_forward(zz, None, _oracle_trunk(tr_blocks), 1, store=torch.float16)
    d = z.double().cpu() - zz
    rms = float(zz.pow(2).mean().sqrt())
    assert float(d.abs().max()) <= 3e-2 * rms and float(d.pow(2).mean().sqrt()) <= 1e-2 * rms
