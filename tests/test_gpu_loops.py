"""GPU tests of the recycling-loop plugins on models shaped like the reference's:
var_6b_hip_loop / var_6b_hip_adaptive (the 6B parcae loop and its early exit,
var_6b_mlx_loop.py:88-236, var_6b_adaptive.py) and var_hip_adaptive_loops (the
AdaptiveTrunk of var_adaptive_loops.py:79-156).

The loop's arithmetic is checked against the oracle loop in test_gpu_recycle.py; here the
plugins' contracts: the loop installed by name, the exit step, the exit step's coda output
handed to forward without a second coda pass, the random stream of a full-length fold, and
for AdaptiveTrunk a converged fold equal to one with fewer loops.
"""

import pytest
import torch

from oracle import recycle as orc
from tests import ref_modules

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _swiglu_blocks(pkg, L, n, seed):
    _, blocks = pkg.workloads.block_stack(L, n_blocks=n, H=256, seed=seed)
    g = torch.Generator().manual_seed(seed + 100)
    for _, _, pt in blocks:
        pt.w2 = torch.randn(256, 128, generator=g) * 128 ** -0.5
    return blocks


def _model6b(pkg, L=20):
    m = ref_modules.Model6BLoop(_swiglu_blocks(pkg, L, 1, 1), _swiglu_blocks(pkg, L, 1, 2),
                                _swiglu_blocks(pkg, L, 1, 3), seed=4).to(DEV)
    pkg.variants.apply_variants(m, ["6b_hip_trunks"])
    return m


def _inputs(L=20, seed=5):
    g = torch.Generator().manual_seed(seed)
    z0, zi, lm_z = (torch.randn(1, L, L, 128, generator=g).to(DEV) for _ in range(3))
    a = torch.rand(128, generator=g).to(DEV)
    bm = (torch.randn(128, 128, generator=g) * 128 ** -0.5).to(DEV)
    return z0, zi, lm_z, a, bm


def _count_calls(module):
    calls = []
    inner = module.forward

    def counted(*a, **k):
        calls.append(1)
        return inner(*a, **k)

    module.forward = counted
    return calls


def test_6b_loop_plugin_runs_every_step(gpu_lib, pkg):
    m = _model6b(pkg)
    z0, zi, lm_z, a, bm = _inputs()
    loop = pkg.variants.apply_variants(m, ["6b_hip_loop"])._hip_loop
    assert m._run_one_loop == loop.run and not isinstance(m.parcae_coda, pkg.var_6b_hip_loop.ExitCache)
    torch.cuda.manual_seed(11)
    out = m(z0, zi, lm_z, None, a, bm, num_loops=2)
    assert loop.steps_run == 3 and out.dtype == torch.float32 and torch.isfinite(out).all()
    # the same loop run directly, then readout -> coda: the same bits
    torch.cuda.manual_seed(11)
    z = pkg.recycle.ParcaeLoop.from_model(m).run(z0, zi, lm_z, None, a, bm, 3)
    ref = m.parcae_coda(m.parcae_readout(z))
    assert torch.equal(out, ref)
    with pytest.raises(NotImplementedError):
        loop.run(z0, zi, lm_z, object(), None, a, bm, None, 2)  # MSA input


@pytest.mark.parametrize("burn", [True, False])
def test_6b_adaptive_exit_hands_coda_output_to_forward(gpu_lib, pkg, burn):
    z0, zi, lm_z, a, bm = _inputs()
    # the full-length fold's output after 2 steps, and the random stream after 4 steps
    full = _model6b(pkg)
    pkg.var_6b_hip_loop.apply(full)
    torch.cuda.manual_seed(3)
    ref2 = full(z0, zi, lm_z, None, a, bm, num_loops=1)
    torch.cuda.manual_seed(3)
    full(z0, zi, lm_z, None, a, bm, num_loops=3)
    after_full = torch.rand(4, device=DEV)
    # adaptive: a threshold every change passes exits at the first comparison (step 2 of 4)
    m = _model6b(pkg)
    loop = pkg.var_6b_hip_adaptive.apply(m, threshold=1e9, burn_rng=burn)
    assert isinstance(m.parcae_coda, pkg.var_6b_hip_loop.ExitCache)
    calls = _count_calls(m.parcae_coda.inner)
    torch.cuda.manual_seed(3)
    out = m(z0, zi, lm_z, None, a, bm, num_loops=3)
    after = torch.rand(4, device=DEV)
    assert loop.steps_run == 2 and len(loop.history) == 1 and "coda_p95" in loop.history[0]
    # the coda ran for the signals of steps 1 and 2 only: forward reused the exit step's output
    assert len(calls) == 2
    assert loop.exit_z is None and loop.exit_out is None  # handed on and cleared
    assert torch.equal(out, ref2)  # the fold of num_loops = 1, bit for bit
    assert torch.equal(after, after_full) == burn  # the skipped steps' dropout masks burnt
    # a threshold nothing passes runs every step and computes signals for steps 1..3
    m2 = _model6b(pkg)
    loop2 = pkg.var_6b_hip_adaptive.apply(m2, threshold=-1.0)
    torch.cuda.manual_seed(3)
    m2(z0, zi, lm_z, None, a, bm, num_loops=3)
    assert loop2.steps_run == 4 and len(loop2.history) == 2


def _model300m(pkg, L=20):
    m = ref_modules.Model300MLoop(_swiglu_blocks(pkg, L, 2, 7), seed=8).to(DEV)
    pkg.var_hip_trunk.apply(m)
    return m


def test_adaptive_trunk_converged_fold_equals_fewer_loops(gpu_lib, pkg):
    L = 20
    zi = torch.randn(1, L, L, 128, generator=torch.Generator().manual_seed(9)).to(DEV)
    ref = _model300m(pkg)(zi, num_loops=1)  # two passes, no plugin
    m = _model300m(pkg)
    trunk = pkg.variants.apply_variants(m, ["hip_adaptive_loops"]).folding_trunk
    assert isinstance(trunk, pkg.var_hip_adaptive_loops.AdaptiveTrunk)
    trunk.threshold = 1e9  # every change passes: converged after min_passes = 2
    calls = _count_calls(trunk.trunk)
    out = m(zi, num_loops=3)
    assert trunk.passes == 2 and len(calls) == 2 and trunk.calls == 4 and trunk.converged
    assert torch.equal(out, ref)
    # a new fold resets the state
    m(zi, num_loops=3)
    assert trunk.passes == 2 and trunk.calls == 4


def test_adaptive_trunk_signal_against_oracle(gpu_lib, pkg):
    L = 20
    zi = torch.randn(1, L, L, 128, generator=torch.Generator().manual_seed(10)).to(DEV)
    m = _model300m(pkg)
    trunk = pkg.var_hip_adaptive_loops.apply(m, threshold=-1.0)  # never converges
    outs = []
    inner = trunk.trunk.forward
    trunk.trunk.forward = lambda *a, **k: outs.append(inner(*a, **k)) or outs[-1]
    m(zi, num_loops=2)
    assert trunk.passes == 3 and len(trunk.history) == 2
    w, b = m.distogram_head.weight.double().cpu(), m.distogram_head.bias.double().cpu()
    eds = [orc.expected_distance(o.double().cpu(), w, b, orc.centers_experimental()) for o in outs]
    for k, h in enumerate(trunk.history):
        ref = float(orc.quantile((eds[k + 1] - eds[k]).abs(), 0.95))
        assert abs(h["disto_p95"] - ref) <= 2e-2 + 1e-2 * ref, (h, ref)


def test_adaptive_trunk_extra_passes_repeat_the_recurrence(gpu_lib, pkg):
    L = 20
    zi = torch.randn(1, L, L, 128, generator=torch.Generator().manual_seed(12)).to(DEV)
    ref = _model300m(pkg)(zi, num_loops=3)  # 4 passes, no plugin
    m = _model300m(pkg)
    trunk = pkg.var_hip_adaptive_loops.apply(m, metric="z_rel", threshold=-1.0, max_extra=2)
    out = m(zi, num_loops=1)  # 2 scheduled passes + 2 extra inside the last call
    assert trunk.passes == 4 and len(trunk.history) == 3 and "z_rel" in trunk.history[0]
    # z_init recovered as input - proj(0): the extra passes continue the same recurrence
    assert float((out - ref).abs().max()) <= 1e-3 * float(ref.abs().max())
