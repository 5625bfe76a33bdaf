"""The recycling-loop plugins' bookkeeping on the CPU, with stand-in trunks (no kernels run):
AdaptiveTrunk (var_adaptive_loops.py:79-156's behaviour) with the "z_rel" signal, and the exit
hand-off of the 6B loop plugin (var_6b_mlx_loop.py:88-113, :229-236's behaviour). The GPU
versions, with the real signal and the HIP trunks, are in test_gpu_loops.py."""

import pytest
import torch
from torch import nn


class _Config:
    num_loops = 3


class _ContractingTrunk(nn.Module):
    """z -> 0.5 z + 1: successive outputs of the recycling converge geometrically."""

    def __init__(self):
        super().__init__()
        self.calls = 0

    def forward(self, pair, pair_attention_mask=None):
        self.calls += 1
        return 0.5 * pair + 1.0


class _Model(nn.Module):
    """upstream's recycling: z = trunk(z_init + pair_loop_proj(z)), num_loops + 1 times from 0."""

    def __init__(self, C=4):
        super().__init__()
        g = torch.Generator().manual_seed(0)
        self.config = _Config()
        self.folding_trunk = _ContractingTrunk()
        self.pair_loop_proj = nn.Linear(C, C)
        self.distogram_head = nn.Linear(C, 128)
        with torch.no_grad():
            self.pair_loop_proj.weight.copy_(0.3 * torch.randn(C, C, generator=g))
            self.pair_loop_proj.bias.copy_(0.1 * torch.randn(C, generator=g))

    def forward(self, z_init, pair_mask=None, num_loops=None):
        n = self.config.num_loops if num_loops is None else num_loops
        z = torch.zeros_like(z_init)
        for _ in range(n + 1):
            z = self.folding_trunk(z_init + self.pair_loop_proj(z), pair_attention_mask=pair_mask)
        return z


def _zi():
    return torch.randn(1, 3, 3, 4, generator=torch.Generator().manual_seed(1))


def test_settled_fold_equals_the_fold_with_fewer_loops(pkg):
    zi = _zi()
    m = _Model()
    trunk = pkg.var_hip_adaptive_loops.apply(m, metric="z_rel", threshold=1e9)
    inner = trunk.trunk
    out = m(zi, num_loops=4)
    assert trunk.passes == 2 and trunk.calls == 5 and trunk.converged and inner.calls == 2
    assert len(trunk.history) == 1 and "z_rel" in trunk.history[0]
    assert torch.equal(out, _Model()(zi, num_loops=1))
    # a new call opens a new fold; the state dict is the model's own
    m(zi, num_loops=2)
    assert trunk.calls == 3 and trunk.passes == 2
    assert set(m.state_dict()) == {k.replace("folding_trunk.", "folding_trunk.trunk.") for k in _Model().state_dict()}


def test_unsettled_fold_runs_every_pass_and_records_each_change(pkg):
    zi = _zi()
    m = _Model()
    trunk = pkg.var_hip_adaptive_loops.apply(m, metric="z_rel", threshold=-1.0)
    out = m(zi)  # config.num_loops = 3: four passes
    assert trunk.passes == 4 and len(trunk.history) == 3 and not trunk.converged
    assert torch.equal(out, _Model()(zi))
    # the contraction halves the change each pass; the recorded signal sees it fall
    ch = [h["z_rel"] for h in trunk.history]
    assert ch[0] > ch[1] > ch[2] > 0


def test_min_passes_gates_the_exit(pkg):
    m = _Model()
    trunk = pkg.var_hip_adaptive_loops.apply(m, metric="z_rel", threshold=1e9, min_passes=3)
    m(_zi(), num_loops=4)
    assert trunk.passes == 3 and trunk.converged


def test_extra_passes_continue_the_recurrence(pkg):
    zi = _zi()
    ref = _Model()(zi, num_loops=3)  # four passes
    m = _Model()
    trunk = pkg.var_hip_adaptive_loops.apply(m, metric="z_rel", threshold=-1.0, max_extra=2)
    out = m(zi, num_loops=1)  # two scheduled passes + two extra inside the last call
    assert trunk.passes == 4 and len(trunk.history) == 3
    assert torch.allclose(out, ref, rtol=1e-6, atol=1e-6)
    # an extra threshold every change passes stops after the first extra pass
    m2 = _Model()
    t2 = pkg.var_hip_adaptive_loops.apply(m2, metric="z_rel", threshold=-1.0, max_extra=3, extra_threshold=1e9)
    m2(zi, num_loops=1)
    assert t2.passes == 3


def test_reapply_replaces_the_wrapper_and_its_hook(pkg):
    m = _Model()
    first = pkg.var_hip_adaptive_loops.apply(m, metric="z_rel", threshold=-1.0)
    second = pkg.var_hip_adaptive_loops.apply(m, metric="z_rel", threshold=1e9)
    assert second.trunk is first.trunk and m.folding_trunk is second
    m(_zi(), num_loops=3)
    assert second.passes == 2 and first.calls == 0  # only the new wrapper's fold hook runs
    assert len(m._forward_pre_hooks) == 1


def test_unknown_metric_is_refused(pkg):
    with pytest.raises(ValueError, match="metric"):
        pkg.var_hip_adaptive_loops.apply(_Model(), metric="disto_mean")


def test_exit_handoff_reuses_the_coda_output_once(pkg):
    L6 = pkg.var_6b_hip_loop
    handoff = L6.ExitHandoff()
    readout = nn.Linear(4, 4, bias=False)
    coda_calls = []

    class Coda(nn.Module):
        def forward(self, x, pair_attention_mask=None):
            coda_calls.append(1)
            return 2 * x

    coda = L6.ExitCache(Coda(), handoff)
    hook = readout.register_forward_hook(handoff.readout_hook)
    z, other = torch.randn(2, 4), torch.randn(2, 4)
    out = torch.randn(2, 4)
    handoff.arm(z, out)
    # another input takes the ordinary path and leaves the hand-off armed
    with torch.no_grad():
        assert torch.equal(coda(readout(other)), 2 * (other @ readout.weight.T))
    assert len(coda_calls) == 1 and handoff.z is z
    # forward's readout -> coda of the exit z: the stored output, no coda pass, hand-off spent
    assert coda(readout(z), pair_attention_mask=None) is out
    assert len(coda_calls) == 1 and handoff.z is None and handoff.out is None
    # spent: the same z now runs the coda
    coda(readout(z))
    assert len(coda_calls) == 2
    hook.remove()
    assert set(coda.state_dict()) == set()  # the wrapper adds no state of its own


def test_exit_policy_checks_and_overrides(pkg):
    L6 = pkg.var_6b_hip_loop
    with pytest.raises(ValueError, match="threshold"):
        L6.ExitPolicy(adaptive=True)
    with pytest.raises(ValueError, match="source"):
        L6.ExitPolicy(source="trunk")
    p = pkg.var_6b_hip_adaptive.POLICY
    assert (p.adaptive, p.threshold, p.source, p.min_steps, p.burn_rng) == (True, 0.5, "coda", 2, True)
    q = L6.with_policy(p, threshold=1e9, burn_rng=False)
    assert (q.threshold, q.burn_rng, q.min_steps) == (1e9, False, 2) and p.threshold == 0.5
    assert q.hands_off_coda and not L6.with_policy(p, source="readout").hands_off_coda
