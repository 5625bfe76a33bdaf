"""The package's synthetic workload generators draw exactly the oracle's inputs (the GPU
leg of the benchmark and the smoke run use the package's; the checks use the oracle's)."""

import numpy as np
import torch

from oracle import q8, tmu


def test_pair_inputs_match_the_oracle(pkg):
    for kw in ({"L": 17, "seed": 3, "dtype": torch.float16}, {"L": 9, "seed": 0, "dtype": torch.float32, "B": 2,
                                                                 "pad_from": 6}):
        z, m, po, pi = pkg.workloads.pair_inputs(C=128, c=128, **kw)
        z2, m2, po2, pi2 = tmu.make_pair_inputs(C=128, c=128, **kw)
        assert torch.equal(z, z2)
        assert (m is None and m2 is None) or torch.equal(m, m2)
        for a, b in ((po, po2), (pi, pi2)):
            for f in ("w_bundle", "w_emit", "w_gate", "ln_in_w", "ln_in_b", "ln_mix_w", "ln_mix_b"):
                assert torch.equal(getattr(a, f), getattr(b, f)), f
            assert a.outgoing == b.outgoing and a.ln_in_eps == b.ln_in_eps and a.ln_mix_eps == b.ln_mix_eps


def test_q8_inputs_match_the_oracle(pkg):
    got = pkg.workloads.q8_inputs(5, 256, 64, seed=11)
    ref = q8.make_q8_inputs(5, 256, 64, seed=11)
    for a, b in zip(got, ref):
        assert np.array_equal(a.numpy(), b)


def test_block_stack_matches_the_oracle(pkg):
    from oracle import transition as otr
    z, blocks = pkg.workloads.block_stack(9, n_blocks=3, H=256, seed=5)
    g = torch.Generator().manual_seed(5)
    z2 = torch.randn(1, 9, 9, 128, generator=g).half()
    ref = otr.draw_blocks(g, 3, 128, 128, 256)
    assert torch.equal(z, z2)
    for (po, pi, pt), rb in zip(blocks, ref):
        for a, b in ((po, rb.tri_out), (pi, rb.tri_in)):
            for f in ("w_bundle", "w_emit", "w_gate"):
                assert torch.equal(getattr(a, f), getattr(b, f))
        for f in ("ln_w", "ln_b", "w1", "w3"):
            assert torch.equal(getattr(pt, f), getattr(rb.trans, f))
        assert pt.w2 is None and rb.trans.w2 is None
