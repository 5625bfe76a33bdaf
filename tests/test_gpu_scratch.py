"""GPU tests of the device's shared scratch (scratch.py): calls on two streams with no
synchronisation of their own are ordered through the buffer and give the single-stream bits,
a grown buffer stays valid for work queued on every stream that used it, and split-K partials
handed out in the scratch are refused once it has been reused."""

import pytest
import torch

from oracle import q8

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _pair(pkg, L, seed):
    z, _, po, pi = pkg.workloads.pair_inputs(L, 128, 128, seed=seed, dtype=torch.float16)
    T = pkg.trimul
    return z.to(DEV), T.TriMulPair(T.TriMul.from_weights(po, device=DEV), T.TriMul.from_weights(pi, device=DEV))


def test_two_streams_are_ordered_through_the_scratch(gpu_lib, pkg):
    cases = [_pair(pkg, L, seed) for L, seed in ((96, 1), (160, 2), (64, 3))]
    refs = [m(z) for z, m in cases]
    torch.cuda.synchronize()
    pkg.scratch.release(DEV)  # start small: the calls below grow the buffer while streams alternate
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for rep in range(3):
        for k, (z, m) in enumerate(cases):
            with torch.cuda.stream(s1 if (rep + k) % 2 == 0 else s2):
                outs.append((k, m(z)))
    torch.cuda.synchronize()
    for k, out in outs:
        assert torch.equal(out.view(torch.int16), refs[k].view(torch.int16)), k


def test_stale_partials_are_refused(gpu_lib, pkg):
    x, qq, s, b = q8.make_q8_inputs(238, 10240, 2560, seed=4)
    lin = pkg.q8.Q8Linear(torch.from_numpy(qq), torch.from_numpy(s), torch.from_numpy(b))
    xt = torch.from_numpy(x).to(DEV)
    D = 2560
    res = torch.randn(238, D, device=DEV)
    w, bb = torch.ones(D, device=DEV), torch.zeros(D, device=DEV)
    parts = lin.partials(xt)
    assert parts[1] > 1  # split-K at this shape: the partials live in the scratch
    pkg.kernels.esmc_layer_norm(res, w, bb, 1e-5, y_parts=parts)  # consumed in time: fine
    lin(xt)  # another scratch user
    with pytest.raises(RuntimeError, match="stale"):
        pkg.kernels.esmc_layer_norm(res, w, bb, 1e-5, y_parts=parts)
