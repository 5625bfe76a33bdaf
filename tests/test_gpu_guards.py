"""Caller-provided outputs and auxiliary tensors are size-checked before any launch.

A raw device pointer carries no size, so the Python wrappers check the element count of
every tensor a kernel writes or reads by index; an undersized one is refused with
ESM_ERR_SHAPE (-2) and nothing is launched.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
F16 = torch.float16


def _refused(pkg, fn):
    with pytest.raises(pkg.capi.EsmError) as e:
        fn()
    assert e.value.code == -2, str(e.value)


def test_undersized_outputs_are_refused(gpu_lib, pkg):
    K = pkg.kernels
    L, C = 8, 128
    z = torch.zeros(1, L, L, C, dtype=F16, device=DEV)
    w = torch.zeros(512, C, dtype=F16, device=DEV)
    ones, zeros = torch.ones(C, device=DEV), torch.zeros(C, device=DEV)
    short = torch.zeros(z.numel() - 8, dtype=F16, device=DEV)
    # transition, epilogue
    _refused(pkg, lambda: K.transition(z, ones, zeros, 1e-5, w, w.T.contiguous(), out=short))
    a, b = K.project(z, None, ones, zeros, 1e-5, w, incoming=False)
    x = K.contract(a, b, L)
    wc = torch.zeros(C, C, dtype=F16, device=DEV)
    _refused(pkg, lambda: K.epilogue(x, z, None, ones, zeros, 1e-5, ones, zeros, 1e-5, wc, wc, out=short))
    _refused(pkg, lambda: K.project(z, torch.ones(L * L - 1, dtype=F16, device=DEV), ones, zeros, 1e-5, w, False))
    # q8 linear
    xq = torch.zeros(4, 128, dtype=F16, device=DEV)
    q = torch.zeros(64, 128, dtype=torch.uint8, device=DEV)
    s = torch.zeros(64, 2, dtype=F16, device=DEV)
    _refused(pkg, lambda: K.q8_linear(xq, q, s, s, out=torch.empty(4, 63, dtype=F16, device=DEV)))
    # ESMC kernels
    xe = torch.zeros(4, 128, device=DEV)
    we = torch.ones(128, device=DEV)
    _refused(pkg, lambda: K.esmc_layer_norm(xe, we, None, 1e-5, out=torch.empty(4, 127, dtype=F16, device=DEV)))
    _refused(pkg, lambda: K.esmc_layer_norm(xe, we, None, 1e-5, y=torch.zeros(4, 128, dtype=F16, device=DEV),
                                            x_out=torch.empty(3, 128, device=DEV)))
    qkv = torch.zeros(4, 3 * 128, dtype=F16, device=DEV)
    _refused(pkg, lambda: K.esmc_qk_rope(qkv, we, we, 1e-5, 1, 5, 2))
    hq = torch.zeros(1, 2, 4, 64, dtype=F16, device=DEV)
    _refused(pkg, lambda: K.esmc_attention(hq, hq, hq, torch.zeros(1, 3, dtype=torch.int32, device=DEV)))
    _refused(pkg, lambda: K.esmc_attention(hq, hq, hq, out=torch.empty(1, 4, 64, dtype=F16, device=DEV)))
    _refused(pkg, lambda: K.esmc_swiglu(torch.zeros(4, 64, dtype=F16, device=DEV),
                                        out=torch.empty(4, 31, dtype=F16, device=DEV)))
    # recycling kernels
    zr = torch.zeros(1, L, L, C, device=DEV)
    bm = torch.zeros(C, C, dtype=F16, device=DEV)
    _refused(pkg, lambda: K.parcae_step(zr, zr, zr[:, :4].contiguous(), ones, zeros, 1e-5, ones, bm))
    _refused(pkg, lambda: K.expected_distance(zr, torch.zeros(64, C, dtype=F16, device=DEV), torch.zeros(64, device=DEV),
                                              torch.zeros(64, device=DEV), out=torch.empty(L * L - 1, device=DEV)))
    _refused(pkg, lambda: K.abs_diff_quantile(zr.flatten(), out=torch.empty(2, device=DEV)))
    # the pair driver's out
    T = pkg.trimul
    from oracle import tmu
    p = tmu.draw_weights(torch.Generator().manual_seed(0), C, C, True)
    pi = tmu.draw_weights(torch.Generator().manual_seed(1), C, C, False)
    pair = T.TriMulPair(T.TriMul.from_weights(p), T.TriMul.from_weights(pi))
    _refused(pkg, lambda: pair(z, out=torch.empty(1, L, L - 1, C, dtype=F16, device=DEV)))
    torch.cuda.synchronize()
