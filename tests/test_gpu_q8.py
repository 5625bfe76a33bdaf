"""GPU parity of the 8-bit weight-only linear (kernel d) and its dequantiser.

Bars: dequantised weights bit-exact against RN_fp16(s*q + b); the GEMM within
1e-3 normwise relative error of the fp64 oracle x . W^T (and max|err| within
1e-3 * max|ref|).
"""

import numpy as np
import pytest
import torch

from oracle import q8

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.mark.parametrize("N,K", [(64, 64), (128, 192), (256, 2560)])
def test_dequant_bit_exact(gpu_lib, pkg, N, K):
    _, q, s, b = q8.make_q8_inputs(1, K, N, seed=N + K)
    w = pkg.kernels.q8_dequant(_t(q), _t(s), _t(b)).cpu().numpy()
    assert np.array_equal(w.view(np.uint16), q8.dequant_f16(q, s, b).view(np.uint16))


def test_dequant_special_values(gpu_lib, pkg):
    N, K = 64, 128
    q = np.tile(np.arange(128, dtype=np.uint8) * 2, (N, 1))
    q[:, 0] = 0
    q[:, 1] = 255
    rng = np.random.default_rng(0)
    s = rng.uniform(0.001, 0.01, (N, 2)).astype(np.float16)
    b = rng.normal(0, 0.1, (N, 2)).astype(np.float16)
    s[0] = 0                                     # s = 0 -> b
    b[1] = np.float16(2.0 ** -20)                # subnormal fp16 bias
    s[2], b[2] = np.float16(2.0 ** -14), 0       # tiny products: subnormal results
    b[3] = np.float16(-0.0)
    w = pkg.kernels.q8_dequant(_t(q), _t(s), _t(b)).cpu().numpy()
    assert np.array_equal(w.view(np.uint16), q8.dequant_f16(q, s, b).view(np.uint16))


def _check(y, x, q, s, b):
    ref = q8.q8_linear(x, q, s, b)
    y = y.astype(np.float64)
    assert np.isfinite(y).all()
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel <= 1e-3, f"normwise relative error {rel:.3e}"
    assert np.abs(y - ref).max() <= 1e-3 * np.abs(ref).max()
    # against the fp16-rounded weights the kernel multiplies by: only accumulation order
    # and the output rounding remain
    ref16 = q8.q8_linear(x, q, s, b, weights="f16")
    assert np.linalg.norm(y - ref16) / np.linalg.norm(ref16) <= 3e-4
    return rel


@pytest.mark.parametrize("M,K,N", [(1, 64, 64), (5, 128, 64), (37, 256, 128), (64, 640, 192), (65, 1024, 256),
                                   (238, 2560, 512)])
def test_q8_linear_small(gpu_lib, pkg, M, K, N):
    x, q, s, b = q8.make_q8_inputs(M, K, N, seed=M)
    y = pkg.kernels.q8_linear(_t(x), _t(q), _t(s), _t(b)).cpu().numpy()
    _check(y, x, q, s, b)


@pytest.mark.parametrize("K,N", [(2560, 10240), (10240, 2560)])
def test_q8_linear_esmc_shapes(gpu_lib, pkg, K, N):
    # the ESMC-style linears: [238, 2560] x [2560 -> 10240] and [238, 10240] x [10240 -> 2560]
    x, q, s, b = q8.make_q8_inputs(238, K, N, seed=K)
    y = pkg.kernels.q8_linear(_t(x), _t(q), _t(s), _t(b)).cpu().numpy()
    _check(y, x, q, s, b)


def test_q8_module_and_mlx_packing(gpu_lib, pkg):
    x, q, s, b = q8.make_q8_inputs(10, 128, 64, seed=3)
    words = torch.from_numpy(q.copy()).view(torch.int32)  # four codes per 32-bit word, little-endian
    lin = pkg.q8.Q8Linear.from_packed_u32(words, torch.from_numpy(s), torch.from_numpy(b))
    y = lin(torch.from_numpy(x).to(DEV).float())  # fp32 in -> fp32 out
    assert y.dtype == torch.float32
    _check(y.cpu().numpy(), x, q, s, b)


def test_q8_linear_rejects_bad_shapes(gpu_lib, pkg):
    x, q, s, b = q8.make_q8_inputs(4, 128, 64, seed=0)
    with pytest.raises(Exception):
        pkg.kernels.q8_linear(_t(x[:, :64]), _t(q), _t(s), _t(b))
