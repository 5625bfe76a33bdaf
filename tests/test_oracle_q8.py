"""Pins the q8-linear oracle (oracle/q8.py): exact arithmetic, special cases, brute force."""

from fractions import Fraction

import numpy as np
import pytest

from oracle import q8


def _small(seed=0, M=3, K=128, N=5):
    return q8.make_q8_inputs(M, K, N, seed=seed)


def test_dequant_exact_matches_rational_arithmetic():
    _, q, s, b = _small(seed=1, N=7, K=192)
    W = q8.dequant_exact(q, s, b)
    rng = np.random.default_rng(0)
    for _ in range(400):
        n, k = rng.integers(0, q.shape[0]), rng.integers(0, q.shape[1])
        exact = Fraction(float(s[n, k // 64])) * int(q[n, k]) + Fraction(float(b[n, k // 64]))
        assert Fraction(float(W[n, k])) == exact  # fp64 holds the exact sum


def test_single_rounding_f16_and_f32():
    _, q, s, b = _small(seed=2, N=16, K=256)
    exact = q8.dequant_exact(q, s, b)
    w16, w32 = q8.dequant_f16(q, s, b), q8.dequant_f32(q, s, b)
    assert w16.dtype == np.float16 and w32.dtype == np.float32
    # round-to-nearest: no representable value is closer than the chosen one
    up16 = np.nextafter(w16, np.float16(np.inf)).astype(np.float64)
    dn16 = np.nextafter(w16, np.float16(-np.inf)).astype(np.float64)
    err = np.abs(w16.astype(np.float64) - exact)
    assert np.all(err <= np.abs(up16 - exact)) and np.all(err <= np.abs(dn16 - exact))
    # fp32: s*q is exact in fp32 (11 + 8 bits), so an fp32 FMA and a mul-then-add agree
    s32 = np.repeat(s.astype(np.float32), 64, 1)
    b32 = np.repeat(b.astype(np.float32), 64, 1)
    prod = s32 * q.astype(np.float32)
    assert np.array_equal(prod.astype(np.float64), np.repeat(s.astype(np.float64), 64, 1) * q)
    assert np.array_equal(prod + b32, w32)


def test_special_cases():
    q = np.array([[0, 255, 1, 128] * 16], dtype=np.uint8)
    s = np.array([[0.005]], dtype=np.float16)
    b = np.array([[-0.0312]], dtype=np.float16)
    W = q8.dequant_exact(q, s, b)
    assert W[0, 0] == float(b[0, 0])                              # q = 0 -> b
    assert W[0, 1] == float(s[0, 0]) * 255 + float(b[0, 0])
    W0 = q8.dequant_exact(q, np.zeros_like(s), b)
    assert np.all(W0 == float(b[0, 0]))                            # s = 0 -> b
    Wb = q8.dequant_exact(q, s, np.zeros_like(b))
    assert Wb[0, 1] == float(s[0, 0]) * 255                        # b = 0 -> s*q


def test_group_index_runs_along_k():
    # a different scale per group must only affect that group's 64 columns
    q = np.full((2, 192), 3, dtype=np.uint8)
    s = np.array([[1, 2, 4], [8, 16, 32]], dtype=np.float16)
    b = np.zeros_like(s)
    W = q8.dequant_exact(q, s, b)
    assert np.all(W[0, :64] == 3) and np.all(W[0, 64:128] == 6) and np.all(W[0, 128:] == 12)
    assert np.all(W[1, 128:] == 96)


def test_linear_bruteforce_and_grouped_identity():
    x, q, s, b = _small(seed=3, M=3, K=128, N=4)
    y = q8.q8_linear(x, q, s, b)
    np.testing.assert_allclose(y, q8.q8_linear_bruteforce(x, q, s, b), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(y, q8.q8_linear_grouped(x, q, s, b), rtol=1e-10, atol=1e-10)


def test_linear_is_x_times_w_transpose_not_w():
    # catches a transposed weight: y[m, n] depends on row n of q only
    x, q, s, b = _small(seed=4, M=2, K=64, N=3)
    q2 = q.copy()
    q2[1] = 0
    y, y2 = q8.q8_linear(x, q, s, b), q8.q8_linear(x, q2, s, b)
    assert np.array_equal(y[:, [0, 2]], y2[:, [0, 2]]) and not np.allclose(y[:, 1], y2[:, 1])


def test_input_draws():
    x, q, s, b = q8.make_q8_inputs(8, 2560, 64, seed=0)
    assert x.dtype == np.float16 and q.dtype == np.uint8 and s.dtype == np.float16 and b.dtype == np.float16
    assert s.shape == (64, 40) and 0.001 <= float(s.min()) and float(s.max()) <= 0.01 + 1e-5
    assert q.min() == 0 and q.max() == 255
    assert abs(float(b.astype(np.float64).std()) - 0.1) < 0.02


@pytest.mark.parametrize("which", ["f16"])
def test_f16_weight_rounding_is_within_the_gemm_tolerance(which):
    # rounding W_hat to fp16 is a per-weight relative error of at most 2^-11 (rms about
    # 2^-11/sqrt(3) = 2.8e-4), uncorrelated across k, so y moves by about that much in
    # normwise relative terms: inside the 1e-3 tolerance with room for the fp16 output rounding
    x, q, s, b = q8.make_q8_inputs(16, 2560, 64, seed=5)
    y, y16 = q8.q8_linear(x, q, s, b), q8.q8_linear(x, q, s, b, weights=which)
    rel = np.linalg.norm(y16 - y) / np.linalg.norm(y)
    assert 1e-5 < rel < 4e-4


def test_quantize_affine_hand_computed_groups():
    # a ramp from -1 to 0.5: |min| > |max|, so the edge is -1: scale 1.5/255 = 1/170 exactly
    # representable as -1/-170 after the rescale (q0 = round(-170) = -170), bias -1;
    # code k = round(255 k / 63)
    w = np.linspace(-1, 0.5, 64, dtype=np.float32)
    q, s, b = q8.quantize_affine(w[None])
    assert b[0, 0] == np.float32(-1.0) and s[0, 0] == np.float32(-1.0) / np.float32(-170.0)
    assert q[0, 0] == 0 and q[0, 1] == 4 and q[0, 4] == 16 and q[0, -1] == 255
    # its mirror (from -0.5 up to 1): the edge is +1, the scale negative (-1/170), bias +1,
    # code 0 at w = 1 (the last element), 255 at w = -0.5
    q, s, b = q8.quantize_affine(-w[::-1][None].copy())
    assert b[0, 0] == np.float32(1.0) and s[0, 0] == np.float32(1.0) / np.float32(-170.0)
    assert q[0, -1] == 0 and q[0, 0] == 255 and q[0, -2] == 4
    # a constant group is represented exactly by its bias with code 0; an all-zero group
    # keeps bias 0 (q0 = 0) and the minimum scale magnitude 1e-7
    q, s, b = q8.quantize_affine(np.full((1, 64), 0.3, np.float32))
    assert np.all(q == 0) and b[0, 0] == np.float32(0.3)
    q, s, b = q8.quantize_affine(np.zeros((1, 64), np.float32))
    assert np.all(q == 0) and b[0, 0] == 0 and abs(s[0, 0]) == np.float32(1e-7)


def test_quantize_affine_properties():
    rng = np.random.default_rng(0)
    w = rng.standard_normal((64, 640)).astype(np.float32) * rng.uniform(0.01, 3, (64, 1)).astype(np.float32)
    w[:8] = np.abs(w[:8])          # all-positive groups
    w[8:16] = -np.abs(w[8:16])     # all-negative groups
    w[16, 5] = 40.0                # an outlier
    q, s, b = q8.quantize_affine(w)
    g = w.reshape(64, 10, 64).astype(np.float64)
    qg = q.reshape(64, 10, 64).astype(np.float64)
    s64, b64 = s.astype(np.float64)[..., None], b.astype(np.float64)[..., None]
    # every value within half a step of its reconstruction (fp32 parameters), except that the
    # rescale to put 0 on the grid (step edge / q0, |q0| = |bias / step|) can push the far
    # extreme up to 255 (0.5 / |q0|) steps past code 255, where it is clipped
    err = np.abs(s64 * qg + b64 - g)
    q0 = np.maximum(np.abs(b64 / s64), 1.0)
    assert np.all(err <= np.abs(s64) * (0.5 + 127.5 / q0 + 1e-4))
    inner = (qg > 0) & (qg < 255)
    assert np.all(np.where(inner, err, 0) <= np.abs(s64) * (0.5 + 1e-4))
    # the edge (larger-magnitude extreme) has code 0; the other extreme a code near 255
    lo, hi = g.min(-1), g.max(-1)
    edge_is_min = np.abs(lo) > np.abs(hi)
    edge_idx = np.where(edge_is_min, g.argmin(-1), g.argmax(-1))
    far_idx = np.where(edge_is_min, g.argmax(-1), g.argmin(-1))
    assert np.all(np.take_along_axis(qg, edge_idx[..., None], -1) == 0)
    assert np.all(np.take_along_axis(qg, far_idx[..., None], -1) >= 253)
    # zero is on the grid: -b / s is an integer (to fp32 precision)
    z = -b.astype(np.float64) / s.astype(np.float64)
    assert np.all(np.abs(z - np.rint(z)) <= 1e-3)
    # the scale's magnitude is the range over 255 up to the rescale by round(edge / scale)
    rng_s = (hi - lo) / 255
    assert np.all(np.abs(np.abs(s) - rng_s) <= rng_s * 0.5 / np.maximum(np.abs(np.rint(np.where(edge_is_min, lo, hi) / rng_s)), 1) + 1e-9)
    # fp16 casts of the parameters (the stored layer) stay within their own rounding
    q16, s16, b16 = q8.quantize_f16(w)
    assert np.array_equal(q16, q) and np.array_equal(s16, s.astype(np.float16))


def test_linear_f32_is_dequant_f32_then_matmul():
    # the CPU baseline's torch form: a one-hot x reads single weights, which must be
    # dequant_f32's bits, and y stays within the fp32 error bound of the exact GEMM
    import torch
    x, q, s, b = q8.make_q8_inputs(5, 256, 48, seed=6)
    tq, ts, tb = (torch.from_numpy(a) for a in (q, s, b))
    wt = q8.q8_linear_f32(torch.eye(256, dtype=torch.float16), tq, ts, tb)
    assert np.array_equal(wt.T.numpy(), q8.dequant_f32(q, s, b))
    y = q8.q8_linear_f32(torch.from_numpy(x), tq, ts, tb).double().numpy()
    ref = q8.q8_linear(x, q, s, b)
    bound = 2 * (256 + 1) * 2.0 ** -24 * (np.abs(x.astype(np.float64)) @ np.abs(q8.dequant_exact(q, s, b)).T)
    assert np.all(np.abs(y - ref) <= bound)
    assert np.abs(y - ref).max() > 0  # fp32, not fp64
