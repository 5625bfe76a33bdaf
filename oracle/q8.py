"""Oracle: MLX-affine 8-bit weight-only linear (group 64), restated in numpy.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Reference arithmetic restated here (paths relative to the reference repo):
  mlx_esmc.py:43          GROUP = 64.
  mlx_esmc.py:53-75       weights keep torch's [out, in] layout; groups of 64 run along
                          ``in`` (K); scales and biases are stored fp16.
  mlx_esmc.py:78-81       y = mx.quantized_matmul(x, w, s, b, transpose=True,
                          group_size=64, bits=8) = x @ W_hat^T with
                          W_hat[n, k] = s[n, k // 64] * q[n, k] + b[n, k // 64].
  (mlx 0.32.3 is the third-party library holding quantized_matmul; it is not in
   this container. Its published affine scheme is the formula above; the 8-bit
   codes are packed four per uint32, little-endian, i.e. byte-identical to a
   row-major uint8 [N, K] array, which is the layout used here.)

  mlx_esmc.py:70-74       layer_params quantises each linear from fp32 with
                          mx.quantize(W, group_size=64, bits=8), then casts scales and
                          biases to fp16. mx.quantize's affine scheme (mlx 0.32.3,
                          affine_quantize in mlx/ops.cpp; its published algorithm, restated
                          in ``quantize_affine``): per group, scale = max((max - min)/255,
                          1e-7), signed towards the larger-magnitude extreme ("edge"),
                          q0 = round(edge / scale); unless q0 = 0 the scale becomes
                          edge / q0 and the bias edge (so 0 is on the grid), else bias 0;
                          codes clip(round((w - bias) / scale), 0, 255), round half to even.

Pinned by (tests/test_oracle_q8.py):
  * exactness argument: s*q is exact in fp32 and fp64 (11 + 8 significant bits) and
    the fp64 sum s*q + b is exact at these magnitudes, so dequant_exact is the real
    number s*q + b, and dequant_f16 / dequant_f32 are its single roundings. Checked
    against fractions.Fraction arithmetic on random codes;
  * special cases: q = 0 gives b, s = 0 gives b, q = 255 with b = 0 gives s*255;
  * the GEMM against a pure-Python loop on tiny shapes, and against the
    dequantise-then-matmul identity y = sum_g s_g (x_g . q_g) + b_g sum(x_g);
  * quantize_affine by hand-computed groups (a ramp from -1 to 0.5, its mirror, a
    constant group, an all-zero group) and by what the scheme fixes for every group:
    codes in 0..255, the edge element at code 0, the other extreme at code 255 up to the
    rescale, |s*q + b - w| <= |s|/2 with the fp32 parameters, and 0 exactly on the grid.
    MLX's own GPU kernel may differ in rounding details (its round, its division): that
    exact choice is parity unpinned, as no MLX is installed and the reference holds no
    quantised vectors.
"""

from __future__ import annotations

import numpy as np
import torch

GROUP = 64  # mlx_esmc.py:43


def quantize_affine(w: np.ndarray, group: int = GROUP, bits: int = 8):
    """(codes uint8 [N, K], scales fp32 [N, K/group], biases fp32): mx.quantize's affine scheme,
    restated in fp32 with IEEE division and round-half-to-even (mlx_esmc.py:73)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    assert K % group == 0
    f = np.float32
    g = w.reshape(N, K // group, group)
    w_max, w_min = g.max(-1), g.min(-1)
    n_bins = f((1 << bits) - 1)
    mask = np.abs(w_min) > np.abs(w_max)
    scale = np.maximum((w_max - w_min) / n_bins, f(1e-7)).astype(f)
    scale = np.where(mask, scale, -scale).astype(f)
    edge = np.where(mask, w_min, w_max).astype(f)
    q0 = np.rint(edge / scale).astype(f)
    at_zero = q0 == 0
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(at_zero, scale, edge / np.where(at_zero, f(1), q0)).astype(f)
    bias = np.where(at_zero, f(0), edge).astype(f)
    q = np.clip(np.rint((g - bias[..., None]) / scale[..., None]), 0, n_bins).astype(np.uint8)
    return q.reshape(N, K), scale, bias


def quantize_f16(w: np.ndarray, group: int = GROUP):
    """quantize_affine with the scales and biases cast to fp16, as layer_params stores them
    (mlx_esmc.py:74): the (q, s, b) arrays of an 8-bit layer."""
    q, s, b = quantize_affine(w, group)
    return q, s.astype(np.float16), b.astype(np.float16)


def dequant_exact(q: np.ndarray, s: np.ndarray, b: np.ndarray, group: int = GROUP) -> np.ndarray:
    """W_hat = s*q + b per group of ``group`` along K, in fp64 (exact for fp16 s, b and uint8 q)."""
    N, K = q.shape
    assert K % group == 0 and s.shape == (N, K // group) and b.shape == s.shape
    s64 = np.repeat(s.astype(np.float64), group, axis=1)
    b64 = np.repeat(b.astype(np.float64), group, axis=1)
    return s64 * q.astype(np.float64) + b64


def dequant_f16(q, s, b, group: int = GROUP) -> np.ndarray:
    """RN_fp16(s*q + b): one rounding of the exact value (what an fp16 FMA gives)."""
    return dequant_exact(q, s, b, group).astype(np.float16)


def dequant_f32(q, s, b, group: int = GROUP) -> np.ndarray:
    """RN_fp32(s*q + b): one rounding; identical with or without FMA since s*q is exact in fp32."""
    return dequant_exact(q, s, b, group).astype(np.float32)


def q8_linear_f32(x: torch.Tensor, q: torch.Tensor, s: torch.Tensor, b: torch.Tensor,
                  group: int = GROUP) -> torch.Tensor:
    """The fp32 dequantise-then-matmul on the CPU (the CPU baseline's q8 linear): W_hat =
    RN_fp32(s*q + b) in torch (s*q is exact in fp32, so the add is the one rounding: the bits of
    ``dequant_f32``), then y = x @ W_hat^T with fp32 accumulation (mlx_esmc.py:78-81)."""
    w = torch.repeat_interleave(s.float(), group, dim=1) * q.float() + torch.repeat_interleave(b.float(), group, dim=1)
    return x.float() @ w.T


def q8_linear(x: np.ndarray, q, s, b, group: int = GROUP, weights: str = "exact") -> np.ndarray:
    """y = x @ W_hat^T in fp64 (mlx_esmc.py:78-81). ``weights``: 'exact' or 'f16' (W_hat rounded to fp16)."""
    W = dequant_exact(q, s, b, group) if weights == "exact" else dequant_f16(q, s, b, group).astype(np.float64)
    return x.astype(np.float64) @ W.T


def q8_linear_grouped(x: np.ndarray, q, s, b, group: int = GROUP) -> np.ndarray:
    """Same value by the factored identity y[m,n] = sum_g s[n,g] (x_g . q_g) + b[n,g] sum(x_g)."""
    M, K = x.shape
    N = q.shape[0]
    G = K // group
    xg = x.astype(np.float64).reshape(M, G, group)
    qg = q.astype(np.float64).reshape(N, G, group)
    dots = np.einsum("mgk,ngk->mng", xg, qg)
    sums = xg.sum(-1)  # [M, G]
    return (dots * s.astype(np.float64)[None]).sum(-1) + sums @ b.astype(np.float64).T


def q8_linear_bruteforce(x, q, s, b, group: int = GROUP):
    """Pure-Python loop (tiny shapes only)."""
    M, K = x.shape
    N = q.shape[0]
    y = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                w = float(s[n, k // group]) * int(q[n, k]) + float(b[n, k // group])
                acc += float(x[m, k]) * w
            y[m, n] = acc
    return y


def make_q8_inputs(M: int, K: int, N: int, seed: int = 0, group: int = GROUP):
    """Seeded q8-linear inputs: x [M,K] fp16 ~ N(0,1); q [N,K] uint8 ~ U{0..255};
    s [N,K/g] fp16 ~ U(0.001, 0.01); b [N,K/g] fp16 ~ N(0, 0.1). Drawn in that order."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g, dtype=torch.float32).half()
    q = torch.randint(0, 256, (N, K), generator=g, dtype=torch.int64).to(torch.uint8)
    s = (torch.rand(N, K // group, generator=g, dtype=torch.float32) * 0.009 + 0.001).half()
    b = (torch.randn(N, K // group, generator=g, dtype=torch.float32) * 0.1).half()
    return x.numpy(), q.numpy(), s.numpy(), b.numpy()
