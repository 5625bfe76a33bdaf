"""Oracle: the ESMC transformer block around the 8-bit linear, restated in torch.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restated from mlx_esmc.py:
  :53-75   layer weights: wqkv = [q; k; v] rows, w1 = [gate; up] rows, each linear in
           torch's [out, in] layout, quantised along `in` in groups of 64 (q8.py);
  :84-102  block_forward: pre-LN attention with QK-LayerNorm over the full width
           (weight only), RoPE (NeoX half rotation, base 10000, positions 0..L-1),
           softmax attention with scale hd^-0.5 and a same-chain mask, o-projection
           divided by res_scale and added to the residual; pre-LN SwiGLU (silu(x1) * x2)
           with w2, divided by res_scale and added;
  :108     res_scale = sqrt(n_layers / 36);
  :186-191 the mask: token i attends to j iff sequence_id[i] == sequence_id[j].

Pinned by (tests/test_oracle_esmc.py): `rope` against transformers'
LlamaRotaryEmbedding + apply_rotary_pos_emb (third-party, NeoX rotate_half) and
against a per-element Python loop; `attention` against
torch.nn.functional.scaled_dot_product_attention and a per-element Python loop;
RoPE's relative-position property (a common position offset leaves attention
scores unchanged); the block's composition checked against hand-composed
library routines.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

from . import q8 as oq8

EPS = 1e-5
ROPE_BASE = 10000.0


@dataclass
class Q8Weights:
    """One 8-bit linear: codes q [N, K] uint8, scales s and biases b [N, K/64] fp16 (numpy)."""

    q: np.ndarray
    s: np.ndarray
    b: np.ndarray

    def dense(self, weights: str = "f16") -> torch.Tensor:
        """W [N, K] fp64: the fp16-rounded dequantisation ("f16") or the exact one ("exact")."""
        w = oq8.dequant_f16(self.q, self.s, self.b).astype(np.float64) if weights == "f16" else \
            oq8.dequant_exact(self.q, self.s, self.b)
        return torch.from_numpy(np.asarray(w, dtype=np.float64))


@dataclass
class EsmcBlockWeights:
    ln1_w: torch.Tensor
    ln1_b: torch.Tensor
    q_ln: torch.Tensor
    k_ln: torch.Tensor
    ln2_w: torch.Tensor
    ln2_b: torch.Tensor
    wqkv: Q8Weights   # [3D, D]
    wo: Q8Weights     # [D, D]
    w1: Q8Weights     # [2F, D]: gate rows, then up rows
    w2: Q8Weights     # [D, F]


def rope(x: torch.Tensor, base: float = ROPE_BASE) -> torch.Tensor:
    """NeoX rotary embedding of x [B, H, L, hd] at positions 0..L-1: the two halves
    (i, i + hd/2) rotate by pos * base^(-2i/hd) (mlx.fast.rope, traditional=False)."""
    hd = x.shape[-1]
    half = hd // 2
    inv = base ** (-torch.arange(0, half, dtype=torch.float64) * 2 / hd)
    ang = torch.arange(x.shape[-2], dtype=torch.float64)[:, None] * inv[None, :]
    cos, sin = torch.cos(ang).to(x.dtype), torch.sin(ang).to(x.dtype)
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)


def chain_mask(sequence_id: torch.Tensor | None):
    """[B, 1, L, L] bool, True where attention is allowed (same chain id), or None."""
    if sequence_id is None:
        return None
    return (sequence_id[:, :, None] == sequence_id[:, None, :])[:, None]


def attention(q, k, v, allowed=None, scale=None):
    """softmax(q k^T * scale, masked) v for [B, H, L, hd]; ``allowed`` [B, 1, L, L] bool or None."""
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    s = (q @ k.transpose(-1, -2)) * scale
    if allowed is not None:
        s = s.masked_fill(~allowed, float("-inf"))
    return torch.softmax(s, dim=-1) @ v


def q8_apply(x: torch.Tensor, w: Q8Weights, weights: str = "f16") -> torch.Tensor:
    return x @ w.dense(weights).to(x.dtype).T


def block_forward(p: EsmcBlockWeights, x: torch.Tensor, sequence_id=None, n_heads: int = 40,
                  res_scale: float = 1.0, weights: str = "f16") -> torch.Tensor:
    """mlx_esmc.py:84-102 on a residual x [B, L, D] (any float dtype: fp64 for parity)."""
    B, L, D = x.shape
    hd = D // n_heads
    h = F.layer_norm(x, (D,), p.ln1_w.to(x.dtype), p.ln1_b.to(x.dtype), EPS)
    q, k, v = q8_apply(h, p.wqkv, weights).split(D, dim=-1)
    q = F.layer_norm(q, (D,), p.q_ln.to(x.dtype), None, EPS)
    k = F.layer_norm(k, (D,), p.k_ln.to(x.dtype), None, EPS)
    heads = lambda t: t.reshape(B, L, n_heads, hd).transpose(1, 2)  # noqa: E731
    o = attention(rope(heads(q)), rope(heads(k)), heads(v), chain_mask(sequence_id), hd ** -0.5)
    o = o.transpose(1, 2).reshape(B, L, D)
    x = x + q8_apply(o, p.wo, weights) / res_scale
    h = F.layer_norm(x, (D,), p.ln2_w.to(x.dtype), p.ln2_b.to(x.dtype), EPS)
    x1, x2 = q8_apply(h, p.w1, weights).chunk(2, dim=-1)
    return x + q8_apply(F.silu(x1) * x2, p.w2, weights) / res_scale


def res_scale_for(n_layers: int) -> float:
    return math.sqrt(n_layers / 36)


def quantize(w: torch.Tensor, group: int = 64) -> Q8Weights:
    """An MLX-style affine 8-bit quantisation of W [N, K] fp32 along K (for building test
    weights): per group, scale = (max - min) / 255 and bias = min, rounded to fp16, codes
    round((w - bias) / scale) clipped to 0..255. The kernels take q, s, b as given, so
    only the format matters here, not MLX's exact choice of scale and bias."""
    N, K = w.shape
    g = w.reshape(N, K // group, group).double()
    lo, hi = g.min(-1).values, g.max(-1).values
    s = ((hi - lo) / 255).clamp(min=1e-8).half()
    b = lo.half()
    q = torch.round((g - b.double()[..., None]) / s.double()[..., None]).clamp(0, 255).to(torch.uint8)
    return Q8Weights(q.reshape(N, K).numpy(), s.numpy(), b.numpy())
