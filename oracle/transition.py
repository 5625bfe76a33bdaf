"""Oracle: the pair transition and the pair-trunk block stack, restated in torch.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restated:
  fast_trunk.py:35-42      the reference's SwiGLU transition:
                           x + W3 (silu(W1 LN(x)) * W2 LN(x)), no biases (fast_trunk.py:59).
  mlx_trunk.py:96-99       same, with w12 = [w1 | w2] fused (gate rows first).
  mlx_trunk.py:93-95       block = T_out, T_in, transition, each with a residual.
  ReLU MLP (the block-stack workload's transition, 128 -> 512 -> ReLU -> 128 with a
  residual): transformers' EsmFoldResidueMLP (models/esm/modeling_esmfold.py,
  class EsmFoldResidueMLP: LayerNorm -> Linear -> ReLU -> Linear, + x).

Pinned by (tests/test_oracle_transition.py): transformers' EsmFoldResidueMLP with
the same weights (third-party, in this container); SwiGLU against its closed form
silu(u) = u*sigmoid(u) evaluated per element in Python; the block order against
composing tmu.trimul by hand.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .tmu import EPS, TriMulWeights, draw_weights, layer_norm, trimul


@dataclass
class TransitionWeights:
    ln_w: torch.Tensor      # [C]
    ln_b: torch.Tensor      # [C]
    w1: torch.Tensor        # [H, C]  (ReLU: the up projection; SwiGLU: the silu-gated half)
    w3: torch.Tensor        # [C, H]  down projection
    w2: torch.Tensor | None = None  # [H, C]  SwiGLU's linear half; None = ReLU MLP
    b1: torch.Tensor | None = None
    b3: torch.Tensor | None = None
    eps: float = EPS

    @property
    def swiglu(self) -> bool:
        return self.w2 is not None


def draw_transition(gen: torch.Generator, C: int, H: int) -> TransitionWeights:
    """ReLU MLP weights W1 [H,C] ~ N(0,1/C), W3 [C,H] ~ N(0,1/H) in that order; LN gamma 1, beta 0; no biases."""
    f32 = torch.float32
    w1 = torch.randn(H, C, generator=gen, dtype=f32) * (1.0 / C) ** 0.5
    w3 = torch.randn(C, H, generator=gen, dtype=f32) * (1.0 / H) ** 0.5
    return TransitionWeights(torch.ones(C, dtype=f32), torch.zeros(C, dtype=f32), w1, w3)


def transition(z: torch.Tensor, p: TransitionWeights) -> torch.Tensor:
    """z + MLP(LN(z)): ReLU (EsmFoldResidueMLP) or SwiGLU (fast_trunk.py:35-42)."""
    h = layer_norm(z, p.ln_w, p.ln_b, p.eps)
    u = F.linear(h, p.w1, p.b1)
    if p.swiglu:
        u = F.silu(u) * F.linear(h, p.w2)
    else:
        u = torch.relu(u)
    return z + F.linear(u, p.w3, p.b3)


@dataclass
class BlockWeights:
    tri_out: TriMulWeights
    tri_in: TriMulWeights
    trans: TransitionWeights


def draw_blocks(gen: torch.Generator, n_blocks: int, C: int, c: int, H: int):
    """Per block: T_out's weights, T_in's weights, then the transition's (draw order)."""
    return [BlockWeights(draw_weights(gen, C, c, True), draw_weights(gen, C, c, False), draw_transition(gen, C, H))
            for _ in range(n_blocks)]


def block_forward(z, mask, blk: BlockWeights, store=None):
    """mlx_trunk.py:93-99 order: z += T_out(z); z += T_in(z); z = transition(z).

    ``store`` (e.g. torch.float16) rounds the residual stream to that dtype after every
    residual add, as the reference's fp16 trunk stores every intermediate, the residual
    stream included, in fp16 (mlx_trunk.py:8-19); None keeps the working precision."""
    r = (lambda t: t) if store is None else (lambda t: t.to(store).to(t.dtype))  # noqa: E731
    z = r(z + trimul(z, mask, blk.tri_out, True))
    z = r(z + trimul(z, mask, blk.tri_in, False))
    return r(transition(z, blk.trans))


def stack_forward(z, mask, blocks, recycles: int = 1, store=None):
    """The block stack applied ``recycles`` times with z carried between passes."""
    for _ in range(recycles):
        for blk in blocks:
            z = block_forward(z, mask, blk, store)
    return z


def transition_fp16ref(z: torch.Tensor, p: TransitionWeights) -> torch.Tensor:
    """The transition with the reference's fp16 storage (mlx_trunk_kernels.py:246-249):
    h = RN(LN(z)); u = RN(h @ W1^T) (SwiGLU: s = RN(silu(x1) * x2), fp32 inside, with
    x = RN(h @ [W1; W2]^T)); z' = RN(z + u @ W3^T) in one rounding (mx.addmm). fp16
    weights, fp32 arithmetic."""
    f32 = torch.float32
    r = lambda t: t.to(torch.float16).to(f32)  # noqa: E731
    zf = z.to(f32)
    h = r(layer_norm(zf, r(p.ln_w.to(f32)), r(p.ln_b.to(f32)), p.eps))
    u = r(F.linear(h, r(p.w1.to(f32))))
    if p.swiglu:
        u = r(F.silu(u) * r(F.linear(h, r(p.w2.to(f32)))))
    else:
        u = torch.relu(u)
    return r(zf + F.linear(u, r(p.w3.to(f32)))).to(z.dtype)


def stack_forward_fp16ref(z, mask, blocks, recycles: int = 1):
    """The block stack with the reference's fp16 storage at every op output
    (``tmu.trimul_fp16ref``, ``transition_fp16ref``): the error floor of the reference's
    own fp16 trunk, for comparison with exact arithmetic."""
    from .tmu import trimul_fp16ref
    for _ in range(recycles):
        for blk in blocks:
            z = trimul_fp16ref(z, mask, blk.tri_out, True)
            z = trimul_fp16ref(z, mask, blk.tri_in, False)
            z = transition_fp16ref(z, blk.trans)
    return z
