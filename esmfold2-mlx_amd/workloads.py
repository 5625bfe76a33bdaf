"""Seeded synthetic workloads of the benchmark configurations (generated on the CPU).

There are no checkpoints, so the benchmark, the smoke run and the tests use the same
seeded draws; both sides of a comparison see identical bytes.

* ``pair_inputs``: a pair tensor z [B, L, L, C] ~ N(0, 1), then the outgoing and the
  incoming update's weights: proj_bundle.weight [4c, C], proj_gate.weight [C, C],
  proj_emit.weight [C, c], in that order, each N(0, 1/fan_in); LayerNorm gamma = 1,
  beta = 0 (no draws). fp32 master weights; z cast to ``dtype`` after the fp32 draw.
* ``block_stack``: the pair-trunk block stack: z ~ N(0, 1), then per block the
  outgoing and the incoming update's weights (as above) and the transition's:
  W1 [H, C] ~ N(0, 1/C), W3 [C, H] ~ N(0, 1/H) (ReLU MLP, no biases, LN gamma 1 beta 0).
* ``q8_inputs``: x [M, K] fp16 ~ N(0, 1); codes q [N, K] ~ U{0..255}; scales
  s [N, K/64] ~ U(0.001, 0.01) and biases b ~ N(0, 0.1), fp16; drawn in that order.
* ``esmc_block_inputs``: one ESMC block (width D, FFN width F): x [B, L, D] ~ N(0, 1)
  fp32, LN parameters 1 + N(0, 0.01) and N(0, 0.01), and 8-bit linears wqkv [3D, D],
  wo [D, D], w1 [2F, D], w2 [D, F] with codes U{0..255} and per-group
  s = 2a/255 * U(0.9, 1.1), b = -a * U(0.9, 1.1), a = sqrt(3/K): dequantised weights of
  variance about 1/K, so activations keep unit scale through the block.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

EPS = 1e-5


@dataclass
class TriMulParams:
    """One triangle multiplicative update's weights in torch's [out, in] layout: the
    attributes ``TriMul.from_weights`` reads (the reference's TriangleMultiplicativeBlock
    fields, fast_trunk.py:53-56)."""

    w_bundle: torch.Tensor   # [4c, C], rows [s_a | s_b | g_a | g_b]
    w_emit: torch.Tensor     # [C, c]
    w_gate: torch.Tensor     # [C, C]
    ln_in_w: torch.Tensor    # [C]
    ln_in_b: torch.Tensor    # [C]
    ln_mix_w: torch.Tensor   # [c]
    ln_mix_b: torch.Tensor   # [c]
    outgoing: bool = True
    ln_in_eps: float = EPS
    ln_mix_eps: float = EPS


def tmu_params(gen: torch.Generator, C: int, c: int, outgoing: bool) -> TriMulParams:
    f32 = torch.float32
    w = torch.randn(4 * c, C, generator=gen, dtype=f32) * (1.0 / C) ** 0.5
    wg = torch.randn(C, C, generator=gen, dtype=f32) * (1.0 / C) ** 0.5
    we = torch.randn(C, c, generator=gen, dtype=f32) * (1.0 / c) ** 0.5
    return TriMulParams(w_bundle=w, w_emit=we, w_gate=wg, ln_in_w=torch.ones(C, dtype=f32),
                        ln_in_b=torch.zeros(C, dtype=f32), ln_mix_w=torch.ones(c, dtype=f32),
                        ln_mix_b=torch.zeros(c, dtype=f32), outgoing=outgoing)


def pair_inputs(L: int, C: int = 128, c: int = 128, seed: int = 0, dtype=torch.float16, B: int = 1,
                pad_from: int | None = None):
    """(z, mask, outgoing params, incoming params); mask m[i,j] = (i < pad_from)(j < pad_from)
    as [B, L, L] fp32, or None."""
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(B, L, L, C, generator=g, dtype=torch.float32).to(dtype)
    p_out = tmu_params(g, C, c, True)
    p_in = tmu_params(g, C, c, False)
    mask = None
    if pad_from is not None:
        v = (torch.arange(L) < pad_from).to(torch.float32)
        mask = (v[:, None] * v[None, :]).expand(B, L, L).contiguous()
    return z, mask, p_out, p_in


@dataclass
class TransitionParams:
    """The pair transition's weights: w1 [H, C], w3 [C, H], w2 [H, C] for SwiGLU (None: ReLU)."""

    ln_w: torch.Tensor
    ln_b: torch.Tensor
    w1: torch.Tensor
    w3: torch.Tensor
    w2: torch.Tensor | None = None
    eps: float = EPS


def transition_params(gen: torch.Generator, C: int, H: int) -> TransitionParams:
    f32 = torch.float32
    w1 = torch.randn(H, C, generator=gen, dtype=f32) * (1.0 / C) ** 0.5
    w3 = torch.randn(C, H, generator=gen, dtype=f32) * (1.0 / H) ** 0.5
    return TransitionParams(torch.ones(C, dtype=f32), torch.zeros(C, dtype=f32), w1, w3)


def block_stack(L: int, n_blocks: int = 8, C: int = 128, c: int = 128, H: int = 512, seed: int = 0,
                dtype=torch.float16, B: int = 1):
    """(z, [(T_out params, T_in params, transition params)] per block)."""
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(B, L, L, C, generator=g, dtype=torch.float32).to(dtype)
    blocks = [(tmu_params(g, C, c, True), tmu_params(g, C, c, False), transition_params(g, C, H))
              for _ in range(n_blocks)]
    return z, blocks


def q8_layer(gen: torch.Generator, N: int, K: int, group: int = 64):
    """(q uint8 [N, K], s, b fp16 [N, K/group]) with dequantised weights of variance ~1/K."""
    a = (3.0 / K) ** 0.5
    q = torch.randint(0, 256, (N, K), generator=gen, dtype=torch.int64).to(torch.uint8)
    u = lambda: 0.9 + 0.2 * torch.rand(N, K // group, generator=gen, dtype=torch.float32)  # noqa: E731
    s = (2 * a / 255 * u()).half()
    b = (-a * u()).half()
    return q, s, b


def esmc_block_inputs(L: int, D: int = 2560, F: int = 5120, B: int = 1, seed: int = 0):
    """(x [B, L, D] fp32, LN params dict, {name: (q, s, b)} for wqkv, wo, w1, w2)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, L, D, generator=g, dtype=torch.float32)
    ln = {n: (1.0 if n in ("ln1_w", "q_ln", "k_ln", "ln2_w") else 0.0) +
          0.1 * torch.randn(D, generator=g, dtype=torch.float32)
          for n in ("ln1_w", "ln1_b", "q_ln", "k_ln", "ln2_w", "ln2_b")}
    lin = {"wqkv": q8_layer(g, 3 * D, D), "wo": q8_layer(g, D, D), "w1": q8_layer(g, 2 * F, D),
           "w2": q8_layer(g, D, F)}
    return x, ln, lin


def q8_inputs(M: int, K: int, N: int, seed: int = 0, group: int = 64):
    """(x fp16 [M, K], q uint8 [N, K], s fp16 [N, K/group], b fp16 [N, K/group]) on the CPU."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g, dtype=torch.float32).half()
    q = torch.randint(0, 256, (N, K), generator=g, dtype=torch.int64).to(torch.uint8)
    s = (torch.rand(N, K // group, generator=g, dtype=torch.float32) * 0.009 + 0.001).half()
    b = (torch.randn(N, K // group, generator=g, dtype=torch.float32) * 0.1).half()
    return x, q, s, b
