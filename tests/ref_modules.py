"""Modules shaped like the reference's trunk (attribute names and weight layouts the
reference reads: fast_trunk.py:51-62, mlx_trunk.py:40-69, var_mlx_trunk.py:24-46), built
from seeded weights, for the plugin and drop-in tests. Their own forwards are not used:
the plugins replace them, and the oracle gives the expected values."""

from __future__ import annotations

import torch
from torch import nn


class TriMulBlock(nn.Module):
    """TriangleMultiplicativeBlock's fields: proj_bundle [4c, C] (no bias, rows
    [s_a | s_b | g_a | g_b]), norm_start, norm_mix, proj_emit [C, c], proj_gate [C, C]."""

    def __init__(self, p):
        super().__init__()
        c4, C = p.w_bundle.shape
        c = c4 // 4
        self.latent_channels = c
        self.proj_bundle = nn.Linear(C, 4 * c, bias=False)
        self.norm_start, self.norm_mix = nn.LayerNorm(C), nn.LayerNorm(c)
        self.proj_emit, self.proj_gate = nn.Linear(c, C, bias=False), nn.Linear(C, C, bias=False)
        with torch.no_grad():
            self.proj_bundle.weight.copy_(p.w_bundle)
            self.proj_emit.weight.copy_(p.w_emit)
            self.proj_gate.weight.copy_(p.w_gate)
            self.norm_start.weight.copy_(p.ln_in_w)
            self.norm_start.bias.copy_(p.ln_in_b)
            self.norm_mix.weight.copy_(p.ln_mix_w)
            self.norm_mix.bias.copy_(p.ln_mix_b)


class Wrapped(nn.Module):
    """A wrapper holding the update as ``_engine`` (mlx_trunk.py:41)."""

    def __init__(self, engine):
        super().__init__()
        self._engine = engine


class FFN(nn.Module):
    def __init__(self, w1, w2, w3):
        super().__init__()
        H, C = w1.shape
        self.hidden_features = H
        self.w12 = nn.Linear(C, 2 * H, bias=False)
        self.w3 = nn.Linear(H, C, bias=False)
        with torch.no_grad():
            self.w12.weight.copy_(torch.cat([w1, w2]))
            self.w3.weight.copy_(w3)


class Transition(nn.Module):
    """Transition's fields: norm, ffn.w12 [2H, C] (silu rows first), ffn.w3 [C, H]."""

    def __init__(self, p):
        super().__init__()
        C = p.w1.shape[1]
        self.norm = nn.LayerNorm(C)
        with torch.no_grad():
            self.norm.weight.copy_(p.ln_w)
            self.norm.bias.copy_(p.ln_b)
        self.ffn = FFN(p.w1, p.w2, p.w3)


class PairBlock(nn.Module):
    def __init__(self, po, pi, pt):
        super().__init__()
        self.tri_mul_out = Wrapped(TriMulBlock(po))
        self.tri_mul_in = Wrapped(TriMulBlock(pi))
        self.pair_transition = Transition(pt)


class FoldingTrunk(nn.Module):
    def __init__(self, blocks):
        super().__init__()
        self.blocks = nn.ModuleList([PairBlock(*b) for b in blocks])


class Model(nn.Module):
    def __init__(self, blocks):
        super().__init__()
        self.folding_trunk = FoldingTrunk(blocks)


class ConfidenceHead(nn.Module):
    def __init__(self, blocks):
        super().__init__()
        self.folding_trunk = FoldingTrunk(blocks)


class Model6B(nn.Module):
    """The 6B release model's four trunk stacks (var_6b_mlx_trunks16k.py:29-32); ``lm`` may be
    None (no lm_encoder)."""

    def __init__(self, main, lm, coda, conf):
        super().__init__()
        self.folding_trunk = FoldingTrunk(main)
        self.lm_encoder = FoldingTrunk(lm) if lm is not None else None
        self.parcae_coda = FoldingTrunk(coda)
        self.confidence_head = ConfidenceHead(conf)
