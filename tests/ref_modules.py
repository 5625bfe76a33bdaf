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


class _LMConfig:
    lm_dropout = 0.25
    per_loop_lm_dropout = True


class _Config:
    num_loops = 3
    lm_encoder = _LMConfig()


class Model6BLoop(nn.Module):
    """The 6B release model's recycling fields as the loop plugin reads them
    (var_6b_mlx_loop.py:116-135, :157-207): lm_encoder, folding_trunk and parcae_coda trunks,
    parcae_input_norm, parcae_readout (bias-free), distogram_head (64 bins), config.lm_encoder,
    no msa_encoder. Its forward stands in for upstream's: the loop by name, then readout ->
    coda; upstream's own loop is not modelled (the plugin replaces it)."""

    def __init__(self, lm, main, coda, C: int = 128, nbins: int = 64, seed: int = 0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.config = _Config()
        self.msa_encoder = None
        self.lm_encoder = FoldingTrunk(lm)
        self.folding_trunk = FoldingTrunk(main)
        self.parcae_coda = FoldingTrunk(coda)
        self.confidence_head = ConfidenceHead(coda)
        self.parcae_input_norm = nn.LayerNorm(C)
        self.parcae_readout = nn.Linear(C, C, bias=False)
        self.distogram_head = nn.Linear(C, nbins)
        with torch.no_grad():
            self.parcae_input_norm.weight.copy_(1 + 0.1 * torch.randn(C, generator=g))
            self.parcae_input_norm.bias.copy_(0.1 * torch.randn(C, generator=g))
            self.parcae_readout.weight.copy_(torch.randn(C, C, generator=g) * C ** -0.5)
            self.distogram_head.weight.copy_(torch.randn(nbins, C, generator=g) * 0.1)
            self.distogram_head.bias.copy_(torch.randn(nbins, generator=g))

    def _run_one_loop(self, *a, **k):
        raise NotImplementedError("upstream's loop is not modelled; apply the loop plugin")

    def forward(self, z, z_init, lm_z, pair_mask, a, b_mat, num_loops=None):
        n = self.config.num_loops if num_loops is None else num_loops
        z = self._run_one_loop(z, z_init, lm_z, None, pair_mask, a, b_mat, None, n + 1)
        return self.parcae_coda(self.parcae_readout(z), pair_attention_mask=pair_mask)


class Model300MLoop(nn.Module):
    """The fields the adaptive-recycling plugin reads (var_adaptive_loops.py:79-92, :145-156):
    folding_trunk, pair_loop_proj, distogram_head (128 bins), config.num_loops. Its forward
    stands in for upstream's recycling: z = trunk(z_init + pair_loop_proj(z)), num_loops + 1
    times from z = 0."""

    def __init__(self, main, C: int = 128, nbins: int = 128, seed: int = 0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.config = _Config()
        self.folding_trunk = FoldingTrunk(main)
        self.pair_loop_proj = nn.Linear(C, C)
        self.distogram_head = nn.Linear(C, nbins)
        with torch.no_grad():
            self.pair_loop_proj.weight.copy_(torch.randn(C, C, generator=g) * 0.5 * C ** -0.5)
            self.pair_loop_proj.bias.copy_(0.1 * torch.randn(C, generator=g))
            self.distogram_head.weight.copy_(torch.randn(nbins, C, generator=g) * 0.1)
            self.distogram_head.bias.copy_(torch.randn(nbins, generator=g))

    def forward(self, z_init, pair_mask=None, num_loops=None):
        n = self.config.num_loops if num_loops is None else num_loops
        z = torch.zeros_like(z_init)
        for _ in range(n + 1):
            z = self.folding_trunk(z_init + self.pair_loop_proj(z), pair_attention_mask=pair_mask)
        return z
