"""Pins the ESMC-block oracle (oracle/esmc.py) without the reference (MLX is absent):
RoPE against transformers' NeoX rotary helpers and a per-element loop, attention
against torch's scaled_dot_product_attention and a per-element loop, RoPE's
relative-position property, the chain mask, and the block's composition."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import esmc

D64 = torch.float64


def test_rope_matches_transformers_neox():
    llama = pytest.importorskip("transformers.models.llama.modeling_llama")
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 3, 11, 64, generator=g, dtype=D64)
    hd, base = 64, 10000.0
    inv = 1.0 / (base ** (torch.arange(0, hd, 2, dtype=D64) / hd))
    ang = torch.arange(11, dtype=D64)[:, None] * inv[None, :]
    emb = torch.cat([ang, ang], dim=-1)
    ref, _ = llama.apply_rotary_pos_emb(x, x, emb.cos()[None], emb.sin()[None], unsqueeze_dim=1)
    torch.testing.assert_close(esmc.rope(x), ref, rtol=1e-12, atol=1e-12)


def test_rope_per_element_and_relative_position():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 1, 5, 8, generator=g, dtype=D64)
    out = esmc.rope(x)
    for pos in range(5):
        for i in range(4):
            th = pos * 10000.0 ** (-2 * i / 8)
            a, b = float(x[0, 0, pos, i]), float(x[0, 0, pos, i + 4])
            assert abs(float(out[0, 0, pos, i]) - (a * math.cos(th) - b * math.sin(th))) < 1e-12
            assert abs(float(out[0, 0, pos, i + 4]) - (b * math.cos(th) + a * math.sin(th))) < 1e-12
    # scores depend on relative positions only: q at p, k at p' vs both shifted by 3
    q = torch.randn(1, 1, 1, 8, generator=g, dtype=D64).expand(1, 1, 9, 8)
    k = torch.randn(1, 1, 1, 8, generator=g, dtype=D64).expand(1, 1, 9, 8)
    s = esmc.rope(q) @ esmc.rope(k).transpose(-1, -2)
    torch.testing.assert_close(s[0, 0, 1, 4], s[0, 0, 4, 7], rtol=1e-12, atol=1e-12)
    assert abs(float(s[0, 0, 1, 4] - s[0, 0, 1, 5])) > 1e-6


def test_attention_matches_sdpa_and_loop():
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(2, 3, 7, 16, generator=g, dtype=D64) for _ in range(3))
    sid = torch.tensor([[0, 0, 0, 1, 1, -1, -1], [0] * 7])
    allowed = esmc.chain_mask(sid)
    out = esmc.attention(q, k, v, allowed, 0.25)
    torch.testing.assert_close(out, F.scaled_dot_product_attention(q, k, v, attn_mask=allowed, scale=0.25))
    # per element, batch 0 head 1 query 4 (chain 1: keys 3, 4)
    w = [math.exp(0.25 * float(q[0, 1, 4] @ k[0, 1, j])) for j in (3, 4)]
    ref = (w[0] * v[0, 1, 3] + w[1] * v[0, 1, 4]) / sum(w)
    torch.testing.assert_close(out[0, 1, 4], ref, rtol=1e-12, atol=1e-12)
    assert esmc.chain_mask(None) is None
    assert bool(allowed[0, 0, 5, 6]) and not bool(allowed[0, 0, 5, 0])  # padding (-1) is its own chain


def _block(D=128, F_=192, seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    qz = lambda n, k: esmc.quantize(r(n, k) * k ** -0.5)  # noqa: E731
    return esmc.EsmcBlockWeights(1 + 0.1 * r(D), 0.1 * r(D), 1 + 0.1 * r(D), 1 + 0.1 * r(D), 1 + 0.1 * r(D),
                                 0.1 * r(D), qz(3 * D, D), qz(D, D), qz(2 * F_, D), qz(D, F_))


def test_block_composition():
    D, H = 128, 2
    p = _block(D)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 9, D, generator=g, dtype=D64)
    sid = torch.tensor([[0] * 5 + [1] * 4, [0] * 9])
    got = esmc.block_forward(p, x, sid, n_heads=H, res_scale=1.49)
    W = {n: getattr(p, n).dense() for n in ("wqkv", "wo", "w1", "w2")}
    h = F.layer_norm(x, (D,), p.ln1_w.double(), p.ln1_b.double(), 1e-5)
    qkv = h @ W["wqkv"].T
    q, k, v = qkv[..., :D], qkv[..., D:2 * D], qkv[..., 2 * D:]
    q = F.layer_norm(q, (D,), p.q_ln.double(), None, 1e-5)
    k = F.layer_norm(k, (D,), p.k_ln.double(), None, 1e-5)
    hs = lambda t: t.reshape(2, 9, H, 64).transpose(1, 2)  # noqa: E731
    o = F.scaled_dot_product_attention(esmc.rope(hs(q)), esmc.rope(hs(k)), hs(v),
                                       attn_mask=(sid[:, :, None] == sid[:, None, :])[:, None])
    x1 = x + (o.transpose(1, 2).reshape(2, 9, D) @ W["wo"].T) / 1.49
    h2 = F.layer_norm(x1, (D,), p.ln2_w.double(), p.ln2_b.double(), 1e-5)
    u = h2 @ W["w1"].T
    ref = x1 + ((F.silu(u[..., :192]) * u[..., 192:]) @ W["w2"].T) / 1.49
    torch.testing.assert_close(got, ref, rtol=1e-10, atol=1e-10)
    # the gate/up order of w1 is observable
    u2 = torch.cat([u[..., 192:], u[..., :192]], -1)
    alt = x1 + ((F.silu(u2[..., :192]) * u2[..., 192:]) @ W["w2"].T) / 1.49
    assert not torch.allclose(got, alt)


def test_quantize_round_trip():
    g = torch.Generator().manual_seed(4)
    w = torch.randn(8, 128, generator=g)
    qw = esmc.quantize(w)
    err = (qw.dense("exact") - w.double()).abs().max()
    assert float(err) <= float(torch.from_numpy(qw.s.astype(np.float64)).max()) * 0.51 + 1e-3
    assert qw.q.dtype == np.uint8 and qw.s.shape == (8, 2) and qw.b.dtype == np.float16
