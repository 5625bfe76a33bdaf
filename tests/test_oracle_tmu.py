"""Pins the TMU oracle (oracle/tmu.py) without importing the reference.

Each check is chosen so that a plausible restatement mistake fails at least one:
the mutation tests at the bottom plant such mistakes in a copy of the oracle and
assert that the third-party cross-check catches every one of them.
"""

import types

import pytest
import torch
import torch.nn.functional as F
from hypothesis import given, settings, strategies as st

from oracle import tmu

D = torch.float64


def _rand_weights(gen, C, c, outgoing, ln_random=True):
    p = tmu.draw_weights(gen, C, c, outgoing).to(torch.float64)
    if ln_random:  # non-trivial LayerNorm affine params so a dropped gamma/beta is caught
        p.ln_in_w = 1 + 0.3 * torch.randn(C, generator=gen, dtype=D)
        p.ln_in_b = 0.3 * torch.randn(C, generator=gen, dtype=D)
        p.ln_mix_w = 1 + 0.3 * torch.randn(c, generator=gen, dtype=torch.float64)
        p.ln_mix_b = 0.3 * torch.randn(c, generator=gen, dtype=torch.float64)
    return p


def _rand_mask(gen, B, L):
    return (torch.rand(B, L, L, generator=gen, dtype=torch.float64) > 0.3).to(torch.float64)


def test_layer_norm_matches_torch():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 5, 7, 16, generator=g, dtype=D)
    w, b = torch.randn(16, generator=g, dtype=D), torch.randn(16, generator=g, dtype=D)
    torch.testing.assert_close(tmu.layer_norm(x, w, b, 1e-5), F.layer_norm(x, (16,), w, b, 1e-5), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("L", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("outgoing", [True, False])
def test_contract_bruteforce(L, outgoing):
    g = torch.Generator().manual_seed(L)
    a, b = torch.randn(2, L, L, 3, generator=g, dtype=D), torch.randn(2, L, L, 3, generator=g, dtype=D)
    torch.testing.assert_close(tmu.contract(a, b, outgoing), tmu.contract_bruteforce(a, b, outgoing),
                               rtol=1e-12, atol=1e-12)


def test_contract_L1_is_product():
    g = torch.Generator().manual_seed(2)
    a, b = torch.randn(1, 1, 1, 9, generator=g, dtype=D), torch.randn(1, 1, 1, 9, generator=g, dtype=D)
    for outgoing in (True, False):
        torch.testing.assert_close(tmu.contract(a, b, outgoing), a * b, rtol=0, atol=0)


def test_contract_directions_differ():
    # outgoing and incoming are genuinely different for non-symmetric operands
    g = torch.Generator().manual_seed(3)
    a, b = torch.randn(1, 4, 4, 2, generator=g, dtype=D), torch.randn(1, 4, 4, 2, generator=g, dtype=D)
    assert not torch.allclose(tmu.contract(a, b, True), tmu.contract(a, b, False))


@given(L=st.integers(1, 7), c=st.integers(1, 5), seed=st.integers(0, 2**31 - 1))
@settings(max_examples=30, deadline=None)
def test_contract_in_is_out_of_transposed(L, c, seed):
    g = torch.Generator().manual_seed(seed)
    a, b = torch.randn(1, L, L, c, generator=g, dtype=D), torch.randn(1, L, L, c, generator=g, dtype=D)
    torch.testing.assert_close(tmu.contract(a, b, False),
                               tmu.contract(a.transpose(1, 2), b.transpose(1, 2), True), rtol=1e-12, atol=1e-12)


# --- independent third-party implementation (transformers' OpenFold TMU) ---------------

def _hf_module(p: tmu.TriMulWeights, outgoing: bool):
    from transformers.models.esm.modeling_esmfold import EsmFoldTriangleMultiplicativeUpdate
    C, c = p.C, p.c
    assert C == c, "the HF module has one width for pair and hidden"
    m = EsmFoldTriangleMultiplicativeUpdate(types.SimpleNamespace(pairwise_state_dim=C), _outgoing=outgoing).double()
    with torch.no_grad():
        W = p.w_bundle
        m.linear_a_p.weight.copy_(W[0:c]); m.linear_b_p.weight.copy_(W[c:2 * c])
        m.linear_a_g.weight.copy_(W[2 * c:3 * c]); m.linear_b_g.weight.copy_(W[3 * c:])
        m.linear_z.weight.copy_(p.w_emit); m.linear_g.weight.copy_(p.w_gate)
        for lin in (m.linear_a_p, m.linear_b_p, m.linear_a_g, m.linear_b_g, m.linear_z, m.linear_g):
            lin.bias.zero_()
        m.layer_norm_in.weight.copy_(p.ln_in_w); m.layer_norm_in.bias.copy_(p.ln_in_b)
        m.layer_norm_out.weight.copy_(p.ln_mix_w); m.layer_norm_out.bias.copy_(p.ln_mix_b)
        m.layer_norm_in.eps = p.ln_in_eps; m.layer_norm_out.eps = p.ln_mix_eps
    return m.eval()


def _hf_check(trimul_fn, L=6, C=8, seed=0, masked=True):
    failures = []
    for outgoing in (True, False):
        g = torch.Generator().manual_seed(seed + outgoing)
        p = _rand_weights(g, C, C, outgoing)
        z = torch.randn(2, L, L, C, generator=g, dtype=D)
        mask = _rand_mask(g, 2, L) if masked else None
        with torch.no_grad():
            ref = _hf_module(p, outgoing)(z, mask)
            got = trimul_fn(z, mask, p, outgoing)
        failures.append(not torch.allclose(got, ref, rtol=1e-10, atol=1e-10))
    return failures


@pytest.mark.parametrize("masked", [True, False])
@pytest.mark.parametrize("L,C", [(1, 4), (5, 8), (9, 16)])
def test_trimul_matches_transformers_openfold(L, C, masked):
    assert _hf_check(tmu.trimul, L=L, C=C, masked=masked) == [False, False]


@pytest.mark.parametrize("C", [128, 256])
def test_trimul_matches_transformers_wide(C):
    # the configs' width and ESMFold2's real 256 (mlx_trunk.py:3-5), nonzero LN params and a
    # random mask: still the same algorithm
    g = torch.Generator().manual_seed(11 + C)
    for outgoing in (True, False):
        p = _rand_weights(g, C, C, outgoing)
        z = torch.randn(1, 12, 12, C, generator=g, dtype=D)
        mask = _rand_mask(g, 1, 12)
        with torch.no_grad():
            ref = _hf_module(p, outgoing)(z, mask)
        torch.testing.assert_close(tmu.trimul(z, mask, p, outgoing), ref, rtol=1e-9, atol=1e-9)


# --- invariants ---------------------------------------------------------------------------

@given(L=st.integers(2, 6), seed=st.integers(0, 2**31 - 1), outgoing=st.booleans())
@settings(max_examples=20, deadline=None)
def test_residue_permutation_equivariance(L, seed, outgoing):
    g = torch.Generator().manual_seed(seed)
    p = _rand_weights(g, 6, 6, outgoing)
    z = torch.randn(1, L, L, 6, generator=g, dtype=D)
    mask = _rand_mask(g, 1, L)
    perm = torch.randperm(L, generator=g)
    out = tmu.trimul(z, mask, p, outgoing)
    out_p = tmu.trimul(z[:, perm][:, :, perm], mask[:, perm][:, :, perm], p, outgoing)
    torch.testing.assert_close(out_p, out[:, perm][:, :, perm], rtol=1e-10, atol=1e-10)


def test_layer_norm_power_of_two_scale_invariance():
    # LN(x/s, eps/s^2) == LN(x, eps): the fp16 range scheme's identity (mlx_trunk.py:14-19)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(50, 128, generator=g, dtype=D) * 300
    w, b = torch.randn(128, generator=g, dtype=D), torch.randn(128, generator=g, dtype=D)
    s = 256.0
    torch.testing.assert_close(tmu.layer_norm(x / s, w, b, 1e-5 / s**2), tmu.layer_norm(x, w, b, 1e-5),
                               rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("outgoing", [True, False])
def test_padded_cells_exact_zero_with_zero_beta_mix(outgoing):
    g = torch.Generator().manual_seed(5)
    p = _rand_weights(g, 8, 8, outgoing)
    p.ln_mix_b = torch.zeros(8, dtype=D)
    L, valid = 7, 5
    z = torch.randn(1, L, L, 8, generator=g, dtype=D)
    v = (torch.arange(L) < valid).double()
    mask = (v[:, None] * v[None, :])[None]
    out = tmu.trimul(z, mask, p, outgoing)
    assert torch.count_nonzero(out[:, valid:, :]) == 0 and torch.count_nonzero(out[:, :, valid:]) == 0
    assert torch.count_nonzero(out[:, :valid, :valid]) > 0
    # with beta_mix != 0 the padded cells are not zero (why the output mask is a separate flag)
    p.ln_mix_b = torch.full((8,), 0.5, dtype=D)
    assert torch.count_nonzero(tmu.trimul(z, mask, p, outgoing)[:, valid:, :]) > 0
    assert torch.count_nonzero(tmu.trimul(z, mask, p, outgoing, out_mask=True)[:, valid:, :]) == 0


def test_all_ones_mask_equals_none():
    g = torch.Generator().manual_seed(6)
    p = _rand_weights(g, 8, 8, True)
    z = torch.randn(1, 6, 6, 8, generator=g, dtype=D)
    torch.testing.assert_close(tmu.trimul(z, torch.ones(1, 6, 6, dtype=D), p), tmu.trimul(z, None, p), rtol=0, atol=0)


def test_pair_is_out_then_in_with_residuals():
    z, mask, po, pi = tmu.make_pair_inputs(5, 8, 8, seed=3, dtype=torch.float64)
    po, pi = po.to(D), pi.to(D)
    z1 = z + tmu.trimul(z, mask, po, True)
    torch.testing.assert_close(tmu.trimul_pair(z, mask, po, pi), z1 + tmu.trimul(z1, mask, pi, False))


def test_draw_order_and_scales():
    z, mask, po, pi = tmu.make_pair_inputs(4, 128, 128, seed=0, dtype=torch.float32)
    g = torch.Generator().manual_seed(0)
    z2 = torch.randn(1, 4, 4, 128, generator=g, dtype=torch.float32)
    w = torch.randn(512, 128, generator=g, dtype=torch.float32) * (1.0 / 128) ** 0.5
    assert torch.equal(z, z2) and torch.equal(po.w_bundle, w)
    assert po.outgoing and not pi.outgoing and mask is None
    assert torch.all(po.ln_in_w == 1) and torch.all(po.ln_mix_b == 0)


# --- mutation tests: plausible restatement mistakes must be caught -----------------------

def _mutant(kind):
    def fn(z, mask, p, outgoing):
        c = p.c
        n = tmu.layer_norm(z, p.ln_in_w, p.ln_in_b, p.ln_in_eps)
        W = p.w_bundle
        if kind == "swap_gate_signal":
            W = torch.cat([W[2 * c:], W[:2 * c]])
        sig, gate = F.linear(n, W[:2 * c]), F.linear(n, W[2 * c:])
        routed = sig * torch.sigmoid(gate)
        if mask is not None and kind != "drop_mask":
            routed = routed * mask.unsqueeze(-1)
        a, b = routed[..., :c], routed[..., c:]
        if kind == "swap_ab":
            a, b = b, a
        d = (not outgoing) if kind == "swap_direction" else outgoing
        x = tmu.contract(a, b, d)
        if kind == "transpose_output":
            x = x.transpose(1, 2)
        mix_b = torch.zeros_like(p.ln_mix_b) if kind == "drop_beta_mix" else p.ln_mix_b
        mixed = F.linear(tmu.layer_norm(x, p.ln_mix_w, mix_b, p.ln_mix_eps), p.w_emit)
        gate_in = z if kind == "gate_on_raw_z" else n
        return mixed * torch.sigmoid(F.linear(gate_in, p.w_gate))
    return fn


@pytest.mark.parametrize("kind", ["swap_gate_signal", "drop_mask", "swap_ab", "swap_direction",
                                  "transpose_output", "drop_beta_mix", "gate_on_raw_z"])
def test_crosscheck_catches_planted_mistakes(kind):
    # the unmutated restatement passes (checked above); each mutant must fail for some direction
    assert any(_hf_check(_mutant(kind), L=6, C=8, seed=100))


def test_mutant_harness_is_sound():
    assert _hf_check(_mutant("none"), L=6, C=8, seed=100) == [False, False]


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("out_mask", [False, True])
def test_sampled_cells_equal_the_full_update(outgoing, out_mask):
    # trimul_cells (rows / columns i and j only) against trimul at every sampled cell, B = 2,
    # random mask and LayerNorm parameters; the other direction's value differs
    g = torch.Generator().manual_seed(21 + outgoing)
    p = _rand_weights(g, 16, 16, outgoing)
    B, L = 2, 9
    z = torch.randn(B, L, L, 16, generator=g, dtype=D)
    mask = _rand_mask(g, B, L)
    full = tmu.trimul(z, mask, p, outgoing, out_mask=out_mask)
    cells = [(b, i, j) for b in range(B) for i in (0, 3, L - 1) for j in (0, 4, L - 1)] + [(1, 5, 5)]
    got = tmu.trimul_cells(z, mask, p, cells, outgoing, out_mask=out_mask)
    ref = torch.stack([full[b, i, j] for b, i, j in cells])
    torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)
    other = tmu.trimul_cells(z, mask, p, cells, not outgoing, out_mask=out_mask)
    assert (other - ref).abs().max() > 1e-3
    # no mask == all-ones mask
    torch.testing.assert_close(tmu.trimul_cells(z, None, p, cells, outgoing),
                               tmu.trimul_cells(z, torch.ones(B, L, L, dtype=D), p, cells, outgoing), rtol=0, atol=0)
