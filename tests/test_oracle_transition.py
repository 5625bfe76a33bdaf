"""Pins the transition / block-stack oracle (oracle/transition.py)."""

import math

import torch

from oracle import tmu, transition as tr

D = torch.float64


def test_relu_mlp_matches_transformers_residue_mlp():
    from transformers.models.esm.modeling_esmfold import EsmFoldResidueMLP
    g = torch.Generator().manual_seed(0)
    p = tr.draw_transition(g, 16, 64)
    p.ln_w = 1 + 0.2 * torch.randn(16, generator=g)
    p.ln_b = 0.2 * torch.randn(16, generator=g)
    p.b1 = 0.1 * torch.randn(64, generator=g)
    p.b3 = 0.1 * torch.randn(16, generator=g)
    m = EsmFoldResidueMLP(16, 64).double().eval()
    with torch.no_grad():
        m.mlp[0].weight.copy_(p.ln_w); m.mlp[0].bias.copy_(p.ln_b)
        m.mlp[1].weight.copy_(p.w1); m.mlp[1].bias.copy_(p.b1)
        m.mlp[3].weight.copy_(p.w3); m.mlp[3].bias.copy_(p.b3)
        z = torch.randn(1, 5, 5, 16, generator=g, dtype=D)
        pd = tr.TransitionWeights(*(t.double() for t in (p.ln_w, p.ln_b, p.w1, p.w3)), b1=p.b1.double(),
                                  b3=p.b3.double())
        torch.testing.assert_close(tr.transition(z, pd), m(z), rtol=1e-12, atol=1e-12)


def test_swiglu_closed_form():
    g = torch.Generator().manual_seed(1)
    C, H = 4, 6
    p = tr.TransitionWeights(torch.ones(C, dtype=D), torch.zeros(C, dtype=D),
                             torch.randn(H, C, generator=g, dtype=D), torch.randn(C, H, generator=g, dtype=D),
                             w2=torch.randn(H, C, generator=g, dtype=D))
    z = torch.randn(1, 2, 2, C, generator=g, dtype=D)
    out = tr.transition(z, p)
    h = tmu.layer_norm(z, p.ln_w, p.ln_b, p.eps)[0, 1, 0]
    u1, u2 = p.w1 @ h, p.w2 @ h
    act = torch.tensor([float(a) / (1 + math.exp(-float(a))) * float(bb) for a, bb in zip(u1, u2)], dtype=D)
    torch.testing.assert_close(out[0, 1, 0], z[0, 1, 0] + p.w3 @ act, rtol=1e-12, atol=1e-12)


def test_block_order():
    g = torch.Generator().manual_seed(2)
    blk = tr.draw_blocks(g, 1, 8, 8, 32)[0]
    blk = tr.BlockWeights(blk.tri_out.to(D), blk.tri_in.to(D),
                          tr.TransitionWeights(blk.trans.ln_w.double(), blk.trans.ln_b.double(),
                                               blk.trans.w1.double(), blk.trans.w3.double()))
    z = torch.randn(1, 5, 5, 8, generator=g, dtype=D)
    z1 = z + tmu.trimul(z, None, blk.tri_out, True)
    z2 = z1 + tmu.trimul(z1, None, blk.tri_in, False)
    torch.testing.assert_close(tr.block_forward(z, None, blk), tr.transition(z2, blk.trans))
    # in-then-out is a different function: the order is observable
    z1b = z + tmu.trimul(z, None, blk.tri_in, False)
    z2b = z1b + tmu.trimul(z1b, None, blk.tri_out, True)
    assert not torch.allclose(z2, z2b)


def test_stack_store_and_recycles():
    g = torch.Generator().manual_seed(3)
    blocks = [tr.BlockWeights(b.tri_out.to(D), b.tri_in.to(D),
                              tr.TransitionWeights(b.trans.ln_w.double(), b.trans.ln_b.double(), b.trans.w1.double(),
                                                   b.trans.w3.double()))
              for b in tr.draw_blocks(g, 2, 8, 8, 32)]
    z = torch.randn(1, 4, 4, 8, generator=g, dtype=D)
    # storing at the working precision is the identity
    torch.testing.assert_close(tr.stack_forward(z, None, blocks, 2, store=D), tr.stack_forward(z, None, blocks, 2),
                               rtol=0, atol=0)
    # recycles compose: two passes = one pass applied to one pass's output
    once = tr.stack_forward(z, None, blocks, 1)
    torch.testing.assert_close(tr.stack_forward(z, None, blocks, 2), tr.stack_forward(once, None, blocks, 1),
                               rtol=0, atol=0)
    # an fp16 residual stream leaves every stored value representable in fp16, and stays
    # within fp16 rounding of the fp64 stream
    z16 = tr.stack_forward(z.half().double(), None, blocks, 1, store=torch.float16)
    assert torch.equal(z16, z16.half().double())
    ref = tr.stack_forward(z.half().double(), None, blocks, 1)
    assert float((z16 - ref).abs().max()) <= 0.05 * float(ref.abs().max())
    assert not torch.equal(z16, ref)


def _blocks64(blocks):
    return [tr.BlockWeights(b.tri_out.to(D), b.tri_in.to(D),
                            tr.TransitionWeights(b.trans.ln_w.double(), b.trans.ln_b.double(), b.trans.w1.double(),
                                                 b.trans.w3.double()))
            for b in blocks]


def test_fp16_reference_scheme_matches_exact_arithmetic_for_one_block():
    # the emulation of the reference's fp16 trunk (every op output stored in fp16, s_a / 256,
    # norm_mix eps / 256^2) computes the same function: one block sits within fp16 noise of
    # fp64 (a dropped rescale, a wrong eps or a swapped operand is off by O(1))
    g = torch.Generator().manual_seed(5)
    blocks = tr.draw_blocks(g, 1, 128, 128, 512)
    z = torch.randn(1, 24, 24, 128, generator=g).half()
    emu = tr.stack_forward_fp16ref(z.float(), None, blocks).double()
    ref = tr.stack_forward(z.double(), None, _blocks64(blocks))
    rms = float((ref - z.double()).pow(2).mean().sqrt())
    assert float((emu - ref).abs().max()) <= 1e-2 * rms
    assert torch.equal(emu, emu.half().double())  # every stored value is fp16
    assert not torch.equal(emu, ref)


def test_fp16_reference_scheme_error_floor_of_deep_stacks():
    # the block-stack workload's depth (8 blocks x 3 recycles): the reference's own fp16 scheme,
    # and even exact arithmetic with only the residual stream stored in fp16, sit above
    # 1e-2 x RMS(update) from fp64 in the max norm while staying near 2e-3 normwise, so a
    # max-norm bar of 1e-2 is out of reach for any fp16 trunk at this depth. Measured at the
    # workload's L=238: 1.66e-2 (fp16 stream) and 1.75e-2 (reference scheme); here at L=48.
    g = torch.Generator().manual_seed(0)
    blocks = tr.draw_blocks(g, 8, 128, 128, 512)
    z = torch.randn(1, 48, 48, 128, generator=g).half()
    ref = tr.stack_forward(z.double(), None, _blocks64(blocks), 3)
    rms = float((ref - z.double()).pow(2).mean().sqrt())
    emu = tr.stack_forward_fp16ref(z.float(), None, blocks, 3).double()
    s16 = tr.stack_forward(z.double(), None, _blocks64(blocks), 3, store=torch.float16)
    for got in (emu, s16):
        d = got - ref
        assert 1e-2 * rms < float(d.abs().max()) < 3e-2 * rms
        assert float(d.pow(2).mean().sqrt()) < 3e-3 * rms
