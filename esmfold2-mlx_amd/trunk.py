"""The pair trunk on the HIP path: the transition module, the block stack and the
FoldingTrunk-level drop-in the reference's ``var_mlx_trunk`` variant swaps in.

Reference contract (var_mlx_trunk.py:24-46, mlx_trunk.py:93-115):
  * ``forward(pair, pair_attention_mask=None)`` returns an fp32 tensor on
    ``pair.device``; an all-ones mask is elided (var_mlx_trunk.py:42-44);
  * ``set_chunk_size`` and ``set_kernel_backend`` exist and do nothing;
  * each block is z += T_out(z); z += T_in(z); z = transition(z) (mlx_trunk.py:93-99),
    with the residual stream kept in fp16 (the reference's fp16 trunk; mlx_trunk.py:8-19).

Every op is a gfx950 kernel of the C ABI: per block, three TMU kernels per direction
with the residual fused into the epilogue, then the transition kernel in place. The
stack is a fixed sequence of launches on device buffers the module owns, so it can be
captured once in a HIP graph and replayed (``PairTrunk.graphed``).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn

from . import capi, kernels, scratch
from .trimul import TriMul, prepare, run_pair

F16 = torch.float16


def relay_trunk_setting(inner, name: str, value) -> None:
    """Pass a FoldingTrunk setting (``set_chunk_size``, ``set_kernel_backend``) from a wrapper to
    the module it wraps, when that module takes it; the HIP kernels need neither."""
    setter = getattr(inner, name, None)
    if callable(setter):
        setter(value)


class PairTransition(nn.Module):
    """z + W3 act(W1 LN(z)): ReLU MLP (w2 None) or the reference's SwiGLU (fast_trunk.py:35-42)."""

    def __init__(self, ln_w, ln_b, w1, w3, w2=None, eps: float = 1e-5, device=None):
        super().__init__()
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        H, C = w1.shape
        if tuple(w3.shape) != (C, H) or (w2 is not None and tuple(w2.shape) != (H, C)):
            raise ValueError(f"transition weights: w1 {tuple(w1.shape)}, w3 {tuple(w3.shape)}")
        h = lambda t: t.detach().to(device=dev, dtype=F16).contiguous()  # noqa: E731
        f = lambda t: t.detach().to(device=dev, dtype=torch.float32).contiguous()  # noqa: E731
        self.register_buffer("w1", h(w1))
        self.register_buffer("w3", h(w3))
        self.register_buffer("w2", None if w2 is None else h(w2))
        self.register_buffer("ln_w", f(ln_w))
        self.register_buffer("ln_b", f(ln_b))
        self.eps, self.C, self.H = float(eps), C, H

    @classmethod
    def from_transition(cls, tr, **kw) -> "PairTransition":
        """From the reference's Transition (norm, ffn.w12 [2H, C], ffn.w3 [C, H], no biases;
        fast_trunk.py:58-62: w1 = w12[:H] is the silu branch, w2 = w12[H:] the linear one)."""
        if tr.ffn.w12.bias is not None or tr.ffn.w3.bias is not None:
            raise ValueError("the reference's transition has no biases (fast_trunk.py:59)")
        H = tr.ffn.hidden_features
        w = tr.ffn.w12.weight
        return cls(tr.norm.weight, tr.norm.bias, w[:H], tr.ffn.w3.weight, w2=w[H:],
                   eps=getattr(tr.norm, "eps", 1e-5), **kw)

    @classmethod
    def from_residue_mlp(cls, mlp, **kw) -> "PairTransition":
        """From transformers' EsmFoldResidueMLP (LayerNorm -> Linear -> ReLU -> Linear, + x)
        with zero (or absent) biases: the block-stack workload's transition."""
        ln, up, down = mlp.mlp[0], mlp.mlp[1], mlp.mlp[3]
        for lin in (up, down):
            if lin.bias is not None and bool(torch.any(lin.bias != 0)):
                raise ValueError("the transition kernel has no bias terms")
        return cls(ln.weight, ln.bias, up.weight, down.weight, eps=ln.eps, **kw)

    @classmethod
    def from_weights(cls, p, **kw) -> "PairTransition":
        """From an object with fields ln_w, ln_b, w1, w3, w2 (None for ReLU), eps."""
        return cls(p.ln_w, p.ln_b, p.w1, p.w3, w2=p.w2, eps=p.eps, **kw)

    def run(self, z16: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        return kernels.transition(z16, self.ln_w, self.ln_b, self.eps, self.w1, self.w3, self.w2, out=out)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise capi.EsmError(-5, "x must be on the GPU: the HIP path has no CPU fallback")
        z16 = x.to(F16).contiguous()
        out = self.run(z16, torch.empty_like(z16))
        return out if x.dtype == F16 else out.to(x.dtype)


class TrunkBlock(nn.Module):
    """z += T_out(z); z += T_in(z); z = transition(z)  (mlx_trunk.py:93-99)."""

    def __init__(self, tri_out: TriMul, tri_in: TriMul, transition: PairTransition):
        super().__init__()
        if not tri_out.outgoing or tri_in.outgoing:
            raise ValueError("a block takes an outgoing then an incoming update")
        self.tri_out, self.tri_in, self.transition = tri_out, tri_in, transition

    def run_(self, z16: torch.Tensor, m16: torch.Tensor | None) -> torch.Tensor:
        """In place on a contiguous fp16 [B, L, L, C] device tensor."""
        run_pair(self.tri_out, self.tri_in, z16, m16, z16)
        return self.transition.run(z16, z16)


@dataclass
class _Graph:
    key: tuple
    graph: torch.cuda.CUDAGraph
    z: torch.Tensor
    mask: torch.Tensor | None
    scratch: torch.Tensor | None  # the shared scratch the captured launches use, kept alive


class PairTrunk(nn.Module):
    """A FoldingTrunk-shaped module running the block stack on the HIP kernels
    (the reference's MLXFoldingTrunk, var_mlx_trunk.py:24-46)."""

    def __init__(self, blocks):
        super().__init__()
        self.blocks = nn.ModuleList(blocks)
        self._graph: _Graph | None = None

    @classmethod
    def from_folding_trunk(cls, folding_trunk, device=None) -> "PairTrunk":
        """Weights of every block of a PyTorch FoldingTrunk (mlx_trunk.py:58-69): tri_mul_out,
        tri_mul_in (through their ``_engine`` when wrapped) and pair_transition."""
        blocks = []
        for blk in folding_trunk.blocks:
            eng = lambda m: getattr(m, "_engine", m)  # noqa: E731
            blocks.append(TrunkBlock(TriMul.from_block(eng(blk.tri_mul_out), outgoing=True, device=device),
                                     TriMul.from_block(eng(blk.tri_mul_in), outgoing=False, device=device),
                                     PairTransition.from_transition(blk.pair_transition, device=device)))
        return cls(blocks)

    @classmethod
    def from_weights(cls, block_params, device=None) -> "PairTrunk":
        """From (T_out params, T_in params, transition params) triples (``workloads.block_stack``)."""
        return cls([TrunkBlock(TriMul.from_weights(po, device=device), TriMul.from_weights(pi, device=device),
                               PairTransition.from_weights(pt, device=device)) for po, pi, pt in block_params])

    # FoldingTrunk API that the model calls on its trunk; the kernels need neither.
    def set_chunk_size(self, chunk_size):
        pass

    def set_kernel_backend(self, backend):
        pass

    def run_(self, z16: torch.Tensor, m16: torch.Tensor | None, recycles: int = 1) -> torch.Tensor:
        """The stack ``recycles`` times, in place on fp16 device buffers (z carried)."""
        for _ in range(recycles):
            for blk in self.blocks:
                blk.run_(z16, m16)
        return z16

    def forward(self, pair: torch.Tensor, pair_attention_mask: torch.Tensor | None = None) -> torch.Tensor:
        mask = pair_attention_mask
        if mask is not None and bool(mask.all()):
            mask = None  # a single-chain fold: skip the multiply (var_mlx_trunk.py:42-44)
        z16, m16 = prepare(pair, mask, self.blocks[0].tri_out.C)
        if z16.data_ptr() == pair.data_ptr():
            z16 = z16.clone()  # never write into the caller's tensor
        self.run_(z16, m16)
        return z16.float()

    # --- HIP graph ---------------------------------------------------------------------------
    def graphed(self, z16: torch.Tensor, m16: torch.Tensor | None = None, recycles: int = 1):
        """A callable replaying the whole stack as one HIP graph on the given buffers (the
        stack runs in place on ``z16``; load new inputs into it between replays)."""
        key = (z16.data_ptr(), tuple(z16.shape), None if m16 is None else m16.data_ptr(), recycles)
        if self._graph is None or self._graph.key != key:
            self.run_(z16.clone(), m16, 1)  # allocate every workspace outside the capture
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.run_(z16, m16, recycles)
            self._graph = _Graph(key, g, z16, m16, scratch.current(z16.device))
        return self._graph.graph.replay
