"""Triangle multiplicative update on the HIP path: the module the reference's
variant mechanism swaps in.

The reference binds, per TriangleMultiplicativeBlock, a forward
``forward(pair_grid, visibility=None) -> update`` (fast_trunk.py:19-32, bound at
fast_trunk.py:57), with the weights read from the live module
(fast_trunk.py:53-56; mlx_trunk.py:40-55). ``TriMul`` keeps that call contract:

  * input pair_grid [B, L, L, C], any float dtype, on the GPU;
  * visibility [B, L, L] (the pair mask) or None, which means all ones
    (fast_trunk.py:20-21); it multiplies a and b only, never the output;
  * returns the update without the residual, in pair_grid's dtype;
  * fp16 activations with fp32 accumulation and fp32 LayerNorm statistics, with
    the fp16 range scheme of the reference's fp16 trunk (contraction stored /256,
    norm_mix eps / 256^2; mlx_trunk.py:14-19, :47-48, :114).

Everything runs in three gfx950 kernels behind ``tmu_forward`` of the C ABI.
"""

from __future__ import annotations

import torch
from torch import nn

from . import capi, scratch

F16 = torch.float16


class TriMul(nn.Module):
    """One triangle multiplicative update (outgoing or incoming) on the HIP path."""

    def __init__(self, w_bundle, ln_in_w, ln_in_b, ln_mix_w, ln_mix_b, w_emit, w_gate, outgoing: bool,
                 ln_in_eps: float = 1e-5, ln_mix_eps: float = 1e-5, out_mask: bool = False, device=None):
        super().__init__()
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        c4, C = w_bundle.shape
        c = c4 // 4
        if c4 != 4 * c or tuple(w_emit.shape) != (C, c) or tuple(w_gate.shape) != (C, C):
            raise ValueError(f"weight shapes: proj_bundle {tuple(w_bundle.shape)}, proj_emit {tuple(w_emit.shape)}, "
                             f"proj_gate {tuple(w_gate.shape)}")
        h = lambda t: t.detach().to(device=dev, dtype=F16).contiguous()  # noqa: E731
        f = lambda t: t.detach().to(device=dev, dtype=torch.float32).contiguous()  # noqa: E731
        self.register_buffer("w_bundle", h(w_bundle))
        self.register_buffer("w_emit", h(w_emit))
        self.register_buffer("w_gate", h(w_gate))
        self.register_buffer("ln_in_w", f(ln_in_w))
        self.register_buffer("ln_in_b", f(ln_in_b))
        self.register_buffer("ln_mix_w", f(ln_mix_w))
        self.register_buffer("ln_mix_b", f(ln_mix_b))
        self.C, self.c = C, c
        self.outgoing = bool(outgoing)
        self.ln_in_eps, self.ln_mix_eps = float(ln_in_eps), float(ln_mix_eps)
        self.out_mask = bool(out_mask)

    # --- construction from the reference's module ------------------------------------------
    @classmethod
    def from_block(cls, block, outgoing: bool, **kw) -> "TriMul":
        """From a TriangleMultiplicativeBlock-shaped module: proj_bundle (no bias, rows
        [s_a | s_b | g_a | g_b]), norm_start, norm_mix, proj_emit, proj_gate (weights only,
        as mlx_trunk.py:40-55 copies them)."""
        if getattr(block.proj_bundle, "bias", None) is not None:  # fast_trunk.py:53
            raise ValueError("proj_bundle has a bias; the reference's split-weight path assumes none")
        for lin in (block.proj_emit, block.proj_gate):
            if getattr(lin, "bias", None) is not None and bool(torch.any(lin.bias != 0)):
                raise ValueError("proj_emit / proj_gate biases are not part of the reference's TMU")
        lc = getattr(block, "latent_channels", None)
        if lc is not None and block.proj_bundle.weight.shape[0] != 4 * lc:
            raise ValueError("proj_bundle rows must be 4 * latent_channels")
        dev = kw.pop("device", None) or (block.proj_bundle.weight.device
                                         if block.proj_bundle.weight.is_cuda else None)
        return cls(block.proj_bundle.weight, block.norm_start.weight, block.norm_start.bias, block.norm_mix.weight,
                   block.norm_mix.bias, block.proj_emit.weight, block.proj_gate.weight, outgoing,
                   ln_in_eps=getattr(block.norm_start, "eps", 1e-5), ln_mix_eps=getattr(block.norm_mix, "eps", 1e-5),
                   device=dev, **kw)

    @classmethod
    def from_weights(cls, p, **kw) -> "TriMul":
        """From an object with the oracle's TriMulWeights fields (w_bundle, w_emit, ...)."""
        return cls(p.w_bundle, p.ln_in_w, p.ln_in_b, p.ln_mix_w, p.ln_mix_b, p.w_emit, p.w_gate, p.outgoing,
                   ln_in_eps=p.ln_in_eps, ln_mix_eps=p.ln_mix_eps, **kw)

    # --- forward -----------------------------------------------------------------------------
    def workspace(self, B: int, L: int, device) -> torch.Tensor:
        """The a, b, x planes of one call: a 256-byte aligned view of the device's shared scratch
        (every update of a trunk runs in the same bytes, one after another)."""
        return scratch.get(capi.lib().tmu_workspace_bytes(B, L, self.c), device)

    def run(self, z16: torch.Tensor, mask16: torch.Tensor | None, out: torch.Tensor, residual: bool) -> torch.Tensor:
        """fp16 in/out on the current stream; ``out`` may be ``z16`` itself when ``residual``."""
        lib = capi.lib()
        B, L, _, C = z16.shape
        if tuple(out.shape) != tuple(z16.shape) or out.dtype != F16 or not out.is_contiguous():
            raise capi.EsmError(-2, f"out must be a contiguous fp16 {tuple(z16.shape)} tensor")
        ws = self.workspace(B, L, z16.device)
        capi.check(lib.tmu_forward_ws(z16.data_ptr(), None if mask16 is None else mask16.data_ptr(),
                                      self.ln_in_w.data_ptr(), self.ln_in_b.data_ptr(), self.ln_in_eps,
                                      self.w_bundle.data_ptr(), self.ln_mix_w.data_ptr(), self.ln_mix_b.data_ptr(),
                                      self.ln_mix_eps, self.w_emit.data_ptr(), self.w_gate.data_ptr(),
                                      out.data_ptr(), ws.data_ptr(), ws.numel(), B, L, C, self.c,
                                      int(self.outgoing), int(residual), int(self.out_mask), capi.stream_ptr()))
        return out

    def forward(self, pair_grid: torch.Tensor, visibility: torch.Tensor | None = None,
                residual: bool = False) -> torch.Tensor:
        z16, mask16 = prepare(pair_grid, visibility, self.C)
        out = torch.empty_like(z16)
        self.run(z16, mask16, out, residual)
        return out if pair_grid.dtype == F16 else out.to(pair_grid.dtype)


def prepare(pair_grid: torch.Tensor, visibility: torch.Tensor | None, C: int):
    """Validate and convert (pair_grid, visibility) to contiguous fp16 device tensors."""
    if not pair_grid.is_cuda:
        raise capi.EsmError(-5, "pair_grid must be on the GPU: the HIP path has no CPU fallback")
    if pair_grid.dim() != 4 or pair_grid.shape[1] != pair_grid.shape[2] or pair_grid.shape[3] != C:
        raise ValueError(f"pair_grid must be [B, L, L, {C}], got {tuple(pair_grid.shape)}")
    z16 = pair_grid.to(F16).contiguous()
    mask16 = None
    if visibility is not None:
        if tuple(visibility.shape) != tuple(pair_grid.shape[:3]):
            raise ValueError(f"visibility must be {tuple(pair_grid.shape[:3])}, got {tuple(visibility.shape)}")
        mask16 = visibility.to(device=pair_grid.device, dtype=F16).contiguous()
    return z16, mask16


class TriMulPair(nn.Module):
    """z1 = z + T_out(z); z2 = z1 + T_in(z1) (mlx_trunk.py:93-95) in one ``tmu_pair_forward``
    call: the outgoing update with its residual fused into kernel (c), then the incoming one
    in place."""

    def __init__(self, t_out: TriMul, t_in: TriMul):
        super().__init__()
        if not t_out.outgoing or t_in.outgoing:
            raise ValueError("TriMulPair takes an outgoing then an incoming update")
        if (t_out.C, t_out.c) != (t_in.C, t_in.c):
            raise ValueError(f"the two updates differ in width: {(t_out.C, t_out.c)} vs {(t_in.C, t_in.c)}")
        self.t_out, self.t_in = t_out, t_in

    def forward(self, z: torch.Tensor, mask: torch.Tensor | None = None, out: torch.Tensor | None = None):
        z16, m16 = prepare(z, mask, self.t_out.C)
        if out is not None and (tuple(out.shape) != tuple(z16.shape) or out.dtype != F16 or not out.is_cuda
                                or not out.is_contiguous()):
            raise capi.EsmError(-2, f"out must be a contiguous fp16 device tensor of shape {tuple(z16.shape)}")
        return run_pair(self.t_out, self.t_in, z16, m16, torch.empty_like(z16) if out is None else out)


def run_pair(o: TriMul, i: TriMul, z16: torch.Tensor, mask16: torch.Tensor | None, out: torch.Tensor) -> torch.Tensor:
    """out = z1 + i(z1), z1 = z16 + o(z16) on the current stream (fp16; ``out`` may be ``z16``)."""
    B, L = z16.shape[0], z16.shape[1]
    ws = o.workspace(B, L, z16.device)
    capi.check(capi.lib().tmu_pair_forward_ws(
        z16.data_ptr(), None if mask16 is None else mask16.data_ptr(),
        o.ln_in_w.data_ptr(), o.ln_in_b.data_ptr(), o.ln_in_eps, o.w_bundle.data_ptr(), o.ln_mix_w.data_ptr(),
        o.ln_mix_b.data_ptr(), o.ln_mix_eps, o.w_emit.data_ptr(), o.w_gate.data_ptr(), int(o.out_mask),
        i.ln_in_w.data_ptr(), i.ln_in_b.data_ptr(), i.ln_in_eps, i.w_bundle.data_ptr(), i.ln_mix_w.data_ptr(),
        i.ln_mix_b.data_ptr(), i.ln_mix_eps, i.w_emit.data_ptr(), i.w_gate.data_ptr(), int(i.out_mask),
        out.data_ptr(), ws.data_ptr(), ws.numel(), B, L, o.C, o.c, capi.stream_ptr()))
    return out
