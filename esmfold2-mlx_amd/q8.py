"""8-bit weight-only linear on the HIP path, the contract of the reference's ``_linear``.

The reference computes ``mx.quantized_matmul(x, w, s, b, transpose=True,
group_size=64, bits=8)`` (mlx_esmc.py:78-81) on weights quantised along the
input axis of torch's [out, in] layout with fp16 scales and biases
(mlx_esmc.py:53-75). ``Q8Linear`` takes the same three arrays (codes as uint8
[N, K], which is the little-endian byte view of MLX's uint32 packing) and
computes y = x . W^T with W = s*q + b on the gfx950 kernel: fp16 activations,
fp32 accumulation, fp16 output. The scales and biases are packed once per layer
into the kernel's per-tile layout, and by default the codes too, into the order of
the kernel's matrix-core fragments (a second copy of the codes, N*K bytes: the
kernel then loads them straight into registers; ``pack_codes=False`` keeps one
copy and reads the [N, K] codes through LDS, the same bits). Shapes whose output
tiles cannot fill the GPU split K over more workgroups through the device's
shared scratch (one buffer for every layer, sized for the largest call).
"""

from __future__ import annotations

import torch
from torch import nn

from . import kernels, scratch

GROUP = 64


class Q8Linear(nn.Module):
    def __init__(self, q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, device=None,
                 pack_codes: bool = True):
        super().__init__()
        N, K = q.shape
        if K % GROUP or N % 64 or tuple(scales.shape) != (N, K // GROUP) or tuple(biases.shape) != (N, K // GROUP):
            raise ValueError(f"q8 shapes: q {tuple(q.shape)}, scales {tuple(scales.shape)}, biases {tuple(biases.shape)}")
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.register_buffer("q", q.detach().to(device=dev, dtype=torch.uint8).contiguous())
        self.register_buffer("scales", scales.detach().to(device=dev, dtype=torch.float16).contiguous())
        self.register_buffer("biases", biases.detach().to(device=dev, dtype=torch.float16).contiguous())
        self.in_features, self.out_features = K, N
        self.register_buffer("packed", kernels.q8_pack_scales(self.scales, self.biases, GROUP))
        self.register_buffer("codes_packed", kernels.q8_pack_codes(self.q, GROUP) if pack_codes else None)
        self.pair_rows = False  # packed layouts in SwiGLU pair order (``swiglu_pairs``)

    def swiglu_pairs(self) -> "Q8Linear":
        """Re-packs a [gate; up] linear (the ESMC block's w1) in SwiGLU pair order for ``swiglu``,
        which then gates inside the GEMM; ``forward`` and ``partials`` keep their results and read
        the [N, K] arrays. Returns self."""
        if not self.pair_rows:
            perm = kernels.swiglu_pair_rows(self.out_features, self.q.device)
            self.packed = kernels.q8_pack_scales(self.scales[perm].contiguous(), self.biases[perm].contiguous(), GROUP)
            self.codes_packed = kernels.q8_pack_codes(self.q[perm].contiguous(), GROUP)
            self.pair_rows = True
        return self

    def swiglu(self, x: torch.Tensor) -> torch.Tensor:
        """silu(x W_gate^T) * (x W_up^T), [..., out_features / 2] fp16: the same bits as
        ``kernels.esmc_swiglu(self(x))`` (needs ``swiglu_pairs``)."""
        if not self.pair_rows:
            raise ValueError("Q8Linear.swiglu needs swiglu_pairs() first")
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features).to(torch.float16).contiguous()
        M = x2.shape[0]
        n = kernels.q8_workspace_bytes(M, self.in_features, self.out_features)
        ws = scratch.get(n, x2.device) if n else None
        y = kernels.q8_linear_swiglu(x2, self.codes_packed, self.packed, self.out_features, GROUP, workspace=ws)
        return y.reshape(*lead, self.out_features // 2)

    def _layouts(self):
        """(packed scales, packed codes) for the plain product: none once re-packed in pair order."""
        return (None, None) if self.pair_rows else (self.packed, self.codes_packed)

    @classmethod
    def from_float(cls, w: torch.Tensor, **kw) -> "Q8Linear":
        """Quantised from fp32 weights [N, K] (torch's [out, in] layout) on the GPU, as the
        reference's layer_params quantises each linear from fp32 (mlx_esmc.py:70-74)."""
        dev = kw.get("device")
        dev = torch.device(dev) if dev is not None else torch.device("cuda", torch.cuda.current_device())
        q, s, b = kernels.q8_quantize(w.detach().to(device=dev, dtype=torch.float32).contiguous(), GROUP)
        return cls(q, s, b, **kw)

    @classmethod
    def from_packed_u32(cls, w_u32: torch.Tensor, scales, biases, **kw) -> "Q8Linear":
        """From MLX's packing: [N, K/4] uint32 words, four codes each, little-endian."""
        w = w_u32.detach().cpu().contiguous()
        if w.dtype not in (torch.int32, torch.uint32):
            raise ValueError("packed codes must be 32-bit words")
        q = w.view(torch.uint8).reshape(w.shape[0], w.shape[1] * 4)
        return cls(q, scales, biases, **kw)

    def dequantized(self) -> torch.Tensor:
        return kernels.q8_dequant(self.q, self.scales, self.biases, GROUP)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features).to(torch.float16).contiguous()
        M = x2.shape[0]
        n = kernels.q8_workspace_bytes(M, self.in_features, self.out_features)
        ws = scratch.get(n, x2.device) if n else None  # split-K partials, only while this call runs
        sb, qp = self._layouts()
        y = kernels.q8_linear(x2, self.q, self.scales, self.biases, GROUP, workspace=ws, packed=sb, codes=qp)
        y = y.reshape(*lead, self.out_features)
        return y if x.dtype == torch.float16 else y.to(x.dtype)

    def partials(self, x: torch.Tensor) -> "ScratchParts":
        """(partials [splits, M, N] fp32, splits) of x . W^T for a consumer that sums them in split
        order (``kernels.esmc_layer_norm(..., y_parts=...)``): rounded to fp16, the sum is
        ``forward(x)`` bit for bit. The view lives in the device's shared scratch: it must be
        consumed before the next call of any module that uses the scratch on this device. The
        result carries the scratch generation it was made in, and ``esmc_layer_norm`` refuses it
        once the scratch has been handed out again."""
        x2 = x.reshape(-1, self.in_features).to(torch.float16).contiguous()
        M = x2.shape[0]
        buf = scratch.get(kernels.q8_partials_bytes(M, self.in_features, self.out_features), x2.device)
        gen = scratch.generation(x2.device)
        sb, qp = self._layouts()
        parts, splits = kernels.q8_linear_partials(x2, self.q, self.scales, self.biases, buf, GROUP, packed=sb,
                                                   codes=qp)
        return ScratchParts(parts, splits, gen)


class ScratchParts(tuple):
    """``(partials, splits)`` in the shared scratch, tagged with the scratch generation."""

    def __new__(cls, parts: torch.Tensor, splits: int, generation: int):
        t = super().__new__(cls, (parts, splits))
        t.generation = generation
        return t
