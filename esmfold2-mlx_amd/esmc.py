"""The ESMC language model's transformer blocks on the HIP path: the drop-in for
``model.esmc`` that the reference's MLXEsmc is (mlx_esmc.py:105-200).

Each block is upstream's EsmcUnifiedTransformerBlock as mlx_esmc.py:84-102 restates it:
pre-LN attention with QK-LayerNorm over all heads (weights only) and NeoX RoPE, then
pre-LN SwiGLU, both residual adds divided by sqrt(n_layers / 36). The four linears are
8-bit (``Q8Linear``: group 64, fp16 scales and biases, fp32 accumulation); every other
op is a gfx950 kernel of the C ABI (``esmc_*``). The residual stream is fp32
(the reference's default, ``residual=mx.float32``) and lives in the hidden-states slab
the fold reads: block i reads hidden_states[i] and its second residual add writes
hidden_states[i + 1], fused with the next block's input LayerNorm (or the final norm).
"""

from __future__ import annotations

import math
import os
import re
from types import SimpleNamespace

import torch
from torch import nn

from . import kernels
from .q8 import Q8Linear

EPS = 1e-5
LINEARS = ("wqkv", "wo", "w1", "w2")
NORMS = ("ln1_w", "ln1_b", "q_ln", "k_ln", "ln2_w", "ln2_b")
# every array of one layer in the converted-weight cache: the norms, then per linear the
# packed codes and their fp16 scales and biases (mlx_esmc.py:53-75)
CACHE_NAMES = NORMS + tuple(f"{n}{t}" for n in LINEARS for t in ("", "_s", "_b"))
# HF names of the published fp32 checkpoint, per layer (mlx_esmc.py:56-67): each cache
# linear is the row-wise concatenation of these (q, k, v for wqkv; gate then up for w1)
HF_LINEARS = {
    "wqkv": ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight"),
    "wo": ("self_attn.o_proj.weight",),
    "w1": ("mlp.gate_proj.weight", "mlp.up_proj.weight"),
    "w2": ("mlp.down_proj.weight",),
}
HF_NORMS = {"ln1_w": "input_layernorm.weight", "ln1_b": "input_layernorm.bias", "q_ln": "self_attn.q_norm.weight",
            "k_ln": "self_attn.k_norm.weight", "ln2_w": "post_attention_layernorm.weight",
            "ln2_b": "post_attention_layernorm.bias"}
_LAYER_KEY = re.compile(r"layers\.(\d+)\.([A-Za-z0-9_]+)")


def hf_layer(tensors, i: int, device=None) -> tuple[dict, dict]:
    """One block from the published HF-named fp32 tensors (``tensors[f"esmc.layers.{i}.{name}"]``):
    (LayerNorm parameters by cache name, {linear: Q8Linear}), each linear quantised on the GPU
    from fp32 with MLX's affine 8-bit scheme (layer_params, mlx_esmc.py:53-75)."""
    get = lambda name: tensors[f"esmc.layers.{i}.{name}"]  # noqa: E731
    ln = {n: get(h).detach().float() for n, h in HF_NORMS.items()}
    lin = {}
    for n, parts in HF_LINEARS.items():
        w = torch.cat([get(h).detach().float() for h in parts]) if len(parts) > 1 else get(parts[0]).detach().float()
        lin[n] = Q8Linear.from_float(w, device=device)
    return ln, lin


class EsmcBlock(nn.Module):
    def __init__(self, ln1_w, ln1_b, q_ln, k_ln, ln2_w, ln2_b, wqkv: Q8Linear, wo: Q8Linear, w1: Q8Linear,
                 w2: Q8Linear, n_heads: int, device=None):
        super().__init__()
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        f = lambda t: t.detach().to(device=dev, dtype=torch.float32).contiguous()  # noqa: E731
        for n, t in (("ln1_w", ln1_w), ("ln1_b", ln1_b), ("q_ln", q_ln), ("k_ln", k_ln), ("ln2_w", ln2_w),
                     ("ln2_b", ln2_b)):
            self.register_buffer(n, f(t))
        self.wqkv, self.wo, self.w1, self.w2 = wqkv, wo, w1, w2
        if w1.out_features % (2 * kernels.SWIGLU_HALF) == 0:
            w1.swiglu_pairs()  # the FFN's SwiGLU runs inside w1's GEMM
        self.D = wo.out_features
        self.F = w2.in_features
        self.n_heads = n_heads
        if self.D != n_heads * 64 or wqkv.out_features != 3 * self.D or w1.out_features != 2 * self.F:
            raise ValueError(f"ESMC block shapes: D={self.D}, heads={n_heads}, wqkv {wqkv.out_features}, "
                             f"w1 {w1.out_features}, w2 in {self.F}")

    @classmethod
    def from_params(cls, p: dict, n_heads: int = 40, device=None) -> "EsmcBlock":
        """From one layer's arrays under the reference's names (mlx_esmc.py:53-75): ln1_w, ln1_b,
        q_ln, k_ln, ln2_w, ln2_b, and per linear `name` (uint32 codes [N, K/4], four per word,
        little-endian), `name_s`, `name_b` (fp16 [N, K/64])."""
        t = lambda a: a if isinstance(a, torch.Tensor) else torch.as_tensor(a)  # noqa: E731
        lin = {n: Q8Linear.from_packed_u32(t(p[n]), t(p[n + "_s"]), t(p[n + "_b"]), device=device) for n in LINEARS}
        return cls(t(p["ln1_w"]), t(p["ln1_b"]), t(p["q_ln"]), t(p["k_ln"]), t(p["ln2_w"]), t(p["ln2_b"]),
                   lin["wqkv"], lin["wo"], lin["w1"], lin["w2"], n_heads, device=device)

    @classmethod
    def from_arrays(cls, ln: dict, lin: dict, n_heads: int, device=None) -> "EsmcBlock":
        """From LN parameters by name and {name: (codes uint8 [N, K], scales, biases)}."""
        q = {n: Q8Linear(*lin[n], device=device) for n in LINEARS}
        return cls(ln["ln1_w"], ln["ln1_b"], ln["q_ln"], ln["k_ln"], ln["ln2_w"], ln["ln2_b"], q["wqkv"], q["wo"],
                   q["w1"], q["w2"], n_heads, device=device)

    def params(self) -> dict:
        """The layer's arrays under the reference's names (inverse of ``from_params``)."""
        p = {n: getattr(self, n).detach().cpu() for n in NORMS}
        for n in LINEARS:
            lin = getattr(self, n)
            q = lin.q.detach().cpu().contiguous()
            p[n] = q.view(torch.int32).view(torch.uint32) if hasattr(torch, "uint32") else q.view(torch.int32)
            p[n + "_s"], p[n + "_b"] = lin.scales.detach().cpu(), lin.biases.detach().cpu()
        return p

    def attention(self, x: torch.Tensor, h: torch.Tensor, sid, res_scale: float, x_mid: torch.Tensor,
                  h2: torch.Tensor) -> None:
        """x_mid = x + wo(attn(h)) / res_scale; h2 = LN2(x_mid). x [B, L, D] fp32, h = LN1(x) fp16."""
        B, L, D = x.shape
        qkv = self.wqkv(h)
        q, k, v = kernels.esmc_qk_rope(qkv.view(B * L, 3 * D), self.q_ln, self.k_ln, EPS, B, L, self.n_heads)
        o = kernels.esmc_attention(q, k, v, sid)
        # wo's split-K partials are summed (and rounded to fp16) by the residual + LayerNorm kernel
        kernels.esmc_layer_norm(x, self.ln2_w, self.ln2_b, EPS, y_parts=self.wo.partials(o), alpha=1.0 / res_scale,
                                x_out=x_mid, out=h2)

    def ffn(self, h2: torch.Tensor):
        """w2(silu(x1) * x2) with [x1 | x2] = w1(h2) (before the residual's / res_scale), as w2's
        split-K partials: (partials, splits) for ``esmc_layer_norm(..., y_parts=...)``."""
        act = self.w1.swiglu(h2) if self.w1.pair_rows else kernels.esmc_swiglu(self.w1(h2))
        return self.w2.partials(act)

    def forward(self, x: torch.Tensor, sequence_id=None, res_scale: float = 1.0) -> torch.Tensor:
        """One block on an fp32 residual [B, L, D] (the reference's block_forward, mlx_esmc.py:84-102)."""
        x = x.to(torch.float32).contiguous()
        h = kernels.esmc_layer_norm(x, self.ln1_w, self.ln1_b, EPS)
        x_mid, h2 = torch.empty_like(x), torch.empty_like(h)
        self.attention(x, h, _chain_ids(sequence_id, x.device), res_scale, x_mid, h2)
        out = torch.empty_like(x)
        # out = x_mid + y2 / res_scale (the LN output of this call is not needed)
        kernels.esmc_layer_norm(x_mid, self.ln1_w, self.ln1_b, EPS, y_parts=self.ffn(h2), alpha=1.0 / res_scale,
                                x_out=out, out=torch.empty_like(h))
        return out


def _chain_ids(sequence_id, device):
    """int32 [B, L] chain ids for the attention mask, or None when every token may attend to
    every other (a single chain: the reference skips the mask, mlx_esmc.py:188-191)."""
    if sequence_id is None:
        return None
    sid = sequence_id.to(device=device)
    if bool((sid == sid[:, :1]).all()):
        return None
    return sid.to(torch.int32).contiguous()


class HipEsmc(nn.Module):
    """ESMC on the HIP kernels with 8-bit linears: forward(input_ids, sequence_id,
    output_hidden_states) -> .hidden_states [n_layers + 1, B, L, D] fp32 on the GPU (each
    block's input, then the final LayerNorm), the contract of MLXEsmc (mlx_esmc.py:179-200)."""

    def __init__(self, embed: torch.Tensor, layers, norm_w: torch.Tensor, n_heads: int = 40, device=None):
        super().__init__()
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.register_buffer("embed", embed.detach().to(device=dev, dtype=torch.float32).contiguous())
        self.register_buffer("norm_w", norm_w.detach().to(device=dev, dtype=torch.float32).contiguous())
        self.layers = nn.ModuleList(layers)
        self.n_heads = n_heads
        self.res_scale = math.sqrt(len(layers) / 36)  # mlx_esmc.py:108

    # ---- construction: the reference's converted-weight cache (mlx_esmc.py:116-148) -------------
    @classmethod
    def from_cache(cls, path, n_heads: int = 40, device=None) -> "HipEsmc":
        """From a safetensors file in the reference's converted-weight layout (mlx_esmc.py:116-148):
        "embed" [V, D] and "norm_w" [D] fp32, and for layers 0 .. n-1 every name of
        ``CACHE_NAMES`` under "layers.{i}." (8-bit codes as uint32 words, four per word)."""
        from safetensors.torch import load_file
        flat = load_file(str(path))
        per_layer: dict[int, dict] = {}
        for key, t in flat.items():
            m = _LAYER_KEY.fullmatch(key)
            if m is not None:
                per_layer.setdefault(int(m.group(1)), {})[m.group(2)] = t
            elif key not in ("embed", "norm_w"):
                raise ValueError(f"{path}: unexpected key {key!r} in an ESMC cache")
        for key in ("embed", "norm_w"):
            if key not in flat:
                raise ValueError(f"{path}: missing {key!r}")
        n = len(per_layer)
        if n == 0 or sorted(per_layer) != list(range(n)):
            raise ValueError(f"{path}: layer indices {sorted(per_layer)[:8]}... are not 0..{n - 1}")
        for i in range(n):
            missing = [c for c in CACHE_NAMES if c not in per_layer[i]]
            extra = [c for c in per_layer[i] if c not in CACHE_NAMES]
            if missing or extra:
                raise ValueError(f"{path}: layer {i} missing {missing}, unexpected {extra}")
        layers = [EsmcBlock.from_params(per_layer[i], n_heads, device=device) for i in range(n)]
        return cls(flat["embed"], layers, flat["norm_w"], n_heads, device=device)

    @classmethod
    def from_hf(cls, tensors, n_layers: int | None = None, n_heads: int = 40, cache=None,
                device=None) -> "HipEsmc":
        """From the published fp32 checkpoint's HF-named tensors (any mapping, e.g. a dict or a
        lazy shard reader: "esmc.embed_tokens.weight", "esmc.norm.weight",
        "esmc.layers.{i}.…"), every linear quantised to 8 bits on the GPU (the reference's
        from_shards, mlx_esmc.py:116-137). With ``cache`` (a path): load it when it exists,
        otherwise convert and write it there in the layout ``from_cache`` reads."""
        if cache is not None and os.path.exists(str(cache)):
            return cls.from_cache(cache, n_heads, device=device)
        if n_layers is None:
            idx = {int(m.group(1)) for k in tensors.keys()
                   if (m := re.match(r"esmc\.layers\.(\d+)\.", k)) is not None}
            n_layers = len(idx)
        layers = []
        for i in range(n_layers):
            ln, lin = hf_layer(tensors, i, device=device)
            layers.append(EsmcBlock(ln["ln1_w"], ln["ln1_b"], ln["q_ln"], ln["k_ln"], ln["ln2_w"], ln["ln2_b"],
                                    lin["wqkv"], lin["wo"], lin["w1"], lin["w2"], n_heads, device=device))
        esmc = cls(tensors["esmc.embed_tokens.weight"].detach().float(), layers,
                   tensors["esmc.norm.weight"].detach().float(), n_heads, device=device)
        if cache is not None:
            os.makedirs(os.path.dirname(os.path.abspath(str(cache))), exist_ok=True)
            esmc.save_cache(cache)
        return esmc

    def save_cache(self, path) -> None:
        from safetensors.torch import save_file
        flat = {"embed": self.embed.detach().cpu(), "norm_w": self.norm_w.detach().cpu()}
        for i, blk in enumerate(self.layers):
            flat.update({f"layers.{i}.{k}": v.contiguous() for k, v in blk.params().items()})
        save_file(flat, str(path))

    def nbytes(self) -> int:
        return sum(b.numel() * b.element_size() for b in self.buffers())

    # nn.Module API the fold calls on its ESMC; the weights stay where they are.
    def to(self, *a, **k):
        return self

    # ---- forward ---------------------------------------------------------------------------------
    def hidden_states(self, input_ids: torch.Tensor, sequence_id=None) -> torch.Tensor:
        dev = self.embed.device
        ids = input_ids.to(dev)
        B, L = ids.shape
        n, D = len(self.layers), self.embed.shape[1]
        hs = torch.empty(n + 1, B, L, D, dtype=torch.float32, device=dev)
        hs[0] = self.embed[ids]
        sid = _chain_ids(sequence_id, dev)
        h = kernels.esmc_layer_norm(hs[0], self.layers[0].ln1_w, self.layers[0].ln1_b, EPS)
        h2 = torch.empty_like(h)
        x_mid = torch.empty(B, L, D, dtype=torch.float32, device=dev)
        x_last = torch.empty_like(x_mid)
        for i, blk in enumerate(self.layers):
            blk.attention(hs[i], h, sid, self.res_scale, x_mid, h2)
            y2 = blk.ffn(h2)
            if i + 1 < n:  # second residual into hidden_states[i+1], fused with the next input LN
                nxt = self.layers[i + 1]
                kernels.esmc_layer_norm(x_mid, nxt.ln1_w, nxt.ln1_b, EPS, y_parts=y2, alpha=1.0 / self.res_scale,
                                        x_out=hs[i + 1], out=h)
            else:  # the last block's output is only seen through the final norm (weights only)
                kernels.esmc_layer_norm(x_mid, self.norm_w, None, EPS, y_parts=y2, alpha=1.0 / self.res_scale,
                                        x_out=x_last, out=hs[n], fp32_out=True)
        return hs

    def forward(self, input_ids=None, sequence_id=None, output_hidden_states=True, **_):
        return SimpleNamespace(hidden_states=self.hidden_states(input_ids, sequence_id))
