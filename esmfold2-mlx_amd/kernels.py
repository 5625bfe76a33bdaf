"""Functional wrappers of the C ABI on torch tensors (device memory and streams only).

Each function checks device, dtype and contiguity, allocates its outputs with
torch, passes raw pointers plus the current HIP stream, and raises
``capi.EsmError`` on a non-zero return. No CPU path exists.
"""

from __future__ import annotations

import ctypes

import torch

from . import capi, scratch

F16 = torch.float16


def _dev(t: torch.Tensor, name: str, dtype=None) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise capi.EsmError(-5, f"{name} must be a CUDA(HIP) tensor; the HIP path has no CPU fallback")
    if dtype is not None and t.dtype != dtype:
        raise capi.EsmError(-2, f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise capi.EsmError(-3, f"{name} must be contiguous")
    return t


def _ptr(t):
    return None if t is None else t.data_ptr()


def _out(t: torch.Tensor, name: str, dtype, numel: int) -> torch.Tensor:
    """A caller-provided output or auxiliary tensor: device, dtype, contiguity, and exactly the
    number of elements the kernel writes (a raw pointer carries no size, so an undersized
    tensor would take out-of-bounds device writes)."""
    _dev(t, name, dtype)
    if t.numel() != numel:
        raise capi.EsmError(-2, f"{name} has {t.numel()} elements, the kernel writes {numel}")
    return t


def leading_dim(L: int) -> int:
    return capi.lib().tmu_leading_dim(L)


def workspace_bytes(B: int, L: int, c: int) -> int:
    return capi.lib().tmu_workspace_bytes(B, L, c)


def project(z, mask, ln_w, ln_b, eps, w, incoming: bool, ld: int | None = None):
    """Kernel (a): -> (a, b) [B, c, L, ld] fp16 (transposed storage when ``incoming``)."""
    lib = capi.lib()
    _dev(z, "z", F16)
    B, L, _, C = z.shape
    c = w.shape[0] // 4
    ld = lib.tmu_leading_dim(L) if ld is None else ld
    a = torch.empty(B, c, L, ld, dtype=F16, device=z.device)
    b = torch.empty_like(a)
    if mask is not None:
        _out(mask, "mask", F16, B * L * L)
    capi.check(lib.tmu_project(z.data_ptr(), _ptr(mask), _dev(ln_w, "ln_w", torch.float32).data_ptr(),
                               _dev(ln_b, "ln_b", torch.float32).data_ptr(), float(eps), _dev(w, "w", F16).data_ptr(),
                               a.data_ptr(), b.data_ptr(), B, L, C, c, ld, int(incoming), capi.stream_ptr()))
    return a, b


def contract(a, b, L: int, scale: float = 1.0, ldx: int | None = None):
    """Kernel (b): x[n, i, j] = scale * sum_k a[n, i, k] b[n, j, k]; a, b [..., L, ld] -> x [..., L, ldx]."""
    lib = capi.lib()
    _dev(a, "a", F16)
    _dev(b, "b", F16)
    ld = a.shape[-1]
    batch = a.numel() // (L * ld)
    ldx = lib.tmu_leading_dim(L) if ldx is None else ldx
    x = torch.empty(*a.shape[:-2], L, ldx, dtype=F16, device=a.device)
    capi.check(lib.tmu_contract(a.data_ptr(), b.data_ptr(), x.data_ptr(), batch, L, ld, ldx, float(scale),
                                capi.stream_ptr()))
    return x


def epilogue(x, z, mask, ln_in_w, ln_in_b, eps_in, ln_mix_w, ln_mix_b, eps_mix, w_emit, w_gate,
             residual: bool = False, out_mask: bool = False, out=None):
    """Kernel (c): -> update (or z + update) [B, L, L, C] fp16."""
    lib = capi.lib()
    _dev(x, "x", F16)
    _dev(z, "z", F16)
    B, L, _, C = z.shape
    c = w_emit.shape[1]
    out = torch.empty_like(z) if out is None else _out(out, "out", F16, z.numel())
    if mask is not None:
        _out(mask, "mask", F16, B * L * L)
    capi.check(lib.tmu_epilogue(x.data_ptr(), x.shape[-1], z.data_ptr(), _ptr(mask),
                                _dev(ln_in_w, "ln_in_w", torch.float32).data_ptr(),
                                _dev(ln_in_b, "ln_in_b", torch.float32).data_ptr(), float(eps_in),
                                _dev(ln_mix_w, "ln_mix_w", torch.float32).data_ptr(),
                                _dev(ln_mix_b, "ln_mix_b", torch.float32).data_ptr(), float(eps_mix),
                                _dev(w_emit, "w_emit", F16).data_ptr(), _dev(w_gate, "w_gate", F16).data_ptr(),
                                out.data_ptr(), B, L, C, c, int(residual), int(out_mask), capi.stream_ptr()))
    return out


def transition(z, ln_w, ln_b, eps, w1, w3, w2=None, out=None):
    """Kernel (e): z + W3 act(W1 LN(z)), act = ReLU (``w2`` None) or silu(W1 h) * (W2 h).
    z [B, L, L, C] fp16; w1, w2 [H, C], w3 [C, H] fp16; ``out`` may be ``z`` (in place). Shapes
    outside the register-resident kernel's run the wide path in the device's shared scratch."""
    lib = capi.lib()
    _dev(z, "z", F16)
    B, L, L2, C = z.shape
    if L2 != L:
        raise capi.EsmError(-2, f"transition: z must be [B, L, L, C], got {tuple(z.shape)}")
    H = w1.shape[0]
    _dev(w1, "w1", F16)
    _dev(w3, "w3", F16)
    if w2 is not None:
        _dev(w2, "w2", F16)
    if tuple(w1.shape) != (H, C) or tuple(w3.shape) != (C, H) or (w2 is not None and tuple(w2.shape) != (H, C)):
        raise capi.EsmError(-2, f"transition: w1 {tuple(w1.shape)}, w3 {tuple(w3.shape)} for C={C}")
    out = torch.empty_like(z) if out is None else _out(out, "out", F16, z.numel())
    need = int(lib.pair_transition_workspace_bytes(B, L, C, H, int(w2 is not None)))
    ws = scratch.get(need, z.device) if need else None  # the wide path's LN(z) and hidden planes
    capi.check(lib.pair_transition_ws(z.data_ptr(), out.data_ptr(), _dev(ln_w, "ln_w", torch.float32).data_ptr(),
                                      _dev(ln_b, "ln_b", torch.float32).data_ptr(), float(eps), w1.data_ptr(),
                                      _ptr(w2), w3.data_ptr(), B, L, C, H, _ptr(ws), need, capi.stream_ptr()))
    return out


def esmc_layer_norm(x, w, b, eps, y=None, alpha: float = 1.0, x_out=None, out=None, fp32_out: bool = False,
                    y_parts=None):
    """LN over the last axis of the fp32 residual x [M, D] (after x_out = x + alpha*y when y
    is given) -> fp16 (or fp32) ``out``. Returns out. ``y_parts`` = (partials [splits, M, D]
    fp32, splits) from ``q8_linear_partials`` stands for y = fp16(sum of the partials)."""
    lib = capi.lib()
    _dev(x, "x", torch.float32)
    M, D = x.shape[0] if x.dim() == 2 else x.numel() // x.shape[-1], x.shape[-1]
    if y is not None and y_parts is not None:
        raise capi.EsmError(-2, "esmc_layer_norm: y and y_parts are exclusive")
    if y is not None:
        _out(y, "y", F16, M * D)
    if y_parts is not None:
        _dev(y_parts[0], "y_parts", torch.float32)
        gen = getattr(y_parts, "generation", None)
        if gen is not None:  # partials living in the shared scratch: not overwritten since
            scratch.check_generation(gen, y_parts[0].device, "esmc_layer_norm: y_parts")
        if y_parts[0].numel() < int(y_parts[1]) * M * D:
            raise capi.EsmError(-2, "esmc_layer_norm: y_parts smaller than splits x M x D")
    if y is not None or y_parts is not None:
        x_out = x if x_out is None else _out(x_out, "x_out", torch.float32, M * D)
    dt = torch.float32 if fp32_out else F16
    out = torch.empty(x.shape, dtype=dt, device=x.device) if out is None else _out(out, "out", dt, M * D)
    wp, bp = _dev(w, "w", torch.float32).data_ptr(), None if b is None else _dev(b, "b", torch.float32).data_ptr()
    hp, h32 = (None, out.data_ptr()) if fp32_out else (out.data_ptr(), None)
    if y_parts is not None:
        capi.check(lib.esmc_layer_norm_parts(x.data_ptr(), y_parts[0].data_ptr(), int(y_parts[1]), float(alpha),
                                             _ptr(x_out), wp, bp, float(eps), hp, h32, M, D, capi.stream_ptr()))
    else:
        capi.check(lib.esmc_layer_norm(x.data_ptr(), _ptr(y), float(alpha), _ptr(x_out), wp, bp, float(eps), hp, h32,
                                       M, D, capi.stream_ptr()))
    return out


def esmc_qk_rope(qkv, q_ln, k_ln, eps, B: int, L: int, n_heads: int, base: float = 10000.0, out=None):
    """qkv [B*L, 3D] fp16 -> (q, k, v) [B, H, L, 64] fp16 (QK-LayerNorm + NeoX RoPE on q, k)."""
    lib = capi.lib()
    _dev(qkv, "qkv", F16)
    shape = (B, n_heads, L, 64)
    if qkv.numel() != B * L * 3 * n_heads * 64:
        raise capi.EsmError(-2, f"esmc_qk_rope: qkv has {qkv.numel()} elements for B={B} L={L} heads={n_heads}")
    if out is not None:
        q, k, v = (_out(t, n, F16, B * n_heads * L * 64) for t, n in zip(out, ("q", "k", "v")))
    else:
        q, k, v = tuple(torch.empty(shape, dtype=F16, device=qkv.device) for _ in range(3))
    capi.check(lib.esmc_qk_rope(qkv.data_ptr(), _dev(q_ln, "q_ln", torch.float32).data_ptr(),
                                _dev(k_ln, "k_ln", torch.float32).data_ptr(), float(eps), q.data_ptr(), k.data_ptr(),
                                v.data_ptr(), B, L, n_heads, 64, float(base), capi.stream_ptr()))
    return q, k, v


def esmc_attention(q, k, v, sequence_id=None, scale: float | None = None, out=None):
    """softmax(q k^T * scale, same-chain mask) v: q, k, v [B, H, L, 64] fp16 -> o [B, L, H*64] fp16."""
    lib = capi.lib()
    B, H, L, hd = q.shape
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _dev(t, n, F16)
    for t, n in ((k, "k"), (v, "v")):
        if tuple(t.shape) != tuple(q.shape):
            raise capi.EsmError(-2, f"esmc_attention: {n} {tuple(t.shape)} differs from q {tuple(q.shape)}")
    sid = None if sequence_id is None else _out(sequence_id, "sequence_id", torch.int32, B * L)
    o = torch.empty(B, L, H * hd, dtype=F16, device=q.device) if out is None else _out(out, "out", F16, B * L * H * hd)
    capi.check(lib.esmc_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), _ptr(sid), o.data_ptr(), B, L, H, hd,
                                  float(hd ** -0.5 if scale is None else scale), capi.stream_ptr()))
    return o


def esmc_swiglu(x12, out=None):
    """[M, 2F] fp16 (rows [x1 | x2]) -> silu(x1) * x2 [M, F] fp16."""
    lib = capi.lib()
    _dev(x12, "x12", F16)
    M, F2 = x12.shape[0] if x12.dim() == 2 else x12.numel() // x12.shape[-1], x12.shape[-1]
    y = (torch.empty(*x12.shape[:-1], F2 // 2, dtype=F16, device=x12.device) if out is None
         else _out(out, "out", F16, M * (F2 // 2)))
    capi.check(lib.esmc_swiglu(x12.data_ptr(), y.data_ptr(), M, F2 // 2, capi.stream_ptr()))
    return y


def parcae_step(z, z_init, refined, ln_w, ln_b, eps, a, b_mat, out=None):
    """a * z + LN(z_init + refined) @ B^T: z, z_init, refined [B, L, L, C] fp32; b_mat [C, C] fp16."""
    lib = capi.lib()
    B, L, _, C = z.shape
    for t, n in ((z, "z"), (z_init, "z_init"), (refined, "refined")):
        _out(t, n, torch.float32, z.numel())
    out = torch.empty_like(z) if out is None else _out(out, "out", torch.float32, z.numel())
    capi.check(lib.parcae_step(z.data_ptr(), z_init.data_ptr(), refined.data_ptr(),
                               _dev(ln_w, "ln_w", torch.float32).data_ptr(), _dev(ln_b, "ln_b", torch.float32).data_ptr(),
                               float(eps), _dev(a, "a", torch.float32).data_ptr(), _dev(b_mat, "b_mat", F16).data_ptr(),
                               out.data_ptr(), B, L, C, capi.stream_ptr()))
    return out


def expected_distance(r, w, bias, centers, out=None):
    """softmax((r + r^T) @ W^T + bias) . centers per pair: r [B, L, L, C] fp32, w [nbins, C] fp16."""
    lib = capi.lib()
    _dev(r, "r", torch.float32)
    B, L, _, C = r.shape
    nb = w.shape[0]
    ed = (torch.empty(B, L, L, dtype=torch.float32, device=r.device) if out is None
          else _out(out, "out", torch.float32, B * L * L))
    capi.check(lib.distogram_expected_distance(r.data_ptr(), _dev(w, "w", F16).data_ptr(),
                                               _dev(bias, "bias", torch.float32).data_ptr(),
                                               _dev(centers, "centers", torch.float32).data_ptr(), ed.data_ptr(), B, L,
                                               C, nb, capi.stream_ptr()))
    return ed


def abs_diff_quantile(x, y=None, q: float = 0.95, out=None):
    """The q-th quantile of |x - y| (|x| when y is None), as torch.quantile: a 1-element fp32 tensor."""
    lib = capi.lib()
    _dev(x, "x", torch.float32)
    if y is not None:
        _dev(y, "y", torch.float32)
        if y.numel() != x.numel():
            raise capi.EsmError(-2, "abs_diff_quantile: x and y differ in size")
    out = torch.empty(1, dtype=torch.float32, device=x.device) if out is None else _out(out, "out", torch.float32, 1)
    capi.check(lib.abs_diff_quantile(x.data_ptr(), _ptr(y), x.numel(), float(q), out.data_ptr(), capi.stream_ptr()))
    return out


def q8_workspace_bytes(M: int, K: int, N: int) -> int:
    """Bytes of workspace q8_linear uses to split K at this shape (0: it runs unsplit)."""
    return int(capi.lib().q8_linear_workspace_bytes(M, K, N))


def q8_workspace(M: int, K: int, N: int, device=None):
    """A workspace for q8_linear at this shape, or None when it needs none. Reusable across
    calls of that shape on one stream, not by calls that overlap in time."""
    n = q8_workspace_bytes(M, K, N)
    if n == 0:
        return None
    return torch.empty(n + 256, dtype=torch.uint8, device=device if device is not None else "cuda")


def q8_partials_bytes(M: int, K: int, N: int) -> int:
    """Bytes of the fp32 partials ``q8_linear_partials`` writes at this shape."""
    return int(capi.lib().q8_linear_partials_bytes(M, K, N))


def q8_partials_buffer(M: int, K: int, N: int, device=None):
    """A buffer for ``q8_linear_partials`` at this shape (fp32 partials of every split)."""
    return torch.empty(q8_partials_bytes(M, K, N) + 256, dtype=torch.uint8,
                       device=device if device is not None else "cuda")


def _packed_codes(lib, fn, codes, packed, N, K):
    """Device pointer of packed codes (``q8_pack_codes``), which are read with packed scales."""
    _dev(codes, "codes", torch.uint8)
    if packed is None:
        raise capi.EsmError(-2, f"{fn}: packed codes need the packed scales too")
    if codes.numel() < lib.q8_packed_codes_bytes(N, K):
        raise capi.EsmError(-2, f"{fn}: packed codes too small for this shape")
    return codes.data_ptr()


def q8_linear_partials(x, q, s, b, parts, group: int = 64, packed=None, codes=None):
    """Kernel (d) without its split reduction: returns (partials [splits, M, N] fp32, splits), a view
    of ``parts`` (a uint8 buffer of at least q8_linear_partials_bytes + 256 bytes, e.g. from
    ``q8_partials_buffer`` or ``q8_workspace``). fp16(sum over splits in order) is q8_linear's y.
    ``codes`` (from ``q8_pack_codes``, with ``packed``) reads the weights in the packed order: the
    same bits."""
    lib = capi.lib()
    _dev(x, "x", F16)
    _dev(q, "q", torch.uint8)
    _dev(s, "s", F16)
    _dev(b, "b", F16)
    _dev(parts, "parts", torch.uint8)
    M, K = x.shape
    N = q.shape[0]
    if q.shape[1] != K or s.shape != (N, K // group) or b.shape != s.shape:
        raise capi.EsmError(-2, f"q8_linear_partials: shapes x{tuple(x.shape)} q{tuple(q.shape)} s{tuple(s.shape)}")
    off = (-parts.data_ptr()) % 256
    sbp = None
    if packed is not None:
        _dev(packed, "packed", torch.int32)
        if packed.numel() * 4 < lib.q8_packed_scales_bytes(N, K):
            raise capi.EsmError(-2, "q8_linear_partials: packed scales too small for this shape")
        sbp = packed.data_ptr()
    splits = ctypes.c_int(0)
    if codes is not None:
        qp = _packed_codes(lib, "q8_linear_partials", codes, packed, N, K)
        capi.check(lib.q8_linear_packed_partials(x.data_ptr(), qp, sbp, parts.data_ptr() + off, parts.numel() - off,
                                                 ctypes.byref(splits), M, K, N, group, capi.stream_ptr()))
    else:
        capi.check(lib.q8_linear_partials(x.data_ptr(), q.data_ptr(), s.data_ptr(), b.data_ptr(), sbp,
                                          parts.data_ptr() + off, parts.numel() - off, ctypes.byref(splits), M, K, N,
                                          group, capi.stream_ptr()))
    n = splits.value
    return parts[off:off + 4 * n * M * N].view(torch.float32).view(n, M, N), n


def q8_pack_scales(s, b, group: int = 64):
    """Scales and biases [N, K/64] fp16 packed as q8_linear's per-tile words (a layout cache)."""
    lib = capi.lib()
    _dev(s, "s", F16)
    _dev(b, "b", F16)
    N, G = s.shape
    if b.shape != s.shape:
        raise capi.EsmError(-2, f"q8_pack_scales: s{tuple(s.shape)} b{tuple(b.shape)}")
    n = int(lib.q8_packed_scales_bytes(N, G * group))
    sb = torch.empty(n // 4, dtype=torch.int32, device=s.device)
    capi.check(lib.q8_pack_scales(s.data_ptr(), b.data_ptr(), sb.data_ptr(), N, G * group, group, capi.stream_ptr()))
    return sb


def q8_pack_codes(q, group: int = 64):
    """Codes [N, K] uint8 in the order kernel (d)'s matrix-core fragments take them (a layout
    cache, about N*K bytes; read together with ``q8_pack_scales``' words)."""
    lib = capi.lib()
    _dev(q, "q", torch.uint8)
    N, K = q.shape
    n = int(lib.q8_packed_codes_bytes(N, K))
    if n == 0:
        raise capi.EsmError(-2, f"q8_pack_codes: unsupported shape q{tuple(q.shape)}")
    qp = torch.empty(n, dtype=torch.uint8, device=q.device)
    capi.check(lib.q8_pack_codes(q.data_ptr(), qp.data_ptr(), N, K, group, capi.stream_ptr()))
    return qp


SWIGLU_HALF = 80  # gate (or up) rows per 160-row tile in the SwiGLU pair order


def swiglu_pair_rows(N: int, device=None):
    """Row order of a [gate; up] weight [N, K] (N = 2F, a multiple of 160) in which each 160-row
    tile holds gate rows 80 t .. 80 t + 79 and then up rows F + 80 t .. F + 80 t + 79."""
    if N % (2 * SWIGLU_HALF):
        raise capi.EsmError(-2, f"swiglu_pair_rows: N={N} must be a multiple of {2 * SWIGLU_HALF}")
    F = N // 2
    t = torch.arange(N // (2 * SWIGLU_HALF)).view(-1, 1) * SWIGLU_HALF
    j = torch.arange(SWIGLU_HALF).view(1, -1)
    return torch.cat([t + j, F + t + j], dim=1).reshape(-1).to(device if device is not None else "cpu")


def q8_linear_swiglu(x, codes, packed, N: int, group: int = 64, out=None, workspace=None):
    """silu(x W_gate^T) * (x W_up^T) [M, N/2] from the [gate; up] weight packed in SwiGLU pair
    order (``q8_pack_codes`` / ``q8_pack_scales`` of its rows taken in ``swiglu_pair_rows(N)``):
    the same bits as ``esmc_swiglu(q8_linear(x, ...))`` on the [gate; up] rows."""
    lib = capi.lib()
    _dev(x, "x", F16)
    _dev(packed, "packed", torch.int32)
    M, K = x.shape
    qp = _packed_codes(lib, "q8_linear_swiglu", codes, packed, N, K)
    if packed.numel() * 4 < lib.q8_packed_scales_bytes(N, K):
        raise capi.EsmError(-2, "q8_linear_swiglu: packed scales too small for this shape")
    y = torch.empty(M, N // 2, dtype=F16, device=x.device) if out is None else _out(out, "out", F16, M * (N // 2))
    if workspace is None:
        wp, wn = None, 0
    else:
        _dev(workspace, "workspace", torch.uint8)
        wp = (workspace.data_ptr() + 255) // 256 * 256
        wn = workspace.numel() - (wp - workspace.data_ptr())
    capi.check(lib.q8_linear_swiglu_packed_ws(x.data_ptr(), qp, packed.data_ptr(), y.data_ptr(), M, K, N, group,
                                              wp, wn, capi.stream_ptr()))
    return y


def q8_linear(x, q, s, b, group: int = 64, out=None, workspace=None, packed=None, codes=None):
    """Kernel (d): y = x . W^T, W = s*q + b per group of 64 along K (fp16 in/out, fp32 accumulation).
    ``packed`` (from ``q8_pack_scales``), ``codes`` (from ``q8_pack_codes``, used with ``packed``) and
    ``workspace`` (from ``q8_workspace``) are optional speed-ups; the result is the same bits with
    or without them."""
    lib = capi.lib()
    _dev(x, "x", F16)
    _dev(q, "q", torch.uint8)
    _dev(s, "s", F16)
    _dev(b, "b", F16)
    M, K = x.shape
    N = q.shape[0]
    if q.shape[1] != K or s.shape != (N, K // group) or b.shape != s.shape:
        raise capi.EsmError(-2, f"q8_linear: shapes x{tuple(x.shape)} q{tuple(q.shape)} s{tuple(s.shape)}")
    y = torch.empty(M, N, dtype=F16, device=x.device) if out is None else _out(out, "out", F16, M * N)
    if workspace is None:
        wp, wn = None, 0
    else:
        _dev(workspace, "workspace", torch.uint8)
        wp = (workspace.data_ptr() + 255) // 256 * 256
        wn = workspace.numel() - (wp - workspace.data_ptr())
    sbp = None
    if packed is not None:
        _dev(packed, "packed", torch.int32)
        if packed.numel() * 4 < lib.q8_packed_scales_bytes(N, K):
            raise capi.EsmError(-2, "q8_linear: packed scales too small for this shape")
        sbp = packed.data_ptr()
    if codes is not None:
        qp = _packed_codes(lib, "q8_linear", codes, packed, N, K)
        capi.check(lib.q8_linear_packed_ws(x.data_ptr(), qp, sbp, y.data_ptr(), M, K, N, group, wp, wn,
                                           capi.stream_ptr()))
    else:
        capi.check(lib.q8_linear_ws(x.data_ptr(), q.data_ptr(), s.data_ptr(), b.data_ptr(), sbp, y.data_ptr(), M, K,
                                    N, group, wp, wn, capi.stream_ptr()))
    return y


def q8_quantize(w, group: int = 64):
    """MLX's affine 8-bit quantisation of fp32 W [N, K] along K (mx.quantize(W, 64, 8) with fp16
    scales and biases, mlx_esmc.py:73-74) -> (q uint8 [N, K], s, b fp16 [N, K/64])."""
    lib = capi.lib()
    _dev(w, "w", torch.float32)
    N, K = w.shape
    q = torch.empty(N, K, dtype=torch.uint8, device=w.device)
    s = torch.empty(N, K // group, dtype=F16, device=w.device)
    b = torch.empty_like(s)
    capi.check(lib.q8_quantize(w.data_ptr(), q.data_ptr(), s.data_ptr(), b.data_ptr(), N, K, group,
                               capi.stream_ptr()))
    return q, s, b


def q8_dequant(q, s, b, group: int = 64):
    """W = RN_fp16(s*q + b) [N, K] fp16: the weights q8_linear multiplies by."""
    lib = capi.lib()
    _dev(q, "q", torch.uint8)
    N, K = q.shape
    w = torch.empty(N, K, dtype=F16, device=q.device)
    capi.check(lib.q8_dequant(q.data_ptr(), _dev(s, "s", F16).data_ptr(), _dev(b, "b", F16).data_ptr(),
                              w.data_ptr(), N, K, group, capi.stream_ptr()))
    return w
