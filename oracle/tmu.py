"""Oracle: the triangle multiplicative update (TMU), restated on the CPU in torch.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the reference the HIP path is
verified against and the timed CPU baseline, never part of the product.

Reference arithmetic restated here (paths relative to the reference repo):
  fast_trunk.py:19-32      _trimul_forward: LN_in -> split-weight projections ->
                           signal * sigmoid(gate) * visibility -> fp32 contraction
                           -> proj_emit(norm_mix(.)) * sigmoid(proj_gate(n)); the
                           output is NOT masked and has no residual.
  fast_trunk.py:53-56      proj_bundle has no bias; its rows are split 2c | 2c
                           into signal [s_a | s_b] and gate [g_a | g_b].
  mlx_trunk.py:40-55       same row order ([signal_a | signal_b | gate_a | gate_b]);
                           proj_emit / proj_gate used as weights only (no bias).
  mlx_trunk.py:72-76       a = s_a * sigmoid(g_a), b = s_b * sigmoid(g_b), then * mask.
  mlx_trunk.py:84-88       outgoing: x[d,i,j] = sum_k a[d,i,k] b[d,j,k]
                           incoming: x[d,i,j] = sum_k a[d,k,i] b[d,k,j]
  mlx_trunk.py:89-90       LN over c of x (norm_mix), @ proj_emit^T, * sigmoid(n @ proj_gate^T).
  mlx_trunk.py:93-95       block order: z += T_out(z); z += T_in(z).
  mlx_trunk.py:31-33       EPS = 1e-5 for every LayerNorm.

Pinned by (tests/test_oracle_tmu.py):
  * brute-force triple loops of the contraction at L in {1,2,3,5,8}; L=1 reduces
    to x = a*b per channel;
  * an independent third-party implementation of the same algorithm, Hugging
    Face transformers' EsmFoldTriangleMultiplicativeUpdate (OpenFold Alg. 11/12),
    with its weights mapped from ours and biases zeroed, both directions, masked;
  * invariants: contract_in(a, b) == contract_out(a^T, b^T) (spatial transpose),
    simultaneous residue permutation equivariance, LN(x/s, eps/s^2) == LN(x, eps),
    exactly-zero update on padded cells when beta_mix = 0, all-ones mask == None;
  * LayerNorm against torch.nn.functional.layer_norm.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

EPS = 1e-5  # mlx_trunk.py:31 (esm's _EPS and nn.LayerNorm's default)


@dataclass
class TriMulWeights:
    """Weights of one triangle multiplicative update, in torch's [out, in] layout.

    Mirrors the attributes of the reference's TriangleMultiplicativeBlock
    (fast_trunk.py:53-56, mlx_trunk.py:40-55): proj_bundle.weight [4c, C] with
    rows [s_a | s_b | g_a | g_b]; norm_start (C); norm_mix (c); proj_emit.weight
    [C, c]; proj_gate.weight [C, C].
    """

    w_bundle: torch.Tensor          # [4c, C]
    w_emit: torch.Tensor            # [C, c]
    w_gate: torch.Tensor            # [C, C]
    ln_in_w: torch.Tensor           # [C]
    ln_in_b: torch.Tensor           # [C]
    ln_mix_w: torch.Tensor          # [c]
    ln_mix_b: torch.Tensor          # [c]
    ln_in_eps: float = EPS
    ln_mix_eps: float = EPS
    outgoing: bool = True

    @property
    def C(self) -> int:
        return self.w_bundle.shape[1]

    @property
    def c(self) -> int:
        return self.w_bundle.shape[0] // 4

    def to(self, dtype) -> "TriMulWeights":
        t = lambda x: x.to(dtype)  # noqa: E731
        return TriMulWeights(t(self.w_bundle), t(self.w_emit), t(self.w_gate), t(self.ln_in_w), t(self.ln_in_b),
                             t(self.ln_mix_w), t(self.ln_mix_b), self.ln_in_eps, self.ln_mix_eps, self.outgoing)


def draw_weights(gen: torch.Generator, C: int, c: int, outgoing: bool) -> TriMulWeights:
    """Seeded weights: W[4c,C], W_g[C,C], W_e[C,c] drawn in that order, each N(0, 1/fan_in);
    LayerNorm gamma = 1, beta = 0 (no draws). fp32 master copies."""
    f32 = torch.float32
    w = torch.randn(4 * c, C, generator=gen, dtype=f32) * (1.0 / C) ** 0.5
    wg = torch.randn(C, C, generator=gen, dtype=f32) * (1.0 / C) ** 0.5
    we = torch.randn(C, c, generator=gen, dtype=f32) * (1.0 / c) ** 0.5
    return TriMulWeights(w_bundle=w, w_emit=we, w_gate=wg,
                         ln_in_w=torch.ones(C, dtype=f32), ln_in_b=torch.zeros(C, dtype=f32),
                         ln_mix_w=torch.ones(c, dtype=f32), ln_mix_b=torch.zeros(c, dtype=f32), outgoing=outgoing)


def layer_norm(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, eps: float) -> torch.Tensor:
    """LayerNorm over the last axis, biased variance (nn.LayerNorm; mlx_trunk.py:81)."""
    mean = x.mean(-1, keepdim=True)
    var = ((x - mean) ** 2).mean(-1, keepdim=True)
    return (x - mean) / torch.sqrt(var + eps) * w + b


def project(z: torch.Tensor, mask: torch.Tensor | None, p: TriMulWeights):
    """(n, a, b): n = LN_in(z); a = s_a*sigmoid(g_a)*m; b = s_b*sigmoid(g_b)*m, cell layout [B,L,L,c].

    fast_trunk.py:22-26 (signal/gate split of the weights, mask applied after gating),
    mlx_trunk.py:72-76 and mlx_trunk_kernels.py:60-63 (same order: gate, then mask)."""
    c = p.c
    n = layer_norm(z, p.ln_in_w, p.ln_in_b, p.ln_in_eps)
    signal = F.linear(n, p.w_bundle[: 2 * c])
    gate = F.linear(n, p.w_bundle[2 * c:])
    routed = signal * torch.sigmoid(gate)
    if mask is not None:
        routed = routed * mask.unsqueeze(-1)
    return n, routed[..., :c], routed[..., c:]


def contract(a: torch.Tensor, b: torch.Tensor, outgoing: bool) -> torch.Tensor:
    """Triangle contraction on cell-layout operands a, b [B,L,L,c] -> x [B,L,L,c].

    mlx_trunk.py:84-88: outgoing x[d,i,j] = sum_k a[d,i,k] b[d,j,k];
    incoming x[d,i,j] = sum_k a[d,k,i] b[d,k,j]. Channels-first GEMM per channel."""
    A = a.permute(0, 3, 1, 2)  # [B, c, L, L]
    Bm = b.permute(0, 3, 1, 2)
    X = A @ Bm.transpose(-1, -2) if outgoing else A.transpose(-1, -2) @ Bm
    return X.permute(0, 2, 3, 1)


def contract_bruteforce(a, b, outgoing: bool):
    """Pure-Python triple loop of the same contraction (small L only; pins contract())."""
    B, L, _, c = a.shape
    x = torch.zeros(B, L, L, c, dtype=torch.float64)
    for bi in range(B):
        for d in range(c):
            for i in range(L):
                for j in range(L):
                    s = 0.0
                    for k in range(L):
                        if outgoing:
                            s += float(a[bi, i, k, d]) * float(b[bi, j, k, d])
                        else:
                            s += float(a[bi, k, i, d]) * float(b[bi, k, j, d])
                    x[bi, i, j, d] = s
    return x


def trimul(z: torch.Tensor, mask: torch.Tensor | None, p: TriMulWeights, outgoing: bool | None = None,
           out_mask: bool = False) -> torch.Tensor:
    """One TMU: the update (no residual) for pair z [B,L,L,C]. fast_trunk.py:19-32.

    ``out_mask`` multiplies the update by the pair mask; the reference does not
    (fast_trunk.py:31-32), so it is off by default."""
    if outgoing is None:
        outgoing = p.outgoing
    n, a, b = project(z, mask, p)
    x = contract(a, b, outgoing)
    mixed = F.linear(layer_norm(x, p.ln_mix_w, p.ln_mix_b, p.ln_mix_eps), p.w_emit)
    upd = mixed * torch.sigmoid(F.linear(n, p.w_gate))
    if out_mask and mask is not None:
        upd = upd * mask.unsqueeze(-1)
    return upd


def trimul_cells(z: torch.Tensor, mask: torch.Tensor | None, p: TriMulWeights, cells, outgoing: bool | None = None,
                 out_mask: bool = False) -> torch.Tensor:
    """The update of ``trimul`` at the sampled cells ``cells`` = [(b, i, j), ...] only -> [n, C].

    The same arithmetic (fast_trunk.py:19-32, mlx_trunk.py:84-90), restricted to what one output
    cell reads: outgoing x[d,i,j] = sum_k a[d,i,k] b[d,j,k] needs the operands of rows i and j
    of the pair grid, incoming x[d,i,j] = sum_k a[d,k,i] b[d,k,j] those of columns i and j; the
    gate needs z[b,i,j]. Each distinct line is projected once, so a grid far too large for
    ``trimul`` is checked at a few hundred cells in seconds. Pinned against ``trimul``
    (tests/test_oracle_tmu.py)."""
    if outgoing is None:
        outgoing = p.outgoing
    cells = [(int(b), int(i), int(j)) for b, i, j in cells]

    def line(bi, r):  # the cells of row r (outgoing) or column r (incoming) of batch bi
        return (z[bi, r], None if mask is None else mask[bi, r]) if outgoing else \
            (z[bi, :, r], None if mask is None else mask[bi, :, r])

    a_lines, b_lines = {}, {}
    for bi, i, j in cells:
        if (bi, i) not in a_lines:
            zl, ml = line(bi, i)
            a_lines[(bi, i)] = project(zl, ml, p)[1]   # a of the line: [L, c]
        if (bi, j) not in b_lines:
            zl, ml = line(bi, j)
            b_lines[(bi, j)] = project(zl, ml, p)[2]   # b of the line: [L, c]
    x = torch.stack([(a_lines[(bi, i)] * b_lines[(bi, j)]).sum(0) for bi, i, j in cells])  # [n, c]
    zc = torch.stack([z[bi, i, j] for bi, i, j in cells])                                    # [n, C]
    n = layer_norm(zc, p.ln_in_w, p.ln_in_b, p.ln_in_eps)
    upd = F.linear(layer_norm(x, p.ln_mix_w, p.ln_mix_b, p.ln_mix_eps), p.w_emit) * torch.sigmoid(F.linear(n, p.w_gate))
    if out_mask and mask is not None:
        upd = upd * torch.stack([mask[bi, i, j] for bi, i, j in cells]).unsqueeze(-1)
    return upd


def trimul_pair(z, mask, p_out: TriMulWeights, p_in: TriMulWeights):
    """z1 = z + T_out(z); z2 = z1 + T_in(z1) (mlx_trunk.py:93-95)."""
    z1 = z + trimul(z, mask, p_out, True)
    return z1 + trimul(z1, mask, p_in, False)


CONTRACT_SCALE = 256.0  # mlx_trunk.py:33


def rn16(t: torch.Tensor) -> torch.Tensor:
    """Round to fp16 and back to the working dtype (one storage rounding)."""
    return t.to(torch.float16).to(t.dtype)


def trimul_fp16ref(z: torch.Tensor, mask: torch.Tensor | None, p: TriMulWeights,
                   outgoing: bool | None = None) -> torch.Tensor:
    """z + update with the reference's fp16 storage at every op output: the arithmetic of
    the fp16 MLX trunk with its Metal kernels (mlx_trunk_kernels.py:210-229, weights from
    mlx_trunk.py:40-55 with dtype fp16), computed in fp32 with one fp16 rounding per stored
    tensor. Used to measure how far the reference's own fp16 scheme sits from exact
    arithmetic, the floor any fp16 implementation is compared against.

      weights   fp16; w_in[:, :c] (s_a) pre-divided by 256 (mlx_trunk.py:46-48)
      n         RN(LN_in(z))                                  (mlx_trunk_kernels.py:233)
      proj      RN(n @ w_in)                                  (:214)
      a, b      RN(s * sigmoid(g) * m), fp32 inside           (gate_cf, :60-64)
      x         RN(a @ b^T)  (incoming: a^T @ b)              (:219)
      mixed     RN(RN(LN_mix(x, eps / 256^2)) @ w_emit)       (ln_cf_to_cl :107-147, :224)
      g         RN(n @ w_out_gate)                            (:225)
      z'        RN(z + mixed * sigmoid(g)), fp32 inside       (resgate_ln, :165-190)
    ``z`` holds fp16-representable values in fp32 (or fp64)."""
    if outgoing is None:
        outgoing = p.outgoing
    f32 = torch.float32
    c = p.c
    w = p.w_bundle.to(f32).clone()
    w[:c] /= CONTRACT_SCALE
    w, we, wg = rn16(w), rn16(p.w_emit.to(f32)), rn16(p.w_gate.to(f32))
    g16 = lambda t: rn16(t.to(f32))  # noqa: E731  (LN parameters are stored fp16 too)
    zf = z.to(f32)
    n = rn16(layer_norm(zf, g16(p.ln_in_w), g16(p.ln_in_b), p.ln_in_eps))
    proj = rn16(F.linear(n, w))
    routed = proj[..., :2 * c] * torch.sigmoid(proj[..., 2 * c:])
    if mask is not None:
        routed = routed * mask.to(f32).unsqueeze(-1)
    routed = rn16(routed)
    x = rn16(contract(routed[..., :c], routed[..., c:], outgoing))
    mix_eps = p.ln_mix_eps / CONTRACT_SCALE ** 2
    mixed = rn16(F.linear(rn16(layer_norm(x, g16(p.ln_mix_w), g16(p.ln_mix_b), mix_eps)), we))
    g = rn16(F.linear(n, wg))
    return rn16(zf + mixed * torch.sigmoid(g)).to(z.dtype)


def make_pair_inputs(L: int, C: int, c: int, seed: int = 0, dtype=torch.float16, B: int = 1,
                     pad_from: int | None = None):
    """Seeded inputs of a TMU pair: z [B,L,L,C] ~ N(0,1), then T_out's and T_in's weights.

    Draw order: z, then out (W, W_g, W_e), then in (W, W_g, W_e). ``dtype`` rounds z
    (the fp16 configs cast the fp32 draw with .half()). ``pad_from`` builds the pair mask
    m[i,j] = (i < pad_from)(j < pad_from); None = no mask."""
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(B, L, L, C, generator=g, dtype=torch.float32).to(dtype)
    p_out = draw_weights(g, C, c, True)
    p_in = draw_weights(g, C, c, False)
    mask = None
    if pad_from is not None:
        v = (torch.arange(L) < pad_from).to(torch.float32)
        mask = (v[:, None] * v[None, :]).expand(B, L, L).contiguous()
    return z, mask, p_out, p_in
