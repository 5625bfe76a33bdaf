"""GPU parity of the ESMC block kernels and modules against the oracle (oracle/esmc.py).

Bars: the row kernels (LayerNorm, QK-LN + RoPE, SwiGLU) within a few fp16 roundings of
the fp64 oracle; attention and the block within max|err| <= 1e-2 x RMS of the oracle's
output (the block: of its update x_out - x_in), with the 8-bit weights dequantised to
fp16 as the GEMM multiplies them.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import esmc as oe

pytestmark = pytest.mark.gpu
DEV = "cuda"
D64 = torch.float64


def _gen(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("D,resid,fp32_out", [(256, False, False), (2560, True, False), (2560, True, True),
                                              (640, False, True)])
def test_layer_norm(gpu_lib, pkg, D, resid, fp32_out):
    g = _gen(D)
    x = 3 * torch.randn(7, D, generator=g) + 1
    y = torch.randn(7, D, generator=g).half() if resid else None
    w, b = 1 + 0.1 * torch.randn(D, generator=g), 0.1 * torch.randn(D, generator=g)
    xd = x.to(DEV)
    out = pkg.kernels.esmc_layer_norm(xd, w.to(DEV), b.to(DEV), 1e-5, y=None if y is None else y.to(DEV),
                                      alpha=0.5, fp32_out=fp32_out)
    xr = x.double() + (0.5 * y.double() if resid else 0)
    ref = F.layer_norm(xr, (D,), w.double(), b.double(), 1e-5)
    tol = (2e-6 if fp32_out else 2 ** -10) * float(ref.abs().max())
    assert float((out.double().cpu() - ref).abs().max()) <= tol
    if resid:  # the residual written back in place
        assert float((xd.double().cpu() - xr).abs().max()) <= 1e-6 * float(xr.abs().max())


@pytest.mark.parametrize("B,L,H", [(1, 1, 2), (2, 37, 4), (1, 238, 40), (1, 1100, 4)])
def test_qk_rope(gpu_lib, pkg, B, L, H):
    # (L = 1100: the angle, up to 1099 rad, in revolutions through fp32 and the hardware sine)
    D = 64 * H
    g = _gen(L)
    qkv = torch.randn(B * L, 3 * D, generator=g).half()
    qln, kln = 1 + 0.1 * torch.randn(D, generator=g), 1 + 0.1 * torch.randn(D, generator=g)
    q, k, v = pkg.kernels.esmc_qk_rope(qkv.to(DEV), qln.to(DEV), kln.to(DEV), 1e-5, B, L, H)
    x = qkv.double().reshape(B, L, 3 * D)
    heads = lambda t: t.reshape(B, L, H, 64).transpose(1, 2)  # noqa: E731
    rq = oe.rope(heads(F.layer_norm(x[..., :D], (D,), qln.double(), None, 1e-5)))
    rk = oe.rope(heads(F.layer_norm(x[..., D:2 * D], (D,), kln.double(), None, 1e-5)))
    for got, ref in ((q, rq), (k, rk)):
        assert float((got.double().cpu() - ref).abs().max()) <= 2 ** -9 * float(ref.abs().max())
    assert torch.equal(v.cpu(), heads(qkv.reshape(B, L, 3 * D)[..., 2 * D:]).contiguous())


@pytest.mark.parametrize("L", [1, 5, 31, 64, 130, 238, 300, 512, 513, 700, 1100])
@pytest.mark.parametrize("masked", [False, True])
def test_attention(gpu_lib, pkg, L, masked):
    # beyond 512 tokens the keys go in passes of 512 with an online softmax: the chains then
    # span pass boundaries, and queries of the later chain see no key in the first pass
    B, H = 2, 3
    g = _gen(L + masked)
    q, k, v = (torch.randn(B, H, L, 64, generator=g).half() for _ in range(3))
    sid = None
    if masked:  # two chains and padding (its own chain, -1), per batch element
        sid = torch.zeros(B, L, dtype=torch.int32)
        sid[0, L // 2:] = 1
        sid[1, (2 * L) // 3:] = -1
    o = pkg.kernels.esmc_attention(q.to(DEV), k.to(DEV), v.to(DEV), None if sid is None else sid.to(DEV))
    ref = oe.attention(q.double(), k.double(), v.double(), oe.chain_mask(sid), 0.125)
    ref = ref.transpose(1, 2).reshape(B, L, H * 64)
    err = float((o.double().cpu() - ref).abs().max())
    assert err <= 1e-2 * float(ref.pow(2).mean().sqrt()), err


def test_attention_keys_only_in_a_later_pass(gpu_lib, pkg):
    # L = 1030: tokens 0..599 are chain 0, the rest chain 1, so the chain-1 queries' first
    # visible key is in the second pass (the running max starts at -inf), and a 1-token chain
    # at the end sees only itself
    B, H, L = 1, 2, 1030
    g = _gen(77)
    q, k, v = (3 * torch.randn(B, H, L, 64, generator=g).half() for _ in range(3))
    sid = torch.zeros(B, L, dtype=torch.int32)
    sid[0, 600:] = 1
    sid[0, L - 1] = 2
    o = pkg.kernels.esmc_attention(q.to(DEV), k.to(DEV), v.to(DEV), sid.to(DEV))
    ref = oe.attention(q.double(), k.double(), v.double(), oe.chain_mask(sid), 0.125)
    ref = ref.transpose(1, 2).reshape(B, L, H * 64)
    err = float((o.double().cpu() - ref).abs().max())
    assert err <= 1e-2 * float(ref.pow(2).mean().sqrt()), err
    # the lone token's output is its own value row
    assert torch.allclose(o[0, L - 1].view(H, 64).float().cpu(), v[0, :, L - 1].float(), atol=1e-3)


def test_swiglu(gpu_lib, pkg):
    g = _gen(0)
    x = (2 * torch.randn(9, 2 * 320, generator=g)).half()
    y = pkg.kernels.esmc_swiglu(x.to(DEV)).double().cpu()
    xd = x.double()
    ref = F.silu(xd[:, :320]) * xd[:, 320:]
    assert float((y - ref).abs().max()) <= 2 ** -10 * float(ref.abs().max())


@pytest.mark.parametrize("M,K,N", [(238, 2560, 2560), (238, 5120, 2560), (238, 2560, 10240), (37, 256, 256),
                                   (5, 1024, 64)])
def test_q8_partials_then_layer_norm_equal_unfused(gpu_lib, pkg, M, K, N):
    """q8_linear_partials + esmc_layer_norm_parts give the same bits as q8_linear (with its split-K
    workspace) + esmc_layer_norm: the partials summed in split order and rounded once, then the same
    residual add and LayerNorm. Covers split (M=238, N=2560) and unsplit (N=10240) plans."""
    g = _gen(M + K + N)
    p = oe.quantize(torch.randn(N, K, generator=g) * K ** -0.5)
    lin = pkg.q8.Q8Linear(torch.from_numpy(p.q), torch.from_numpy(p.s), torch.from_numpy(p.b))
    x = torch.randn(M, K, generator=g).half().to(DEV)
    y = lin(x)
    parts, splits = lin.partials(x)
    assert parts.shape == (splits, M, N) and splits >= 1
    acc = parts[0].clone()
    for s_ in range(1, splits):
        acc += parts[s_]
    assert torch.equal(acc.half(), y)
    if N > 8192:  # wider than the LayerNorm supports: the partials alone are the case
        return
    r = (3 * torch.randn(M, N, generator=g) + 1).to(DEV)
    w, b = (1 + 0.1 * torch.randn(N, generator=g)).to(DEV), (0.1 * torch.randn(N, generator=g)).to(DEV)
    for fp32_out in (False, True):
        xo1, xo2 = torch.empty_like(r), torch.empty_like(r)
        h1 = pkg.kernels.esmc_layer_norm(r, w, b, 1e-5, y=y, alpha=0.37, x_out=xo1, fp32_out=fp32_out)
        h2 = pkg.kernels.esmc_layer_norm(r, w, b, 1e-5, y_parts=(parts, splits), alpha=0.37, x_out=xo2,
                                         fp32_out=fp32_out)
        torch.cuda.synchronize()
        assert torch.equal(xo1, xo2) and torch.equal(h1, h2)


def _weights(D, F_, seed):
    g = _gen(seed)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    qz = lambda n, k: oe.quantize(r(n, k) * k ** -0.5)  # noqa: E731
    return oe.EsmcBlockWeights(1 + 0.1 * r(D), 0.1 * r(D), 1 + 0.1 * r(D), 1 + 0.1 * r(D), 1 + 0.1 * r(D),
                               0.1 * r(D), qz(3 * D, D), qz(D, D), qz(2 * F_, D), qz(D, F_))


def _module_block(pkg, p, n_heads):
    lin = {n: pkg.q8.Q8Linear(torch.from_numpy(getattr(p, n).q), torch.from_numpy(getattr(p, n).s),
                              torch.from_numpy(getattr(p, n).b)) for n in ("wqkv", "wo", "w1", "w2")}
    return pkg.esmc.EsmcBlock(p.ln1_w, p.ln1_b, p.q_ln, p.k_ln, p.ln2_w, p.ln2_b, lin["wqkv"], lin["wo"], lin["w1"],
                              lin["w2"], n_heads)


@pytest.mark.parametrize("D,F_,H,L,masked", [(256, 384, 4, 37, True), (640, 1024, 10, 238, False)])
def test_block(gpu_lib, pkg, D, F_, H, L, masked):
    p = _weights(D, F_, seed=D)
    blk = _module_block(pkg, p, H)
    g = _gen(1)
    x = 2 * torch.randn(2, L, D, generator=g)
    sid = None
    if masked:
        sid = torch.zeros(2, L, dtype=torch.int64)
        sid[0, 20:] = 1
    rs = math.sqrt(80 / 36)
    out = blk(x.to(DEV), None if sid is None else sid.to(DEV), res_scale=rs).double().cpu()
    ref = oe.block_forward(p, x.double(), sid, n_heads=H, res_scale=rs, weights="f16")
    upd = ref - x.double()
    err = float((out - ref).abs().max())
    assert err <= 1e-2 * float(upd.pow(2).mean().sqrt()), err


def test_block_real_width(gpu_lib, pkg):
    # the ESMC block at the width the reference runs (D = 2560, 40 heads; FFN 5120), 238 tokens,
    # two chains: every linear at its real shape (wqkv 2560 -> 7680, wo 2560 -> 2560 split-K,
    # w1 2560 -> 10240, w2 5120 -> 2560 split-K)
    D, F_, H, L = 2560, 5120, 40, 238
    p = _weights(D, F_, seed=5)
    blk = _module_block(pkg, p, H)
    x = 2 * torch.randn(1, L, D, generator=_gen(9))
    sid = torch.zeros(1, L, dtype=torch.int64)
    sid[0, 150:] = 1
    rs = math.sqrt(80 / 36)
    out = blk(x.to(DEV), sid.to(DEV), res_scale=rs).double().cpu()
    ref = oe.block_forward(p, x.double(), sid, n_heads=H, res_scale=rs, weights="f16")
    upd = ref - x.double()
    err = float((out - ref).abs().max())
    assert err <= 1e-2 * float(upd.pow(2).mean().sqrt()), err


def test_block_graph_replay(gpu_lib, pkg):
    """The block captured as one HIP graph: every replay equals the eager result bit for bit,
    with eager launches of the block between the replays."""
    D, F_, H, L = 256, 384, 4, 37
    blk = _module_block(pkg, _weights(D, F_, seed=3), H)
    x = (2 * torch.randn(1, L, D, generator=_gen(7))).to(DEV)
    ref = blk(x, None, res_scale=1.5)  # also allocates the layers' workspaces outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = blk(x, None, res_scale=1.5)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), i
        other = blk(x * (i + 2), None, res_scale=1.5)  # eager work between the replays
        torch.cuda.synchronize()
        assert not torch.equal(other, ref)


def test_hip_esmc_hidden_states_and_cache(gpu_lib, pkg, tmp_path):
    D, F_, H, n = 256, 384, 4, 3
    ps = [_weights(D, F_, seed=10 + i) for i in range(n)]
    g = _gen(5)
    embed = torch.randn(33, D, generator=g)
    norm_w = 1 + 0.1 * torch.randn(D, generator=g)
    model = pkg.esmc.HipEsmc(embed, [_module_block(pkg, p, H) for p in ps], norm_w, n_heads=H)
    assert model.to("cpu") is model
    ids = torch.randint(0, 33, (2, 29), generator=g)
    sid = torch.zeros(2, 29, dtype=torch.int64)
    sid[1, 15:] = 1
    hs = model(input_ids=ids.to(DEV), sequence_id=sid.to(DEV), output_hidden_states=True).hidden_states
    assert hs.shape == (n + 1, 2, 29, D) and hs.dtype == torch.float32
    # the oracle: each block's input, then the final LayerNorm (weights only)
    rs = math.sqrt(n / 36)
    x = embed.double()[ids]
    for i, p in enumerate(ps):
        assert float((hs[i].double().cpu() - x).abs().max()) <= 1e-2 * float(x.pow(2).mean().sqrt()) + 1e-6
        x = oe.block_forward(p, x, sid, n_heads=H, res_scale=rs, weights="f16")
    last = F.layer_norm(x, (D,), norm_w.double(), None, 1e-5)
    assert float((hs[n].double().cpu() - last).abs().max()) <= 1e-2 * float(last.pow(2).mean().sqrt())
    # the reference's converted-weight cache layout: save, reload, same hidden states
    path = tmp_path / "esmc_q8.safetensors"
    model.save_cache(path)
    from safetensors.torch import load_file
    flat = load_file(str(path))
    assert {"embed", "norm_w", "layers.0.wqkv", "layers.0.wqkv_s", "layers.0.wqkv_b", "layers.2.w2_b",
            "layers.1.q_ln"} <= set(flat)
    assert flat["layers.0.wqkv"].shape == (3 * D, D // 4) and flat["layers.0.wqkv_s"].dtype == torch.float16
    again = pkg.esmc.HipEsmc.from_cache(path, n_heads=H)
    hs2 = again(input_ids=ids.to(DEV), sequence_id=sid.to(DEV)).hidden_states
    assert torch.equal(hs, hs2)


def test_hip_esmc_from_hf_weights(gpu_lib, pkg, tmp_path):
    # the product quantiser: HF-named fp32 tensors -> 8-bit layers (wqkv = [q; k; v], w1 = [gate; up],
    # group 64 along in, fp16 scales and biases) -> the cache layout, as the reference's
    # layer_params / from_shards (mlx_esmc.py:53-75, :116-137)
    from oracle import q8 as oq8
    D, F_, H, n = 128, 256, 2, 2
    g = _gen(21)
    hf = {"esmc.embed_tokens.weight": torch.randn(33, D, generator=g),
          "esmc.norm.weight": 1 + 0.1 * torch.randn(D, generator=g)}
    shapes = {"self_attn.q_proj.weight": (D, D), "self_attn.k_proj.weight": (D, D), "self_attn.v_proj.weight": (D, D),
              "self_attn.o_proj.weight": (D, D), "mlp.gate_proj.weight": (F_, D), "mlp.up_proj.weight": (F_, D),
              "mlp.down_proj.weight": (D, F_)}
    for i in range(n):
        for name, shp in shapes.items():
            hf[f"esmc.layers.{i}.{name}"] = torch.randn(*shp, generator=g) * shp[1] ** -0.5
        for name in ("input_layernorm", "post_attention_layernorm"):
            hf[f"esmc.layers.{i}.{name}.weight"] = 1 + 0.1 * torch.randn(D, generator=g)
            hf[f"esmc.layers.{i}.{name}.bias"] = 0.1 * torch.randn(D, generator=g)
        for name in ("q_norm", "k_norm"):
            hf[f"esmc.layers.{i}.self_attn.{name}.weight"] = 1 + 0.1 * torch.randn(D, generator=g)
    path = tmp_path / "cache" / "esmc_q8.safetensors"
    model = pkg.esmc.HipEsmc.from_hf(hf, n_heads=H, cache=path)
    assert len(model.layers) == n and path.exists()
    # the row layout of the fused linears and the quantised arrays, against the oracle's quantiser
    for i, blk in enumerate(model.layers):
        for lin, parts in (("wqkv", ("q_proj", "k_proj", "v_proj")), ("w1", ("gate_proj", "up_proj"))):
            pre = "self_attn" if lin == "wqkv" else "mlp"
            w = torch.cat([hf[f"esmc.layers.{i}.{pre}.{p}.weight"] for p in parts]).numpy()
            qr, sr, br = oq8.quantize_f16(w)
            m = getattr(blk, lin)
            assert np.array_equal(m.q.cpu().numpy(), qr)
            assert np.array_equal(m.scales.cpu().numpy().view(np.uint16), sr.view(np.uint16))
            assert np.array_equal(m.biases.cpu().numpy().view(np.uint16), br.view(np.uint16))
    # hidden states against the oracle blocks built from the oracle's quantisation
    ps = []
    for i in range(n):
        lw = lambda nm: hf[f"esmc.layers.{i}.{nm}"]  # noqa: E731
        qw = {}
        for lin, names in (("wqkv", ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight")),
                           ("wo", ("self_attn.o_proj.weight",)), ("w1", ("mlp.gate_proj.weight", "mlp.up_proj.weight")),
                           ("w2", ("mlp.down_proj.weight",))):
            qw[lin] = oe.Q8Weights(*oq8.quantize_f16(torch.cat([lw(nm) for nm in names]).numpy()))
        ps.append(oe.EsmcBlockWeights(lw("input_layernorm.weight"), lw("input_layernorm.bias"),
                                      lw("self_attn.q_norm.weight"), lw("self_attn.k_norm.weight"),
                                      lw("post_attention_layernorm.weight"), lw("post_attention_layernorm.bias"),
                                      qw["wqkv"], qw["wo"], qw["w1"], qw["w2"]))
    ids = torch.randint(0, 33, (1, 40), generator=g)
    hs = model(input_ids=ids.to(DEV)).hidden_states
    x = hf["esmc.embed_tokens.weight"].double()[ids]
    rs = math.sqrt(n / 36)
    for i, p in enumerate(ps):
        assert float((hs[i].double().cpu() - x).abs().max()) <= 1e-2 * float(x.pow(2).mean().sqrt()) + 1e-6
        x = oe.block_forward(p, x, None, n_heads=H, res_scale=rs, weights="f16")
    last = F.layer_norm(x, (D,), hf["esmc.norm.weight"].double(), None, 1e-5)
    assert float((hs[n].double().cpu() - last).abs().max()) <= 1e-2 * float(last.pow(2).mean().sqrt())
    # the cache written on conversion loads back (from_hf finds it) with the same hidden states
    again = pkg.esmc.HipEsmc.from_hf({}, n_heads=H, cache=path)
    assert torch.equal(again(input_ids=ids.to(DEV)).hidden_states, hs)
