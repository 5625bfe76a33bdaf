"""GPU parity of the 8-bit weight-only linear (kernel d) and its dequantiser.

Bars: dequantised weights bit-exact against RN_fp16(s*q + b); the GEMM within
1e-3 normwise relative error of the fp64 oracle x . W^T (and max|err| within
1e-3 * max|ref|).
"""

import contextlib

import numpy as np
import pytest
import torch

from oracle import q8

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@contextlib.contextmanager
def _tile_rows(pkg, rows):
    # every q8 plan in the block uses output tiles of `rows` weight rows (0: the plan's choice)
    lib = pkg.capi.lib()
    pkg.capi.check(lib.q8_set_tile_rows(rows))
    try:
        yield
    finally:
        pkg.capi.check(lib.q8_set_tile_rows(0))


@pytest.mark.parametrize("N,K", [(64, 64), (128, 192), (256, 2560)])
def test_dequant_bit_exact(gpu_lib, pkg, N, K):
    _, q, s, b = q8.make_q8_inputs(1, K, N, seed=N + K)
    w = pkg.kernels.q8_dequant(_t(q), _t(s), _t(b)).cpu().numpy()
    assert np.array_equal(w.view(np.uint16), q8.dequant_f16(q, s, b).view(np.uint16))


def test_dequant_special_values(gpu_lib, pkg):
    N, K = 64, 128
    q = np.tile(np.arange(128, dtype=np.uint8) * 2, (N, 1))
    q[:, 0] = 0
    q[:, 1] = 255
    rng = np.random.default_rng(0)
    s = rng.uniform(0.001, 0.01, (N, 2)).astype(np.float16)
    b = rng.normal(0, 0.1, (N, 2)).astype(np.float16)
    s[0] = 0                                     # s = 0 -> b
    b[1] = np.float16(2.0 ** -20)                # subnormal fp16 bias
    s[2], b[2] = np.float16(2.0 ** -14), 0       # tiny products: subnormal results
    b[3] = np.float16(-0.0)
    w = pkg.kernels.q8_dequant(_t(q), _t(s), _t(b)).cpu().numpy()
    assert np.array_equal(w.view(np.uint16), q8.dequant_f16(q, s, b).view(np.uint16))


def _check(y, x, q, s, b):
    ref = q8.q8_linear(x, q, s, b)
    y = y.astype(np.float64)
    assert np.isfinite(y).all()
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel <= 1e-3, f"normwise relative error {rel:.3e}"
    assert np.abs(y - ref).max() <= 1e-3 * np.abs(ref).max()
    # against the fp16-rounded weights the kernel multiplies by: only accumulation order
    # and the output rounding remain
    ref16 = q8.q8_linear(x, q, s, b, weights="f16")
    assert np.linalg.norm(y - ref16) / np.linalg.norm(ref16) <= 3e-4
    return rel


@pytest.mark.parametrize("M,K,N", [(1, 64, 64), (5, 128, 64), (37, 256, 128), (64, 640, 192), (65, 1024, 256),
                                   (238, 2560, 512)])
def test_q8_linear_small(gpu_lib, pkg, M, K, N):
    x, q, s, b = q8.make_q8_inputs(M, K, N, seed=M)
    y = pkg.kernels.q8_linear(_t(x), _t(q), _t(s), _t(b)).cpu().numpy()
    _check(y, x, q, s, b)


@pytest.mark.parametrize("K,N", [(2560, 10240), (10240, 2560)])
def test_q8_linear_esmc_shapes(gpu_lib, pkg, K, N):
    # the ESMC-style linears: [238, 2560] x [2560 -> 10240] and [238, 10240] x [10240 -> 2560]
    x, q, s, b = q8.make_q8_inputs(238, K, N, seed=K)
    y = pkg.kernels.q8_linear(_t(x), _t(q), _t(s), _t(b)).cpu().numpy()
    _check(y, x, q, s, b)


def test_q8_module_and_mlx_packing(gpu_lib, pkg):
    x, q, s, b = q8.make_q8_inputs(10, 128, 64, seed=3)
    words = torch.from_numpy(q.copy()).view(torch.int32)  # four codes per 32-bit word, little-endian
    lin = pkg.q8.Q8Linear.from_packed_u32(words, torch.from_numpy(s), torch.from_numpy(b))
    y = lin(torch.from_numpy(x).to(DEV).float())  # fp32 in -> fp32 out
    assert y.dtype == torch.float32
    _check(y.cpu().numpy(), x, q, s, b)


def test_q8_linear_rejects_bad_shapes(gpu_lib, pkg):
    x, q, s, b = q8.make_q8_inputs(4, 128, 64, seed=0)
    with pytest.raises(Exception):
        pkg.kernels.q8_linear(_t(x[:, :64]), _t(q), _t(s), _t(b))


@pytest.mark.parametrize("M,K,N", [(238, 10240, 2560), (5, 1024, 64), (64, 4096, 320), (130, 512, 192)])
def test_q8_linear_split_k(gpu_lib, pkg, M, K, N):
    # shapes whose 64-row output tiles cannot fill the GPU split K over workgroups through
    # the workspace; a second kernel sums the fp32 partials in split order
    nbytes = pkg.kernels.q8_workspace_bytes(M, K, N)
    assert nbytes > 0, "this shape is expected to split K"
    ws = pkg.kernels.q8_workspace(M, K, N)
    x, q, s, b = q8.make_q8_inputs(M, K, N, seed=M + K)
    x2 = np.random.default_rng(1).standard_normal((M, K)).astype(np.float16)
    args = (_t(q), _t(s), _t(b))
    y1 = pkg.kernels.q8_linear(_t(x), *args, workspace=ws).cpu().numpy()
    _check(y1, x, q, s, b)
    # the workspace is left ready: a second call (other x) and a repeat of the first
    y2 = pkg.kernels.q8_linear(_t(x2), *args, workspace=ws).cpu().numpy()
    _check(y2, x2, q, s, b)
    y3 = pkg.kernels.q8_linear(_t(x), *args, workspace=ws).cpu().numpy()
    assert np.array_equal(y1.view(np.uint16), y3.view(np.uint16)), "split-K result depends on arrival order"
    # the unsplit kernel (no workspace) agrees to the accumulation-order bound
    y0 = pkg.kernels.q8_linear(_t(x), *args).cpu().numpy()
    _check(y0, x, q, s, b)


def test_q8_workspace_sizes_and_errors(gpu_lib, pkg):
    assert pkg.kernels.q8_workspace_bytes(238, 2560, 10240) == 0  # 256 tiles: no split
    M, K, N = 5, 1024, 64
    x, q, s, b = q8.make_q8_inputs(M, K, N, seed=2)
    small = torch.zeros(64 + 256, dtype=torch.uint8, device=DEV)
    with pytest.raises(pkg.capi.EsmError):
        pkg.kernels.q8_linear(_t(x), _t(q), _t(s), _t(b), workspace=small)


def test_q8_module_split_k_workspace(gpu_lib, pkg):
    # the split-K partials run in the device's shared scratch
    x, q, s, b = q8.make_q8_inputs(238, 4096, 640, seed=9)
    lin = pkg.q8.Q8Linear(torch.from_numpy(q), torch.from_numpy(s), torch.from_numpy(b))
    xt = torch.from_numpy(x).to(DEV)
    assert pkg.kernels.q8_workspace_bytes(238, 4096, 640) > 0
    y = lin(xt)
    assert pkg.scratch.reserved(DEV) >= pkg.kernels.q8_workspace_bytes(238, 4096, 640)
    _check(y.cpu().numpy(), x, q, s, b)
    _check(lin(xt).cpu().numpy(), x, q, s, b)


def test_q8_memory_stops_growing_over_row_counts(gpu_lib, pkg):
    # many layers and many sequence lengths share one scratch buffer: device memory stays
    # flat once the largest shape has run, and results are unchanged by the sharing
    K, N = 4096, 640
    layers = [pkg.q8.Q8Linear(*(torch.from_numpy(a) for a in q8.make_q8_inputs(8, K, N, seed=40 + i)[1:]))
              for i in range(4)]
    xs = {M: torch.from_numpy(q8.make_q8_inputs(M, K, N, seed=M)[0]).to(DEV) for M in (256, 31, 97, 200, 5)}
    first = {M: [lin(x) for lin in layers] for M, x in xs.items()}
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    for rnd in range(3):
        for M, x in xs.items():
            for lin, y0 in zip(layers, first[M]):
                assert torch.equal(lin(x).view(torch.int16), y0.view(torch.int16))
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() <= base, f"round {rnd}: {torch.cuda.memory_allocated()} > {base}"
    _check(first[97][2].cpu().numpy(), *q8.make_q8_inputs(97, K, N, seed=97)[:1],
           *q8.make_q8_inputs(8, K, N, seed=42)[1:])


@pytest.mark.parametrize("M,K,N", [(238, 2560, 640), (238, 10240, 320), (7, 192, 192)])
def test_q8_packed_scales_same_bits(gpu_lib, pkg, M, K, N):
    # the packed-scale layout is a cache: same bits as the [N, K/64] arrays, split or not
    x, q, s, b = (_t(a) for a in q8.make_q8_inputs(M, K, N, seed=N))
    sb = pkg.kernels.q8_pack_scales(s, b)
    # layout: word (j, g, r) = b[32 j + r, g] << 16 | s[32 j + r, g], 0 past N
    s16, b16 = s.cpu().numpy().view(np.uint16), b.cpu().numpy().view(np.uint16)
    T, G = -(-N // 32), K // 64
    ref = np.zeros((T, G, 32), dtype=np.uint32)
    for t in range(T):
        rows = np.arange(32 * t, min(32 * t + 32, N))
        ref[t, :, :len(rows)] = (b16[rows].astype(np.uint32).T << 16) | s16[rows].astype(np.uint32).T
    assert np.array_equal(sb.cpu().numpy().view(np.uint32).reshape(T, G, 32), ref)
    ws = pkg.kernels.q8_workspace(M, K, N)
    y_plain = pkg.kernels.q8_linear(x, q, s, b, workspace=ws)
    y_packed = pkg.kernels.q8_linear(x, q, s, b, workspace=ws, packed=sb)
    assert torch.equal(y_plain.view(torch.int16), y_packed.view(torch.int16))
    _check(y_packed.cpu().numpy(), *q8.make_q8_inputs(M, K, N, seed=N))


@pytest.mark.parametrize("M,K,N", [(238, 2560, 640), (238, 10240, 320), (238, 5120, 2560), (7, 192, 192),
                                   (100, 64, 64), (65, 320, 448)])
def test_q8_packed_codes_same_bits(gpu_lib, pkg, M, K, N):
    # the packed-code layout is a cache: the same MFMAs in the same order as the [N, K] codes,
    # so y and the split partials are the same bits; odd group counts (a step's second group
    # past K), N not a multiple of 160 and split-K shapes included
    x, q, s, b = (_t(a) for a in q8.make_q8_inputs(M, K, N, seed=N + K))
    sb = pkg.kernels.q8_pack_scales(s, b)
    qp = pkg.kernels.q8_pack_codes(q)
    ws = pkg.kernels.q8_workspace(M, K, N)
    y_ref = pkg.kernels.q8_linear(x, q, s, b, workspace=ws, packed=sb)
    y_pc = pkg.kernels.q8_linear(x, q, s, b, workspace=ws, packed=sb, codes=qp)
    assert torch.equal(y_ref.view(torch.int16), y_pc.view(torch.int16))
    # without a workspace the tile runs unsplit (another summation order): again equal across layouts
    y_ref1 = pkg.kernels.q8_linear(x, q, s, b, packed=sb)
    y_pc1 = pkg.kernels.q8_linear(x, q, s, b, packed=sb, codes=qp)
    assert torch.equal(y_ref1.view(torch.int16), y_pc1.view(torch.int16))
    buf_a, buf_b = pkg.kernels.q8_partials_buffer(M, K, N), pkg.kernels.q8_partials_buffer(M, K, N)
    pa, na = pkg.kernels.q8_linear_partials(x, q, s, b, buf_a, packed=sb)
    pb, nb = pkg.kernels.q8_linear_partials(x, q, s, b, buf_b, packed=sb, codes=qp)
    assert na == nb and torch.equal(pa.view(torch.int32), pb.view(torch.int32))
    if M * K * N <= 238 * 2560 * 640:
        _check(y_pc.cpu().numpy(), *q8.make_q8_inputs(M, K, N, seed=N + K))


def test_q8_packed_codes_layout(gpu_lib, pkg):
    # chunk ((j S + s) 4 + w), lane l: row 32 j + l % 32, k = 128 s + 16 w + 8 (l / 32) + 0..7,
    # then k + 64; zeros past N and past K (N = 200: a partial last block; 3 groups: the second
    # step's upper half is past K)
    N, K = 200, 192
    rng = np.random.default_rng(3)
    q = rng.integers(0, 256, (N, K), dtype=np.uint8)
    qp = pkg.kernels.q8_pack_codes(_t(q)).cpu().numpy()
    J, S = 7, 2
    qz = np.zeros((J * 32, S * 128), dtype=np.uint8)
    qz[:N, :K] = q
    ref = np.zeros((J, S, 4, 64, 16), dtype=np.uint8)
    for j in range(J):
        for st in range(S):
            for w in range(4):
                for ln in range(64):
                    n, k0 = 32 * j + ln % 32, 128 * st + 16 * w + 8 * (ln // 32)
                    ref[j, st, w, ln, :8] = qz[n, k0:k0 + 8]
                    ref[j, st, w, ln, 8:] = qz[n, k0 + 64:k0 + 72]
    assert np.array_equal(qp, ref.reshape(-1))


@pytest.mark.parametrize("M,K,N", [(238, 2560, 7680), (238, 2560, 10240), (238, 5120, 2560), (7, 192, 320),
                                   (65, 320, 448), (100, 64, 64)])
def test_q8_tile_widths_same_bits(gpu_lib, pkg, M, K, N):
    # 128- and 160-row tiles differ only in which workgroup computes an output: unsplit, the same
    # bits (both code layouts); split, each within the oracle bars
    K_, lib = pkg.kernels, pkg.capi.lib()
    x, q, s, b = (_t(a) for a in q8.make_q8_inputs(M, K, N, seed=M + 3 * N))
    sb, qp = K_.q8_pack_scales(s, b), K_.q8_pack_codes(q)
    assert lib.q8_tile_rows(M, K, N) in (128, 160)
    ys = {}
    for rows in (128, 160):
        with _tile_rows(pkg, rows):
            assert lib.q8_tile_rows(M, K, N) == rows
            ys[rows] = (K_.q8_linear(x, q, s, b, packed=sb), K_.q8_linear(x, q, s, b, packed=sb, codes=qp),
                        K_.q8_linear(x, q, s, b, packed=sb, codes=qp, workspace=K_.q8_workspace(M, K, N)))
    for y in ys[128][:2] + ys[160][:2]:
        assert torch.equal(y.view(torch.int16), ys[160][0].view(torch.int16))
    if M * K * N <= 238 * 2560 * 2560:
        for rows in (128, 160):
            _check(ys[rows][2].cpu().numpy(), *q8.make_q8_inputs(M, K, N, seed=M + 3 * N))


@pytest.mark.parametrize("M,K,N", [(238, 2560, 10240), (50, 2560, 10240), (7, 192, 320), (100, 640, 640)])
def test_q8_swiglu_fused_same_bits(gpu_lib, pkg, M, K, N):
    # w1 then SwiGLU in one call (rows in SwiGLU pair order) against the two calls on [gate; up]:
    # unsplit (the GEMM's epilogue gates) and split-K (the reduction gates), same bits
    K_ = pkg.kernels
    x, q, s, b = (_t(a) for a in q8.make_q8_inputs(M, K, N, seed=M + N))
    ws = K_.q8_workspace(M, K, N)
    with _tile_rows(pkg, 160):  # the pair order's tile, so both calls split K alike
        ref = K_.esmc_swiglu(K_.q8_linear(x, q, s, b, workspace=ws))
    perm = K_.swiglu_pair_rows(N, DEV)
    sbp = K_.q8_pack_scales(s[perm].contiguous(), b[perm].contiguous())
    qpp = K_.q8_pack_codes(q[perm].contiguous())
    got = K_.q8_linear_swiglu(x, qpp, sbp, N, workspace=ws)
    assert got.shape == (M, N // 2)
    assert torch.equal(ref.view(torch.int16), got.view(torch.int16))
    got1 = K_.q8_linear_swiglu(x, qpp, sbp, N)  # no workspace: unsplit
    ref1 = K_.esmc_swiglu(K_.q8_linear(x, q, s, b))
    assert torch.equal(ref1.view(torch.int16), got1.view(torch.int16))
    # and against the fp64 oracle of silu(x W_g) * (x W_u)
    xs, qs, ss, bs = q8.make_q8_inputs(M, K, N, seed=M + N)
    y = q8.q8_linear(xs, qs, ss, bs)
    g, u = y[:, :N // 2], y[:, N // 2:]
    want = g / (1 + np.exp(-g)) * u
    rel = np.linalg.norm(got.cpu().numpy().astype(np.float64) - want) / np.linalg.norm(want)
    assert rel <= 3e-3, f"normwise relative error {rel:.3e}"  # the GEMM's ~3e-4 and two fp16 roundings


def test_q8_module_swiglu_pairs(gpu_lib, pkg):
    x, q, s, b = (_t(a) for a in q8.make_q8_inputs(238, 640, 1280, seed=9))
    lin = pkg.q8.Q8Linear(q, s, b, device=DEV)
    y0 = lin(x)
    lin.swiglu_pairs()
    assert torch.equal(lin(x).view(torch.int16), y0.view(torch.int16))  # forward unchanged
    assert torch.equal(lin.swiglu(x).view(torch.int16), pkg.kernels.esmc_swiglu(y0).view(torch.int16))


def test_q8_module_packed_codes_option(gpu_lib, pkg):
    x, q, s, b = (_t(a) for a in q8.make_q8_inputs(238, 2560, 512, seed=5))
    on = pkg.q8.Q8Linear(q, s, b, device=DEV)
    off = pkg.q8.Q8Linear(q, s, b, device=DEV, pack_codes=False)
    assert on.codes_packed is not None and off.codes_packed is None
    assert torch.equal(on(x).view(torch.int16), off(x).view(torch.int16))
    pa, na = on.partials(x)
    pa = pa.clone()
    pb, nb = off.partials(x)
    assert na == nb and torch.equal(pa.view(torch.int32), pb.view(torch.int32))


def _quant_cases():
    rng = np.random.default_rng(7)
    w = rng.standard_normal((96, 640)).astype(np.float32) * rng.uniform(0.01, 3, (96, 1)).astype(np.float32)
    w[0, :64] = np.linspace(-1, 0.5, 64)          # hand-computed group: bias -1, step 1/170
    w[1, :64] = 0.3                                # constant group: code 0, bias 0.3
    w[2, :64] = 0.0                                # all-zero group: bias 0 (q0 = 0)
    w[3] = np.abs(w[3])                            # all-positive groups
    w[4] = -np.abs(w[4])                           # all-negative groups
    w[5, 70] = 40.0                                # an outlier
    w[6, :64] = rng.integers(-3, 4, 64) * 0.25     # ties at half steps
    return w


def test_quantize_matches_oracle_bit_exact(gpu_lib, pkg):
    # the GPU quantiser (MLX's affine scheme, mlx_esmc.py:73-74) gives the oracle's codes, fp16
    # scales and fp16 biases bit for bit; its dequantised weights sit within the scheme's bound
    w = _quant_cases()
    q, s, b = pkg.kernels.q8_quantize(_t(w))
    qr, sr, br = q8.quantize_f16(w)
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(s.cpu().numpy().view(np.uint16), sr.view(np.uint16))
    assert np.array_equal(b.cpu().numpy().view(np.uint16), br.view(np.uint16))
    wd = pkg.kernels.q8_dequant(q, s, b).float().cpu().numpy()
    step = np.repeat(np.abs(sr.astype(np.float32)), 64, axis=1)
    assert np.all(np.abs(wd - w) <= 1.5 * step + 1e-3 * np.abs(w) + 1e-6)
    # a larger layer, and the module built from fp32 weights computes with exactly these arrays
    w2 = np.random.default_rng(8).standard_normal((640, 2560)).astype(np.float32) / 50
    lin = pkg.q8.Q8Linear.from_float(torch.from_numpy(w2))
    qr, sr, br = q8.quantize_f16(w2)
    assert np.array_equal(lin.q.cpu().numpy(), qr)
    assert np.array_equal(lin.scales.cpu().numpy().view(np.uint16), sr.view(np.uint16))
    x = np.random.default_rng(9).standard_normal((238, 2560)).astype(np.float16)
    _check(lin(_t(x)).cpu().numpy(), x, qr, sr, br)
