"""CPU tests of the C ABI: the library loads, exports every declared symbol, and
rejects bad arguments before launching anything (no GPU needed for these paths)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "esmfold2_amd.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*([a-z_0-9]+)\s*\(", src, flags=re.M)))


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg.capi.lib(require_gpu=False)


def test_header_declares_the_entry_points():
    names = declared_functions()
    for n in ("tmu_project", "tmu_contract", "tmu_epilogue", "tmu_forward", "q8_linear", "q8_linear_ws",
              "q8_linear_workspace_bytes", "q8_pack_scales", "q8_packed_scales_bytes",
              "pair_transition", "q8_dequant", "esm_last_error", "esm_version", "tmu_workspace_bytes", "tmu_leading_dim",
              "tmu_pair_forward"):
        assert n in names


def test_every_declared_symbol_is_exported_and_bound(pkg, lib):
    handle = ctypes.CDLL(pkg.capi.lib_path())
    for name in declared_functions():
        assert hasattr(handle, name), f"{name} declared in the header but not exported"
        assert name in pkg.capi.SIGNATURES, f"{name} has no ctypes signature"
    assert set(pkg.capi.SIGNATURES) == set(declared_functions())


def test_version_and_sizes(lib):
    assert b"gfx950" in lib.esm_version()
    assert lib.tmu_leading_dim(238) == 240 and lib.tmu_leading_dim(240) == 240 and lib.tmu_leading_dim(1) == 8
    # 3 planes, each B*c times the larger of L*ld and the fragment layout's rbn*kbn*512
    # halfs (L=238: 8 x 15 tiles of 32 rows x 16 k), fp16, rounded to 256 bytes
    plane = 1 * 128 * max(238 * 240, 8 * 15 * 512) * 2
    assert lib.tmu_workspace_bytes(1, 238, 128) == 3 * ((plane + 255) // 256 * 256)
    assert lib.tmu_workspace_bytes(1, 256, 128) == 3 * 128 * 256 * 256 * 2   # both layouts 256 x 256
    assert lib.tmu_workspace_bytes(0, 238, 128) == 0


def _err(lib):
    return lib.esm_last_error().decode()


def test_rejects_unsupported_channels(lib):
    rc = lib.tmu_project(None, None, None, None, 1e-5, None, None, None, 1, 8, 256, 256, 8, 0, None)
    assert rc == -4 and "supported" in _err(lib)
    rc = lib.tmu_forward(*([None] * 4), 1e-5, None, None, None, 1e-5, None, None, None, None, 1, 8, 64, 64, 1, 0, 0,
                         None)
    assert rc == -4
    # the wide path needs C = c (the reference's TMU has c = C)
    rc = lib.tmu_forward(*([None] * 4), 1e-5, None, None, None, 1e-5, None, None, None, None, 1, 8, 256, 128, 1, 0,
                         0, None)
    assert rc == -4
    rc = lib.tmu_forward(*([None] * 4), 1e-5, None, None, None, 1e-5, None, None, None, None, 1, 8, 256, 256, 1, 0,
                         0, None)
    assert rc == -1


def test_rejects_null_and_bad_shapes(lib):
    assert lib.tmu_project(None, None, None, None, 1e-5, None, None, None, 1, 8, 128, 128, 8, 0, None) == -1
    assert lib.tmu_contract(None, None, None, 4, 8, 8, 8, 1.0, None) == -1
    assert lib.tmu_contract(None, None, None, -1, 8, 8, 8, 1.0, None) == -2
    assert lib.q8_linear(None, None, None, None, None, 4, 100, 64, 64, None) == -2  # K % 64
    assert lib.q8_linear(None, None, None, None, None, 4, 128, 64, 32, None) == -4  # group 32
    assert lib.q8_dequant(None, None, None, None, 64, 64, 64, None) == -1
    assert lib.q8_linear_ws(None, None, None, None, None, None, 5, 1024, 64, 64, None, 0, None) == -1
    assert lib.pair_transition(None, None, None, None, 1e-5, None, None, None, 1, 8, 128, 512, None) == -1
    # widths the wide path does not cover: C not a multiple of 128 (or above 512), H not of 32
    assert lib.pair_transition(None, None, None, None, 1e-5, None, None, None, 1, 8, 192, 512, None) == -4
    assert lib.pair_transition(None, None, None, None, 1e-5, None, None, None, 1, 8, 640, 512, None) == -4
    assert lib.pair_transition(None, None, None, None, 1e-5, None, ctypes.c_void_p(4096), None, 1, 8, 256, 100,
                               None) == -4
    # 256 wide, or SwiGLU at H = 512: supported through the wide path (NULL pointers checked)
    assert lib.pair_transition(None, None, None, None, 1e-5, None, None, None, 1, 8, 256, 512, None) == -1
    assert lib.pair_transition_ws(None, None, None, None, 1e-5, None, ctypes.c_void_p(4096), None, 1, 8, 128, 512,
                                  None, 0, None) == -1
    assert lib.pair_transition_workspace_bytes(1, 8, 128, 512, 0) == 0       # the register-resident kernel
    assert lib.pair_transition_workspace_bytes(1, 8, 128, 512, 1) == 2 * 8 * 8 * 128 + 2 * 8 * 8 * 512
    assert lib.tmu_workspace_bytes(1, 8, 256) == 4 * 256 * 512 * 2  # a, b, x and LN_in(z); one fragment tile
    assert lib.pair_transition(None, None, None, None, 1e-5, None, None, None, 0, 8, 128, 512, None) == 0
    # the partials entry points: a NULL split count, a short buffer, a bad split count
    assert lib.q8_linear_partials(None, None, None, None, None, None, 0, None, 4, 128, 64, 64, None) == -1
    splits = ctypes.c_int(7)
    assert lib.q8_linear_partials(fake16 := ctypes.c_void_p(4096), fake16, fake16, fake16, None,
                                  ctypes.c_void_p(1 << 20), 16, ctypes.byref(splits), 5, 1024, 64, 64, None) == -2
    assert splits.value == 0 and "partials" in _err(lib)
    assert lib.q8_linear_partials_bytes(5, 1024, 64) >= 5 * 64 * 4 and lib.q8_linear_partials_bytes(5, 100, 64) == 0
    assert lib.esmc_layer_norm_parts(fake16, fake16, 0, 1.0, fake16, fake16, None, 1e-5, fake16, None, 4, 64,
                                     None) == -2
    assert lib.esmc_layer_norm_parts(fake16, None, 2, 1.0, fake16, fake16, None, 1e-5, fake16, None, 4, 64,
                                     None) == -1
    # a negative or NaN eps is refused by every LayerNorm entry point, before any pointer is used
    for eps in (-1e-5, float("nan")):
        assert lib.pair_transition(None, None, None, None, eps, None, None, None, 1, 8, 128, 512, None) == -2
        assert lib.esmc_layer_norm(None, None, 0.0, None, None, None, eps, None, None, 4, 64, None) == -2
        assert lib.esmc_qk_rope(None, None, None, eps, None, None, None, 1, 8, 4, 64, 10000.0, None) == -2
        assert lib.parcae_step(*([None] * 5), eps, None, None, None, 1, 8, 128, None) == -2
        assert "eps" in _err(lib)
    assert lib.q8_pack_scales(None, None, None, 64, 128, 64, None) == -1
    assert lib.q8_pack_scales(None, None, None, 64, 100, 64, None) == -2
    # per 32-row block and 64-group, 32 words
    assert lib.q8_packed_scales_bytes(64, 128) == 2 * 2 * 32 * 4 and lib.q8_packed_scales_bytes(161, 64) == 6 * 32 * 4
    # split-K workspace: too small, then misaligned (both rejected before any launch)
    need = lib.q8_linear_workspace_bytes(5, 1024, 64)
    assert need > 0 and lib.q8_linear_workspace_bytes(238, 2560, 10240) == 0
    assert lib.q8_linear_workspace_bytes(5, 100, 64) == 0  # unsupported K
    ws = ctypes.c_void_p(1 << 20)
    assert lib.q8_linear_ws(fake16 := ctypes.c_void_p(4096), fake16, fake16, fake16, None, fake16, 5, 1024, 64, 64,
                            ws, need - 1, None) == -2
    assert "workspace" in _err(lib)
    assert lib.q8_linear_ws(fake16, fake16, fake16, fake16, None, fake16, 5, 1024, 64, 64,
                            ctypes.c_void_p((1 << 20) + 16), need, None) == -3
    # misaligned leading dimension (not a multiple of 8): checked before any pointer is used
    fake = ctypes.c_void_p(4096)
    assert lib.tmu_contract(fake, fake, fake, 1, 10, 12, 16, 1.0, None) == -2
    assert "multiples of 8" in _err(lib)
    # x columns past roundup(L, 64) would never be written: refused
    assert lib.tmu_contract(fake, fake, fake, 1, 8, 8, 136, 1.0, None) == -2
    assert "ldx <= 64" in _err(lib)
    # misaligned pointers
    odd = ctypes.c_void_p(4096 + 2)
    assert lib.tmu_contract(odd, fake, fake, 1, 10, 16, 16, 1.0, None) == -3


def test_packed_codes_entry_points_validate(lib):
    # sizes: per 32-row block and step of two 64-groups, 4 chunks of 1 KB
    assert lib.q8_packed_codes_bytes(160, 128) == 5 * 4096
    assert lib.q8_packed_codes_bytes(161, 192) == 6 * 2 * 4096  # 3 groups -> 2 steps, 6 blocks
    assert lib.q8_packed_codes_bytes(64, 100) == 0 and lib.q8_packed_codes_bytes(0, 64) == 0
    assert lib.q8_pack_codes(None, None, 64, 128, 64, None) == -1
    assert lib.q8_pack_codes(None, None, 64, 128, 32, None) == -4
    assert lib.q8_pack_codes(None, None, 64, 100, 64, None) == -2
    assert lib.q8_pack_codes(None, None, 0, 128, 64, None) == 0  # empty: a no-op
    fake = ctypes.c_void_p(4096)
    assert lib.q8_pack_codes(ctypes.c_void_p(4096 + 4), fake, 64, 128, 64, None) == -3  # q not 8-byte aligned
    # the GEMM: packed codes and packed scales are both required; q, s, b are not read
    assert lib.q8_linear_packed_ws(fake, None, fake, fake, 5, 1024, 64, 64, None, 0, None) == -1
    assert "packed codes" in _err(lib)
    assert lib.q8_linear_packed_ws(fake, fake, None, fake, 5, 1024, 64, 64, None, 0, None) == -1
    assert lib.q8_linear_packed_ws(fake, ctypes.c_void_p(4096 + 8), fake, fake, 5, 1024, 64, 64, None, 0, None) == -3
    assert lib.q8_linear_packed_ws(fake, fake, fake, fake, 5, 1024, 64, 32, None, 0, None) == -4
    need = lib.q8_linear_workspace_bytes(5, 1024, 64)
    assert lib.q8_linear_packed_ws(fake, fake, fake, fake, 5, 1024, 64, 64, ctypes.c_void_p(1 << 20), need - 1,
                                   None) == -2
    splits = ctypes.c_int(3)
    assert lib.q8_linear_packed_partials(fake, fake, fake, fake, 16, ctypes.byref(splits), 5, 1024, 64, 64,
                                         None) == -2
    assert splits.value == 0
    assert lib.q8_linear_packed_partials(fake, fake, fake, fake, 1 << 20, None, 5, 1024, 64, 64, None) == -1


def test_swiglu_pair_rows_and_checks(pkg, lib):
    perm = pkg.kernels.swiglu_pair_rows(320)
    # tile 0: gate rows 0..79 then up rows 160..239; tile 1: gate 80..159 then up 240..319
    assert perm[:80].tolist() == list(range(80)) and perm[80:160].tolist() == list(range(160, 240))
    assert perm[160:240].tolist() == list(range(80, 160)) and perm[240:].tolist() == list(range(240, 320))
    assert sorted(perm.tolist()) == list(range(320))
    fake = ctypes.c_void_p(4096)
    assert lib.q8_linear_swiglu_packed_ws(fake, None, fake, fake, 5, 128, 320, 64, None, 0, None) == -1
    assert lib.q8_linear_swiglu_packed_ws(fake, fake, fake, fake, 5, 128, 192, 64, None, 0, None) == -2
    assert "multiple of 160" in _err(lib)


def test_pair_forward_validates_before_launching(lib):
    f, ws = ctypes.c_void_p(4096), ctypes.c_void_p(1 << 20)

    def pair(z=f, mask=None, workspace=ws, B=1, L=8, C=128, c=128, o_mask=0, i_mask=0, eps=1e-5, out=f, i_w=f):
        o = [f, f, eps, f, f, f, eps, f, f, o_mask]
        i = [f, f, eps, i_w, f, f, eps, f, f, i_mask]
        return lib.tmu_pair_forward(z, mask, *o, *i, out, workspace, B, L, C, c, None)

    assert pair(C=192, c=192) == -4 and pair(C=256, c=128) == -4
    assert pair(C=256, c=256, z=None) == -1
    assert pair(B=0) == 0 and pair(L=0) == 0
    assert pair(z=None) == -1 and pair(workspace=None) == -1
    assert pair(workspace=ctypes.c_void_p((1 << 20) + 16)) == -3
    assert pair(o_mask=1) == -1 and "mask" in _err(lib)
    assert pair(i_mask=1) == -1                     # the incoming update's arguments: before any launch
    assert pair(i_w=None) == -1 and pair(i_w=ctypes.c_void_p(4096 + 2)) == -3
    assert pair(eps=-1.0) == -2 and pair(eps=float("nan")) == -2
    assert pair(L=5000) == -2
    assert pair(z=ctypes.c_void_p(4096 + 2)) == -3
    assert pair(B=600) == -2                        # B * c beyond the contraction's grid


def test_sized_forward_refuses_a_small_workspace(lib):
    f, ws = ctypes.c_void_p(4096), ctypes.c_void_p(1 << 20)
    o = [f, f, 1e-5, f, f, f, 1e-5, f, f, 0]

    def fwd(nbytes, B=1, L=8, C=128, c=128):
        return lib.tmu_forward_ws(f, None, f, f, 1e-5, f, f, f, 1e-5, f, f, f, ws, nbytes, B, L, C, c, 1, 1, 0, None)

    def pair(nbytes, B=1, L=8, C=128, c=128):
        return lib.tmu_pair_forward_ws(f, None, *o, *o, f, ws, nbytes, B, L, C, c, None)

    for call in (fwd, pair):
        need = lib.tmu_workspace_bytes(2, 40, 256)
        assert call(need - 1, B=2, L=40, C=256, c=256) == -2 and "workspace" in _err(lib)
        # a buffer sized for c = 128 is too small for the 256-wide path
        assert call(lib.tmu_workspace_bytes(2, 40, 128), B=2, L=40, C=256, c=256) == -2
        # empty and unsupported shapes keep the unsized forms' answers
        assert call(0, B=0) == 0 and call(0, L=0) == 0
        assert call(1 << 40, C=192, c=192) == -4


def test_library_matches_its_sources(pkg):
    # the in-tree library carries the content hash of the sources it was compiled from
    lib = pkg.capi.lib(require_gpu=False)
    assert lib.esm_source_hash().decode() == pkg.build.source_hash() == pkg.build.library_hash()
    assert pkg.build.up_to_date()


def test_empty_inputs_are_a_no_op(lib):
    assert lib.tmu_project(None, None, None, None, 1e-5, None, None, None, 0, 0, 128, 128, 0, 0, None) == 0
    assert lib.tmu_contract(None, None, None, 0, 0, 0, 0, 1.0, None) == 0
    assert lib.q8_linear(None, None, None, None, None, 0, 64, 64, 64, None) == 0
    assert _err(lib) == ""


def test_python_wrappers_refuse_cpu_tensors(pkg):
    import torch
    from oracle import tmu
    p = tmu.draw_weights(torch.Generator().manual_seed(0), 128, 128, True)
    with pytest.raises(Exception):
        pkg.trimul.TriMul.from_weights(p, device="cpu")(torch.zeros(1, 4, 4, 128))


def test_q8_tile_rows_plan_and_override(lib):
    # without a GPU the plan assumes 256 CUs: 4 m-tiles x 60 (128 rows) fit one round; 4 x 80 take
    # two where 4 x 64 (160 rows) take one; tiny shapes take 128
    assert lib.q8_tile_rows(238, 2560, 7680) == 128 and lib.q8_tile_rows(238, 2560, 10240) == 160
    assert lib.q8_tile_rows(7, 64, 64) == 128
    # split K: 7 steps per workgroup in 3 splits (128 rows) against 5 in 4 (160 rows) and one
    # split's partials less to write and read: 128; at K = 5120 (14 against 10) and K = 10240
    # (27 against 20) the steps outweigh the partials: 160
    assert lib.q8_tile_rows(238, 2560, 2560) == 128
    assert lib.q8_tile_rows(238, 5120, 2560) == 160 and lib.q8_tile_rows(238, 10240, 2560) == 160
    # 16 m-tiles: 960 narrow (4 rounds) against 768 wide (3 rounds): 3 x 10 <= 4 x 9 -> 160
    assert lib.q8_tile_rows(1024, 2560, 7680) == 160
    assert lib.q8_tile_rows(0, 64, 64) == 0
    assert lib.q8_set_tile_rows(96) == -2 and "q8_set_tile_rows" in _err(lib)
    try:
        assert lib.q8_set_tile_rows(160) == 0 and lib.q8_tile_rows(238, 2560, 7680) == 160
        assert lib.q8_set_tile_rows(128) == 0 and lib.q8_tile_rows(238, 2560, 10240) == 128
    finally:
        assert lib.q8_set_tile_rows(0) == 0
    assert lib.q8_tile_rows(238, 2560, 10240) == 160
    # the workspace covers the SwiGLU plan too (160-row tiles: more K splits at small M)
    assert lib.q8_linear_workspace_bytes(50, 2560, 10240) == 4 * 50 * 10240 * 4
