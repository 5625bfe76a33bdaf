"""ctypes binding of libesmfold2_amd.so (the C ABI declared in include/esmfold2_amd.h).

There is no fallback: if the library is missing, fails to load, or no GPU is
present when one is required, this raises. Every wrapper checks the return code
and raises ``EsmError`` with the library's message.
"""

from __future__ import annotations

import ctypes
import os
import sys
import threading

from . import build as _build

_vp, _int, _f32, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/esmfold2_amd.h
SIGNATURES = {
    "esm_last_error": (ctypes.c_char_p, []),
    "esm_version": (ctypes.c_char_p, []),
    "esm_source_hash": (ctypes.c_char_p, []),
    "esm_timing_begin": (_int, [_int]),
    "esm_timing_end": (_int, [_vp, _int, _vp]),
    "esm_timing_name": (ctypes.c_char_p, [_int]),
    "tmu_workspace_bytes": (_sz, [_int, _int, _int]),
    "tmu_leading_dim": (_int, [_int]),
    "tmu_project": (_int, [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _int, _int, _int, _int, _int, _int, _vp]),
    "tmu_contract": (_int, [_vp, _vp, _vp, _int, _int, _int, _int, _f32, _vp]),
    "tmu_frag_plane_elems": (_sz, [_int]),
    "tmu_project_frag": (_int, [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _int, _int, _int, _int, _int, _vp]),
    "tmu_contract_frag": (_int, [_vp, _vp, _vp, _int, _int, _int, _f32, _vp]),
    "tmu_epilogue": (_int, [_vp, _int, _vp, _vp, _vp, _vp, _f32, _vp, _vp, _f32, _vp, _vp, _vp, _int, _int, _int,
                            _int, _int, _int, _vp]),
    "tmu_forward": (_int, [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _int, _int, _int,
                           _int, _int, _int, _int, _vp]),
    "tmu_pair_forward": (_int, [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _f32, _vp, _vp, _int,
                                _vp, _vp, _f32, _vp, _vp, _vp, _f32, _vp, _vp, _int,
                                _vp, _vp, _int, _int, _int, _int, _vp]),
    "tmu_forward_ws": (_int, [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _sz, _int, _int,
                              _int, _int, _int, _int, _int, _vp]),
    "tmu_pair_forward_ws": (_int, [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _f32, _vp, _vp, _int,
                                   _vp, _vp, _f32, _vp, _vp, _vp, _f32, _vp, _vp, _int,
                                   _vp, _vp, _sz, _int, _int, _int, _int, _vp]),
    "pair_transition": (_int, [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _int, _int, _int, _int, _vp]),
    "pair_transition_ws": (_int, [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _int, _int, _int, _int, _vp, _sz, _vp]),
    "pair_transition_workspace_bytes": (_sz, [_int, _int, _int, _int, _int]),
    "esmc_layer_norm": (_int, [_vp, _vp, _f32, _vp, _vp, _vp, _f32, _vp, _vp, _int, _int, _vp]),
    "esmc_layer_norm_parts": (_int, [_vp, _vp, _int, _f32, _vp, _vp, _vp, _f32, _vp, _vp, _int, _int, _vp]),
    "esmc_qk_rope": (_int, [_vp, _vp, _vp, _f32, _vp, _vp, _vp, _int, _int, _int, _int, _f32, _vp]),
    "esmc_attention": (_int, [_vp, _vp, _vp, _vp, _vp, _int, _int, _int, _int, _f32, _vp]),
    "esmc_swiglu": (_int, [_vp, _vp, _int, _int, _vp]),
    "parcae_step": (_int, [_vp, _vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _int, _int, _int, _vp]),
    "distogram_expected_distance": (_int, [_vp, _vp, _vp, _vp, _vp, _int, _int, _int, _int, _vp]),
    "abs_diff_quantile": (_int, [_vp, _vp, _sz, _f32, _vp, _vp]),
    "q8_linear": (_int, [_vp, _vp, _vp, _vp, _vp, _int, _int, _int, _int, _vp]),
    "q8_linear_ws": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _int, _int, _int, _int, _vp, _sz, _vp]),
    "q8_linear_noalloc": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _int, _int, _int, _int, _vp]),
    "q8_linear_workspace_bytes": (_sz, [_int, _int, _int]),
    "q8_linear_partials_bytes": (_sz, [_int, _int, _int]),
    "q8_tile_rows": (_int, [_int, _int, _int]),
    "q8_set_tile_rows": (_int, [_int]),
    "q8_linear_partials": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _int, _int, _int, _int, _vp]),
    "q8_packed_scales_bytes": (_sz, [_int, _int]),
    "q8_pack_scales": (_int, [_vp, _vp, _vp, _int, _int, _int, _vp]),
    "q8_packed_codes_bytes": (_sz, [_int, _int]),
    "q8_pack_codes": (_int, [_vp, _vp, _int, _int, _int, _vp]),
    "q8_linear_packed_ws": (_int, [_vp, _vp, _vp, _vp, _int, _int, _int, _int, _vp, _sz, _vp]),
    "q8_linear_packed_partials": (_int, [_vp, _vp, _vp, _vp, _sz, _vp, _int, _int, _int, _int, _vp]),
    "q8_linear_swiglu_packed_ws": (_int, [_vp, _vp, _vp, _vp, _int, _int, _int, _int, _vp, _sz, _vp]),
    "q8_dequant": (_int, [_vp, _vp, _vp, _vp, _int, _int, _int, _vp]),
    "q8_quantize": (_int, [_vp, _vp, _vp, _vp, _int, _int, _int, _vp]),
}

ERRORS = {-1: "ESM_ERR_NULL", -2: "ESM_ERR_SHAPE", -3: "ESM_ERR_ALIGN", -4: "ESM_ERR_UNSUPPORTED",
          -5: "ESM_ERR_DEVICE"}


class EsmError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{ERRORS.get(code, f'hipError {code}')}] {msg}")
        self.code = code


_lock = threading.Lock()
_lib = None
_gpu_ok = False


def lib_path() -> str:
    return _build.LIB_PATH


def _load() -> ctypes.CDLL:
    """Load the in-tree library, building it first when it is missing or was compiled from other
    sources than the ones beside it (compared by content hash, so copies keep their state)."""
    if not _build.up_to_date():
        stale = os.path.exists(_build.LIB_PATH)
        if stale:
            print(f"[esmfold2_amd] {_build.LIB_PATH} was built from other sources: rebuilding", file=sys.stderr,
                  flush=True)
        _build.build(force=True)
    handle = ctypes.CDLL(_build.LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)  # AttributeError if a declared symbol is missing
        fn.restype, fn.argtypes = res, args
    if handle.esm_source_hash().decode() != _build.source_hash():
        raise EsmError(-5, f"{_build.LIB_PATH} does not match its sources after the build")
    return handle


def lib(reload: bool = False, require_gpu: bool = True) -> ctypes.CDLL:
    """The loaded library (built on first use when missing or stale). With ``require_gpu`` the
    first call checks that a ROCm GPU is visible; later calls return the cached handle."""
    global _lib, _gpu_ok
    h = _lib
    if h is not None and not reload and (_gpu_ok or not require_gpu):
        return h
    with _lock:
        if _lib is None or reload:
            _lib = _load()
        if require_gpu and not _gpu_ok:
            import torch
            if not torch.cuda.is_available():
                raise EsmError(-5, "no ROCm GPU visible: the HIP path has no CPU fallback")
            _gpu_ok = True
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise EsmError(rc, _lib.esm_last_error().decode())


def stream_ptr(stream=None) -> int:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


class KernelTimes:
    """Kernel durations stamped by the runtime (``esm_timing_begin`` / ``esm_timing_end``):

        with capi.KernelTimes(max_launches) as kt:
            ...launches through this library...
        kt.records  # [(kernel name, microseconds)] in launch order

    Each timed launch carries start/stop events that the runtime stamps with the kernel's own
    begin and end, so the figures are a profiler's kernel-trace durations, measured live."""

    def __init__(self, max_launches: int):
        self.max_launches = int(max_launches)
        self.records: list[tuple[str, float]] = []

    def __enter__(self):
        check(lib().esm_timing_begin(self.max_launches))
        return self

    def __exit__(self, *exc):
        h = lib()
        us = (ctypes.c_float * max(self.max_launches, 1))()
        n = ctypes.c_int(0)
        rc = h.esm_timing_end(us, self.max_launches, ctypes.byref(n))
        if exc[0] is None:
            check(rc)
        self.records = [(h.esm_timing_name(i).decode(), float(us[i])) for i in range(n.value)]
        return False

    def by_kernel(self) -> dict[str, list[float]]:
        out: dict[str, list[float]] = {}
        for name, t in self.records:
            out.setdefault(name, []).append(t)
        return out
