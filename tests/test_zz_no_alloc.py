"""The allocation-free 8-bit linear, q8_linear_noalloc, through the C ABI against the entry
point it mirrors, q8_linear_ws with a caller workspace: the same bits, on two calls in a row
(the second smaller, so it runs in the scratch the first one left behind), for a split-K
shape (the 238 x 10240 -> 2560 ESMC linear) and one that runs unsplit.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(pkg, M, K, N, seed):
    x, q, s, b = pkg.workloads.q8_inputs(M, K, N, seed=seed)
    return tuple(t.to(DEV) for t in (x, q, s, b))


def _noalloc(pkg, lib, x, q, s, b, sb):
    M, K = x.shape
    N = q.shape[0]
    y = torch.empty(M, N, dtype=torch.float16, device=DEV)
    rc = lib.q8_linear_noalloc(x.data_ptr(), q.data_ptr(), s.data_ptr(), b.data_ptr(),
                               None if sb is None else sb.data_ptr(), y.data_ptr(), M, K, N, 64,
                               pkg.capi.stream_ptr())
    assert rc == 0, lib.esm_last_error().decode()
    return y


@pytest.mark.parametrize("shapes", [((238, 10240, 2560), (97, 10240, 2560)), ((238, 2560, 10240), (40, 2560, 640))])
@pytest.mark.parametrize("packed", [True, False])
def test_noalloc_matches_workspace_entry_point(gpu_lib, pkg, shapes, packed):
    lib = pkg.capi.lib()
    K_ = pkg.kernels
    for i, (M, K, N) in enumerate(shapes):
        x, q, s, b = _inputs(pkg, M, K, N, seed=100 * i + M)
        sb = K_.q8_pack_scales(s, b) if packed else None
        ws = K_.q8_workspace(M, K, N, device=DEV)
        y_ws = K_.q8_linear(x, q, s, b, workspace=ws, packed=sb)
        y_na = _noalloc(pkg, lib, x, q, s, b, sb)
        torch.cuda.synchronize()
        assert torch.equal(y_na.view(torch.int16), y_ws.view(torch.int16)), f"call {i}: {M}x{K}->{N}"


def test_noalloc_allocates_nothing(gpu_lib, pkg):
    # after a first call (which loads nothing new), further calls leave torch's device memory
    # untouched except for the outputs the caller allocated
    lib = pkg.capi.lib()
    x, q, s, b = _inputs(pkg, 238, 10240, 2560, seed=7)
    y = torch.empty(238, 2560, dtype=torch.float16, device=DEV)
    args = (x.data_ptr(), q.data_ptr(), s.data_ptr(), b.data_ptr(), None, y.data_ptr(), 238, 10240, 2560, 64)
    assert lib.q8_linear_noalloc(*args, pkg.capi.stream_ptr()) == 0
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    free_before = torch.cuda.mem_get_info()[0]  # the device's own count: sees a hipMalloc too
    for _ in range(3):
        assert lib.q8_linear_noalloc(*args, pkg.capi.stream_ptr()) == 0
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before
    assert torch.cuda.mem_get_info()[0] == free_before
    # argument checks come first, as for the other entry points
    assert lib.q8_linear_noalloc(None, None, None, None, None, None, 4, 128, 64, 64, None) == -1
    assert lib.q8_linear_noalloc(*args[:9], 32, pkg.capi.stream_ptr()) == -4
    bad = ctypes.c_void_p(y.data_ptr() + 2)
    assert lib.q8_linear_noalloc(*args[:5], bad, 238, 10240, 2560, 64, None) == -3


def test_noalloc_captures_into_a_graph(gpu_lib, pkg):
    """Captured with torch's default (global) capture mode, in which an allocation by the
    library would fail the capture; every replay, with eager calls that share the static
    scratch in between, equals the eager result bit for bit."""
    lib = pkg.capi.lib()
    x, q, s, b = _inputs(pkg, 238, 10240, 2560, seed=9)
    x2, q2, s2, b2 = _inputs(pkg, 97, 10240, 2560, seed=10)
    ref = _noalloc(pkg, lib, x, q, s, b, None)
    ref2 = _noalloc(pkg, lib, x2, q2, s2, b2, None)
    torch.cuda.synchronize()
    y = torch.empty(238, 2560, dtype=torch.float16, device=DEV)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = lib.q8_linear_noalloc(x.data_ptr(), q.data_ptr(), s.data_ptr(), b.data_ptr(), None, y.data_ptr(),
                                   238, 10240, 2560, 64, pkg.capi.stream_ptr())
    assert rc == 0, lib.esm_last_error().decode()
    for i in range(3):
        y.zero_()
        g.replay()
        mid = _noalloc(pkg, lib, x2, q2, s2, b2, None)  # eager work on the same scratch between replays
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"replay {i}"
        assert torch.equal(mid.view(torch.int16), ref2.view(torch.int16)), f"eager call after replay {i}"
