"""One device-memory scratch buffer per GPU, shared by every module of this package.

The kernels' scratch (the triangle update's a, b and x planes, the 8-bit linear's
split-K partials) is live only during one call, so a trunk of many updates, or an
ESMC of many linears, needs one buffer sized for its largest call rather than one
per module (a 6B fold's 68 updates at L=512 would otherwise hold 68 x 201 MB).

Rules:
  * ``get`` returns a 256-byte aligned view of the device's buffer with at least the
    requested bytes, growing the buffer when a call needs more; a buffer that is
    replaced is dropped, and torch's stream-ordered allocator keeps its memory until
    the work already queued on it is done.
  * Calls that use the scratch on one device must be ordered: one stream, or streams the
    caller synchronises. Two calls that overlap in time would share the bytes.
  * A HIP graph that captured calls keeps the buffers they used alive: ``current`` gives
    the buffer to hold next to the graph.
"""

from __future__ import annotations

import threading

import torch

ALIGN = 256
_lock = threading.Lock()
_bufs: dict[int, torch.Tensor] = {}


def _index(device) -> int:
    d = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    if d.type != "cuda":
        raise ValueError(f"scratch lives in device memory, got {d}")
    return torch.cuda.current_device() if d.index is None else d.index


def get(nbytes: int, device=None) -> torch.Tensor:
    """A uint8 view of ``nbytes`` (>= 1) at a 256-byte aligned address of the device's scratch."""
    idx = _index(device)
    need = max(int(nbytes), 1) + ALIGN
    with _lock:
        buf = _bufs.get(idx)
        if buf is None or buf.numel() < need:
            # grow geometrically so a slowly rising size does not reallocate every call
            size = need if buf is None else max(need, buf.numel() + buf.numel() // 4)
            buf = _bufs[idx] = torch.empty(size, dtype=torch.uint8, device=torch.device("cuda", idx))
    off = (-buf.data_ptr()) % ALIGN
    return buf[off:off + max(int(nbytes), 1)]


def current(device=None) -> torch.Tensor | None:
    """The device's scratch buffer now (None before the first ``get``)."""
    with _lock:
        return _bufs.get(_index(device))


def reserved(device=None) -> int:
    """Bytes held by the device's scratch buffer."""
    b = current(device)
    return 0 if b is None else b.numel()


def release(device=None) -> None:
    """Drop the device's scratch buffer (the next call allocates a new one)."""
    with _lock:
        _bufs.pop(_index(device), None)
