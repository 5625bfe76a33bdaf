"""One device-memory scratch buffer per GPU, shared by every module of this package.

The kernels' scratch (the triangle update's a, b and x planes, the 8-bit linear's
split-K partials) is live only during one call, so a trunk of many updates, or an
ESMC of many linears, needs one buffer sized for its largest call rather than one
per module (a 6B fold's 68 updates at L=512 would otherwise hold 68 x 201 MB).

Rules:
  * ``get`` returns a 256-byte aligned view of the device's buffer with at least the
    requested bytes, growing the buffer when a call needs more. Every stream that has used
    the buffer is recorded on it (``Tensor.record_stream``), so when a grown buffer replaces
    it the caching allocator keeps the old memory until the work queued on each of those
    streams is done.
  * Calls on one device are ordered through the buffer: when ``get`` is called on a stream
    other than the buffer's last user, that stream first waits for the work already queued on
    the last user (``wait_stream``), so two streams never run their scratch users at once.
    Under HIP-graph capture no wait is recorded (the caller orders the capture).
  * Each ``get`` starts a new generation: a view handed out earlier (``Q8Linear.partials``)
    is valid only until the next ``get`` on that device, which ``check_generation`` tells.
  * A HIP graph that captured calls keeps the buffers they used alive: ``current`` gives
    the buffer to hold next to the graph.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass

import torch

ALIGN = 256
_lock = threading.Lock()


@dataclass
class _Slot:
    buf: torch.Tensor
    stream: torch.cuda.Stream          # the last stream that called get()
    generation: int = 0


_slots: dict[int, _Slot] = {}


def _index(device) -> int:
    d = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    if d.type != "cuda":
        raise ValueError(f"scratch lives in device memory, got {d}")
    return torch.cuda.current_device() if d.index is None else d.index


def get(nbytes: int, device=None) -> torch.Tensor:
    """A uint8 view of ``nbytes`` (>= 1) at a 256-byte aligned address of the device's scratch."""
    idx = _index(device)
    need = max(int(nbytes), 1) + ALIGN
    stream = torch.cuda.current_stream(idx)
    capturing = torch.cuda.is_current_stream_capturing()
    with _lock:
        slot = _slots.get(idx)
        if slot is not None and slot.stream != stream and not capturing:
            stream.wait_stream(slot.stream)  # the previous user's queued work first
        if slot is None or slot.buf.numel() < need:
            # grow geometrically so a slowly rising size does not reallocate every call; the
            # old buffer is freed here, and record_stream has told the allocator who used it
            size = need if slot is None else max(need, slot.buf.numel() + slot.buf.numel() // 4)
            buf = torch.empty(size, dtype=torch.uint8, device=torch.device("cuda", idx))
            slot = _slots[idx] = _Slot(buf, stream, 0 if slot is None else slot.generation)
        elif slot.stream != stream:
            if not capturing:
                slot.buf.record_stream(stream)
            slot.stream = stream
        slot.generation += 1
        buf = slot.buf
    off = (-buf.data_ptr()) % ALIGN
    return buf[off:off + max(int(nbytes), 1)]


def generation(device=None) -> int:
    """How many times the device's scratch has been handed out (0 before the first ``get``)."""
    with _lock:
        slot = _slots.get(_index(device))
        return 0 if slot is None else slot.generation


def check_generation(gen: int, device=None, what: str = "a scratch view") -> None:
    """Raise if the scratch was handed out again since ``gen``: a view from then is overwritten."""
    now = generation(device)
    if now != gen:
        raise RuntimeError(f"{what} is stale: the device scratch was reused ({now - gen} later call(s)) "
                           "before it was consumed")


def current(device=None) -> torch.Tensor | None:
    """The device's scratch buffer now (None before the first ``get``)."""
    with _lock:
        slot = _slots.get(_index(device))
        return None if slot is None else slot.buf


def reserved(device=None) -> int:
    """Bytes held by the device's scratch buffer."""
    b = current(device)
    return 0 if b is None else b.numel()


def release(device=None) -> None:
    """Drop the device's scratch buffer (the next call allocates a new one)."""
    with _lock:
        _slots.pop(_index(device), None)
