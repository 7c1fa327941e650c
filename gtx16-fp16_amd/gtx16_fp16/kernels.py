"""Kernel runtime: entry-point lookup, argument marshalling, streams and split-reduction workspaces.

MI355X counterpart of the reference's NVRTC/cuLaunchKernel runtime (src/gtx16_fp16/kernels.py:253-355).
The kernels are compiled ahead of time for gfx950 into ``libg16.so``; each reference kernel name
maps to one C entry point of that library (``include/g16.h``) that picks its own launch shape and
enqueues on the stream it is given. Nothing is compiled at run time.
"""
from __future__ import annotations

import threading

import torch

from . import _clib

# kernels.py:253 -- M <= 8 takes the skinny path (fp32 math on unquantised activations).
SKINNY_MAX_M = 8

# Reference kernel names (kernels.py:139-250) -> C entry points of libg16.so.
KERNELS = {
    "rowscale_f32": "g16_rowscale_f32",
    "rowscale_f16": "g16_rowscale_f16",
    "hgemm_f32out": "g16_hgemm_f32out",
    "hgemm_f16out": "g16_hgemm_f16out",
    "hgemm_splitk": "g16_hgemm_splitk",
    "skinny_f32in": "g16_skinny_f32in",
    "skinny_f16in": "g16_skinny_f16in",
}


def get_kernel(name: str, device: torch.device | None = None):
    """The bound C entry point replacing reference kernel ``name`` (kernels.py:341-355). The
    library holds code for every device it supports, so ``device`` only exists for signature
    compatibility."""
    del device
    try:
        sym = KERNELS[name]
    except KeyError:
        raise KeyError(f"unknown kernel {name!r}; known: {sorted(KERNELS)}") from None
    return getattr(_clib.load(), sym)


def stream_handle(device_index: int) -> int:
    """Raw handle of torch's current HIP stream on ``device_index`` (kernels.py:294-296)."""
    return torch._C._cuda_getCurrentRawStream(device_index)


def _arg(a):
    if isinstance(a, torch.Tensor):
        return a.data_ptr()
    return a


def launch(kernel, args: list, what: str = "g16 kernel") -> None:
    """Call a C entry point with tensors passed as device pointers and ``None`` as NULL; raise
    ``RuntimeError`` on a nonzero status (kernels.py:299-321)."""
    _clib.check(kernel(*[_arg(a) for a in args]), what)


class PreparedLaunch:
    """A bound entry point whose per-call Python work is only the call itself: for the
    token-by-token FastLinear path (kernels.py:324-338)."""

    __slots__ = ("fn", "what")

    def __init__(self, fn, what: str):
        self.fn = fn
        self.what = what

    def __call__(self, *args) -> None:
        status = self.fn(*args)
        if status != 0:
            _clib.check(status, self.what)


# ---- split-reduction buffers ----------------------------------------------------------------
# The split-K GEMM and the skinny GEMV sum their K slices through two buffers: fp32 partials (no
# initialisation needed) and per-tile arrival counters, which must be zero before first use and
# which every call leaves zero again. One pair is kept per (device, stream) and grown on demand:
# calls on one stream are ordered, so they can share it; calls on different streams get
# different buffers.
#   A buffer that is replaced by a larger one is kept alive, never freed: a HIP graph captured
# while it was current still writes to it on every replay, and if its memory went back to the
# caching allocator, a later tensor could be placed there and overwritten by such a replay.
# Growth doubles the size, so the retired buffers of a key add up to less than its current one.
_ws_lock = threading.Lock()
_partials: dict[tuple[int, int], torch.Tensor] = {}
_counters: dict[tuple[int, int], torch.Tensor] = {}
_scratch: dict[tuple[int, int], torch.Tensor] = {}
_retired: list[torch.Tensor] = []
# (device index, stream) -> (partial bytes, counter bytes, the pointer tuple split_buffers returns):
# the per-call lookup of a stream whose buffers are already large enough
_current: dict[tuple[int, int], tuple] = {}
_MIN_PARTIAL_BYTES = 1 << 20
_MIN_COUNTER_BYTES = 64 << 10
# mm_t's cast scratch is kept per stream up to this size (small GEMMs are bound by host time, and
# an allocation is ~1.3 us of it); larger casts are allocated per call like the reference's
_MAX_CACHED_SCRATCH = 16 << 20


def _grown(table: dict, key, nbytes: int, floor: int, device, zero: bool) -> torch.Tensor:
    buf = table.get(key)
    if buf is None or buf.numel() < nbytes:
        with _ws_lock:
            buf = table.get(key)
            if buf is None or buf.numel() < nbytes:
                size = max(nbytes, floor, 0 if buf is None else 2 * buf.numel())
                if buf is not None:
                    _retired.append(buf)
                # Allocated (and zero-filled) on the current stream, so ordered before the kernels.
                make = torch.zeros if zero else torch.empty
                buf = make(size, dtype=torch.uint8, device=device)
                table[key] = buf
    return buf


def split_buffers(device: torch.device, stream: int, partial_bytes: int, counter_bytes: int):
    """(partials ptr, partials size, counters ptr, counters size) for a split reduction on
    ``stream``; (0, 0, 0, 0) when the call needs none."""
    if partial_bytes <= 0 and counter_bytes <= 0:
        return 0, 0, 0, 0
    key = (device.index or 0, stream)
    hit = _current.get(key)
    if hit is not None and hit[0] >= partial_bytes and hit[1] >= counter_bytes:
        return hit[2]
    part = _grown(_partials, key, partial_bytes, _MIN_PARTIAL_BYTES, device, zero=False)
    cnt = _grown(_counters, key, counter_bytes, _MIN_COUNTER_BYTES, device, zero=True)
    ptrs = (part.data_ptr(), part.numel(), cnt.data_ptr(), cnt.numel())
    _current[key] = (part.numel(), cnt.numel(), ptrs)
    return ptrs


def scratch_buffer(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """A uint8 device buffer of at least ``nbytes`` for the cast of one mm_t call on ``stream``:
    kept per (device, stream) and reused by the next call there (calls on one stream are ordered)
    up to 16 MiB; above that a fresh allocation per call. A buffer that is outgrown stays alive,
    like the split buffers, since a captured graph may still use it."""
    if nbytes > _MAX_CACHED_SCRATCH:
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    key = (device.index or 0, stream)
    buf = _scratch.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = _grown(_scratch, key, nbytes, 1 << 20, device, zero=False)
    return buf


def release_workspaces() -> None:
    """Drop every cached split-reduction buffer, the retired ones included (they are re-created on
    demand). Only safe when no captured HIP graph that used them will be replayed again."""
    with _ws_lock:
        _partials.clear()
        _counters.clear()
        _scratch.clear()
        _current.clear()
        _retired.clear()
