"""Kernel runtime: entry-point lookup, argument marshalling, streams and split-reduction workspaces.

MI355X counterpart of the reference's NVRTC/cuLaunchKernel runtime (src/gtx16_fp16/kernels.py:253-355).
The kernels are compiled ahead of time for gfx950 into ``libg16.so``; each reference kernel name
maps to one C entry point of that library (``include/g16.h``) that picks its own launch shape and
enqueues on the stream it is given. Nothing is compiled at run time.
"""
from __future__ import annotations

import contextlib
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


class Kernel:
    """A reference kernel (kernels.py:139-250) bound to the library entry point that replaces it.
    ``launch`` and ``PreparedLaunch`` take it with the reference's grid, block and argument list;
    calling it directly calls the entry point with the C ABI's own arguments (``include/g16.h``)."""

    __slots__ = ("name", "fn", "device_index")

    def __init__(self, name: str, fn, device_index: int | None):
        self.name = name
        self.fn = fn
        self.device_index = device_index

    def __call__(self, *args):
        return self.fn(*args)

    def __repr__(self) -> str:
        return f"Kernel({self.name!r} -> {KERNELS[self.name]}, device={self.device_index})"


_kernels: dict[tuple[str, int | None], Kernel] = {}


def get_kernel(name: str, device: torch.device | int | None = None) -> Kernel:
    """The reference kernel ``name`` (kernels.py:341-355) on ``device``: the library holds code for
    every device it supports, so nothing is compiled; the device only keys the split buffers of
    the launches that need them (the current device at launch time when None)."""
    if name not in KERNELS:
        raise KeyError(f"unknown kernel {name!r}; known: {sorted(KERNELS)}")
    idx = None if device is None else (torch.device(device).index or 0)
    k = _kernels.get((name, idx))
    if k is None:
        k = _kernels[(name, idx)] = Kernel(name, getattr(_clib.load(), KERNELS[name]), idx)
    return k


def stream_handle(device_index: int) -> int:
    """Raw handle of torch's current HIP stream on ``device_index`` (kernels.py:294-296)."""
    return torch._C._cuda_getCurrentRawStream(device_index)


def _arg(a):
    if isinstance(a, torch.Tensor):
        return a.data_ptr()
    return a


def call(fn, args: list, what: str = "g16 kernel") -> None:
    """Call a C entry point with tensors passed as device pointers and ``None`` as NULL; raise
    ``RuntimeError`` on a nonzero status (kernels.py:299-302)."""
    _clib.check(fn(*[_arg(a) for a in args]), what)


class PreparedCall:
    """A bound entry point whose per-call Python work is only the call itself, for the
    token-by-token FastLinear path; raises ``RuntimeError`` on a nonzero status."""

    __slots__ = ("fn", "what")

    def __init__(self, fn, what: str):
        self.fn = fn
        self.what = what

    def __call__(self, *args) -> None:
        status = self.fn(*args)
        if status != 0:
            _clib.check(status, self.what)


# ---- the reference's launch interface (kernels.py:299-338) --------------------------------------
# The reference launches its seven kernels with an explicit grid and block and the kernel's own
# parameter list. Here each entry point plans its own launch shape, so grid and block are read
# only for the sizes the reference passes through them (the rowscale kernel's row count, the
# split count of the split-K and skinny kernels); the block is not used. Per kernel, the reference
# arguments and what the call computes:
#   rowscale_f32/_f16 [X, Y, S, K, thresh], grid (M, 1, 1): the same cast bits as the reference.
#   hgemm_f32out/_f16out [A, B, C, bias, rscale, M, N, K]: C = rscale * (A @ B) + bias.
#   hgemm_splitk [A, B, C, rscale, M, N, K, kchunk], grid z = slices: C += rscale * (A @ B), as the
#     reference's fp32 atomics add into its prefilled C; the slices are summed in a fixed order
#     into a temporary, which is then added to C (C must be a tensor).
#   skinny_f32in/_f16in [A, B, C, bias, M, N, K, kchunk], grid y = slices: C = A @ B + bias. The
#     reference adds into C and requires it zeroed (kernels.py:158); the result on a zeroed C is
#     the same, and here C needs no zero-fill.
_cus: dict[int, int] = {}


def _num_cus(idx: int) -> int:
    n = _cus.get(idx)
    if n is None:
        n = _cus[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return n


def _device_index(kernel: Kernel, args) -> int:
    if kernel.device_index is not None:
        return kernel.device_index
    for a in args:
        if isinstance(a, torch.Tensor) and a.is_cuda:
            return a.device.index or 0
    return torch.cuda.current_device()


def _slices(K: int, kchunk: int, grid_slices: int) -> int:
    if K <= 0:
        return 1
    return max(1, -(-K // kchunk)) if kchunk > 0 else max(1, grid_slices)


def _run(kernel: Kernel, grid, args: list, stream: int) -> None:
    name, fn = kernel.name, kernel.fn
    what = f"{name} ({KERNELS[name]})"
    if name.startswith("rowscale"):
        X, Y, S, K, thresh = args
        _clib.check(fn(_arg(X), _arg(Y), _arg(S), int(grid[0]), int(K), float(thresh), stream), what)
    elif name in ("hgemm_f32out", "hgemm_f16out"):
        A, B, C, bias, rscale, M, N, K = args
        _clib.check(fn(_arg(A), _arg(B), _arg(C), _arg(bias), _arg(rscale), int(M), int(N), int(K), stream), what)
    elif name.startswith("skinny"):
        A, B, C, bias, M, N, K, kchunk = args
        M, N, K = int(M), int(N), int(K)
        ks = _slices(K, int(kchunk), int(grid[1]))
        lib = _clib.load()
        dev = torch.device("cuda", _device_index(kernel, args))
        ws = split_buffers(dev, stream, lib.g16_skinny_workspace_bytes(M, N, K, ks),
                           lib.g16_skinny_counter_bytes(M, N, K, ks))
        _clib.check(fn(_arg(A), _arg(B), _arg(C), _arg(bias), M, N, K, ks, *ws, stream), what)
    elif name == "hgemm_splitk":
        A, B, C, rscale, M, N, K, kchunk = args
        if not isinstance(C, torch.Tensor) or C.dtype != torch.float32:
            raise TypeError("hgemm_splitk adds into C: pass C as an fp32 tensor (through launch())")
        M, N, K = int(M), int(N), int(K)
        ks = _slices(K, int(kchunk), int(grid[2]))
        lib = _clib.load()
        idx = _device_index(kernel, args)
        dev = torch.device("cuda", idx)
        cus = _num_cus(idx)
        ws = split_buffers(dev, stream, lib.g16_hgemm_splitk_workspace_bytes(M, N, K, ks, cus),
                           lib.g16_hgemm_splitk_counter_bytes(M, N, K, ks, cus))
        # the temporary and the addition run on the launch's stream, after the GEMM
        on = (contextlib.nullcontext() if stream == stream_handle(idx)
              else torch.cuda.stream(torch.cuda.ExternalStream(stream, device=dev)))
        with on:
            tmp = torch.empty(M, N, device=dev, dtype=torch.float32)
            _clib.check(fn(_arg(A), _arg(B), tmp.data_ptr(), 0, None, _arg(rscale), M, N, K, ks, cus, *ws, stream),
                        what)
            C.view(M, N).add_(tmp)
    else:  # pragma: no cover - KERNELS and this dispatch list the same seven names
        raise KeyError(name)


def launch(kernel: Kernel, grid: tuple[int, int, int], block: tuple[int, int, int], args: list, stream: int) -> None:
    """The reference's launch (kernels.py:315-321): ``kernel`` from ``get_kernel``, its grid and
    block, its argument list (tensors, None for NULL, ints, floats) and a raw stream handle
    (``stream_handle``). Raises ``RuntimeError`` when the entry point returns a nonzero status."""
    del block
    _run(kernel, grid, list(args), stream)


class PreparedLaunch:
    """The reference's prepared launch (kernels.py:324-338): built once with the kernel, grid,
    block and one character per argument ('p' pointer, 'i' int32, 'f' float32); each call passes
    the stream handle and the argument values (pointers as ints or None)."""

    __slots__ = ("kernel", "grid", "block", "kinds")

    def __init__(self, kernel: Kernel, grid, block, kinds: str):
        if len(kinds) != _ARITY[kernel.name] or set(kinds) - {"p", "i", "f"}:
            raise ValueError(f"{kernel.name} takes {_ARITY[kernel.name]} arguments, kinds {kinds!r}")
        if kernel.name == "hgemm_splitk":
            raise TypeError("hgemm_splitk adds into C: launch it through launch() with C as a tensor")
        self.kernel, self.grid, self.block, self.kinds = kernel, grid, block, kinds

    def __call__(self, stream: int, *args) -> None:
        _run(self.kernel, self.grid, list(args), stream)


_ARITY = {"rowscale_f32": 5, "rowscale_f16": 5, "hgemm_f32out": 8, "hgemm_f16out": 8, "hgemm_splitk": 8,
          "skinny_f32in": 8, "skinny_f16in": 8}


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
