"""ctypes binding of libg16.so, the C ABI declared in ``include/g16.h``.

The library is loaded lazily on first use, after ``torch``: it depends on ``libamdhip64.so.7`` by
SONAME, and binding it to the HIP runtime torch has already loaded is what lets it share torch's
device context and streams. A missing or stale library raises ``RuntimeError``; there is no
fallback implementation behind this module.
"""
from __future__ import annotations

import ctypes
import importlib.util
import sysconfig
import threading
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime before libg16.so)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libg16.so"
ABI_VERSION = 16

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); one entry per function of include/g16.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "g16_abi_version": (_I, []),
    "g16_strerror": (ctypes.c_char_p, [_I]),
    "g16_rowscale_f32": (_I, [_P, _P, _P, _I, _I, _F, _P]),
    "g16_rowscale_f16": (_I, [_P, _P, _P, _I, _I, _F, _P]),
    "g16_hgemm_f32out": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "g16_hgemm_f16out": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "g16_packed_a_bytes": (_SZ, [_I, _I]),
    "g16_rowscale_pack_f32": (_I, [_P, _P, _P, _I, _I, _F, _P]),
    "g16_rowscale_pack_f16": (_I, [_P, _P, _P, _I, _I, _F, _P]),
    "g16_hgemm_packed_f32out": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "g16_hgemm_packed_f16out": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "g16_hgemm_use_packed": (_I, [_I, _I, _I, _I]),
    "g16_hgemm_use_packed_b": (_I, [_I, _I, _I, _I]),
    "g16_mm_t_scratch_bytes": (_SZ, [_I, _I, _I, _I]),
    "g16_mm_t_gemm": (_I, [_P, _I, _P, _P, _I, _P, _F, _I, _I, _I, _I, _P, _SZ, _P, _SZ, _P, _SZ, _P]),
    "g16_mm_t_spec_history": (_I, [_P]),
    "g16_mm_t_spec_paused": (_I, [_P, _P]),
    "g16_packed_b_bytes": (_SZ, [_I, _I]),
    "g16_pack_weight": (_I, [_P, _P, _I, _I, _P]),
    "g16_hgemm_packed_ab_f32out": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "g16_hgemm_packed_ab_f16out": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "g16_hgemm_splitk": (_I, [_P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _P, _SZ, _P, _SZ, _P]),
    "g16_hgemm_splitk_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "g16_hgemm_splitk_counter_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "g16_hgemm_plan": (_I, [_I, _I, _I, _I]),
    "g16_hgemm_tile": (_I, [_I, _I, _I, _I, _P, _P]),
    "g16_skinny_f32in": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _SZ, _P, _SZ, _P]),
    "g16_skinny_f16in": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _SZ, _P, _SZ, _P]),
    "g16_skinny_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "g16_skinny_counter_bytes": (_SZ, [_I, _I, _I, _I]),
    "g16_skinny_plan": (_I, [_I, _I, _I, _I]),
    "g16_skinny_strip_cols": (_I, [_I, _I]),
    "g16_skinny_f32in_noalloc": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "g16_pack_decode_weight": (_I, [_P, _P, _I, _I, _P]),
    "g16_skinny_strips_f32in": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "g16_skinny_strips_f16in": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "g16_skinny_strips_route": (_I, [_I, _I, _I, _I]),
    "g16_gemm_clock": (_I, [_P, _P]),
    "g16_peak_flops_per_lane_iter": (ctypes.c_double, [_I]),
    "g16_peak_run": (_I, [_I, _I, _I, _P, _P]),
    "g16_peak_run_clocked": (_I, [_I, _I, _I, _P, _P, _P]),
    "g16_stream_read": (_I, [_P, _SZ, _I, _P, _P]),
    "g16_peak_mfma_data": (_I, [_I, _I, _P, _I, _P, _P, _P]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and return the library with every signature of ``SIGNATURES`` applied."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"gtx16_fp16: HIP library {p} is missing; build it with "
                "`python gtx16-fp16_amd/build_lib.py` (or __graft_entry__.build())")
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.g16_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"gtx16_fp16: {p} has ABI version {ver}, expected {ABI_VERSION}; rebuild it")
        if path is None:
            _lib = lib
        return lib


_fast = None


def fast():
    """The CPython extension ``_g16fast`` (built next to the library from ``csrc/fastcall.c``), bound
    to the loaded library: ``skinny_f32in``, ``skinny_strips_f32in`` and ``mm_t_gemm`` take the same arguments as the C
    entry points (pointers as ints or None) and return their status, with argument conversion
    that costs a few ns per argument instead of ctypes' ~0.1 us. Missing -> ``RuntimeError``."""
    global _fast
    if _fast is not None:
        return _fast
    lib = load()
    with _lock:
        if _fast is None:
            p = LIB_PATH.parent / ("_g16fast" + sysconfig.get_config_var("EXT_SUFFIX"))
            if not p.exists():
                raise RuntimeError(
                    f"gtx16_fp16: extension {p} is missing; build it with "
                    "`python gtx16-fp16_amd/build_lib.py` (or __graft_entry__.build())")
            spec = importlib.util.spec_from_file_location("_g16fast", p)
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            mod.bind(ctypes.cast(lib.g16_skinny_f32in, ctypes.c_void_p).value,
                     ctypes.cast(lib.g16_mm_t_gemm, ctypes.c_void_p).value,
                     ctypes.cast(lib.g16_skinny_strips_f32in, ctypes.c_void_p).value)
            _fast = mod
    return _fast


def strerror(status: int) -> str:
    return load().g16_strerror(status).decode()


def check(status: int, what: str) -> None:
    """Raise ``RuntimeError`` for a nonzero status (the reference raises on a nonzero
    cuLaunchKernel result, src/gtx16_fp16/kernels.py:299-302)."""
    if status != 0:
        raise RuntimeError(f"{what} failed with status {status}: {strerror(status)}")
