"""Host-side dispatch: support checks, path selection, launches on the current torch stream.

Mirrors the reference's src/gtx16_fp16/ops.py (same names, arguments, dtype rules and fallbacks);
the kernels behind it are the gfx950 ones of libg16.so.
"""
from __future__ import annotations

import weakref

import torch

from . import _clib
from .kernels import SKINNY_MAX_M, scratch_buffer, split_buffers, stream_handle

# ops.py:14-16 -- rows whose |max| exceeds this are scaled down by a power of two before the fp16
# cast (GEMM path); the result is scaled back in fp32.
ROW_SCALE_THRESHOLD = 1024.0

# The gfx target libg16.so is built for.
TARGET_ARCH = "gfx950"

_cus: dict[int, int] = {}
_arch_ok: dict[int, bool] = {}
# Devices whose speculation history (g16_mm_t_spec_history) is enabled.
_spec_history: set[int] = set()


def tensor_version(t: torch.Tensor) -> int | None:
    """torch's in-place write counter of ``t``; None for an inference tensor (one made under
    ``torch.inference_mode()``), which has no counter."""
    return None if t.is_inference() else t._version


def _dev_index(device) -> int:
    if device is None:
        return torch.cuda.current_device()
    d = torch.device(device) if not isinstance(device, int) else torch.device("cuda", device)
    return d.index if d.index is not None else torch.cuda.current_device()


def _is_target(idx: int) -> bool:
    ok = _arch_ok.get(idx)
    if ok is None:
        arch = getattr(torch.cuda.get_device_properties(idx), "gcnArchName", "") or ""
        ok = torch.version.hip is not None and arch.split(":")[0] == TARGET_ARCH
        _arch_ok[idx] = ok
    return ok


def is_affected(device: torch.device | int | None = None) -> bool:
    """True when the device is one these kernels target: an MI355X-class gfx950 GPU.

    (The reference's predicate selects Turing TU116/TU117 devices, ops.py:19-26; here it decides
    whether ``patch`` swaps layers by default.)"""
    if not torch.cuda.is_available():
        return False
    return _is_target(_dev_index(device))


def supported(x2d: torch.Tensor, w_t: torch.Tensor) -> bool:
    """x2d: [M, K] fp16/fp32 contiguous GPU tensor; w_t: [K, N] fp16 contiguous, 16-byte aligned;
    K % 8 == 0 and N % 8 == 0 (ops.py:29-35). Additionally the device must be the gfx950 target
    of libg16.so, so other GPUs take the torch fallback instead of failing to launch."""
    K, N = w_t.shape
    return (x2d.is_cuda and x2d.dim() == 2 and x2d.dtype in (torch.float16, torch.float32)
            and w_t.dtype == torch.float16 and x2d.is_contiguous() and w_t.is_contiguous()
            and x2d.shape[1] == K and K % 8 == 0 and N % 8 == 0 and w_t.data_ptr() % 16 == 0
            and w_t.device == x2d.device and _is_target(x2d.device.index or 0))


def _sm_count(device: torch.device) -> int:
    """Compute units of ``device`` (cached; ops.py:38-42)."""
    i = device.index or 0
    if i not in _cus:
        _cus[i] = torch.cuda.get_device_properties(i).multi_processor_count
    return _cus[i]


def skinny_config(N: int, K: int, sms: int) -> tuple[tuple[int, int, int], int]:
    """Grid and K rows per workgroup of the skinny kernel for ``sms`` compute units
    (ops.py:45-51): column strips of 8 wavefronts (g16_skinny_strip_cols wide), K split so that
    about one workgroup lands on every CU."""
    lib = _clib.load()
    ksplit = lib.g16_skinny_plan(1, N, K, sms)
    cols = lib.g16_skinny_strip_cols(1, N)
    rows = 0 if K == 0 else -(-(-(-K // ksplit)) // 8) * 8
    ksplit = 1 if K == 0 else -(-K // rows)
    return ((N + cols - 1) // cols * ksplit, 1, 1), rows


# (M, N, K, device index) -> the GEMM route mm_t takes for that shape, computed once per shape:
# ("packed", packed-activation bytes) | ("splitk", ksplit, partial bytes, counter bytes) | ("plain",);
# skinny shapes are keyed (-M, N, K, device index) -> (ksplit, partial bytes, counter bytes).
_routes: dict[tuple[int, int, int, int], tuple] = {}


def _gemm_route(lib, M: int, N: int, K: int, dev: torch.device) -> tuple:
    """(route, scratch bytes, ksplit, split workspace bytes, split counter bytes) of the GEMM path
    for this shape: the plan g16_mm_t_gemm follows for the same compute-unit count."""
    key = (M, N, K, dev.index or 0)
    r = _routes.get(key)
    if r is None:
        cus = _sm_count(dev)
        scratch = lib.g16_mm_t_scratch_bytes(M, N, K, cus)
        if lib.g16_hgemm_use_packed(M, N, K, cus):
            r = ("packed", scratch, 1, 0, 0)
        else:
            ksplit = lib.g16_hgemm_plan(M, N, K, cus)
            if ksplit > 1:
                r = ("splitk", scratch, ksplit, lib.g16_hgemm_splitk_workspace_bytes(M, N, K, ksplit, cus),
                     lib.g16_hgemm_splitk_counter_bytes(M, N, K, ksplit, cus))
            else:
                r = ("plain", scratch, 1, 0, 0)
        _remember(key, r)
    return r


def _remember(key: tuple, value: tuple) -> None:
    if len(_routes) > 4096:  # bounded: shapes are few in practice
        _routes.clear()
    _routes[key] = value


def _check_operands(x2d: torch.Tensor, w_t: torch.Tensor, bias: torch.Tensor | None) -> None:
    # The reference leaves validation to supported() (ops.py:29-35, "Check supported() first"); a
    # call that skips it must still not hand the kernels a pointer they cannot read (a bias or
    # weight on another device, a misaligned weight), so those are rejected here.
    if not (x2d.is_cuda and x2d.dim() == 2 and x2d.dtype in (torch.float16, torch.float32)):
        raise ValueError("mm_t: x2d must be a 2-D fp16 or fp32 CUDA tensor")
    if not (w_t.dim() == 2 and w_t.dtype == torch.float16 and w_t.device == x2d.device and w_t.is_contiguous()
            and w_t.data_ptr() % 16 == 0):
        raise ValueError("mm_t: w_t must be a contiguous, 16-byte aligned fp16 tensor on x2d's device")
    K, N = w_t.shape
    if x2d.shape[1] != K or K % 8 or N % 8:
        raise ValueError(f"mm_t: shapes x2d {tuple(x2d.shape)} and w_t {tuple(w_t.shape)} are not supported "
                         "(K and N must match and be multiples of 8)")
    if bias is not None and (bias.device != x2d.device or bias.numel() != N):
        raise ValueError(f"mm_t: bias must hold {N} values on x2d's device")


def _cast_scratch(xbytes: int, M: int, dev: torch.device) -> tuple[torch.Tensor, int, int]:
    # The fp16 copy of x (row-major or tile-packed, xbytes) and the M fp32 row scales share one
    # allocation, 256-byte aligned parts: one caching-allocator call instead of two on a path whose
    # per-call cost is host time at small shapes. Returns (owner, copy pointer, scales pointer).
    off = (xbytes + 255) // 256 * 256
    buf = torch.empty(off + 4 * M, device=dev, dtype=torch.uint8)
    ptr = buf.data_ptr()
    return buf, ptr, ptr + off


def _aligned(x: torch.Tensor) -> torch.Tensor:
    # The kernels read activations as M*K contiguous values with 16-byte (rowscale) or dword
    # (skinny) loads from a 16-byte aligned base; supported() checks the weight's alignment only,
    # as the reference does, so a misaligned or non-contiguous activation view (an expanded one
    # may own fewer than M*K values) is copied into a fresh allocation.
    if not x.is_contiguous():
        return x.contiguous()
    return x if x.data_ptr() % 16 == 0 else x.clone()


def mm_t(x2d: torch.Tensor, w_t: torch.Tensor, bias: torch.Tensor | None = None,
         out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """out[M,N] = x2d[M,K] @ w_t[K,N] + bias[N]  (ops.py:65-108).

    x2d fp16 or fp32; w_t fp16; bias fp32 (or None); out fp32 or fp16. Check supported() first.
    M <= 8: fp32 math on the unquantised x (skinny path). M > 8: rows with |max| > 1024 are scaled
    by a power of two, cast to fp16, multiplied on the matrix cores with fp32 accumulation and
    scaled back; shapes with too few output tiles split K with a deterministic reduction."""
    if out_dtype not in (torch.float32, torch.float16):
        raise ValueError(f"out_dtype must be float32 or float16, got {out_dtype}")
    _check_operands(x2d, w_t, bias)
    lib = _clib.load()
    M, K = x2d.shape
    N = w_t.shape[1]
    dev = x2d.device
    stream = stream_handle(dev.index or 0)
    b = None if bias is None else bias.float().contiguous()
    bptr = None if b is None else b.data_ptr()

    x2d = _aligned(x2d)
    if M <= SKINNY_MAX_M:  # memory-bound path, fp32 math
        out = torch.empty(M, N, device=dev, dtype=torch.float32)
        key = (-M, N, K, dev.index or 0)
        plan = _routes.get(key)
        if plan is None:
            ksplit = lib.g16_skinny_plan(M, N, K, _sm_count(dev))
            plan = (ksplit, lib.g16_skinny_workspace_bytes(M, N, K, ksplit),
                    lib.g16_skinny_counter_bytes(M, N, K, ksplit))
            _remember(key, plan)
        ksplit = plan[0]
        bufs = split_buffers(dev, stream, plan[1], plan[2])
        fn = _clib.fast().skinny_f32in if x2d.dtype == torch.float32 else lib.g16_skinny_f16in
        _clib.check(fn(x2d.data_ptr(), w_t.data_ptr(), out.data_ptr(), bptr, M, N, K, ksplit, *bufs, stream),
                    "skinny GEMM")
        return out if out_dtype == torch.float32 else out.to(out_dtype)

    # GEMM path: fp16 inputs, with per-row power-of-two scaling for rows that would overflow. One
    # library call runs the rowscale cast into `scratch` and the GEMM on the planned route: the
    # tile-packed 256-row tiles for large outputs, split-K where the tiles leave CUs idle, else the
    # plain tiles (the cast, scales and GEMM of ops.py:86-108); on the unsplit 32x128 tile with
    # K <= 1280 the GEMM casts fp32 rows into LDS, and fp16 x on the 32-, 64- and 128-row tiles is
    # streamed as it is (a row within the threshold is its own cast): one launch in both cases.
    # The speculation history lets a weight whose fp16 call needed a tile computed again take the
    # two-launch route for a while; it is enabled once per device (a small pinned allocation,
    # retried on a later call if this one is being captured into a graph).
    if x2d.dtype == torch.float16 and dev.index not in _spec_history:
        if lib.g16_mm_t_spec_history(stream) == 0:
            _spec_history.add(dev.index)
    kind, scratch_bytes, _ks, ws_bytes, cnt_bytes = _gemm_route(lib, M, N, K, dev)
    out = torch.empty(M, N, device=dev, dtype=out_dtype)
    # no scratch where the GEMM casts its own rows into LDS (one launch, the unsplit small tile)
    scratch = scratch_buffer(dev, stream, scratch_bytes) if scratch_bytes else None
    bufs = split_buffers(dev, stream, ws_bytes, cnt_bytes) if kind == "splitk" else (None, 0, None, 0)
    _clib.check(_clib.fast().mm_t_gemm(x2d.data_ptr(), 1 if x2d.dtype == torch.float32 else 0, w_t.data_ptr(),
                                  out.data_ptr(), 1 if out_dtype == torch.float16 else 0, bptr, ROW_SCALE_THRESHOLD,
                                  M, N, K, _sm_count(dev), None if scratch is None else scratch.data_ptr(),
                                  scratch_bytes, *bufs, stream), "GEMM")
    return out


def prepacked_route(M: int, N: int, K: int, device: torch.device) -> bool:
    """True where mm_t takes the tile-packed route on the 256x256 tile, the one a prepacked weight
    serves."""
    return _gemm_route(_clib.load(), M, N, K, device)[0] == "packed" and \
        _clib.load().g16_hgemm_use_packed_b(M, N, K, _sm_count(device)) == 1


def pack_weight(w_t: torch.Tensor) -> torch.Tensor:
    """w_t [K, N] fp16 (CUDA, contiguous, K and N multiples of 8) -> its prepacked form for
    mm_t_prepacked: w_t transposed into the GEMM's tile-packed layout, a 1-D fp16 tensor."""
    if not (w_t.is_cuda and w_t.dim() == 2 and w_t.dtype == torch.float16 and w_t.is_contiguous()
            and w_t.data_ptr() % 16 == 0 and w_t.shape[0] % 8 == 0 and w_t.shape[1] % 8 == 0):
        raise ValueError("pack_weight: w_t must be a contiguous, 16-byte aligned fp16 CUDA tensor "
                         "with both dimensions multiples of 8")
    lib = _clib.load()
    K, N = w_t.shape
    wp = torch.empty(lib.g16_packed_b_bytes(K, N) // 2, device=w_t.device, dtype=torch.float16)
    _clib.check(lib.g16_pack_weight(w_t.data_ptr(), wp.data_ptr(), K, N, stream_handle(w_t.device.index or 0)),
                "weight packing")
    return wp


STRIPS_MAX_M = 4  # G16_STRIPS_MAX_M


def pack_decode_weight(w_t: torch.Tensor) -> torch.Tensor:
    """w_t [K, N] fp16 (CUDA, contiguous, K and N multiples of 8) -> its decode layout for
    ``skinny_strips``: N/8 strips of 8 columns, each all K rows long and contiguous, as an
    [N/8, K, 8] fp16 tensor (``wd[s, k, c] == w_t[k, 8 * s + c]``)."""
    if not (w_t.is_cuda and w_t.dim() == 2 and w_t.dtype == torch.float16 and w_t.is_contiguous()
            and w_t.data_ptr() % 16 == 0 and w_t.shape[0] % 8 == 0 and w_t.shape[1] % 8 == 0):
        raise ValueError("pack_decode_weight: w_t must be a contiguous, 16-byte aligned fp16 CUDA tensor "
                         "with both dimensions multiples of 8")
    lib = _clib.load()
    K, N = w_t.shape
    wd = torch.empty(N // 8, K, 8, device=w_t.device, dtype=torch.float16)
    _clib.check(lib.g16_pack_decode_weight(w_t.data_ptr(), wd.data_ptr(), K, N, stream_handle(w_t.device.index or 0)),
                "decode-layout packing")
    return wd


def skinny_strips(x2d: torch.Tensor, wd: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """The skinny product on a weight's decode layout ``wd = pack_decode_weight(w_t)``: fp32
    ``x2d @ w_t + bias`` for 1 <= M <= STRIPS_MAX_M rows of fp32 or fp16 activations, in fp32
    arithmetic on the activations as given (the skinny path's semantics, one workgroup per strip of
    8 columns over all of K)."""
    if not (wd.is_cuda and wd.dim() == 3 and wd.shape[2] == 8 and wd.dtype == torch.float16 and wd.is_contiguous()):
        raise ValueError("skinny_strips: wd must be a decode-layout weight (pack_decode_weight)")
    N, K = wd.shape[0] * 8, wd.shape[1]
    if not (x2d.dim() == 2 and x2d.shape[1] == K and 1 <= x2d.shape[0] <= STRIPS_MAX_M
            and x2d.dtype in (torch.float32, torch.float16) and x2d.device == wd.device):
        raise ValueError(f"skinny_strips: x2d must be [M, {K}] fp32 or fp16 on {wd.device}, 1 <= M <= {STRIPS_MAX_M}")
    if bias is not None and not (bias.dtype == torch.float32 and bias.numel() == N and bias.device == wd.device):
        raise ValueError(f"skinny_strips: bias must be fp32 with {N} elements on {wd.device}")
    x2d = _aligned(x2d)
    bias = None if bias is None else bias.contiguous()
    M = x2d.shape[0]
    out = torch.empty(M, N, device=wd.device, dtype=torch.float32)
    lib = _clib.load()
    fn = lib.g16_skinny_strips_f32in if x2d.dtype == torch.float32 else lib.g16_skinny_strips_f16in
    _clib.check(fn(x2d.data_ptr(), wd.data_ptr(), out.data_ptr(), None if bias is None else bias.data_ptr(),
                   M, N, K, stream_handle(wd.device.index or 0)), "skinny GEMM (decode layout)")
    return out


# The latest tile-packed rowscale cast per (device index, stream): (weak reference to the tensor the
# caller named as its source, that tensor's version, (data pointer, M, K, dtype) of the activations
# cast, owning buffer, packed-cast pointer, row-scales pointer). Consecutive calls that name the same
# unmodified source (a transformer's Q, K and V projections all read the same hidden states) reuse
# it instead of casting again. The weak reference makes a freed tensor miss even when a new one
# gets its address; the version counter makes any in-place write through torch (the tensor or a
# view of it) miss.
_cast_cache: dict[tuple[int, int], tuple] = {}


def release_cast_cache() -> None:
    """Drop the cached activation casts (they are rebuilt on demand)."""
    _cast_cache.clear()


def _packed_cast(lib, x2d: torch.Tensor, M: int, K: int, dev: torch.device, stream: int, source=None):
    """(owner, packed-cast pointer, row-scales pointer) of x2d's tile-packed rowscale cast, enqueued
    on ``stream``, or the cached one of the previous call on this stream when ``source`` is the same
    unmodified tensor. Not cached while the stream is being captured into a graph, nor for an
    inference tensor (no version counter to tell whether it was written since)."""
    key = (dev.index or 0, stream)
    meta = (x2d.data_ptr(), M, K, x2d.dtype)
    capturing = torch.cuda.is_current_stream_capturing()
    if source is not None and source.is_inference():
        source = None
    if source is not None and not capturing:
        hit = _cast_cache.get(key)
        if hit is not None and hit[0]() is source and hit[1] == source._version and hit[2] == meta:
            return hit[3], hit[4], hit[5]
    owner, xp, rscale = _cast_scratch(lib.g16_packed_a_bytes(M, K), M, dev)
    rs_fn = lib.g16_rowscale_pack_f32 if x2d.dtype == torch.float32 else lib.g16_rowscale_pack_f16
    _clib.check(rs_fn(x2d.data_ptr(), xp, rscale, M, K, ROW_SCALE_THRESHOLD, stream), "rowscale cast")
    if source is not None and not capturing:
        _cast_cache[key] = (weakref.ref(source), source._version, meta, owner, xp, rscale)
    else:
        _cast_cache.pop(key, None)
    return owner, xp, rscale


def mm_t_prepacked(x2d: torch.Tensor, w_t: torch.Tensor, wp: torch.Tensor, bias: torch.Tensor | None = None,
                   out_dtype: torch.dtype = torch.float32, _cast_source: torch.Tensor | None = None) -> torch.Tensor:
    """mm_t for a weight that also has its prepacked form ``wp = pack_weight(w_t)``: same contract and
    the same result bits as ``mm_t(x2d, w_t, bias, out_dtype)``. On the large-GEMM route the GEMM
    reads ``wp`` instead of ``w_t`` (plain 16-byte LDS reads for both operands); elsewhere it is
    exactly mm_t. Check supported(x2d, w_t) first.

    ``_cast_source`` (used by FastLinear) names the tensor x2d was taken from: consecutive calls on
    one stream with the same unmodified source share one rowscale cast of it."""
    if out_dtype not in (torch.float32, torch.float16):
        raise ValueError(f"out_dtype must be float32 or float16, got {out_dtype}")
    _check_operands(x2d, w_t, bias)
    M, K = x2d.shape
    N = w_t.shape[1]
    dev = x2d.device
    if M <= SKINNY_MAX_M or not prepacked_route(M, N, K, dev):
        return mm_t(x2d, w_t, bias, out_dtype)
    lib = _clib.load()
    if wp.dtype != torch.float16 or wp.device != dev or not wp.is_contiguous() or \
            wp.numel() * 2 < lib.g16_packed_b_bytes(K, N) or wp.data_ptr() % 16 != 0:
        raise ValueError("wp is not a packed weight for this w_t (use pack_weight(w_t))")
    stream = stream_handle(dev.index or 0)
    b = None if bias is None else bias.float().contiguous()
    x2d = _aligned(x2d)
    out = torch.empty(M, N, device=dev, dtype=out_dtype)
    _scratch, xp, rscale = _packed_cast(lib, x2d, M, K, dev, stream, _cast_source)
    fn = lib.g16_hgemm_packed_ab_f32out if out_dtype == torch.float32 else lib.g16_hgemm_packed_ab_f16out
    _clib.check(fn(xp, wp.data_ptr(), out.data_ptr(), None if b is None else b.data_ptr(), rscale, M, N, K, stream),
                "GEMM")
    return out


def matmul(a: torch.Tensor, b: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Drop-in for a @ b with 2-D fp16 inputs; falls back to torch.matmul when the shape is not
    supported. Default output dtype: fp16, like torch (ops.py:111-119)."""
    out_dtype = out_dtype or torch.float16
    if a.dim() == 2 and b.dim() == 2 and a.dtype == b.dtype == torch.float16 and a.is_cuda:
        a_c, b_c = a.contiguous(), b.contiguous()
        if supported(a_c, b_c):
            return mm_t(a_c, b_c, None, out_dtype)
    return torch.matmul(a, b).to(out_dtype)
