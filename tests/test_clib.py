"""CPU tests of libg16.so's C ABI: it loads, exports every function include/g16.h declares, and
rejects bad arguments before any launch (so these calls need no GPU)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from gtx16_fp16 import _clib, kernels

HEADER = Path(__file__).resolve().parents[1] / "include" / "g16.h"


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(g16_\w+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    return _clib.load()


def test_header_and_binding_agree():
    assert declared_functions() == set(_clib.SIGNATURES)


_CTYPE = {"int": ctypes.c_int, "float": ctypes.c_float, "double": ctypes.c_double, "size_t": ctypes.c_size_t}


def _ctype(decl: str, ret: bool = False):
    # a C parameter or return type of the header as the ctypes type that passes it: any pointer is
    # c_void_p (c_char_p for the strerror string), the scalars by name
    decl = decl.strip()
    if "*" in decl:
        return ctypes.c_char_p if ret and "char" in decl else ctypes.c_void_p
    words = [w for w in decl.split() if w != "const"]
    base = words[0] if ret else " ".join(words[:-1])
    return _CTYPE[base]


def header_prototypes() -> dict[str, tuple[object, list[object]]]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"#.*", "", text)
    out = {}
    for ret, name, args in re.findall(r"([\w\s\*]+?)\b(g16_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [a for a in (s.strip() for s in args.split(",")) if a and a != "void"]
        out[name] = (_ctype(ret, ret=True), [_ctype(p) for p in params])
    return out


def test_binding_types_match_the_header_prototypes():
    # every argument and result type the ctypes binding declares is the one the C prototype has
    # (a size_t bound as c_int, say, would pass the low half of the register and garbage above it)
    protos = header_prototypes()
    assert set(protos) == set(_clib.SIGNATURES)
    for name, (res, args) in _clib.SIGNATURES.items():
        assert protos[name] == (res, args), name


def test_integration_ctypes_stub_matches_the_binding():
    # the stub INTEGRATION.md shows a maintainer (route 2) binds the same types as this package
    doc = (HEADER.parents[1] / "INTEGRATION.md").read_text()
    block = doc.split("# src/gtx16_fp16/_rocm.py")[1].split("```")[0]
    alias = {"P": ctypes.c_void_p, "I": ctypes.c_int, "F": ctypes.c_float, "SZ": ctypes.c_size_t}
    seen = {}
    for name, args in re.findall(r'"(g16_\w+)":\s*\[([^\]]*)\]', block):
        seen[name] = [alias[a.strip()] for a in args.split(",") if a.strip()]
    for names, args in re.findall(r"for name in \(([^)]*)\):\s*\n\s*fn = getattr\(_lib, name\); "
                                  r"fn\.argtypes, fn\.restype = \[([^\]]*)\]", block):
        for name in re.findall(r'"(g16_\w+)"', names):
            seen[name] = [alias[a.strip()] for a in args.split(",")]
    for name, args in re.findall(r"_lib\.(g16_\w+)\.argtypes, _lib\.\1\.restype = \[([^\]]*)\]", block):
        seen[name] = [alias[a.strip()] for a in args.split(",")]
    assert len(seen) >= 14
    for name, args in seen.items():
        assert args == list(_clib.SIGNATURES[name][1]), name


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_abi_version_and_strerror(lib):
    assert lib.g16_abi_version() == _clib.ABI_VERSION
    assert b"aligned" in lib.g16_strerror(-2)
    assert b"workspace" in lib.g16_strerror(-4)
    assert lib.g16_strerror(-99) == b"unknown g16 status"


def test_argument_errors_need_no_gpu(lib):
    A = 0x1000  # never dereferenced: every call below is rejected before a launch
    assert lib.g16_hgemm_f32out(A, A, A, None, None, 64, 64, 60, None) == -1      # K % 8
    assert lib.g16_hgemm_f32out(A, A, A, None, None, 64, 60, 64, None) == -1      # N % 8
    assert lib.g16_hgemm_f32out(A + 2, A, A, None, None, 64, 64, 64, None) == -2  # alignment
    assert lib.g16_hgemm_f32out(None, A, A, None, None, 64, 64, 64, None) == -3   # NULL
    assert lib.g16_hgemm_f32out(A, A, A, None, None, 0, 64, 64, None) == 0        # M == 0: no-op
    assert lib.g16_hgemm_splitk(A, A, A, 0, None, None, 64, 64, 1024, 4, 0, None, 0, None, 0, None) == -4
    assert lib.g16_hgemm_splitk(A, A, A, 0, None, None, 64, 64, 1024, 0, 0, None, 0, None, 0, None) == -5
    assert lib.g16_skinny_f32in(A, A, A, None, 9, 64, 64, 1, None, 0, None, 0, None) == -1   # M > 8
    assert lib.g16_skinny_f32in(A, A, A, None, 4, 4096, 4096, 8, A, 1 << 30, None, 0, None) == -4
    assert lib.g16_skinny_f32in(A, A, A + 4, None, 1, 64, 64, 1, None, 0, None, 0, None) == -2  # C alignment
    # split partials beyond a 2 GiB workspace (8 x 65536 x 1024 slices x 4 bytes) are refused
    assert lib.g16_skinny_f32in(A, A, A, None, 8, 65536, 8192, 1024, A, 1 << 40, A, 1 << 20, None) == -5
    need = lib.g16_mm_t_scratch_bytes(64, 64, 2048, 256)
    assert need == 64 * 2048 * 2 + 64 * 4                                      # cast + row scales
    assert lib.g16_mm_t_gemm(A, 1, A, A, 0, None, 1024.0, 64, 64, 2048, 256, A, need - 1, None, 0, None, 0, None) == -4
    assert lib.g16_mm_t_gemm(A, 1, A, A, 0, None, 1024.0, 64, 64, 2048, 256, A + 8, need, None, 0, None, 0, None) == -2
    assert lib.g16_mm_t_gemm(A, 1, A, A, 0, None, 1024.0, 64, 60, 2048, 256, A, need, None, 0, None, 0, None) == -1
    assert lib.g16_mm_t_gemm(A, 1, A, A, 0, None, 1024.0, 0, 64, 2048, 256, A, need, None, 0, None, 0, None) == 0
    # the one-launch route (no scratch): misaligned x and a threshold that is not 2^k are refused
    assert lib.g16_mm_t_scratch_bytes(64, 64, 64, 256) == 0
    assert lib.g16_mm_t_gemm(A + 4, 1, A, A, 0, None, 1024.0, 64, 64, 64, 256, None, 0, None, 0, None, 0, None) == -2
    assert lib.g16_mm_t_gemm(A, 1, A, A, 0, None, 1000.0, 64, 64, 64, 256, None, 0, None, 0, None, 0, None) == -1
    assert lib.g16_mm_t_gemm(A, 1, A, None, 0, None, 1024.0, 64, 64, 64, 256, None, 0, None, 0, None, 0, None) == -3
    # the no-allocation skinny variant refuses splits past its static scratch before any HIP call:
    # 32 slices x 8 x 16384 x 4 bytes = 16 MiB of partials > 4 MiB; N = 131080 needs 257 counter lines
    assert lib.g16_skinny_f32in_noalloc(A, A, A, None, 8, 16384, 4096, 32, None) == -7
    assert lib.g16_skinny_f32in_noalloc(A, A, A, None, 1, 131080, 4096, 2, None) == -7
    assert lib.g16_skinny_f32in_noalloc(A, A, A, None, 9, 64, 64, 1, None) == -1
    assert lib.g16_skinny_f32in_noalloc(A, A, A, None, 0, 64, 64, 1, None) == 0
    assert b"static scratch" in lib.g16_strerror(-7)
    assert lib.g16_gemm_clock(None, None) == -3
    assert lib.g16_gemm_clock(A + 4, None) == -2
    assert lib.g16_rowscale_f32(A, A, A, 4, 64, 1000.0, None) == -1               # threshold not 2^k
    assert lib.g16_rowscale_f32(A, A, A, 4, 64, -1024.0, None) == -1
    # the decode layout: M <= 4, K and N multiples of 8, 16-byte alignment, non-NULL operands
    assert lib.g16_skinny_strips_f32in(A, A, A, None, 5, 64, 64, None) == -1
    assert lib.g16_skinny_strips_f16in(A, A, A, None, 1, 64, 60, None) == -1
    assert lib.g16_skinny_strips_f32in(A, A, A + 4, None, 1, 64, 64, None) == -2
    assert lib.g16_skinny_strips_f32in(None, A, A, None, 1, 64, 64, None) == -3
    assert lib.g16_skinny_strips_f32in(A, A, A, None, 0, 64, 64, None) == 0
    assert lib.g16_pack_decode_weight(A, A, 60, 64, None) == -1
    assert lib.g16_pack_decode_weight(A, A + 8, 64, 64, None) == -2
    assert lib.g16_pack_decode_weight(A, None, 64, 64, None) == -3
    assert lib.g16_pack_decode_weight(A, A, 0, 64, None) == 0


def test_gemm_size_limits_refused_before_launch(lib):
    # Operand offsets are 32-bit inside the GEMM's buffer descriptors: K past 2^22 - 8 or N past
    # 2^24 - 8 would read zeros silently, so every GEMM entry point refuses them (G16_E_SHAPE).
    A = 0x1000
    big_k, big_n = (1 << 22), (1 << 24)
    for fn in (lib.g16_hgemm_f32out, lib.g16_hgemm_f16out, lib.g16_hgemm_packed_f32out,
               lib.g16_hgemm_packed_ab_f16out):
        assert fn(A, A, A, None, None, 64, 64, big_k, None) == -1
        assert fn(A, A, A, None, None, 64, big_n, 64, None) == -1
    assert lib.g16_hgemm_splitk(A, A, A, 0, None, None, 64, 64, big_k, 2, 0, A, 1 << 40, A, 1 << 20, None) == -1
    assert lib.g16_mm_t_gemm(A, 1, A, A, 0, None, 1024.0, 64, 64, big_k, 256, A, 1 << 40, None, 0, None, 0,
                             None) == -1
    assert lib.g16_mm_t_gemm(A, 1, A, A, 0, None, 1024.0, 64, big_n, 64, 256, A, 1 << 40, None, 0, None, 0,
                             None) == -1


def test_splitk_launch_checks_buffers_against_the_callers_cu_count(lib):
    # M=300, N=264: 256 CUs take 25 tiles of 64x64 (padded 320 x 320), 10 CUs take 9 tiles of
    # 128x128 (384 x 384), so the 10-CU plan needs more workspace. A launch for 10 CUs handed the
    # 256-CU workspace must be refused (it used to plan with the device's own count instead).
    A = 0x1000
    M, N, K = 300, 264, 1024
    ws256 = lib.g16_hgemm_splitk_workspace_bytes(M, N, K, 2, 256)
    ws10 = lib.g16_hgemm_splitk_workspace_bytes(M, N, K, 2, 10)
    assert ws256 == 2 * 320 * 320 * 4 and ws10 == 2 * 384 * 384 * 4
    cnt10 = lib.g16_hgemm_splitk_counter_bytes(M, N, K, 2, 10)
    assert cnt10 == 9 * 256 and lib.g16_hgemm_splitk_counter_bytes(M, N, K, 2, 256) == 25 * 256
    assert lib.g16_hgemm_splitk(A, A, A, 0, None, None, M, N, K, 2, 10, A, ws256, A, cnt10, None) == -4
    # counters sized for 10 CUs are too few for the 256-CU grid
    assert lib.g16_hgemm_splitk(A, A, A, 0, None, None, M, N, K, 2, 256, A, ws256, A, cnt10, None) == -4
    # num_cus <= 0 in a size query means the current device's count (256 when there is none)
    assert lib.g16_hgemm_splitk_workspace_bytes(M, N, K, 2, 0) in (ws256, lib.g16_hgemm_splitk_workspace_bytes(
        M, N, K, 2, _device_cus()))


def _device_cus() -> int:
    import torch

    return torch.cuda.get_device_properties(0).multi_processor_count if torch.cuda.is_available() else 256


def test_plans_and_buffer_sizes(lib):
    assert lib.g16_skinny_plan(1, 4096, 4096, 256) >= 8
    assert lib.g16_hgemm_plan(4096, 4096, 4096, 256) == 1           # enough tiles: no split
    assert lib.g16_hgemm_plan(64, 1024, 4096, 256) > 1              # few tiles: split K
    # measured-best splits (the modelled choice for M > 64; g16_hgemm_plan(M, N, K))
    assert lib.g16_hgemm_plan(1024, 1024, 1024, 256) == 1            # 256 tiles of 64x64
    assert lib.g16_hgemm_plan(1024, 1024, 2048, 256) == 1
    assert lib.g16_hgemm_plan(512, 512, 512, 256) == 1               # 64 tiles of 64x64: a split costs more than it saves
    assert lib.g16_hgemm_plan(64, 1024, 1024, 256) == 4
    assert lib.g16_hgemm_plan(64, 1024, 4096, 256) == 8
    # tiles that leave CUs idle split as far as pays off within one workgroup per CU
    assert lib.g16_hgemm_plan(512, 4096, 4096, 256) == 1             # 256 tiles of 64x128
    assert lib.g16_hgemm_plan(128, 4096, 4096, 256) == 2             # 128 tiles of 64x64, 2 slices
    assert lib.g16_hgemm_plan(192, 512, 4096, 256) == 8              # 24 tiles of 64x64, 8 slices
    assert lib.g16_hgemm_plan(384, 4096, 4096, 256) == 1             # 192 tiles of 64x128
    assert lib.g16_hgemm_plan(768, 4096, 4096, 256) == 1             # 192 tiles of 128x128: 2 slices would overflow
    # 128 tiles of 256x256 would leave half the CUs idle: 256 tiles of 256x128 instead, packed A
    # (and a packed weight, whose blocks the 128-column tiles read by halves), no split
    assert lib.g16_hgemm_plan(2048, 4096, 4096, 256) == 1
    assert lib.g16_hgemm_plan(2048, 4096, 8192, 256) == 1
    assert lib.g16_hgemm_use_packed(2048, 4096, 4096, 256) == 1
    assert lib.g16_hgemm_use_packed_b(2048, 4096, 4096, 256) == 1
    assert lib.g16_hgemm_use_packed_b(4096, 4096, 4096, 256) == 1
    assert lib.g16_hgemm_use_packed_b(1536, 4096, 4096, 256) == 1    # 128x128 tiles would need 1.5 rounds
    assert lib.g16_hgemm_use_packed_b(1536, 4096, 1024, 256) == 0    # short K: 128x128 tiles, not packed
    # skinny: 256-column strips up to N = 8192, 512 above; whole 16-row blocks per wavefront, at
    # most one workgroup per CU
    assert lib.g16_skinny_strip_cols(1, 4096) == 256 and lib.g16_skinny_strip_cols(8, 8192) == 256
    assert lib.g16_skinny_strip_cols(1, 8200) == 512 and lib.g16_skinny_strip_cols(4, 14336) == 512
    assert lib.g16_skinny_plan(1, 4096, 4096, 256) == 16             # 16 strips x 16 slices
    assert lib.g16_skinny_plan(4, 4096, 4096, 256) == 16
    assert lib.g16_skinny_plan(1, 14336, 4096, 256) == 8             # 28 strips: 8 x 28 <= 256
    ks = lib.g16_skinny_plan(4, 4096, 4096, 256)
    assert lib.g16_skinny_workspace_bytes(4, 4096, 4096, ks) == ks * 4 * 4096 * 4
    assert lib.g16_skinny_counter_bytes(4, 4096, 4096, ks) == (4096 // 256) * 256
    assert lib.g16_skinny_counter_bytes(4, 14336, 4096, 8) == (14336 // 512) * 256
    assert lib.g16_skinny_workspace_bytes(4, 4096, 4096, 1) == 0
    assert lib.g16_hgemm_splitk_workspace_bytes(64, 1024, 1024, 1, 0) == 0
    assert lib.g16_hgemm_splitk_counter_bytes(64, 1024, 1024, 4, 0) > 0


def test_one_launch_route_needs_no_scratch(lib):
    # mm_t's GEMM path is one launch (the cast in LDS, no scratch) exactly where the plan is the
    # unsplit 32x128 tile and K <= 1280
    for M, N, K in [(64, 1024, 1000), (50, 1000, 1000), (20, 32768, 1280), (20, 1024, 256), (20, 1024, 512),
                    (33, 1024, 8)]:
        assert lib.g16_mm_t_scratch_bytes(M, N, K, 256) == 0, (M, N, K)
    for M, N, K in [(1024, 1024, 1024), (20, 32768, 1288), (1024, 1024, 2048), (20, 1024, 1024), (64, 1024, 1024),
                    (4096, 4096, 4096)]:
        assert lib.g16_mm_t_scratch_bytes(M, N, K, 256) > 0, (M, N, K)


def test_fast_extension_matches_the_c_entry_points(lib):
    # _g16fast forwards its arguments unchanged: the same rejected calls give the same statuses
    fast = _clib.fast()
    A = 0x1000
    assert fast.skinny_f32in(A, A, A, None, 9, 64, 64, 1, None, 0, None, 0, None) == -1
    assert fast.skinny_f32in(A, A, A + 4, None, 1, 64, 64, 1, None, 0, None, 0, None) == -2
    assert fast.skinny_f32in(A, A, A, None, 4, 4096, 4096, 8, A, 1 << 30, None, 0, None) == -4
    assert fast.skinny_f32in(A, A, A, None, 8, 65536, 8192, 1024, A, 1 << 40, A, 1 << 20, None) == -5
    need = lib.g16_mm_t_scratch_bytes(64, 64, 2048, 256)
    assert fast.mm_t_gemm(A, 1, A, A, 0, None, 1024.0, 64, 64, 2048, 256, A, need - 1, None, 0, None, 0, None) == -4
    assert fast.mm_t_gemm(A, 1, A, A, 0, None, 1024.0, 64, 64, 2048, 256, A + 8, need, None, 0, None, 0, None) == -2
    assert fast.mm_t_gemm(A, 1, A, A, 0, None, 1024.0, 64, 60, 2048, 256, A, need, None, 0, None, 0, None) == -1
    assert fast.mm_t_gemm(A, 1, A, A, 0, None, 1000.0, 64, 64, 64, 256, None, 0, None, 0, None, 0, None) == -1
    assert fast.mm_t_gemm(A, 1, A, A, 0, None, 1024.0, 0, 64, 2048, 256, A, need, None, 0, None, 0, None) == 0
    assert fast.skinny_strips_f32in(A, A, A, None, 5, 64, 64, None) == -1
    assert fast.skinny_strips_f32in(A, A, A + 4, None, 1, 64, 64, None) == -2
    assert fast.skinny_strips_f32in(A, A, A, None, 0, 64, 64, None) == 0
    with pytest.raises(TypeError):
        fast.skinny_f32in(A, A, A)
    with pytest.raises(TypeError):
        fast.skinny_strips_f32in(A, A, A, None, 1, 64, 64)
    with pytest.raises(OverflowError):
        fast.skinny_f32in(A, A, A, None, 1 << 40, 64, 64, 1, None, 0, None, 0, None)
    with pytest.raises(TypeError):
        fast.mm_t_gemm(A, 1, A, A, 0, None, "x", 64, 64, 64, 256, A, need, None, 0, None, 0, None)


def test_nonzero_status_raises_runtime_error():
    # kernels.py:299-302 convention: a failed launch raises RuntimeError naming the status
    with pytest.raises(RuntimeError, match="status 98"):
        kernels.call(lambda *a: 98, [1, 2], "fake kernel")
    with pytest.raises(RuntimeError, match="skinny"):
        kernels.PreparedCall(lambda *a: -4, "skinny GEMM")(1, 2)
    kernels.PreparedCall(lambda *a: 0, "ok")()


def test_launch_interface_has_the_reference_signatures():
    # kernels.py:315 launch(kernel, grid, block, args, stream); kernels.py:327-336
    # PreparedLaunch(kernel, grid, block, kinds) called as (stream, *args)
    import inspect

    assert list(inspect.signature(kernels.launch).parameters) == ["kernel", "grid", "block", "args", "stream"]
    assert list(inspect.signature(kernels.PreparedLaunch).parameters) == ["kernel", "grid", "block", "kinds"]
    assert list(inspect.signature(kernels.PreparedLaunch.__call__).parameters) == ["self", "stream", "args"]
    assert list(inspect.signature(kernels.get_kernel).parameters) == ["name", "device"]


def _recording(name, status=0):
    """A kernel of the reference's name whose entry point records its C arguments."""
    seen = []

    def fn(*a):
        seen.append(a)
        return status

    return kernels.Kernel(name, fn, 0), seen


def test_launch_maps_reference_arguments_to_the_entry_points():
    # the argument lists ops.py builds (ops.py:89-90, 106-108) reach the C entry points in their
    # order (include/g16.h), with the row count taken from the rowscale grid
    k, seen = _recording("rowscale_f32")
    kernels.launch(k, (48, 1, 1), (256, 1, 1), [0x1000, 0x2000, 0x3000, 64, 1024.0], 7)
    assert seen == [(0x1000, 0x2000, 0x3000, 48, 64, 1024.0, 7)]
    k, seen = _recording("hgemm_f16out")
    kernels.launch(k, (2, 3, 1), (256, 1, 1), [0x10, 0x20, 0x30, None, 0x40, 300, 256, 64], 9)
    assert seen == [(0x10, 0x20, 0x30, None, 0x40, 300, 256, 64, 9)]
    k, seen = _recording("hgemm_f32out", status=4)
    with pytest.raises(RuntimeError, match="hgemm_f32out"):
        kernels.launch(k, (1, 1, 1), (256, 1, 1), [0x10, 0x20, 0x30, None, None, 8, 8, 8], 0)


def test_prepared_launch_checks_its_kinds_and_refuses_accumulating_split_k():
    k, seen = _recording("rowscale_f16")
    pl = kernels.PreparedLaunch(k, (4, 1, 1), (256, 1, 1), "pppif")
    pl(5, 0x100, 0x200, 0x300, 16, 1024.0)
    assert seen == [(0x100, 0x200, 0x300, 4, 16, 1024.0, 5)]
    with pytest.raises(ValueError):
        kernels.PreparedLaunch(k, (4, 1, 1), (256, 1, 1), "ppp")
    with pytest.raises(TypeError, match="adds into C"):
        kernels.PreparedLaunch(kernels.Kernel("hgemm_splitk", None, 0), (1, 1, 2), (256, 1, 1), "ppppiiii")


def test_split_counts_follow_the_reference_kchunk():
    # ops.py:48-50, 95-97: slices = ceil(K / kchunk); the grid's slice count when kchunk is 0
    assert kernels._slices(4096, 512, 99) == 8
    assert kernels._slices(4100, 520, 99) == 8
    assert kernels._slices(64, 0, 3) == 3
    assert kernels._slices(0, 0, 5) == 1


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="missing"):
        _clib.load(tmp_path / "libg16.so")


def test_get_kernel_names_match_reference_kernels():
    assert set(kernels.KERNELS) == {"rowscale_f32", "rowscale_f16", "hgemm_f32out", "hgemm_f16out",
                                    "hgemm_splitk", "skinny_f32in", "skinny_f16in"}
    k = kernels.get_kernel("hgemm_f32out")
    assert k.name == "hgemm_f32out" and k.fn is not None and kernels.get_kernel("hgemm_f32out") is k
    with pytest.raises(KeyError):
        kernels.get_kernel("hgemm")


def test_decode_layout_route_rule(lib):
    # g16_skinny_strips_route: the measured rule for FastLinear's decode layout (M <= 2 always; M = 3,
    # 4 for weights up to 2^22 elements; beyond that only fp16 activations, M = 4 up to N = 8192)
    r = lib.g16_skinny_strips_route
    assert r(1, 4096, 4096, 1) == 1 and r(2, 14336, 4096, 1) == 1 and r(1, 8, 8, 0) == 1
    assert r(3, 2048, 2048, 1) == 1 and r(4, 1024, 3072, 1) == 1
    assert r(3, 4096, 4096, 1) == 0 and r(4, 4096, 4096, 1) == 0
    assert r(3, 4096, 4096, 0) == 1 and r(4, 4096, 4096, 0) == 1 and r(3, 14336, 4096, 0) == 1
    assert r(4, 11008, 4096, 0) == 0 and r(4, 8192, 8192, 0) == 1
    assert r(5, 64, 64, 0) == 0 and r(0, 64, 64, 1) == 0 and r(1, 0, 64, 1) == 0 and r(1, 64, 0, 1) == 0
