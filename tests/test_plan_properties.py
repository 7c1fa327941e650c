"""CPU property tests of the launch plans (g16_hgemm_plan, g16_skinny_plan): for any shape the
plans stay inside the limits the kernels and their buffers are sized for, and the plan, the tile
and the buffer sizes the library reports agree with each other. No GPU needed: the plans are host
functions of the library. The tile is read from the library (its split-buffer sizes), not
recomputed here."""
from __future__ import annotations

import pytest

hypothesis = pytest.importorskip("hypothesis")
from hypothesis import given, settings, strategies as st  # noqa: E402

from gtx16_fp16 import _clib  # noqa: E402
from _plan import tile as planned_tile  # noqa: E402


@pytest.fixture(scope="module")
def lib():
    return _clib.load()


def _ceil(a: int, b: int) -> int:
    return -(-a // b)


# The GEMM tiles the library has kernels for, by (rows, columns).
TILES = {(32, 128), (64, 128), (64, 64), (128, 128), (256, 128), (256, 256)}


def _tile(lib, M: int, N: int, K: int, num_cus: int) -> tuple[int, int, int]:
    """(rows, columns, count) of the tile the library plans for this shape on num_cus CUs, from
    g16_hgemm_tile, checked against the library's own split-buffer sizes for a 2-way split (the tile
    does not depend on the split): the counters hold one 256-byte line per tile and the partials
    2 slices x tile x 4 bytes. (Split slices start on multiples of 64 K, so K < 128 cannot split
    and has no split sizes to check.)"""
    bm, bn = planned_tile(lib, M, N, K, num_cus)
    ntiles = _ceil(M, bm) * _ceil(N, bn)
    if K >= 128:
        assert lib.g16_hgemm_splitk_counter_bytes(M, N, K, 2, num_cus) == ntiles * 256
        assert lib.g16_hgemm_splitk_workspace_bytes(M, N, K, 2, num_cus) == ntiles * 2 * bm * bn * 4
    return bm, bn, ntiles


dims = st.integers(min_value=1, max_value=1 << 15).map(lambda v: v * 8)
cus = st.sampled_from([64, 120, 256, 304])


@settings(max_examples=400, deadline=None)
@given(M=st.integers(min_value=9, max_value=70000), N=dims, K=dims, num_cus=cus)
def test_gemm_plan_limits(lib, M, N, K, num_cus):
    ks = lib.g16_hgemm_plan(M, N, K, num_cus)
    bm, bn, tiles = _tile(lib, M, N, K, num_cus)
    # one of the compiled tiles, covering the output exactly once
    assert (bm, bn) in TILES
    assert tiles == _ceil(M, bm) * _ceil(N, bn)
    # a 256-row tile only where the rows fill it at least twice over; tiles never taller than
    # needed below that (32-row tiles serve M <= 32)
    assert bm < 256 or M >= 512
    assert M > 32 or bm == 32
    # the packed route is exactly the unsplit 256-row tiles (their packed stage images)
    assert lib.g16_hgemm_use_packed(M, N, K, num_cus) == (1 if (bm == 256 and ks == 1) else 0)
    assert 1 <= ks <= 8
    # the 4-wavefront tiles' grid fits one round of the CUs whenever one of them can
    if 32 < M and bm < 256 and min(_ceil(M, r) * _ceil(N, c) for r, c in TILES if r < 256) <= num_cus:
        assert tiles * ks <= num_cus
    if ks > 1:
        # split only when tiles leave CUs idle, never past one workgroup per CU, >= 256 K a slice
        assert tiles < num_cus
        assert tiles * ks <= num_cus
        assert _ceil(K, ks) >= 256
        assert lib.g16_hgemm_splitk_workspace_bytes(M, N, K, ks, num_cus) == tiles * ks * bm * bn * 4
        assert lib.g16_hgemm_splitk_counter_bytes(M, N, K, ks, num_cus) == tiles * 256
    # the one-call path's scratch holds the cast (row-major, or packed in 256-row blocks of 32-wide
    # K steps) plus the row scales; none where the unsplit 32x128 tile keeps the cast in LDS
    # (K <= 1280: 20 K steps of 64)
    if bm == 32 and ks == 1 and K <= 1280:
        assert lib.g16_mm_t_scratch_bytes(M, N, K, num_cus) == 0
    else:
        cast = (_ceil(M, 256) * 256 * _ceil(K, 32) * 32 * 2 if ks == 1 and bm == 256 else M * K * 2)
        assert lib.g16_mm_t_scratch_bytes(M, N, K, num_cus) == _ceil(cast, 256) * 256 + 4 * M


@settings(max_examples=400, deadline=None)
@given(M=st.integers(min_value=1, max_value=8), N=dims, K=dims, num_cus=cus)
def test_skinny_plan_limits(lib, M, N, K, num_cus):
    ks = lib.g16_skinny_plan(M, N, K, num_cus)
    cols = lib.g16_skinny_strip_cols(M, N)
    assert cols in (256, 512)
    strips = _ceil(N, cols)
    assert ks >= 1
    # every wavefront gets rows (8 wavefronts per slice), and the grid stays within one
    # workgroup per CU whenever the strips alone do
    assert ks * 8 <= max(K, 8)
    if strips <= num_cus:
        assert strips * ks <= num_cus
    ws = lib.g16_skinny_workspace_bytes(M, N, K, ks)
    assert ws == (0 if ks == 1 else ks * M * N * 4)
    # one 256-byte counter line per strip
    assert lib.g16_skinny_counter_bytes(M, N, K, ks) == (0 if ks == 1 else strips * 256)
