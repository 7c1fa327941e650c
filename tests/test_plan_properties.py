"""CPU property tests of the launch plans (g16_hgemm_plan, g16_skinny_plan): for any shape the
plans stay inside the limits the kernels and their buffers are sized for. No GPU needed: the plans
are host functions of the library."""
from __future__ import annotations

import pytest

hypothesis = pytest.importorskip("hypothesis")
from hypothesis import given, settings, strategies as st  # noqa: E402

from gtx16_fp16 import _clib  # noqa: E402


@pytest.fixture(scope="module")
def lib():
    return _clib.load()


def _ceil(a: int, b: int) -> int:
    return -(-a // b)


def _tiles(M: int, N: int, K: int, num_cus: int) -> int:
    # the library's tile choice (choose_tile): 32x128, 64x128, 256x256, 256x128 or 128x128
    if M <= 32:
        return _ceil(N, 128)
    if M <= 64:  # two rows of 32x128 tiles while they fill at most half the CUs, else 64x128
        return 2 * _ceil(N, 128) if 4 * _ceil(N, 128) <= num_cus else _ceil(N, 128)
    t256 = _ceil(M, 256) * _ceil(N, 256)
    if M >= 1024 and N >= 256 and 2 * t256 > num_cus:
        return t256
    if M >= 1024 and N >= 256 and 8 * t256 > 3 * num_cus:
        return _ceil(M, 256) * _ceil(N, 128)
    for bm in (32, 64):  # short K: the smallest 4-wavefront tile whose grid fits one round
        if K <= 3072 and _ceil(M, bm) * _ceil(N, 128) <= num_cus:
            return _ceil(M, bm) * _ceil(N, 128)
    return _ceil(M, 128) * _ceil(N, 128)


dims = st.integers(min_value=1, max_value=1 << 15).map(lambda v: v * 8)
cus = st.sampled_from([64, 120, 256, 304])


@settings(max_examples=400, deadline=None)
@given(M=st.integers(min_value=9, max_value=70000), N=dims, K=dims, num_cus=cus)
def test_gemm_plan_limits(lib, M, N, K, num_cus):
    ks = lib.g16_hgemm_plan(M, N, K, num_cus)
    tiles = _tiles(M, N, K, num_cus)
    assert 1 <= ks <= 8
    if ks > 1:
        # split only when tiles leave CUs idle, never past one workgroup per CU, >= 256 K a slice
        assert tiles < num_cus
        assert tiles * ks <= num_cus
        assert _ceil(K, ks) >= 256
        assert lib.g16_hgemm_use_packed(M, N, K, num_cus) == 0
        assert lib.g16_hgemm_splitk_workspace_bytes(M, N, K, ks) > 0
        assert lib.g16_hgemm_splitk_counter_bytes(M, N, K, ks) > 0


@settings(max_examples=400, deadline=None)
@given(M=st.integers(min_value=1, max_value=8), N=dims, K=dims, num_cus=cus)
def test_skinny_plan_limits(lib, M, N, K, num_cus):
    ks = lib.g16_skinny_plan(M, N, K, num_cus)
    strips = _ceil(N, 512)
    assert ks >= 1
    # every wavefront gets rows (8 wavefronts per slice), and the grid stays within one
    # workgroup per CU whenever the strips alone do
    assert ks * 8 <= max(K, 8)
    if strips <= num_cus:
        assert strips * ks <= num_cus
    ws = lib.g16_skinny_workspace_bytes(M, N, K, ks)
    assert ws == (0 if ks == 1 else ks * M * N * 4)
