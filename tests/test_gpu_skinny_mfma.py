"""Skinny path, M = 8 on the matrix cores (skinny.hip's MF form) against the oracle.

mm_t with M = 8 and N <= 8192 runs the split skinny kernel; where each wavefront gets 32..128 K rows
its multiplies run as v_mfma_f32_16x16x32_f16 on an fp16 hi/lo split of the row-scaled activations
(reference semantics: fp32 math on the unquantised activations, kernels.py:160-219). The shapes below
take that form (checked from the plan); the bar is the skinny bar of every other skinny test, and
infinities and NaNs must land where the oracle's fp64 products put them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _inputs import randn

pytestmark = pytest.mark.gpu

SKINNY_TOL = 1e-5


@pytest.fixture(scope="module")
def g():
    import gtx16_fp16
    return gtx16_fp16


@pytest.fixture(scope="module")
def lib():
    from gtx16_fp16 import _clib
    return _clib.load()


@pytest.fixture(scope="module")
def cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def _rows_per_wave(lib, cuda, M, N, K):
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    ks = lib.g16_skinny_plan(M, N, K, cus)
    return -(-(-(-K // ks)) // 8), ks


def _takes_matrix_cores(lib, cuda, M, N, K):
    # use_mf in skinny.hip: M = 8, 256-column strips (N <= 8192), 32..128 K rows per wavefront
    rpw, _ = _rows_per_wave(lib, cuda, M, N, K)
    return M == 8 and lib.g16_skinny_strip_cols(M, N) == 256 and 32 <= rpw <= 128


def _same_nonfinite_pattern(got, want):
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isposinf(got), np.isposinf(want))
    assert np.array_equal(np.isneginf(got), np.isneginf(want))
    fin = np.isfinite(want)
    if fin.any():
        assert oracle.rel_err(got[fin], want[fin]) <= SKINNY_TOL


# K x N: one batch per wavefront (4096^2, 16384 x 1024), two (4096 x 8192), three with a partial last
# one (11008 x 4096: 86 rows), and a last strip of 8 columns with 64-row wavefronts (12288 x 2056)
MF_SHAPES = [(4096, 4096), (16384, 1024), (4096, 8192), (11008, 4096), (12288, 2056)]


@pytest.mark.parametrize("K,N", MF_SHAPES)
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("with_bias", [False, True])
def test_m8_matrix_core_matches_oracle(g, lib, cuda, K, N, x_dtype, with_bias):
    M = 8
    assert _takes_matrix_cores(lib, cuda, M, N, K)
    x = randn((M, K), seed=K + N, dtype=torch.float32)
    x[1, ::97] *= 3e4 if x_dtype == torch.float32 else 5e3  # a wide row (its scale follows the largest)
    x[5] = 0.0                               # an all-zero row
    if x_dtype == torch.float32:
        x[2] *= 1e-30                        # rows far from fp16's range, scaled exactly
        x[3] *= 1e20
    x = x.to(x_dtype)
    w = randn((K, N), seed=K, scale=0.02, dtype=torch.float16)
    b = randn((N,), seed=N, scale=0.02) if with_bias else None
    y = g.mm_t(x.to(cuda), w.to(cuda), None if b is None else b.to(cuda), torch.float32)
    torch.cuda.synchronize()
    ref = oracle.skinny(_np(x), _np(w), None if b is None else _np(b))
    assert np.isfinite(_np(y)).all()
    assert oracle.rel_err(_np(y), ref) <= SKINNY_TOL
    # each row on its own scale: the tiny and huge rows are as accurate as the others
    for m in (1, 2, 3):
        if np.linalg.norm(ref[m]) > 0:
            assert oracle.rel_err(_np(y)[m], ref[m]) <= SKINNY_TOL, m
    assert not _np(y)[5].any() or with_bias


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.float16])
def test_m8_matrix_core_nonfinite_weights(lib, cuda, x_dtype):
    # +-inf and NaN weights against activations that are positive, zero, exactly representable in
    # fp16 (a hi/lo split with a zero lo part) or tiny: the products must be the fp64 oracle's
    # infinities and NaNs (inf * 0 = NaN, inf + -inf = NaN), never a NaN from a zero split part
    M, K, N = 8, 16384, 1024
    assert _takes_matrix_cores(lib, cuda, M, N, K)
    x = randn((M, K), seed=5).abs() + 0.25
    x[:, 100] = 0.0
    x[:, 37] = 1.5
    if x_dtype == torch.float32:
        x[:, 38] = 1e-30
    x = x.to(x_dtype)
    w = randn((K, N), seed=6, scale=0.02, dtype=torch.float16)
    for (k, n, v) in [(0, 3, "inf"), (31, 7, "-inf"), (100, 11, "inf"), (K - 1, 13, "inf"), (2048, 17, "nan"),
                      (5, 19, "inf"), (6, 19, "-inf"), (37, 23, "-inf"), (38, 29, "inf"), (32, 31, "inf")]:
        w[k, n] = float(v)
    _, ks = _rows_per_wave(lib, cuda, M, N, K)
    xd, wd = x.to(cuda), w.to(cuda)
    part = torch.empty(max(lib.g16_skinny_workspace_bytes(M, N, K, ks), 16), dtype=torch.uint8, device=cuda)
    cnt = torch.zeros(max(lib.g16_skinny_counter_bytes(M, N, K, ks), 256), dtype=torch.uint8, device=cuda)
    out = torch.full((M, N), float("nan"), device=cuda)
    st = torch.cuda.current_stream(cuda).cuda_stream
    fn = lib.g16_skinny_f32in if x_dtype == torch.float32 else lib.g16_skinny_f16in
    assert fn(xd.data_ptr(), wd.data_ptr(), out.data_ptr(), None, M, N, K, ks, part.data_ptr(), part.numel(),
              cnt.data_ptr(), cnt.numel(), st) == 0
    torch.cuda.synchronize()
    with np.errstate(invalid="ignore"):  # inf * 0 and inf - inf in the fp64 oracle: expected NaNs
        want = oracle.skinny(_np(x), _np(w), None)
    assert not np.isfinite(want).all()
    _same_nonfinite_pattern(_np(out), want)


def test_m8_matrix_core_repeat_runs_bitwise_equal(lib, cuda):
    M, K, N = 8, 11008, 4096
    assert _takes_matrix_cores(lib, cuda, M, N, K)
    _, ks = _rows_per_wave(lib, cuda, M, N, K)
    x = randn((M, K), seed=1).to(cuda)
    w = randn((K, N), seed=2, scale=0.02, dtype=torch.float16).to(cuda)
    b = randn((N,), seed=3, scale=0.02).to(cuda)
    part = torch.empty(max(lib.g16_skinny_workspace_bytes(M, N, K, ks), 16), dtype=torch.uint8, device=cuda)
    cnt = torch.zeros(max(lib.g16_skinny_counter_bytes(M, N, K, ks), 256), dtype=torch.uint8, device=cuda)
    st = torch.cuda.current_stream(cuda).cuda_stream
    outs = []
    for _ in range(4):
        c = torch.full((M, N), float("nan"), device=cuda)
        assert lib.g16_skinny_f32in(x.data_ptr(), w.data_ptr(), c.data_ptr(), b.data_ptr(), M, N, K, ks,
                                    part.data_ptr(), part.numel(), cnt.data_ptr(), cnt.numel(), st) == 0
        outs.append(c)
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    assert oracle.rel_err(_np(outs[0]), oracle.skinny(_np(x), _np(w), _np(b))) <= SKINNY_TOL


def test_m8_one_wavefront_with_an_infinity_falls_back(g, lib, cuda):
    # An inf among one wavefront's activations sends that wavefront (only) to the fp32 FMA loop; its
    # partial sums and the matrix-core ones of the others add up to the oracle's answer: +-inf where
    # the row meets it, finite elsewhere
    M, K, N = 8, 4096, 4096
    assert _takes_matrix_cores(lib, cuda, M, N, K)
    x = randn((M, K), seed=9)
    x[4, 40] = float("inf")
    w = randn((K, N), seed=10, scale=0.02, dtype=torch.float16)
    y = g.mm_t(x.to(cuda), w.to(cuda), None, torch.float32)
    torch.cuda.synchronize()
    want = oracle.skinny(_np(x), _np(w), None)
    _same_nonfinite_pattern(_np(y), want)
    assert np.isfinite(_np(y)[[0, 1, 2, 3, 5, 6, 7]]).all()
