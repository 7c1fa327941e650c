"""GPU parity at the size limits of the GEMM entry points (include/g16.h: K <= G16_GEMM_MAX_K =
2^22 - 8 and N <= G16_GEMM_MAX_N = 2^24 - 8, set by the 32-bit offsets of the kernels' buffer
descriptors), where an offset computed in too narrow a type would read zeros or drop stores without
any error. Operands are generated on the GPU; rows (and columns) are independent, so the fp64
oracle runs on sampled rows and columns, always including the first and last ones.

* mm_t at K = G16_GEMM_MAX_K on the split 32x128 tile (fp16 and fp32 activations: the row-major
  cast scratch is then 512 MiB) and on the split 128x128 tile (a 4 GiB cast scratch);
* the tile-packed 256x256 GEMM through the C ABI at K = G16_GEMM_MAX_K: the last K step's packed
  offset is 2^31 - 16 KiB, the descriptor's last 16 KiB;
* mm_t at N = G16_GEMM_MAX_N on the 32x128 and 64x128 tiles and on the skinny path (M = 1 and 8);
* an fp32 output of 2 GiB (M = 512, N = 2^20).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

MAX_K = (1 << 22) - 8
MAX_N = (1 << 24) - 8
GEMM_TOL = 1e-3
SKINNY_TOL = 1e-5


@pytest.fixture(scope="module")
def g(cuda):
    import gtx16_fp16

    return gtx16_fp16


@pytest.fixture(scope="module")
def lib(cuda):
    from gtx16_fp16 import _clib

    return _clib.load()


@pytest.fixture(autouse=True)
def _free(cuda):
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _gen(shape, seed, dtype, device, scale=1.0):
    gen = torch.Generator(device=device).manual_seed(seed)
    t = torch.randn(shape, generator=gen, device=device, dtype=dtype)
    return t.mul_(scale) if scale != 1.0 else t


def _sample(n, k, seed):
    idx = np.random.default_rng(seed).choice(n, min(k, n), replace=False)
    return np.unique(np.concatenate([idx, [0, n - 1]]))


def _check(y, x, w, b, rows, cols):
    # the sampled block of y, with the rows of x and the columns of w and b it depends on
    xr = x[torch.from_numpy(rows).to(x.device)].cpu().numpy()
    wc = w[:, torch.from_numpy(cols).to(w.device)].cpu().numpy()
    bc = None if b is None else b[torch.from_numpy(cols).to(b.device)].cpu().numpy()
    got = y[torch.from_numpy(rows).to(y.device)][:, torch.from_numpy(cols).to(y.device)].float().cpu().numpy()
    return got, xr, wc, bc


@pytest.mark.parametrize("x_dtype", [torch.float16, torch.float32])
def test_mm_t_at_max_k_on_the_split_32x128_tile(g, lib, cuda, x_dtype):
    M, K, N = 64, MAX_K, 128
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    assert lib.g16_hgemm_plan(M, N, K, cus) > 1
    x = _gen((M, K), 1, x_dtype, cuda)
    x[3, K - 1] = 3.0e4  # a rescaled row whose largest value sits in the last K step
    w = _gen((K, N), 2, torch.float16, cuda, 0.02)
    b = _gen((N,), 3, torch.float32, cuda, 0.02)
    y = g.mm_t(x, w, b, torch.float32)
    torch.cuda.synchronize()
    rows, cols = np.array([0, 3, 31, 32, M - 1]), _sample(N, 24, 4)
    got, xr, wc, bc = _check(y, x, w, b, rows, cols)
    # the GEMM semantics of the full call (M > 8): rowscale the sampled rows, then the quantised GEMM
    y16, S, _ = oracle.rowscale(xr)
    want = oracle.gemm(y16, S, wc, bc, "float32")
    assert np.isfinite(got).all()
    assert oracle.rel_err(got, want) <= GEMM_TOL


def test_mm_t_at_max_k_on_the_split_128x128_tile(g, lib, cuda):
    M, K, N = 512, MAX_K, 1024
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    assert lib.g16_hgemm_plan(M, N, K, cus) > 1
    x = _gen((M, K), 5, torch.float16, cuda)
    w = _gen((K, N), 6, torch.float16, cuda, 0.02)
    y = g.mm_t(x, w, None, torch.float32)
    torch.cuda.synchronize()
    rows, cols = _sample(M, 6, 7), _sample(N, 14, 8)
    got, xr, wc, _ = _check(y, x, w, None, rows, cols)
    y16, S, _ = oracle.rowscale(xr)
    assert oracle.rel_err(got, oracle.gemm(y16, S, wc, None, "float32")) <= GEMM_TOL


def test_packed_gemm_at_max_k(lib, cuda):
    M, K, N = 256, MAX_K, 256
    st = torch.cuda.current_stream(cuda).cuda_stream
    x = _gen((M, K), 9, torch.float16, cuda)
    x[200, K - 5] = -5.0e3
    w = _gen((K, N), 10, torch.float16, cuda, 0.02)
    xp = torch.empty(lib.g16_packed_a_bytes(M, K) // 2, dtype=torch.float16, device=cuda)
    s = torch.empty(M, dtype=torch.float32, device=cuda)
    c = torch.full((M, N), float("nan"), device=cuda)
    assert lib.g16_rowscale_pack_f16(x.data_ptr(), xp.data_ptr(), s.data_ptr(), M, K, 1024.0, st) == 0
    assert lib.g16_hgemm_packed_f32out(xp.data_ptr(), w.data_ptr(), c.data_ptr(), None, s.data_ptr(), M, N, K, st) == 0
    torch.cuda.synchronize()
    rows, cols = np.array([0, 1, 127, 200, 255]), _sample(N, 14, 11)
    got, xr, wc, _ = _check(c, x, w, None, rows, cols)
    y16, S, _ = oracle.rowscale(xr)
    assert np.array_equal(s.cpu().numpy()[rows], S)
    assert oracle.rel_err(got, oracle.gemm(y16, S, wc, None, "float32")) <= GEMM_TOL


@pytest.mark.parametrize("M", [16, 64])
def test_mm_t_at_max_n(g, cuda, M):
    K, N = 64, MAX_N
    x = _gen((M, K), 12, torch.float32, cuda)
    w = _gen((K, N), 13, torch.float16, cuda, 0.02)
    b = _gen((N,), 14, torch.float32, cuda, 0.02)
    y = g.mm_t(x, w, b, torch.float32)
    torch.cuda.synchronize()
    rows = np.arange(M)
    cols = np.unique(np.concatenate([np.arange(64), np.arange(N - 64, N), _sample(N, 256, 15)]))
    got, xr, wc, bc = _check(y, x, w, b, rows, cols)
    assert oracle.rel_err(got, oracle.mm_t(xr, wc, bc, "float32")) <= GEMM_TOL


@pytest.mark.parametrize("M", [1, 8])
def test_skinny_at_max_n(g, cuda, M):
    K, N = 64, MAX_N
    x = _gen((M, K), 16, torch.float32, cuda)
    w = _gen((K, N), 17, torch.float16, cuda, 0.02)
    b = _gen((N,), 18, torch.float32, cuda, 0.02)
    y = g.mm_t(x, w, b, torch.float32)
    torch.cuda.synchronize()
    rows = np.arange(M)
    cols = np.unique(np.concatenate([np.arange(64), np.arange(N - 64, N), _sample(N, 256, 19)]))
    got, xr, wc, bc = _check(y, x, w, b, rows, cols)
    assert oracle.rel_err(got, oracle.mm_t(xr, wc, bc, "float32")) <= SKINNY_TOL


def test_mm_t_with_a_2_gib_output(g, cuda):
    M, K, N = 512, 264, 1 << 20
    x = _gen((M, K), 20, torch.float32, cuda)
    w = _gen((K, N), 21, torch.float16, cuda, 0.02)
    y = g.mm_t(x, w, None, torch.float32)
    torch.cuda.synchronize()
    assert y.numel() * 4 == 1 << 31
    rows = _sample(M, 14, 22)
    cols = np.unique(np.concatenate([np.arange(32), np.arange(N - 32, N), _sample(N, 128, 23)]))
    got, xr, wc, _ = _check(y, x, w, None, rows, cols)
    y16, S, _ = oracle.rowscale(xr)
    assert oracle.rel_err(got, oracle.gemm(y16, S, wc, None, "float32")) <= GEMM_TOL
