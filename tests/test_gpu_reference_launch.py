"""GPU tests of the reference's launch interface (src/gtx16_fp16/kernels.py:299-355): each of the
seven kernels obtained with ``get_kernel`` and launched through ``launch`` or ``PreparedLaunch``
with the grid, block and argument list the reference's own call sites build (ops.py:78-108,
linear.py:49-64), checked against the fp64 oracle: the rowscale cast bit for bit, the GEMMs within
a relative Frobenius error of 1e-3 and the skinny kernels within 1e-5 (the tolerances of the other
parity tests)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _inputs import randn

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-3
SKINNY_TOL = 1e-5


@pytest.fixture(scope="module")
def k(cuda):
    from gtx16_fp16 import kernels

    return kernels


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def _cast(k, x, cuda):
    """ops.py:86-90: the rowscale launch with grid (M, 1, 1)."""
    M, K = x.shape
    x16 = torch.empty(M, K, device=cuda, dtype=torch.float16)
    rscale = torch.empty(M, device=cuda, dtype=torch.float32)
    name = "rowscale_f32" if x.dtype == torch.float32 else "rowscale_f16"
    k.launch(k.get_kernel(name, cuda), (M, 1, 1), (256, 1, 1), [x, x16, rscale, K, 1024.0],
             k.stream_handle(cuda.index or 0))
    return x16, rscale


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_rowscale_launch_is_bitwise_the_oracle_cast(k, cuda, dtype):
    x = randn((96, 1032), seed=3, dtype=dtype)
    x[5] *= 3000.0  # a rescaled row
    x[17, 40] = float("inf")
    xd = x.to(cuda)
    x16, rscale = _cast(k, xd, cuda)
    torch.cuda.synchronize()
    y16, S, _ = oracle.rowscale(_np(x))
    assert np.array_equal(_np(x16).view(np.uint16), y16.view(np.uint16))
    assert np.array_equal(_np(rscale), S)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_hgemm_launch_as_ops_builds_it(k, cuda, out_dtype):
    # ops.py:103-108: grid ((N+127)/128, (M+127)/128, 1), [x16, w_t, out, b, rscale, M, N, K]
    M, K, N = 320, 1024, 384
    x = randn((M, K), seed=0).to(cuda)
    x[7] *= 5000.0
    w = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).to(cuda)
    b = randn((N,), seed=2, scale=0.02).to(cuda)
    x16, rscale = _cast(k, x, cuda)
    out = torch.empty(M, N, device=cuda, dtype=out_dtype)
    name = "hgemm_f32out" if out_dtype == torch.float32 else "hgemm_f16out"
    k.launch(k.get_kernel(name, cuda), ((N + 127) // 128, (M + 127) // 128, 1), (256, 1, 1),
             [x16, w, out, b, rscale, M, N, K], k.stream_handle(cuda.index or 0))
    torch.cuda.synchronize()
    ref = oracle.mm_t(_np(x), _np(w), _np(b), "float32" if out_dtype == torch.float32 else "float16")
    assert oracle.rel_err(_np(out), ref) <= GEMM_TOL


@pytest.mark.parametrize("with_bias", [True, False])
def test_hgemm_splitk_launch_adds_into_the_prefilled_output(k, cuda, with_bias):
    # ops.py:92-101: out prefilled with the bias rows (or zeros), the split launch adds the product
    M, K, N = 64, 4096, 1024
    x = randn((M, K), seed=4).to(cuda)
    w = randn((K, N), seed=5, scale=0.02, dtype=torch.float16).to(cuda)
    b = randn((N,), seed=6, scale=0.02).to(cuda) if with_bias else None
    x16, rscale = _cast(k, x, cuda)
    tiles = ((N + 127) // 128) * ((M + 127) // 128)
    sms = torch.cuda.get_device_properties(cuda).multi_processor_count
    ksplit = min((2 * sms + tiles - 1) // tiles, K // 128)
    kchunk = ((K + ksplit - 1) // ksplit + 15) // 16 * 16
    ksplit = (K + kchunk - 1) // kchunk
    out = torch.empty(M, N, device=cuda, dtype=torch.float32)
    if b is None:
        out.zero_()
    else:
        out.copy_(b.float().expand(M, N))
    k.launch(k.get_kernel("hgemm_splitk", cuda), ((N + 127) // 128, (M + 127) // 128, ksplit), (256, 1, 1),
             [x16, w, out, rscale, M, N, K, kchunk], k.stream_handle(cuda.index or 0))
    torch.cuda.synchronize()
    ref = oracle.mm_t(_np(x), _np(w), None if b is None else _np(b), "float32")
    assert oracle.rel_err(_np(out), ref) <= GEMM_TOL
    # a second launch adds the product again, as the reference's atomics would
    k.launch(k.get_kernel("hgemm_splitk", cuda), ((N + 127) // 128, (M + 127) // 128, ksplit), (256, 1, 1),
             [x16, w, out, rscale, M, N, K, kchunk], k.stream_handle(cuda.index or 0))
    torch.cuda.synchronize()
    twice = oracle.mm_t(_np(x), _np(w), None, "float32").astype(np.float64) * 2.0
    if b is not None:
        twice = twice + _np(b).astype(np.float64)[None, :]
    assert oracle.rel_err(_np(out), twice) <= GEMM_TOL


@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (4, 1024, 3072), (8, 3072, 1024)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_skinny_launch_as_ops_builds_it(k, cuda, M, K, N, dtype):
    # ops.py:78-84: zeroed fp32 out, grid and kchunk from skinny_config
    from gtx16_fp16.ops import skinny_config

    x = randn((M, K), seed=7, dtype=dtype).to(cuda)
    w = randn((K, N), seed=8, scale=0.02, dtype=torch.float16).to(cuda)
    b = randn((N,), seed=9, scale=0.02).to(cuda)
    sms = torch.cuda.get_device_properties(cuda).multi_processor_count
    grid, kchunk = skinny_config(N, K, sms)
    out = torch.zeros(M, N, device=cuda, dtype=torch.float32)
    name = "skinny_f32in" if dtype == torch.float32 else "skinny_f16in"
    k.launch(k.get_kernel(name, cuda), grid, (256, 1, 1), [x, w, out, b, M, N, K, kchunk],
             k.stream_handle(cuda.index or 0))
    torch.cuda.synchronize()
    assert oracle.rel_err(_np(out), oracle.skinny(_np(x), _np(w), _np(b))) <= SKINNY_TOL


def test_prepared_skinny_launch_as_linear_builds_it(k, cuda):
    # linear.py:55-63: a PreparedLaunch of skinny_f32in with kinds "ppppiiii", called with the
    # stream handle and raw pointers; repeated calls give the same bits
    from gtx16_fp16.ops import skinny_config

    M, K, N = 2, 1024, 768
    x = randn((M, K), seed=10).to(cuda)
    w = randn((K, N), seed=11, scale=0.02, dtype=torch.float16).to(cuda)
    sms = torch.cuda.get_device_properties(cuda).multi_processor_count
    grid, kchunk = skinny_config(N, K, sms)
    pl = k.PreparedLaunch(k.get_kernel("skinny_f32in", cuda), grid, (256, 1, 1), "ppppiiii")
    outs = []
    for _ in range(3):
        out = torch.zeros(M, N, device=cuda, dtype=torch.float32)
        pl(k.stream_handle(cuda.index or 0), x.data_ptr(), w.data_ptr(), out.data_ptr(), None, M, N, K, kchunk)
        outs.append(out)
    torch.cuda.synchronize()
    assert oracle.rel_err(_np(outs[0]), oracle.skinny(_np(x), _np(w))) <= SKINNY_TOL
    assert all(torch.equal(o, outs[0]) for o in outs[1:])
