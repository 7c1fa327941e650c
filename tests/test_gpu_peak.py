"""GPU smoke tests of the peak microbenchmark entry points (bench.py --peak): every kind runs,
returns OK and leaves finite values; the stream read covers the buffer it is given."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib(cuda):
    from gtx16_fp16 import _clib

    return _clib.load()


@pytest.mark.parametrize("kind", [0, 1, 2, 3, 4, 5, 6, 7])
def test_peak_kernels_run(lib, cuda, kind):
    blocks = 8
    out = torch.full((blocks * 256,), float("nan"), device=cuda)
    st = torch.cuda.current_stream(cuda).cuda_stream
    assert lib.g16_peak_run(kind, blocks, 10, out.data_ptr(), st) == 0
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert lib.g16_peak_flops_per_lane_iter(kind) > 0


@pytest.mark.parametrize("kind", [0, 4, 6])
def test_peak_clock_readout(lib, cuda, kind):
    # workgroup 0's loop: shader cycles and 100 MHz reference ticks give a clock in the part's range
    blocks, iters = 8, 20000
    out = torch.empty(blocks * 256, device=cuda)
    clocks = torch.zeros(2, dtype=torch.int64, device=cuda)
    st = torch.cuda.current_stream(cuda).cuda_stream
    assert lib.g16_peak_run_clocked(kind, blocks, iters, out.data_ptr(), clocks.data_ptr(), st) == 0
    torch.cuda.synchronize()
    cyc, ticks = clocks.tolist()
    assert cyc > 0 and ticks > 0
    assert 300.0 < 100.0 * cyc / ticks < 3500.0
    assert torch.isfinite(out).all()


def test_peak_fp32_fma_value(lib, cuda):
    # x <- fma(x, a, b) with a = 0.999, b = 0.001, 8 chains seeded tid + i, summed: an fp32 model
    blocks, iters = 1, 7
    out = torch.empty(blocks * 256, device=cuda)
    st = torch.cuda.current_stream(cuda).cuda_stream
    assert lib.g16_peak_run(0, blocks, iters, out.data_ptr(), st) == 0
    torch.cuda.synchronize()
    a, b = np.float32(0.999), np.float32(0.001)
    x = (np.arange(256, dtype=np.float64)[:, None] + np.arange(8)[None, :]).astype(np.float32)
    for _ in range(iters):  # fmaf: one rounding of the exact product-sum
        x = (x.astype(np.float64) * np.float64(a) + np.float64(b)).astype(np.float32)
    s = np.zeros(256, dtype=np.float32)
    for i in range(8):
        s = (s + x[:, i]).astype(np.float32)
    assert np.array_equal(out.cpu().numpy(), s)


@pytest.mark.parametrize("iters", [1, 3])
def test_peak_lds_read_value(lib, cuda, iters):
    # kind 6: word 4i of the 32 KB buffer holds i + 1; lane t reads 16-byte elements
    # t + 256 d (d < 8) every iteration and XORs their first words
    blocks = 2
    out = torch.empty(blocks * 256, device=cuda)
    st = torch.cuda.current_stream(cuda).cuda_stream
    assert lib.g16_peak_run(6, blocks, iters, out.data_ptr(), st) == 0
    torch.cuda.synchronize()
    t = np.arange(256, dtype=np.uint32)
    acc = np.zeros(256, dtype=np.uint32)
    for it in range(iters):
        for d in range(8):
            acc ^= t + 256 * d + 1
    want = np.tile((acc & 0xFF).astype(np.float32), blocks)
    assert np.array_equal(out.cpu().numpy(), want)


def test_stream_read_and_rejects(lib, cuda):
    buf = torch.ones(1 << 20, dtype=torch.uint8, device=cuda)
    out = torch.empty(4 * 256, device=cuda)
    st = torch.cuda.current_stream(cuda).cuda_stream
    assert lib.g16_stream_read(buf.data_ptr(), buf.numel(), 4, out.data_ptr(), st) == 0
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert lib.g16_stream_read(buf.data_ptr(), 17, 4, out.data_ptr(), st) == -1
    assert lib.g16_peak_run(9, 1, 1, out.data_ptr(), st) == -6
