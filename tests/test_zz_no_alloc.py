"""GPU test of g16_skinny_f32in_noalloc, the allocation-free variant of g16_skinny_f32in: through the
C ABI, its output is bitwise equal to the buffered entry point's on the same plan (same kernels,
same summation order), on consecutive calls whose second input is smaller than the first (the
static scratch keeps the first call's contents), and within 1e-5 of the fp64 oracle. The first call
is M = 8 at 4096^2, which runs the matrix-core form of the skinny kernel (16 K slices on 256-column
strips); the FMA-loop form follows at M = 4 and M = 1. Splits that do not fit the static scratch are
refused before any launch."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _inputs import randn

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib(cuda):
    from gtx16_fp16 import _clib

    return _clib.load()


def _buffered(lib, x, w, b, ks, st):
    M, K = x.shape
    N = w.shape[1]
    ws = torch.empty(max(lib.g16_skinny_workspace_bytes(M, N, K, ks), 16), dtype=torch.uint8, device=x.device)
    cnt = torch.zeros(max(lib.g16_skinny_counter_bytes(M, N, K, ks), 16), dtype=torch.uint8, device=x.device)
    out = torch.empty(M, N, device=x.device)
    assert lib.g16_skinny_f32in(x.data_ptr(), w.data_ptr(), out.data_ptr(), b.data_ptr(), M, N, K, ks,
                                ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(), st) == 0
    return out


def test_noalloc_matches_the_buffered_entry_point(lib, cuda):
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    st = torch.cuda.current_stream(cuda).cuda_stream
    # larger call first, then smaller ones: M, K and N all shrink, so stale partials and a
    # different strip count would show if the scratch were not handled per call
    for seed, (M, K, N) in enumerate(((8, 4096, 4096), (4, 4096, 4096), (1, 1024, 3072), (4, 4096, 4096))):
        x = randn((M, K), seed=10 + seed).to(cuda)
        w = randn((K, N), seed=20 + seed, scale=0.02, dtype=torch.float16).to(cuda)
        b = randn((N,), seed=30 + seed, scale=0.02).to(cuda)
        ks = lib.g16_skinny_plan(M, N, K, cus)
        assert ks > 1  # the split path: the scratch partials and counters are used
        ref = _buffered(lib, x, w, b, ks, st)
        outs = []
        for _ in range(2):
            out = torch.full((M, N), float("nan"), device=cuda)
            assert lib.g16_skinny_f32in_noalloc(x.data_ptr(), w.data_ptr(), out.data_ptr(), b.data_ptr(), M, N, K,
                                                ks, st) == 0
            outs.append(out)
        torch.cuda.synchronize()
        for out in outs:
            assert torch.equal(out, ref), (M, K, N)
        want = oracle.mm_t(x.cpu().numpy(), w.cpu().numpy(), b.cpu().numpy(), "float32")
        assert oracle.rel_err(outs[0].cpu().numpy(), want) <= 1e-5


def test_noalloc_refuses_splits_past_its_scratch(lib, cuda):
    st = torch.cuda.current_stream(cuda).cuda_stream
    x = torch.zeros(8, 4096, device=cuda)
    w = torch.zeros(4096, 16384, dtype=torch.float16, device=cuda)
    out = torch.full((8, 16384), 7.0, device=cuda)
    # 32 slices x 8 rows x 16384 columns x 4 bytes = 16 MiB of partials > 4 MiB
    assert lib.g16_skinny_f32in_noalloc(x.data_ptr(), w.data_ptr(), out.data_ptr(), None, 8, 16384, 4096, 32,
                                        st) == -7
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())  # nothing was launched
    # the same shape with one slice needs no split buffers at all
    assert lib.g16_skinny_f32in_noalloc(x.data_ptr(), w.data_ptr(), out.data_ptr(), None, 8, 16384, 4096, 1,
                                        st) == 0
    torch.cuda.synchronize()
    assert bool((out == 0.0).all())
