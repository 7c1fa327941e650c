"""One-launch small GEMMs: where mm_t's plan is the unsplit 32x128 tile and K <= 1280,
g16_mm_t_gemm runs a single GEMM launch and needs no scratch. For fp32 x its workgroups cast their
own rows of x into LDS (no fp16 copy in HBM, no rowscale launch); for fp16 x it is the speculative
launch that streams x itself (test_gpu_speculative.py covers it in depth, and the LDS cast of fp16
x, which the speculation history selects after a recomputation). Either way the result must equal
the reference's two-step sequence (rowscale cast, then GEMM: ops.py:86-108), run here through the
separate entry points g16_rowscale_* and g16_hgemm_*, bit for bit -- including rows that are
rescaled, +inf and NaN entries, ragged M, N and K, fp16 and fp32 activations and outputs. Also:
repeat calls bitwise equal, the public mm_t on this route, the fp64 oracle, and HIP-graph replays.
"""
from __future__ import annotations

import pytest
import torch

import oracle
from _inputs import outlier_rows, randn

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-3


@pytest.fixture(scope="module")
def lib(cuda):
    from gtx16_fp16 import _clib

    return _clib.load()


@pytest.fixture(scope="module")
def cus(cuda):
    return torch.cuda.get_device_properties(cuda).multi_processor_count


def _inputs(M, K, N, x_dtype, special: bool, seed: int, out16: bool):
    # outlier rows (rescaled by the cast) within the input's range, small enough that an fp16
    # output stays finite
    hi = 8e3 if out16 else (2e5 if x_dtype == torch.float32 else 6e4)
    x = outlier_rows(randn((M, K), seed=seed), 0.1, 2e3, hi, seed=seed + 3)
    if special and M >= 3:
        x[1, K // 2] = float("inf")
        x[2, 0] = float("nan")
        x[2, K - 1] = -3e3
    return x.to(x_dtype), randn((K, N), seed=seed + 1, scale=0.05, dtype=torch.float16)


def _one_launch(lib, x, w, bias, out16, num_cus):
    M, K = x.shape
    N = w.shape[1]
    assert lib.g16_mm_t_scratch_bytes(M, N, K, num_cus) == 0  # the one-launch route
    out = torch.empty(M, N, dtype=torch.float16 if out16 else torch.float32, device=x.device)
    st = lib.g16_mm_t_gemm(x.data_ptr(), 1 if x.dtype == torch.float32 else 0, w.data_ptr(), out.data_ptr(),
                           1 if out16 else 0, None if bias is None else bias.data_ptr(), 1024.0, M, N, K, num_cus,
                           None, 0, None, 0, None, 0, torch.cuda.current_stream(x.device).cuda_stream)
    assert st == 0, lib.g16_strerror(st)
    return out


def _two_launches(lib, x, w, bias, out16):
    """The reference's sequence through the separate entry points: rowscale, then the GEMM."""
    M, K = x.shape
    N = w.shape[1]
    dev = x.device
    stream = torch.cuda.current_stream(dev).cuda_stream
    y = torch.empty(M, K, dtype=torch.float16, device=dev)
    s = torch.empty(M, dtype=torch.float32, device=dev)
    rs = lib.g16_rowscale_f32 if x.dtype == torch.float32 else lib.g16_rowscale_f16
    assert rs(x.data_ptr(), y.data_ptr(), s.data_ptr(), M, K, 1024.0, stream) == 0
    out = torch.empty(M, N, dtype=torch.float16 if out16 else torch.float32, device=dev)
    gm = lib.g16_hgemm_f16out if out16 else lib.g16_hgemm_f32out
    assert gm(y.data_ptr(), w.data_ptr(), out.data_ptr(), None if bias is None else bias.data_ptr(), s.data_ptr(),
              M, N, K, stream) == 0
    return out


# (M, K, N, x dtype, fp16 out, bias, special values)
CASES = [
    (64, 1000, 1024, torch.float16, True, False, False),     # two tile rows, ragged K
    (50, 1000, 1000, torch.float32, False, True, True),      # ragged M, N, K tail; inf / NaN rows
    (20, 1280, 32768, torch.float32, False, False, False),   # 20 resident K steps, the most
    (20, 256, 1024, torch.float16, True, True, False),       # fewer rows than one tile
    (33, 8, 1024, torch.float32, False, True, False),        # one K step of 8
    (64, 1016, 2048, torch.float16, False, True, True),      # ragged K, fp16 specials
    (64, 1000, 1024, torch.float32, True, True, False),
]


@pytest.mark.parametrize("M,K,N,xdt,out16,use_bias,special", CASES)
def test_one_launch_equals_the_two_step_sequence_bitwise(lib, cus, cuda, M, K, N, xdt, out16, use_bias, special):
    if cus != 256:
        pytest.skip(f"the case table is for 256 CUs (this device has {cus})")
    x, w = _inputs(M, K, N, xdt, special, seed=M + K + N, out16=out16)
    bias = randn((N,), seed=7, scale=0.1) if use_bias else None
    xd, wd = x.to(cuda), w.to(cuda)
    bd = None if bias is None else bias.to(cuda)
    bits = (lambda t: t.view(torch.int16)) if out16 else (lambda t: t.view(torch.int32))
    two = _two_launches(lib, xd, wd, bd, out16)
    one = _one_launch(lib, xd, wd, bd, out16, cus)
    torch.cuda.synchronize()
    assert torch.equal(bits(one), bits(two))
    again = [_one_launch(lib, xd, wd, bd, out16, cus) for _ in range(5)]
    torch.cuda.synchronize()
    for o in again:
        assert torch.equal(bits(o), bits(one))
    import gtx16_fp16 as g

    pub = g.mm_t(xd, wd, bd, torch.float16 if out16 else torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(bits(pub), bits(one))
    if not special:
        ref = oracle.mm_t(x.numpy(), w.numpy(), None if bias is None else bias.numpy(),
                          "float16" if out16 else "float32")
        assert oracle.rel_err(one.cpu().numpy(), ref) <= GEMM_TOL


def test_graph_replays_of_one_launch_mm_t_match_eager(cuda):
    import gtx16_fp16 as g

    shapes = [(64, 1000, 1024, torch.float16), (50, 1000, 1000, torch.float32), (20, 256, 1024, torch.float32)]
    xs = [randn((M, K), seed=20 + i).to(dt).to(cuda) for i, (M, K, N, dt) in enumerate(shapes)]
    ws = [randn((K, N), seed=30 + i, scale=0.05, dtype=torch.float16).to(cuda) for i, (M, K, N, dt) in enumerate(shapes)]
    eager = [g.mm_t(x, w, None, torch.float32) for x, w in zip(xs, ws)]
    s = torch.cuda.Stream(cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        for x, w in zip(xs, ws):
            g.mm_t(x, w, None, torch.float32)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            outs = [g.mm_t(x, w, None, torch.float32) for x, w in zip(xs, ws)]
    torch.cuda.current_stream(cuda).wait_stream(s)
    torch.cuda.synchronize()
    for _ in range(3):
        for o in outs:
            o.fill_(0.0)
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e)
        extra = g.mm_t(xs[0], ws[0], None, torch.float32)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(extra, eager[0])
