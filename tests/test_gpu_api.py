"""GPU tests of the public API (FastLinear, patch, matmul) on gfx950, mirroring the reference's
tests/test_correctness.py but checked against the fp64 oracle on the same fp16 weights."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def g(cuda):
    import gtx16_fp16

    return gtx16_fp16


@pytest.fixture(scope="module")
def lib(cuda):
    from gtx16_fp16 import _clib

    return _clib.load()


def _ref_linear(x: torch.Tensor, fl) -> np.ndarray:
    x2 = x.detach().reshape(-1, fl.in_features).float().cpu().numpy()
    w = fl.weight_t.cpu().numpy()
    b = None if fl.bias is None else fl.bias.cpu().numpy()
    return oracle.mm_t(x2, w, b, "float32").reshape(*x.shape[:-1], fl.out_features)


def test_is_affected_on_gfx950(g, cuda):
    assert g.is_affected() is True
    assert g.is_affected(0) is True and g.is_affected(cuda) is True


@pytest.mark.parametrize("shape", [(4, 50, 1024), (1, 1, 1024), (2, 1024), (7, 1024), (8, 1024), (9, 1024)])
def test_fast_linear_matches_oracle(g, cuda, shape):
    # tests/test_correctness.py:69-78 (both the decode fast path and the reshape path)
    torch.manual_seed(0)
    fl = g.FastLinear.from_linear(nn.Linear(1024, 768).to(cuda))
    x = torch.randn(*shape, device=cuda)
    with torch.no_grad():
        y = fl(x)
    torch.cuda.synchronize()
    assert y.dtype == torch.float32 and y.shape == (*shape[:-1], 768)
    M = int(np.prod(shape[:-1]))
    tol = 1e-5 if M <= 8 else 1e-3
    assert oracle.rel_err(y.cpu().numpy(), _ref_linear(x, fl)) <= tol


def test_fast_linear_is_deterministic_across_calls(g, cuda):
    # tests/test_correctness.py:52-59, tightened to bitwise equality (no float atomics here)
    fl = g.FastLinear.from_linear(nn.Linear(1024, 768).to(cuda))
    x = torch.randn(1, 1024, device=cuda)
    with torch.no_grad():
        outs = [fl(x) for _ in range(4)]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


def test_fast_linear_decode_after_half_and_bias_swap(g, cuda):
    # .half() makes the bias buffer fp16 and replaces it: the token-by-token path must notice the
    # new tensor and not hand its pointer to a kernel that reads an fp32 bias
    torch.manual_seed(0)
    fl = g.FastLinear.from_linear(nn.Linear(1024, 768).to(cuda))
    x = torch.randn(2, 1024, device=cuda)
    with torch.no_grad():
        fl(x)
        fl.half()
        assert fl.bias.dtype == torch.float16 and fl.weight_t.dtype == torch.float16
        y = fl(x)
        torch.cuda.synchronize()
        assert oracle.rel_err(y.cpu().numpy(), _ref_linear(x, fl)) <= 1e-5
        fl.bias = torch.randn(768, device=cuda)          # a new fp32 bias: the fast path again
        y2 = fl(x)
        torch.cuda.synchronize()
        assert fl._decode_entry(2, x.device)[0] is not None
        assert oracle.rel_err(y2.cpu().numpy(), _ref_linear(x, fl)) <= 1e-5


def test_fast_linear_falls_back_when_grad_needed(g, cuda):
    fl = g.FastLinear.from_linear(nn.Linear(256, 256).to(cuda))
    x = torch.randn(4, 256, device=cuda, requires_grad=True)
    fl(x).sum().backward()
    assert x.grad is not None


def test_fast_linear_fp16_input(g, cuda):
    fl = g.FastLinear.from_linear(nn.Linear(512, 256).to(cuda))
    x = torch.randn(300, 512, device=cuda).half()
    with torch.no_grad():
        y = fl(x)
    torch.cuda.synchronize()
    assert y.dtype == torch.float16
    assert oracle.rel_err(y.float().cpu().numpy(), _ref_linear(x, fl)) <= 1e-3


def test_patch_replaces_linear_layers(g, cuda):
    # tests/test_correctness.py:89-100
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(512, 1024), nn.GELU(), nn.Linear(1024, 512), nn.Linear(512, 10)).to(cuda).eval()
    x = torch.randn(64, 512, device=cuda)
    with torch.no_grad():
        ref = model(x)
    n = g.patch(model, min_features=256, force=True)
    assert n == 2
    assert isinstance(model[0], g.FastLinear) and isinstance(model[3], nn.Linear)
    with torch.no_grad():
        y = model(x)
    assert ((y - ref).norm() / ref.norm()).item() < 3e-3


def test_patch_default_on_gfx950_and_skip(g, cuda):
    model = nn.Sequential(nn.Linear(512, 512), nn.Linear(512, 512)).to(cuda)
    assert g.patch(model, skip=("1",)) == 1  # is_affected is True on gfx950, no force needed
    assert isinstance(model[0], g.FastLinear) and isinstance(model[1], nn.Linear)


@pytest.mark.parametrize("M", [1, 2, 8, 64, 1000])
def test_bias_and_inputs_are_not_modified(g, cuda, M):
    # tests/test_correctness.py:38-49
    x = torch.randn(M, 512, device=cuda).half()
    w = torch.randn(512, 768, device=cuda).half()
    b = torch.randn(768, device=cuda)
    x0, w0, b0 = x.clone(), w.clone(), b.clone()
    for _ in range(3):
        g.mm_t(x, w, b, torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(x, x0) and torch.equal(w, w0) and torch.equal(b, b0)


@pytest.mark.parametrize("M", [4, 64, 600])
def test_mm_t_on_non_contiguous_views(g, cuda, M):
    # an expanded view owns only K values and a transposed one has row stride 1: both are copied
    # to a contiguous buffer before a kernel reads M*K contiguous values
    w = torch.randn(512, 256, device=cuda).half()
    for x in (torch.randn(1, 512, device=cuda).expand(M, 512), torch.randn(512, M, device=cuda).t()):
        assert not x.is_contiguous()
        assert torch.equal(g.mm_t(x, w), g.mm_t(x.contiguous(), w))


def test_matmul_fp16_drop_in(g, cuda):
    a = torch.randn(256, 384, device=cuda).half()
    b = torch.randn(384, 128, device=cuda).half()
    y = g.matmul(a, b)
    torch.cuda.synchronize()
    assert y.dtype == torch.float16 and y.shape == (256, 128)
    ref = oracle.mm_t(a.cpu().numpy(), b.cpu().numpy(), None, "float32")
    assert oracle.rel_err(y.float().cpu().numpy(), ref) <= 1e-3
    # non-contiguous inputs are made contiguous first (ops.py:116)
    y2 = g.matmul(a.t().contiguous().t(), b)
    assert torch.equal(y2, y)


def test_matmul_fallback_for_odd_shapes(g, cuda):
    a = torch.randn(33, 13, device=cuda).half()
    b = torch.randn(13, 7, device=cuda).half()
    assert not g.supported(a, b)
    torch.testing.assert_close(g.matmul(a, b), (a @ b), rtol=1e-2, atol=1e-2)


def test_misaligned_activation_view(g, cuda):
    # supported() does not check the activation's alignment (ops.py:29-35); a misaligned view must
    # still give the right answer on both paths.
    base = torch.randn(16 * 256 + 1, device=cuda)
    w = (0.05 * torch.randn(256, 128, device=cuda)).half()
    for M in (4, 16):
        x = base[1:1 + M * 256].view(M, 256)
        assert x.data_ptr() % 16 != 0 and x.is_contiguous()
        y = g.mm_t(x, w, None, torch.float32)
        torch.cuda.synchronize()
        ref = oracle.mm_t(x.cpu().numpy(), w.cpu().numpy(), None, "float32")
        assert oracle.rel_err(y.cpu().numpy(), ref) <= (1e-5 if M <= 8 else 1e-3)


def test_empty_and_tiny_shapes(g, cuda):
    w = torch.randn(8, 8, device=cuda).half()
    b = torch.randn(8, device=cuda)
    for M in (1, 9):
        y = g.mm_t(torch.zeros(M, 0, device=cuda), torch.zeros(0, 8, device=cuda).half(), b, torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(y, b.expand(M, 8))
    y = g.mm_t(torch.ones(9, 8, device=cuda), w, None, torch.float32)
    torch.cuda.synchronize()
    ref = oracle.mm_t(np.ones((9, 8), np.float32), w.cpu().numpy(), None, "float32")
    assert oracle.rel_err(y.cpu().numpy(), ref) <= 1e-3


def test_graph_capture_replays_match_eager(g, cuda):
    # The kernels allocate nothing and use no memset, so the decode path can be captured in a HIP
    # graph; replays with the program's own eager work in between must keep matching eager.
    fl = g.FastLinear.from_linear(nn.Linear(1024, 1024).to(cuda))
    x = torch.randn(1, 1024, device=cuda)
    with torch.no_grad():
        eager = fl(x).clone()
        fl(x)  # warm the decode cache and the split buffers for this stream
        s = torch.cuda.Stream(cuda)
        s.wait_stream(torch.cuda.current_stream(cuda))
        with torch.cuda.stream(s):
            fl(x)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out = fl(x)
        for i in range(4):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), i
            with torch.no_grad():
                assert torch.equal(fl(x), eager)


def test_graph_of_every_mm_t_route_replays_bitwise(g, lib, cuda):
    # One graph holding mm_t on every route: the tile-packed 256x256 GEMM in one round and as a
    # persistent grid (cast + GEMM), the one-launch fp16 route, the resident one-launch fp32 route,
    # and the skinny kernel at M = 4 (FMA loop) and M = 8 (matrix cores). Replayed several times with
    # other eager mm_t work in between, every replay must equal the eager results bit for bit.
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    cases = [(2304, 256, 4096, torch.float32), (2560, 512, 8192, torch.float32), (1024, 1024, 1024, torch.float16),
             (48, 768, 1024, torch.float32), (4, 4096, 4096, torch.float32), (8, 4096, 4096, torch.float32)]
    if cus == 256:
        assert lib.g16_hgemm_use_packed(2304, 4096, 256, cus) == 1 and lib.g16_hgemm_use_packed(2560, 8192, 512, cus) == 1
        assert lib.g16_mm_t_scratch_bytes(48, 1024, 768, cus) == 0  # the resident route
    gens = [torch.Generator(cuda).manual_seed(70 + i) for i in range(len(cases))]
    xs = [torch.randn(M, K, device=cuda, generator=gn).to(dt) for (M, K, N, dt), gn in zip(cases, gens)]
    for x in xs[:2]:
        x[7] *= 3000.0  # a rescaled row on the packed route
    ws = [(torch.randn(K, N, device=cuda, generator=gn) * 0.02).half() for (M, K, N, dt), gn in zip(cases, gens)]
    bs = [torch.randn(N, device=cuda, generator=gn) * 0.02 for (M, K, N, dt), gn in zip(cases, gens)]
    eager = [g.mm_t(x, w, b, torch.float32) for x, w, b in zip(xs, ws, bs)]
    s = torch.cuda.Stream(cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(s):
        for x, w, b in zip(xs, ws, bs):
            g.mm_t(x, w, b, torch.float32)  # eager on the capture stream first: its buffers exist
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        outs = [g.mm_t(x, w, b, torch.float32) for x, w, b in zip(xs, ws, bs)]
    other_x = torch.randn(300, 512, device=cuda)
    other_w = (torch.randn(512, 384, device=cuda) * 0.02).half()
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        for k, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e), (i, cases[k][:3])
        g.mm_t(other_x, other_w)  # the program's own eager work between replays
        g.mm_t(xs[4], ws[4], bs[4])
        torch.cuda.synchronize()


def test_graphs_of_mm_t_keep_their_buffers_when_a_later_capture_outgrows_them(g, cuda):
    # mm_t keeps its cast scratch and split buffers per stream and grows them on demand; a graph
    # captured before a larger capture on the same stream must keep replaying correctly (the
    # outgrown buffers stay alive and are never handed to anything else).
    small = [(64, 1024, 1024), (100, 2048, 520)]          # split-K route; plain route with a cast
    large = [(64, 4096, 11008), (1536, 4096, 1024)]      # more partials; a larger cast
    s = torch.cuda.Stream(cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))

    def capture(shapes, seed):
        xs = [torch.randn(M, K, device=cuda, generator=torch.Generator(cuda).manual_seed(seed + i))
              for i, (M, K, N) in enumerate(shapes)]
        ws = [(torch.randn(K, N, device=cuda, generator=torch.Generator(cuda).manual_seed(seed + 9 + i)) * 0.02).half()
              for i, (M, K, N) in enumerate(shapes)]
        with torch.cuda.stream(s):
            for x, w in zip(xs, ws):
                g.mm_t(x, w)  # eager on the capture stream first: its buffers exist
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=s):
                outs = [g.mm_t(x, w) for x, w in zip(xs, ws)]
        torch.cuda.current_stream(cuda).wait_stream(s)
        torch.cuda.synchronize()
        eager = [g.mm_t(x, w) for x, w in zip(xs, ws)]
        return graph, outs, eager, (xs, ws)  # the graph reads xs and ws: keep them alive

    g1, outs1, eager1, keep1 = capture(small, 100)
    g2, outs2, eager2, keep2 = capture(large, 200)
    for _ in range(3):
        for o in outs1 + outs2:
            o.fill_(0.0)
        g1.replay()
        g2.replay()
        g1.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs1, eager1):
            assert torch.equal(o, e)
        for o, e in zip(outs2, eager2):
            assert torch.equal(o, e)


@pytest.mark.parametrize("shapes", [
    ((64, 4096, 1024, torch.float16), (64, 4096, 1024, torch.float16)),  # one split-K route on both
    ((64, 4096, 1024, torch.float32), (4, 4096, 4096, torch.float32)),  # split-K cast + GEMM; skinny
    ((2304, 256, 4096, torch.float32), (8, 4096, 4096, torch.float32)),  # packed cast + GEMM; skinny (matrix cores)
    ((2560, 512, 8192, torch.float32), (2560, 512, 8192, torch.float32)),  # the persistent packed grid on both
])
def test_concurrent_streams_keep_their_own_split_buffers(g, cuda, shapes):
    # Calls on different streams may run at the same time, so each stream has its own split
    # partials, counters and cast scratch: interleaved launches on two streams give the serial
    # results bit for bit.
    ins = []
    for i, (M, K, N, dt) in enumerate(shapes):
        gen = torch.Generator(cuda).manual_seed(300 + i)
        x = torch.randn(M, K, device=cuda, generator=gen).to(dt)
        w = (torch.randn(K, N, device=cuda, generator=gen) * 0.02).half()
        b = torch.randn(N, device=cuda, generator=gen) * 0.02
        ins.append((x, w, b))
    ref = [g.mm_t(x, w, b) for x, w, b in ins]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(cuda) for _ in ins]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream(cuda))
    outs = [[] for _ in ins]
    for _ in range(25):
        for s, (x, w, b), o in zip(streams, ins, outs):
            with torch.cuda.stream(s):
                o.append(g.mm_t(x, w, b))
    torch.cuda.synchronize()
    for r, o in zip(ref, outs):
        for k, y in enumerate(o):
            assert torch.equal(y, r), k


def test_gemm_clock_stamps_give_a_plausible_clock(cuda):
    # g16_gemm_clock: workgroup 0's main-loop shader cycles and 100 MHz ticks of the latest GEMM
    from gtx16_fp16 import _clib

    lib = _clib.load()
    a = torch.randn(1024, 1024, device=cuda).half()
    st = torch.cuda.current_stream(cuda).cuda_stream
    c = torch.empty(1024, 1024, device=cuda)
    dst = torch.zeros(2, dtype=torch.int64, device=cuda)
    assert lib.g16_gemm_clock(dst.data_ptr() + 4, st) == -2
    assert lib.g16_gemm_clock(None, st) == -3
    for _ in range(3):
        assert lib.g16_hgemm_f32out(a.data_ptr(), a.data_ptr(), c.data_ptr(), None, None, 1024, 1024, 1024, st) == 0
    assert lib.g16_gemm_clock(dst.data_ptr(), st) == 0
    cyc, ticks = dst.tolist()
    assert cyc > 0 and ticks > 0
    assert 300.0 <= 100.0 * cyc / ticks <= 3000.0
