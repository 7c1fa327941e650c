"""One-launch small GEMMs for fp16 activations: on the 4-wavefront tiles (32x128, 64x128, 64x64,
128x128, split or not), g16_mm_t_gemm streams x itself as A. A row whose |max| is within the threshold has
scale 1, so its rowscale cast is x and the result is exactly the cast path's; where some |x| of a
tile exceeds the threshold (or is NaN), that tile is computed again with its A fragments rescaled in
registers, by the rows' exponents taken from the maxima the first pass tracked (by the
last-arriving slice, over every slice, for split tiles). No scratch buffer is used.

Every case is compared bit for bit with the reference's two-step sequence (rowscale cast, then
GEMM: ops.py:86-108) run through the separate entry points g16_rowscale_f16 and g16_hgemm_* /
g16_hgemm_splitk on the same planned route: tiles within the threshold (the streamed path) and
tiles with rows above it (the recomputation), the threshold's edge, +inf and NaN entries (alone
and in rows that also exceed the threshold), ragged M, N and K, fp16 and fp32 output with and
without bias, and thresholds from 2^-8 (row exponents up to 24: subnormal factors) to 2^20. Also:
repeat calls bitwise equal and the split counters left zero, the public mm_t, the fp64 oracle, and
HIP-graph replays.
"""
from __future__ import annotations

import pytest
import torch

import oracle
from _inputs import outlier_rows, randn
from _plan import tile as planned_tile

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-3


@pytest.fixture(scope="module")
def lib(cuda):
    from gtx16_fp16 import _clib

    return _clib.load()


@pytest.fixture(scope="module")
def cus(cuda):
    return torch.cuda.get_device_properties(cuda).multi_processor_count




def _bufs(lib, M, N, K, num_cus, dev):
    ks = lib.g16_hgemm_plan(M, N, K, num_cus)
    wsb = lib.g16_hgemm_splitk_workspace_bytes(M, N, K, ks, num_cus) if ks > 1 else 0
    cb = lib.g16_hgemm_splitk_counter_bytes(M, N, K, ks, num_cus) if ks > 1 else 0
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
    cnt = torch.zeros(max(cb, 16), dtype=torch.uint8, device=dev)
    return ks, ws, wsb, cnt, cb


def _one_launch(lib, x, w, bias, out16, num_cus, bufs, thresh=1024.0):
    """g16_mm_t_gemm with no scratch: the speculative route needs none."""
    M, K = x.shape
    N = w.shape[1]
    ks, ws, wsb, cnt, cb = bufs
    out = torch.empty(M, N, dtype=torch.float16 if out16 else torch.float32, device=x.device)
    st = lib.g16_mm_t_gemm(x.data_ptr(), 0, w.data_ptr(), out.data_ptr(), 1 if out16 else 0,
                           None if bias is None else bias.data_ptr(), thresh, M, N, K, num_cus,
                           None, 0, ws.data_ptr() if wsb else None, wsb,
                           cnt.data_ptr() if cb else None, cb, torch.cuda.current_stream(x.device).cuda_stream)
    assert st == 0, lib.g16_strerror(st)
    return out


def _two_launches(lib, x, w, bias, out16, num_cus, bufs, thresh=1024.0):
    """The reference's sequence through the separate entry points: rowscale, then the GEMM on the
    planned route (split-K where the plan splits)."""
    M, K = x.shape
    N = w.shape[1]
    dev = x.device
    stream = torch.cuda.current_stream(dev).cuda_stream
    ks, ws, wsb, cnt, cb = bufs
    y = torch.empty(M, K, dtype=torch.float16, device=dev)
    s = torch.empty(M, dtype=torch.float32, device=dev)
    assert lib.g16_rowscale_f16(x.data_ptr(), y.data_ptr(), s.data_ptr(), M, K, thresh, stream) == 0
    out = torch.empty(M, N, dtype=torch.float16 if out16 else torch.float32, device=dev)
    b = None if bias is None else bias.data_ptr()
    if ks > 1:
        assert lib.g16_hgemm_splitk(y.data_ptr(), w.data_ptr(), out.data_ptr(), 1 if out16 else 0, b, s.data_ptr(),
                                    M, N, K, ks, num_cus, ws.data_ptr(), wsb, cnt.data_ptr(), cb, stream) == 0
    else:
        gm = lib.g16_hgemm_f16out if out16 else lib.g16_hgemm_f32out
        assert gm(y.data_ptr(), w.data_ptr(), out.data_ptr(), b, s.data_ptr(), M, N, K, stream) == 0
    return out


def _inputs(M, K, N, kind: str, seed: int, out16: bool):
    """fp16 x: 'within' every |x| <= 1024 (the streamed path); 'over' some rows above it (the
    recomputation); 'edge' one row at exactly 1024 and one a step above; 'special' +inf and NaN;
    'nan_over' NaN in a row above the threshold (its exponent comes from its other values) and in
    a row within it."""
    x = randn((M, K), seed=seed)
    if kind == "over":
        x = outlier_rows(x, 0.1, 2e3, 8e3 if out16 else 6e4, seed=seed + 3)
    elif kind == "edge":
        x[0, K // 3] = 1024.0                         # at the threshold: scale 1
        if M > 1:
            x[M - 1, 0] = 1025.0                      # fp16 1025: above it, scale 2
    elif kind == "special":
        x[M // 2, K // 2] = float("inf")
        if M > 2:
            x[1, 0] = float("nan")
    elif kind == "nan_over":
        r = M // 2
        x[r, K - 1] = float("nan")
        x[r, K // 3] = -2500.0                        # exponent 2 from this entry, NaN dropped
        x[0, K // 2] = float("nan")                   # a NaN row within the threshold
        if M > 40:
            x[40, 3] = -float("nan")
    return x.to(torch.float16), randn((K, N), seed=seed + 1, scale=0.05, dtype=torch.float16)


# (M, K, N, tile on 256 CUs, planned split on 256 CUs)
ROUTES = [
    (1024, 1024, 1024, (64, 64), 1),     # C1: the square tile, unsplit
    (64, 1024, 1024, (32, 128), 4),      # C3
    (64, 4096, 1024, (32, 128), 8),      # C3
    (1000, 1000, 1000, (64, 64), 1),     # ragged M, N, K on the square tile
    (100, 2048, 3072, (64, 64), 2),      # the square tile split twice, ragged M
    (320, 4056, 1024, (64, 64), 3),      # ... 3 ways, ragged last K step
    (72, 3072, 264, (64, 64), 8),        # ... 8 ways, ragged M and N
    (100, 1000, 264, (32, 128), 3),      # ragged M, N, K
    (64, 4096, 11008, (64, 128), 2),     # 64x128 split twice
    (128, 8192, 4096, (64, 128), 4),     # 64x128 split 4 ways at M > 64
    (256, 11008, 264, (32, 128), 8),     # 32x128 split 8 ways at M > 64
    (320, 8192, 4096, (128, 128), 2),    # 128x128 split twice
    (384, 4056, 3072, (128, 128), 3),    # 128x128 split 3 ways, ragged last K step
    (768, 4056, 4096, (128, 128), 1),    # 128x128 unsplit, ragged K tail
    (40, 8, 136, (32, 128), 1),          # one K step of 8
]
KINDS = ["within", "over", "edge", "special", "nan_over"]


@pytest.mark.parametrize("M,K,N,tile,ks", ROUTES)
@pytest.mark.parametrize("kind", KINDS)
def test_one_launch_equals_the_two_step_sequence_bitwise(lib, cus, cuda, M, K, N, tile, ks, kind):
    if cus != 256:
        pytest.skip(f"the route table is for 256 CUs (this device has {cus})")
    assert planned_tile(lib, M, N, K, cus) == tile
    assert lib.g16_hgemm_plan(M, N, K, cus) == ks
    out16 = (M + K) % 2 == 0
    use_bias = (N // 8) % 2 == 1
    x, w = _inputs(M, K, N, kind, seed=M + K + N, out16=out16)
    bias = randn((N,), seed=7, scale=0.1) if use_bias else None
    xd, wd = x.to(cuda), w.to(cuda)
    bd = None if bias is None else bias.to(cuda)
    bits = (lambda t: t.view(torch.int16)) if out16 else (lambda t: t.view(torch.int32))
    bufs = _bufs(lib, M, N, K, cus, cuda)
    two = _two_launches(lib, xd, wd, bd, out16, cus, bufs)
    one = _one_launch(lib, xd, wd, bd, out16, cus, bufs)
    torch.cuda.synchronize()
    assert torch.equal(bits(one), bits(two))
    again = [_one_launch(lib, xd, wd, bd, out16, cus, bufs) for _ in range(5)]
    torch.cuda.synchronize()
    for o in again:
        assert torch.equal(bits(o), bits(one))
    assert int(bufs[3].count_nonzero()) == 0  # split counters (and their flag) left zero
    import gtx16_fp16 as g

    pub = g.mm_t(xd, wd, bd, torch.float16 if out16 else torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(bits(pub), bits(one))
    if kind in ("within", "over", "edge"):
        ref = oracle.mm_t(x.numpy(), w.numpy(), None if bias is None else bias.numpy(),
                          "float16" if out16 else "float32")
        assert oracle.rel_err(one.cpu().numpy(), ref) <= GEMM_TOL


# (M, K, N, threshold): the exponents of rows up to 6e4 reach 16 - log2(threshold), 24 at 2^-8
THRESHOLDS = [
    (100, 1000, 264, 2.0 ** -8),
    (64, 4096, 1024, 2.0 ** -8),
    (1024, 1024, 1024, 2.0 ** -3),
    (64, 1024, 1024, 1.0),
    (512, 4096, 4096, 32768.0),
    (1024, 2048, 1024, 2.0 ** 20),
]


@pytest.mark.parametrize("M,K,N,thresh", THRESHOLDS)
def test_one_launch_thresholds_bitwise(lib, cus, cuda, M, K, N, thresh):
    x = randn((M, K), seed=M + N)
    x = outlier_rows(x, 0.1, 2e3, 6e4, seed=M + 5)
    x[M // 3, 1] = 65504.0                            # the largest fp16: exponent 16 - log2(thresh)
    x[M // 3, 2] = 3e-8                               # rounds to an fp16 subnormal, then underflows
    x16 = x.to(torch.float16)
    w = randn((K, N), seed=M + 2, scale=0.05, dtype=torch.float16)
    xd, wd = x16.to(cuda), w.to(cuda)
    bufs = _bufs(lib, M, N, K, cus, cuda)
    two = _two_launches(lib, xd, wd, None, False, cus, bufs, thresh)
    one = _one_launch(lib, xd, wd, None, False, cus, bufs, thresh)
    torch.cuda.synchronize()
    assert torch.equal(one.view(torch.int32), two.view(torch.int32))
    assert int(bufs[3].count_nonzero()) == 0


def test_thresholds_below_two_to_minus_8_take_the_two_launch_route(lib, cus, cuda):
    """2^-9: a row exponent can reach 25, whose factor is below the fp16 range; the library runs the
    cast and the GEMM as two launches, which need the scratch buffer."""
    M, K, N = 64, 1024, 1024
    x16 = randn((M, K), seed=3).to(torch.float16).to(cuda)
    x16[5, 5] = 60000.0
    wd = randn((K, N), seed=4, scale=0.05, dtype=torch.float16).to(cuda)
    bufs = _bufs(lib, M, N, K, cus, cuda)
    ks, ws, wsb, cnt, cb = bufs
    out = torch.empty(M, N, device=cuda)
    stream = torch.cuda.current_stream(cuda).cuda_stream
    st = lib.g16_mm_t_gemm(x16.data_ptr(), 0, wd.data_ptr(), out.data_ptr(), 0, None, 2.0 ** -9, M, N, K, cus,
                           None, 0, ws.data_ptr() if wsb else None, wsb, cnt.data_ptr() if cb else None, cb, stream)
    assert st == -3  # G16_E_NULL: the two-launch route's cast needs the scratch
    sb = lib.g16_mm_t_scratch_bytes(M, N, K, cus)
    scratch = torch.empty(sb, dtype=torch.uint8, device=cuda)
    st = lib.g16_mm_t_gemm(x16.data_ptr(), 0, wd.data_ptr(), out.data_ptr(), 0, None, 2.0 ** -9, M, N, K, cus,
                           scratch.data_ptr(), sb, ws.data_ptr() if wsb else None, wsb,
                           cnt.data_ptr() if cb else None, cb, stream)
    assert st == 0, lib.g16_strerror(st)
    two = _two_launches(lib, x16, wd, None, False, cus, bufs, 2.0 ** -9)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), two.view(torch.int32))


@pytest.mark.parametrize("M,K,N,with_scratch", [(64, 4096, 1024, True), (64, 1000, 1024, False)])
def test_a_recomputed_weight_takes_the_other_route_for_63_calls(lib, cus, cuda, M, K, N, with_scratch):
    """After a call whose tile was computed again, the weight's next 63 calls take the other route
    -- the two-launch one where the caller passed the scratch it needs (64x4096x1024), the resident
    one-launch cast into LDS where the plan allows it (64x1000x1024, no scratch) -- then speculation
    resumes; every call's result is the two-step sequence's, bit for bit."""
    xo, w = _inputs(M, K, N, "over", seed=11, out16=False)
    xw, _ = _inputs(M, K, N, "within", seed=12, out16=False)
    xo, xw, wd = xo.to(cuda), xw.to(cuda), w.to(cuda)
    bufs = _bufs(lib, M, N, K, cus, cuda)
    ks, ws, wsb, cnt, cb = bufs
    stream = torch.cuda.current_stream(cuda).cuda_stream
    assert lib.g16_mm_t_spec_history(stream) == 0   # enabled once per device (idempotent)
    assert lib.g16_mm_t_spec_history(stream) == 0
    sb = lib.g16_mm_t_scratch_bytes(M, N, K, cus)
    assert (sb > 0) == with_scratch
    scratch = torch.empty(max(sb, 16), dtype=torch.uint8, device=cuda)

    def call(x):
        out = torch.empty(M, N, device=cuda)
        st = lib.g16_mm_t_gemm(x.data_ptr(), 0, wd.data_ptr(), out.data_ptr(), 0, None, 1024.0, M, N, K, cus,
                               scratch.data_ptr() if sb else None, sb, ws.data_ptr() if wsb else None, wsb,
                               cnt.data_ptr() if cb else None, cb, stream)
        assert st == 0, lib.g16_strerror(st)
        return out

    ref_o = _two_launches(lib, xo, wd, None, False, cus, bufs)
    ref_w = _two_launches(lib, xw, wd, None, False, cus, bufs)
    # leave the slot clear first: calls within the threshold until no pause is left
    for _ in range(70):
        call(xw)
    torch.cuda.synchronize()
    assert lib.g16_mm_t_spec_paused(wd.data_ptr(), stream) == 0
    o = call(xo)                      # speculative, computed again: the slot records it
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int32), ref_o.view(torch.int32))
    assert lib.g16_mm_t_spec_paused(wd.data_ptr(), stream) == 1
    outs = [call(xo if i % 2 else xw) for i in range(63)]   # the other route: no new miss is noted
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert torch.equal(o.view(torch.int32), (ref_o if i % 2 else ref_w).view(torch.int32))
    assert lib.g16_mm_t_spec_paused(wd.data_ptr(), stream) == 1
    o = call(xw)                      # the 64th: speculative again, and within the threshold
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int32), ref_w.view(torch.int32))
    assert lib.g16_mm_t_spec_paused(wd.data_ptr(), stream) == 0
    assert int(cnt.count_nonzero()) == 0


def test_without_scratch_a_split_shape_always_speculates(lib, cus, cuda):
    """No scratch and no resident plan: the two-launch route is not available, so a weight whose call
    was computed again keeps the one-launch route (and its result bits)."""
    M, K, N = 64, 1024, 1024
    xo, w = _inputs(M, K, N, "over", seed=21, out16=False)
    xo, wd = xo.to(cuda), w.to(cuda)
    bufs = _bufs(lib, M, N, K, cus, cuda)
    ref = _two_launches(lib, xo, wd, None, False, cus, bufs)
    outs = [_one_launch(lib, xo, wd, None, False, cus, bufs) for _ in range(3)]
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o.view(torch.int32), ref.view(torch.int32))


def test_graph_replays_of_speculative_mm_t_match_eager(cuda):
    import gtx16_fp16 as g

    shapes = [(1024, 1024, 1024, "within"), (64, 4096, 1024, "over"), (100, 1000, 264, "over"),
              (512, 4096, 4096, "within")]
    xs, ws = [], []
    for i, (M, K, N, kind) in enumerate(shapes):
        x, w = _inputs(M, K, N, kind, seed=40 + i, out16=False)
        xs.append(x.to(cuda))
        ws.append(w.to(cuda))
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
        extra = g.mm_t(xs[1], ws[1], None, torch.float32)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(extra, eager[1])
