"""GPU tests of the prepacked-weight route (FastLinear's large-batch GEMM): the weight packer
against the numpy model of the layout, and mm_t_prepacked / FastLinear bitwise equal to mm_t on the
unpacked weight (same values, same MFMA order), including a weight modified in place."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from _inputs import outlier_rows, randn
from _packing import pack_a

pytestmark = pytest.mark.gpu

# shapes on the tile-packed 256x256 route (ragged M, K and N included)
# the last two run 256x128 tiles (128 tiles of 256x256 would leave half the CUs idle), which read the
# packed weight by half blocks; (1800, 136, 3896) also has a ragged last half block
ROUTE_SHAPES = [(4096, 4096, 4096), (2300, 264, 4096), (4100, 1000, 2056), (2048, 264, 4096), (1800, 136, 3896)]


@pytest.fixture(scope="module")
def ops(cuda):
    from gtx16_fp16 import ops

    return ops


@pytest.mark.parametrize("K,N", [(8, 8), (136, 264), (1000, 2056), (4096, 4096)])
def test_pack_weight_bitexact(ops, cuda, K, N):
    w = randn((K, N), seed=K + N, scale=0.02, dtype=torch.float16)
    wp = ops.pack_weight(w.to(cuda))
    torch.cuda.synchronize()
    expect = pack_a(w.numpy().T.copy())
    got = wp.cpu().numpy()
    assert got.shape == expect.shape
    assert np.array_equal(got.view(np.uint16), expect.view(np.uint16))


@pytest.mark.parametrize("M,K,N", ROUTE_SHAPES)
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("in_dtype", [torch.float32, torch.float16])
def test_mm_t_prepacked_bitwise_equals_mm_t(ops, cuda, M, K, N, out_dtype, in_dtype):
    assert ops.prepacked_route(M, N, K, cuda)
    hi = 2e5 if out_dtype == torch.float32 and in_dtype == torch.float32 else 1e4
    x = outlier_rows(randn((M, K), seed=0), 0.01, 2e3, hi, seed=3).to(in_dtype).to(cuda)
    w = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).to(cuda)
    bias = randn((N,), seed=2, scale=0.02).to(cuda)
    wp = ops.pack_weight(w)
    for b in (bias, None):
        y0 = ops.mm_t(x, w, b, out_dtype)
        y1 = ops.mm_t_prepacked(x, w, wp, b, out_dtype)
        torch.cuda.synchronize()
        assert torch.equal(y0, y1)
    ref = oracle.mm_t(x.cpu().numpy(), w.cpu().numpy(), bias.cpu().numpy(),
                      "float32" if out_dtype == torch.float32 else "float16")
    y = ops.mm_t_prepacked(x, w, wp, bias, out_dtype)
    assert oracle.rel_err(y.float().cpu().numpy(), ref.astype(np.float64)) <= 1e-3


@pytest.mark.parametrize("M,K,N", [(2300, 264, 4096), (1800, 136, 3896)])
@pytest.mark.parametrize("in_dtype", [torch.float32, torch.float16])
def test_mm_t_prepacked_nonfinite_rows_bitwise_equal_mm_t(ops, cuda, M, K, N, in_dtype):
    # Rows holding +-inf or NaN (their output rows are NaN) on both 256-row tiles: the prepacked
    # route gives mm_t's result bit for bit, NaN rows included, and the oracle's NaN rows.
    assert ops.prepacked_route(M, N, K, cuda)
    x = randn((M, K), seed=7)
    for r, v, k in ((0, "inf", 5), (255, "nan", K - 1), (256, "-inf", 0), (M - 1, "nan", K // 2)):
        x[r, k] = float(v)
    x[700, 3] = 5e3  # a rescaled row
    x = x.to(in_dtype).to(cuda)
    w = randn((K, N), seed=8, scale=0.02, dtype=torch.float16).to(cuda)
    bias = randn((N,), seed=9, scale=0.02).to(cuda)
    wp = ops.pack_weight(w)
    for out_dtype, view in ((torch.float32, torch.int32), (torch.float16, torch.int16)):
        y0 = ops.mm_t(x, w, bias, out_dtype)
        y1 = ops.mm_t_prepacked(x, w, wp, bias, out_dtype)
        torch.cuda.synchronize()
        assert torch.equal(y0.view(view), y1.view(view))
        nan_rows = torch.isnan(y1).all(dim=1).cpu().numpy()
        want = oracle.mm_t(x.cpu().numpy(), w.cpu().numpy(), bias.cpu().numpy(),
                           "float32" if out_dtype == torch.float32 else "float16")
        assert np.array_equal(nan_rows, np.isnan(want).all(axis=1))
        assert nan_rows.sum() == 4 and torch.isfinite(y1[~torch.from_numpy(nan_rows).to(cuda)]).all()


def test_mm_t_prepacked_off_route_is_mm_t(ops, cuda):
    # small and skinny shapes ignore wp and take mm_t's own route
    for M, K, N in [(300, 136, 264), (4, 1024, 1024)]:
        x = randn((M, K), seed=5).to(cuda)
        w = randn((K, N), seed=6, scale=0.02, dtype=torch.float16).to(cuda)
        wp = ops.pack_weight(w)
        assert torch.equal(ops.mm_t_prepacked(x, w, wp), ops.mm_t(x, w))


def test_mm_t_prepacked_rejects_a_wrong_packed_weight(ops, cuda):
    M = K = N = 4096
    x = torch.randn(M, K, device=cuda)
    w = torch.randn(K, N, device=cuda).half()
    with pytest.raises(ValueError):
        ops.mm_t_prepacked(x, w, torch.empty(16, dtype=torch.float16, device=cuda))


def test_mm_t_rejects_operands_the_kernels_cannot_read(ops, cuda):
    # a bias or weight on another device, or a misaligned weight view, raises instead of launching
    x = torch.randn(64, 256, device=cuda)
    w = torch.randn(256, 128, device=cuda).half()
    with pytest.raises(ValueError, match="bias"):
        ops.mm_t(x, w, torch.zeros(128))
    with pytest.raises(ValueError, match="bias"):
        ops.mm_t(x, w, torch.zeros(64, device=cuda))
    with pytest.raises(ValueError, match="w_t"):
        ops.mm_t(x, w.cpu())
    wide = torch.randn(256 * 128 + 4, device=cuda).half()
    with pytest.raises(ValueError, match="w_t"):
        ops.mm_t(x, wide[4:].view(256, 128))   # 8-byte aligned base
    with pytest.raises(ValueError, match="pack_weight"):
        ops.pack_weight(wide[4:].view(256, 128))


def test_fast_linear_large_batch_uses_prepacked_weight_and_tracks_changes(cuda):
    import gtx16_fp16 as g
    from gtx16_fp16 import ops

    torch.manual_seed(0)
    fl = g.FastLinear.from_linear(nn.Linear(768, 3072).to(cuda))
    x = torch.randn(64, 256, 768, device=cuda)  # M = 16384 rows: the packed route
    assert ops.prepacked_route(16384, 3072, 768, cuda)
    with torch.no_grad():
        y = fl(x)
        assert fl._wp is not None
        assert torch.equal(y.reshape(-1, 3072), ops.mm_t(x.reshape(-1, 768), fl.weight_t, fl.bias))
        fl.weight_t.mul_(0.5)            # in place: the packed copy must be rebuilt
        y2 = fl(x)
        assert torch.equal(y2.reshape(-1, 3072), ops.mm_t(x.reshape(-1, 768), fl.weight_t, fl.bias))
        assert not torch.equal(y, y2)
        fl.prepack_weight = False
        assert torch.equal(fl(x), y2)
    assert "_wp" not in fl.state_dict() and set(fl.state_dict()) == {"weight_t", "bias"}


def _qkv(cuda, K=768, N=768, seed=0):
    # three layers with the opt-in shared cast turned on
    torch.manual_seed(seed)
    layers = [FastLinearT.from_linear(nn.Linear(K, N).to(cuda)) for _ in range(3)]
    for fl in layers:
        fl.share_cast = True
    return layers


FastLinearT = None


@pytest.fixture(scope="module", autouse=True)
def _fast_linear_cls(cuda):
    global FastLinearT
    from gtx16_fp16 import FastLinear

    FastLinearT = FastLinear


def _unshared(layers, x):
    for fl in layers:
        fl.share_cast = False
    try:
        with torch.no_grad():
            return [fl(x) for fl in layers]
    finally:
        for fl in layers:
            fl.share_cast = True


def test_shared_cast_across_layers_is_bitwise_the_unshared_result(ops, cuda):
    # Q, K and V projections of one hidden-states tensor (11264 token rows, on the tile-packed route,
    # with outlier rows): the second and third layer reuse the first one's rowscale cast
    layers = _qkv(cuda)
    x = outlier_rows(randn((11264, 768), seed=3), 0.02, 2e3, 2e5, seed=4).reshape(44, 256, 768).to(cuda)
    assert ops.prepacked_route(11264, 768, 768, cuda)
    ops.release_cast_cache()
    with torch.no_grad():
        shared = [fl(x) for fl in layers]
    assert len(ops._cast_cache) == 1
    want = _unshared(layers, x)
    torch.cuda.synchronize()
    for a, b in zip(shared, want):
        assert torch.equal(a, b)
    xs = x.reshape(-1, 768)[:1024].cpu().numpy()  # the oracle on the first 1024 rows (outliers among them)
    ref = oracle.mm_t(xs, layers[1].weight_t.cpu().numpy(), layers[1].bias.cpu().numpy(), "float32")
    assert oracle.rel_err(shared[1].reshape(-1, 768)[:1024].cpu().numpy(), ref) <= 1e-3


def test_shared_cast_misses_after_in_place_write_and_for_a_new_tensor(ops, cuda):
    layers = _qkv(cuda, seed=1)
    x = randn((11264, 768), seed=5).to(cuda)
    assert ops.prepacked_route(11264, 768, 768, cuda)
    with torch.no_grad():
        layers[0](x)                      # cached cast of x
        x.mul_(3000.0)                    # in place: version changes, rows now need the rescale
        got = layers[1](x)
    want = _unshared(layers[1:2], x)[0]
    assert torch.equal(got, want)
    ptr = x.data_ptr()
    with torch.no_grad():
        layers[0](x)
    del x
    # a new tensor, often at the same address, with other values: the dead weak reference misses
    y = randn((11264, 768), seed=6).to(cuda)
    with torch.no_grad():
        got = layers[1](y)
    want = _unshared(layers[1:2], y)[0]
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"same address as the cached tensor: {y.data_ptr() == ptr}"


def test_no_shared_cast_under_graph_capture(ops, cuda):
    layers = _qkv(cuda, seed=2)
    x = randn((11264, 768), seed=7).to(cuda)
    want = _unshared(layers, x)
    s = torch.cuda.Stream(cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.stream(s):
        for fl in layers:
            fl(x)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            outs = [fl(x) for fl in layers]
    torch.cuda.current_stream(cuda).wait_stream(s)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, want):
            assert torch.equal(a, b)


def test_shared_cast_is_off_by_default(ops, cuda):
    # share_cast is opt-in: a default layer casts its own input on every call
    torch.manual_seed(3)
    layers = [FastLinearT.from_linear(nn.Linear(768, 768).to(cuda)) for _ in range(2)]
    assert not any(fl.share_cast for fl in layers)
    x = randn((11264, 768), seed=8).to(cuda)
    ops.release_cast_cache()
    with torch.no_grad():
        got = [fl(x) for fl in layers]
    assert len(ops._cast_cache) == 0
    for fl, y in zip(layers, got):
        assert torch.equal(y, ops.mm_t(x, fl.weight_t, fl.bias))


def test_large_batch_under_inference_mode(ops, cuda):
    # Inference tensors carry no version counter: the prepacked route and the opt-in shared cast
    # must still run (the cast is then never shared), also for a layer built under inference_mode,
    # whose weight_t is itself an inference tensor.
    torch.manual_seed(4)
    lin = nn.Linear(768, 768).to(cuda)
    layers = _qkv(cuda, seed=4)
    x = randn((11264, 768), seed=9).to(cuda)
    want = _unshared(layers, x)
    with torch.inference_mode():
        xi = x.clone()
        assert xi.is_inference()
        got = [fl(xi) for fl in layers]
        built = FastLinearT.from_linear(lin)
        assert built.weight_t.is_inference()
        yb = built(xi)
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert torch.equal(a, b)
    ref = FastLinearT.from_linear(lin)  # the same weights, built outside inference_mode
    assert torch.equal(yb, ops.mm_t(x, ref.weight_t, ref.bias))
    assert built._wp is not None


def test_no_prepacked_copy_is_built_under_graph_capture(ops, cuda):
    # The first large-batch call of a layer inside a capture takes mm_t on weight_t (the pack kernel
    # is not recorded into the graph); replays match eager and the layer builds its copy eagerly later.
    torch.manual_seed(5)
    fl = FastLinearT.from_linear(nn.Linear(768, 768).to(cuda))
    x = randn((11264, 768), seed=10).to(cuda)
    want = ops.mm_t(x, fl.weight_t, fl.bias)
    s = torch.cuda.Stream(cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.stream(s):
        ops.mm_t(x, fl.weight_t, fl.bias)  # the stream's cast scratch exists before capture
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            out = fl(x)
    torch.cuda.current_stream(cuda).wait_stream(s)
    assert fl._wp is None
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
    with torch.no_grad():
        y = fl(x)
    torch.cuda.synchronize()
    assert fl._wp is not None and torch.equal(y, want)
