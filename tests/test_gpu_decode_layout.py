"""GPU tests of FastLinear's decode layout (csrc/decode.hip): the strip-major weight copy and the
skinny product on it, for the token-by-token branch of FastLinear.forward (reference
src/gtx16_fp16/linear.py:49-64, skinny semantics kernels.py:153-219).

* The layout is bit-exact against its numpy model (wd[s, k, c] == w_t[k, 8 s + c]).
* The product is within the skinny path's tolerance of the fp64 oracle (relative Frobenius error
  <= 1e-5) for M = 1..4, fp32 and fp16 activations, with and without bias, on shapes with ragged K
  (rows that end inside a wavefront's 64-row group, wavefronts with no rows at all) and N from one
  strip to 11008 columns, and bitwise repeatable.
* FastLinear (with the opt-in ``prepack_decode``) takes the route where the library's rule says
  so, keeps the copy outside its state_dict, and rebuilds it when weight_t is modified in place or
  replaced; it builds no copy under graph capture and works under ``torch.inference_mode()``.
* Non-finite activations: lanes past the end of a wavefront's rows add nothing, so a +-inf in the
  last row of a wavefront's range (or at K - 1) gives the oracle's +-inf (or NaN) per column, not a
  NaN from inf * 0.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from _inputs import randn

pytestmark = pytest.mark.gpu

SKINNY_TOL = 1e-5

SHAPES = [(4096, 4096), (1024, 3072), (3072, 1024), (8, 8), (72, 200), (520, 8), (1032, 776), (4104, 264),
          (2040, 4096), (4096, 11008)]


@pytest.fixture(scope="module")
def ops(cuda):
    from gtx16_fp16 import ops

    return ops


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("K,N", SHAPES)
def test_decode_layout_is_the_strip_major_copy(ops, cuda, K, N):
    w = randn((K, N), seed=K + N, scale=0.02, dtype=torch.float16)
    wd = ops.pack_decode_weight(w.to(cuda))
    torch.cuda.synchronize()
    assert wd.shape == (N // 8, K, 8)
    want = _np(w).reshape(K, N // 8, 8).transpose(1, 0, 2)
    assert np.array_equal(_np(wd).view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("K,N", SHAPES)
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.float16])
def test_strips_match_oracle_and_repeat(ops, cuda, K, N, M, x_dtype):
    x = randn((M, K), seed=M + K, dtype=x_dtype)
    w = randn((K, N), seed=K + N, scale=0.02, dtype=torch.float16)
    b = randn((N,), seed=N, scale=0.02)
    wd = ops.pack_decode_weight(w.to(cuda))
    xd, bd = x.to(cuda), b.to(cuda)
    ys = [ops.skinny_strips(xd, wd, bd) for _ in range(3)]
    y0 = ops.skinny_strips(xd, wd, None)
    torch.cuda.synchronize()
    assert oracle.rel_err(_np(ys[0]), oracle.skinny(_np(x), _np(w), _np(b))) <= SKINNY_TOL
    assert oracle.rel_err(_np(y0), oracle.skinny(_np(x), _np(w), None)) <= SKINNY_TOL
    assert all(torch.equal(y, ys[0]) for y in ys[1:])


def test_strips_use_only_the_rows_of_k(ops, cuda):
    # Lanes past the last row re-read that row and must add nothing: with a weight of ones and one
    # activation 1 in row K - 1, every column is exactly bias + 1, whatever K is.
    for K in (8, 64, 72, 136, 520, 1032, 2040):
        w = torch.ones(K, 16, dtype=torch.float16, device=cuda)
        x = torch.zeros(1, K, device=cuda)
        x[0, K - 1] = 1.0
        b = torch.full((16,), 0.5, device=cuda)
        y = ops.skinny_strips(x, ops.pack_decode_weight(w), b)
        torch.cuda.synchronize()
        assert torch.equal(y, torch.full((1, 16), 1.5, device=cuda)), K


def test_fast_linear_takes_the_decode_layout_and_rebuilds_it(cuda):
    import gtx16_fp16 as g
    from gtx16_fp16 import _clib

    lib = _clib.load()
    torch.manual_seed(0)
    fl = g.FastLinear.from_linear(nn.Linear(1024, 3072).to(cuda))
    assert not fl.prepack_decode          # opt-in
    fl.prepack_decode = True
    assert lib.g16_skinny_strips_route(1, 3072, 1024, 1) == 1
    x = torch.randn(1, 1024, device=cuda)

    def ref():
        return oracle.skinny(_np(x), _np(fl.weight_t), _np(fl.bias))

    with torch.no_grad():
        y = fl(x)
        torch.cuda.synchronize()
        assert fl._wd is not None and fl._decode_entry(1, x.device)[5]
        assert oracle.rel_err(_np(y), ref()) <= SKINNY_TOL
        assert set(fl.state_dict()) == {"weight_t", "bias"}
        fl.weight_t.mul_(2.0)                          # in place: the copy must be rebuilt
        y2 = fl(x)
        torch.cuda.synchronize()
        assert oracle.rel_err(_np(y2), ref()) <= SKINNY_TOL
        fl.weight_t = (torch.randn(1024, 3072, device=cuda) * 0.02).half()   # replaced
        y3 = fl(x)
        torch.cuda.synchronize()
        assert oracle.rel_err(_np(y3), ref()) <= SKINNY_TOL
        # off: the split kernel on weight_t, no copy built on a fresh layer
        fl2 = g.FastLinear.from_linear(nn.Linear(1024, 3072).to(cuda))
        fl2.prepack_decode = False
        y4 = fl2(x)
        torch.cuda.synchronize()
        assert fl2._wd is None and not fl2._decode_entry(1, x.device)[5]
        assert oracle.rel_err(_np(y4), oracle.skinny(_np(x), _np(fl2.weight_t), _np(fl2.bias))) <= SKINNY_TOL


def test_fast_linear_keeps_the_split_kernel_where_the_rule_says_so(cuda):
    import gtx16_fp16 as g

    fl = g.FastLinear.from_linear(nn.Linear(4096, 4096).to(cuda))
    fl.prepack_decode = True
    x = torch.randn(4, 4096, device=cuda)              # fp32 activations, M = 4, 2^24 weights
    with torch.no_grad():
        y = fl(x)
    torch.cuda.synchronize()
    assert fl._wd is None and not fl._decode_entry(4, x.device)[5]
    assert oracle.rel_err(_np(y), oracle.skinny(_np(x), _np(fl.weight_t), _np(fl.bias))) <= SKINNY_TOL


def test_fast_linear_fp16_activations_take_the_decode_layout(cuda):
    # fp16 activations skip the fp32 fast path; the general path takes the decode layout for them
    # too (fp32 product, cast to fp16 at the end like the skinny path's fp16 output)
    import gtx16_fp16 as g

    torch.manual_seed(1)
    fl = g.FastLinear.from_linear(nn.Linear(1024, 3072).to(cuda))
    fl.prepack_decode = True
    x = torch.randn(2, 1, 1024, device=cuda).half()
    with torch.no_grad():
        y = fl(x)
    torch.cuda.synchronize()
    assert fl._wd is not None
    assert y.dtype == torch.float16 and y.shape == (2, 1, 3072)
    ref = oracle.skinny(_np(x).reshape(2, 1024), _np(fl.weight_t), _np(fl.bias))
    assert oracle.rel_err(_np(y.float()).reshape(2, 3072), ref) <= 1e-3
    fl2 = g.FastLinear.from_linear(nn.Linear(1024, 3072).to(cuda))
    with torch.no_grad():
        fl2.weight_t.copy_(fl.weight_t)
        fl2.bias.copy_(fl.bias)
        fl2.prepack_decode = False
        y2 = fl2(x)
    torch.cuda.synchronize()
    assert fl2._wd is None
    # the two routes differ only in the order of the fp32 additions (then one fp16 rounding each):
    # both within the fp16 output's tolerance of the oracle, and close to each other
    assert oracle.rel_err(_np(y2.float()).reshape(2, 3072), ref) <= 1e-3
    assert oracle.rel_err(_np(y.float()), _np(y2.float()).astype(np.float64)) <= 1e-3


def _rows_per_wave(K):
    # rows per wavefront of the decode kernel: K over its 8 wavefronts in whole 64-row groups
    return -(-(-(-K // 8)) // 64) * 64


def _assert_same_nonfinite(got, want):
    # same NaN positions, same infinities with the same signs, finite values within the skinny bar
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isposinf(got), np.isposinf(want))
    assert np.array_equal(np.isneginf(got), np.isneginf(want))
    fin = np.isfinite(want)
    if fin.any():
        assert oracle.rel_err(got[fin], want[fin]) <= SKINNY_TOL


@pytest.mark.parametrize("K", [3072, 11008])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("with_bias", [True, False])
def test_strips_nonfinite_activation_at_a_wavefronts_last_row(ops, cuda, K, M, x_dtype, with_bias):
    # +inf / -inf at the last row of a wavefront's range (where that wavefront's last batch of row
    # loads is partial: the lanes past it re-read that row) and at K - 1: every column must be the
    # oracle's +-inf (NaN only where the weight is 0), not NaN from the dead lanes' inf * 0.
    N = 1024
    rpw = _rows_per_wave(K)
    rows = [min(K, w * rpw + rpw) - 1 for w in range(8) if w * rpw < K] + [K - 1]
    x = randn((M, K), seed=K + M, dtype=x_dtype)
    for m in range(M):
        x[m, rows[(3 * m) % len(rows)]] = float("inf") if m % 2 == 0 else float("-inf")
    w = randn((K, N), seed=K, scale=0.02, dtype=torch.float16)
    b = randn((N,), seed=N, scale=0.02) if with_bias else None
    wd = ops.pack_decode_weight(w.to(cuda))
    y = ops.skinny_strips(x.to(cuda), wd, None if b is None else b.to(cuda))
    torch.cuda.synchronize()
    want = oracle.skinny(_np(x), _np(w), None if b is None else _np(b))
    assert not np.isfinite(want).any()
    _assert_same_nonfinite(_np(y).astype(np.float64), want)


@pytest.mark.parametrize("K", [3072, 11008])
@pytest.mark.parametrize("M", [1, 2])
def test_fast_linear_decode_route_nonfinite_activation(cuda, K, M):
    # the same through FastLinear's token-by-token fast path on its decode layout
    import gtx16_fp16 as g

    N = 1024
    torch.manual_seed(K)
    fl = g.FastLinear.from_linear(nn.Linear(K, N).to(cuda))
    fl.prepack_decode = True
    x = torch.randn(M, K, device=cuda)
    rpw = _rows_per_wave(K)
    x[0, rpw - 1] = float("inf")
    x[M - 1, K - 1] = float("-inf")
    with torch.no_grad():
        y = fl(x)
    torch.cuda.synchronize()
    assert fl._decode_entry(M, x.device)[5] is not None and fl._wd is not None
    with np.errstate(invalid="ignore"):  # at M = 1 the row holds both infinities: NaN columns expected
        want = oracle.skinny(_np(x), _np(fl.weight_t), _np(fl.bias))
    _assert_same_nonfinite(_np(y).astype(np.float64), want)


def test_fast_linear_decode_layout_under_inference_mode_and_capture(cuda):
    # inference_mode: weight_t built there is an inference tensor (no version counter); capture:
    # no copy is built inside a capture (the split kernel on weight_t serves the call), and the
    # copy is built on the next eager call. All within the skinny bar of the oracle.
    import gtx16_fp16 as g

    torch.manual_seed(7)
    lin = nn.Linear(1024, 1024).to(cuda)
    x = torch.randn(1, 1024, device=cuda)
    with torch.inference_mode():
        fl = g.FastLinear.from_linear(lin)
        fl.prepack_decode = True
        y = fl(x)
        y2 = fl(x.half())
    torch.cuda.synchronize()
    assert fl._wd is not None
    ref = oracle.skinny(_np(x), _np(fl.weight_t), _np(fl.bias))
    assert oracle.rel_err(_np(y), ref) <= SKINNY_TOL
    assert oracle.rel_err(_np(y2.float()), oracle.skinny(_np(x.half()), _np(fl.weight_t), _np(fl.bias))) <= 1e-3

    fl2 = g.FastLinear.from_linear(lin)
    fl2.prepack_decode = True
    s = torch.cuda.Stream(cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.stream(s):
        fl2.prepack_decode = False
        fl2(x)                              # the split kernel's buffers exist on this stream
        fl2.prepack_decode = True
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            out = fl2(x)
    torch.cuda.current_stream(cuda).wait_stream(s)
    assert fl2._wd is None
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert oracle.rel_err(_np(out), ref) <= SKINNY_TOL
    with torch.no_grad():
        y3 = fl2(x)
    torch.cuda.synchronize()
    assert fl2._wd is not None and oracle.rel_err(_np(y3), ref) <= SKINNY_TOL
