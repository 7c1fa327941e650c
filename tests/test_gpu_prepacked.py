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
