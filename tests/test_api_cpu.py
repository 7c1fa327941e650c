"""CPU tests of the host-side API: fallback routing, dtype rules and model patching.

On CPU tensors every entry point takes the reference's torch fallback (ops.py:33,119;
linear.py:45-46,69-70), so these run without a GPU and mirror tests/test_correctness.py.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn

import gtx16_fp16 as g
from gtx16_fp16 import _clib, ops


def test_exports_and_version():
    assert set(g.__all__) == {"FastLinear", "patch", "is_affected", "matmul", "mm_t", "supported"}
    assert g.__version__ == "0.1.0"
    assert ops.ROW_SCALE_THRESHOLD == 1024.0
    from gtx16_fp16.kernels import SKINNY_MAX_M

    assert SKINNY_MAX_M == 8


def test_is_affected_reports_bool():
    # tests/test_correctness.py:129-130
    assert isinstance(g.is_affected(), bool)
    if not torch.cuda.is_available():
        assert g.is_affected() is False


def test_supported_rejects_cpu_tensors():
    x = torch.randn(16, 64)
    w = torch.randn(64, 32).half()
    assert not g.supported(x, w)


def test_mm_t_rejects_bad_out_dtype_before_any_device_work():
    # ops.py:70-71
    with pytest.raises(ValueError):
        g.mm_t(torch.randn(4, 8), torch.randn(8, 8).half(), None, torch.bfloat16)


def test_mm_t_and_pack_weight_reject_host_tensors():
    # without supported() in front, a host tensor must be refused before any pointer reaches a kernel
    x, w = torch.randn(16, 64), torch.randn(64, 32).half()
    with pytest.raises(ValueError, match="x2d"):
        g.mm_t(x, w)
    with pytest.raises(ValueError, match="x2d"):
        ops.mm_t_prepacked(x, w, torch.empty(0, dtype=torch.float16))
    with pytest.raises(ValueError, match="pack_weight"):
        ops.pack_weight(w)


def test_matmul_fallback_for_odd_shapes():
    # tests/test_correctness.py:62-66 (CPU tensors always take the fallback)
    a = torch.randn(33, 13).half()
    b = torch.randn(13, 7).half()
    assert not g.supported(a, b)
    y = g.matmul(a, b)
    assert y.dtype == torch.float16
    torch.testing.assert_close(y, a @ b, rtol=1e-2, atol=1e-2)
    assert g.matmul(a, b, torch.float32).dtype == torch.float32


def test_fast_linear_from_linear_layout_and_state_dict():
    torch.manual_seed(0)
    lin = nn.Linear(64, 48)
    fl = g.FastLinear.from_linear(lin)
    assert fl.weight_t.shape == (64, 48) and fl.weight_t.dtype == torch.float16
    assert fl.bias.dtype == torch.float32
    assert torch.equal(fl.weight_t, lin.weight.detach().t().half())
    assert torch.equal(fl.weight, fl.weight_t.t())
    sd = fl.state_dict()
    assert set(sd) == {"weight_t", "bias"}
    fl2 = g.FastLinear(64, 48)
    fl2.load_state_dict(sd)
    assert torch.equal(fl2.weight_t, fl.weight_t) and torch.equal(fl2.bias, fl.bias)
    assert "in_features=64" in repr(fl)
    assert g.FastLinear(8, 8, bias=False).bias is None


@pytest.mark.parametrize("shape", [(4, 50, 64), (1, 1, 64), (2, 64), (7, 64), (0, 64)])
def test_fast_linear_cpu_fallback_matches_nn_linear(shape):
    # tests/test_correctness.py:69-78 on the CPU fallback path
    torch.manual_seed(0)
    lin = nn.Linear(64, 48)
    fl = g.FastLinear.from_linear(lin)
    x = torch.randn(*shape)
    with torch.no_grad():
        y = fl(x)
        ref = nn.functional.linear(x, lin.weight.half().float(), lin.bias)
    assert y.dtype == torch.float32 and y.shape == (*shape[:-1], 48)
    torch.testing.assert_close(y, ref, rtol=1e-5, atol=1e-5)


def test_fast_linear_output_dtype_rules():
    # linear.py:44: fp16 in -> fp16 out, other dtypes -> fp32 out
    fl = g.FastLinear.from_linear(nn.Linear(32, 16))
    with torch.no_grad():
        assert fl(torch.randn(3, 32).half()).dtype == torch.float16
        assert fl(torch.randn(3, 32).bfloat16()).dtype == torch.float32
        assert fl(torch.randn(3, 32)).dtype == torch.float32


def test_fast_linear_falls_back_when_grad_needed():
    # tests/test_correctness.py:81-86
    fl = g.FastLinear.from_linear(nn.Linear(256, 256))
    x = torch.randn(4, 256, requires_grad=True)
    fl(x).sum().backward()
    assert x.grad is not None and x.grad.shape == x.shape


def test_patch_skips_cpu_models_and_respects_filters():
    model = nn.Sequential(nn.Linear(512, 1024), nn.GELU(), nn.Linear(1024, 512), nn.Linear(512, 10))
    assert g.patch(model) == 0                 # no GPU parameters -> nothing affected
    assert g.patch(model, force=True) == 0     # force still requires GPU layers (linear.py:93)
    assert all(isinstance(m, (nn.Linear, nn.GELU)) for m in model)


def test_skinny_config_covers_k():
    lib = _clib.load()
    for N, K in [(4096, 4096), (3072, 1024), (520, 2048), (8, 8), (14336, 4096)]:
        (gx, gy, gz), rows = ops.skinny_config(N, K, 256)
        cols = lib.g16_skinny_strip_cols(1, N)
        assert cols == (256 if N <= 8192 else 512)
        nstrips = (N + cols - 1) // cols
        assert gy == gz == 1 and gx % nstrips == 0
        assert (gx // nstrips) * rows >= K > (gx // nstrips - 1) * rows


def test_fast_linear_caches_are_opt_in_and_cpu_layers_build_none():
    # The decode-layout copy and the shared activation cast are off unless a caller turns them on;
    # a layer on the CPU (torch fallback) never builds a weight copy, whatever the flags.
    assert g.FastLinear.prepack_decode is False and g.FastLinear.share_cast is False
    assert g.FastLinear.prepack_weight is True
    fl = g.FastLinear.from_linear(nn.Linear(64, 48))
    fl.prepack_decode = fl.share_cast = True
    with torch.no_grad():
        fl(torch.randn(1, 64))
        fl(torch.randn(300, 64))
    assert fl._wp is None and fl._wd is None
    fl.release_copies()  # nothing to free: no synchronisation needed, no error on a CPU layer
    assert fl._wp is None and fl._wd is None


def test_tensor_version_of_inference_tensors():
    # inference tensors carry no version counter: the caches key them as None instead of raising
    t = torch.zeros(4)
    v0 = ops.tensor_version(t)
    t.add_(1)
    assert ops.tensor_version(t) == v0 + 1
    with torch.inference_mode():
        ti = torch.zeros(4)
        assert ti.is_inference() and ops.tensor_version(ti) is None
        with torch.no_grad():
            fl = g.FastLinear.from_linear(nn.Linear(16, 8))
        assert fl.weight_t.is_inference()
        y = fl(torch.randn(2, 16))  # CPU fallback under inference_mode
    assert y.shape == (2, 8)
