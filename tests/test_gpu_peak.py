"""GPU tests of the peak microbenchmark entry points (bench.py --peak): every kind runs, returns OK
and leaves finite values; the stream read covers the buffer it is given; and the arithmetic the
instruction probes time is the arithmetic they claim: the fp32 FMA chains, the LDS reads, and the
MFMA probes (kinds 2-5 and the GEMM-order probe on supplied operands) against a numpy model of
the same products, built from the documented operand and accumulator lane layouts of
v_mfma_f32_32x32x16_f16 and v_mfma_f32_16x16x32_f16. A wrong lane layout, a dropped or repeated
MFMA, or operands other than the ones described moves the values far outside the tolerance."""
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


# ---- numpy model of the two MFMA forms (one wavefront of 64 lanes, 8 fp16 operands per lane) ----

def _mfma32_regs(afr: np.ndarray, bfr: np.ndarray) -> np.ndarray:
    """v_mfma_f32_32x32x16_f16 on lanes' fragments afr, bfr [64, 8] -> the 16 output registers of
    each lane [64, 16]: lane l holds A row l % 32 and B column l % 32 over k = 8 (l // 32) .. + 7;
    register r of lane l is C[8 (r // 4) + 4 (l // 32) + r % 4, l % 32]."""
    A = np.zeros((32, 16))
    B = np.zeros((16, 32))
    for l in range(64):
        A[l % 32, 8 * (l // 32):8 * (l // 32) + 8] = afr[l]
        B[8 * (l // 32):8 * (l // 32) + 8, l % 32] = bfr[l]
    C = A @ B
    return np.array([[C[8 * (r // 4) + 4 * (l // 32) + r % 4, l % 32] for r in range(16)] for l in range(64)])


def _mfma16_regs(afr: np.ndarray, bfr: np.ndarray) -> np.ndarray:
    """v_mfma_f32_16x16x32_f16 -> [64, 4]: lane l holds A row l % 16 and B column l % 16 over
    k = 8 (l // 16) .. + 7; register r of lane l is C[4 (l // 16) + r, l % 16]."""
    A = np.zeros((16, 32))
    B = np.zeros((32, 16))
    for l in range(64):
        A[l % 16, 8 * (l // 16):8 * (l // 16) + 8] = afr[l]
        B[8 * (l // 16):8 * (l // 16) + 8, l % 16] = bfr[l]
    C = A @ B
    return np.array([[C[4 * (l // 16) + r, l % 16] for r in range(4)] for l in range(64)])


def _random_half(x: np.ndarray) -> np.ndarray:
    """The probe's random fp16 bit pattern of index x (a 32-bit integer hash; random sign and
    mantissa, exponent in [2^-3, 2^0))."""
    x = x.astype(np.uint32)
    with np.errstate(over="ignore"):
        x ^= x >> np.uint32(16)
        x = (x * np.uint32(0x7FEB352D)).astype(np.uint32)
        x ^= x >> np.uint32(15)
        x = (x * np.uint32(0x846CA68B)).astype(np.uint32)
        x ^= x >> np.uint32(16)
    bits = (x & np.uint32(0x83FF)) | ((np.uint32(12) + ((x >> np.uint32(10)) & np.uint32(3))) << np.uint32(10))
    return bits.astype(np.uint16).view(np.float16).astype(np.float64)


def _probe_operands(kind: int, block: int) -> tuple[np.ndarray, np.ndarray]:
    """a, b [256, 8] of one workgroup for kinds 2-5 (the probe's mfma_operands)."""
    t = np.arange(256)
    i = np.arange(8)
    if kind in (2, 3):
        seed = np.float32(1e-3)
        a = (seed * (t[:, None] + i[None, :]).astype(np.float32)).astype(np.float16)
        b = np.broadcast_to((seed * i.astype(np.float32)).astype(np.float16), (256, 8))
        return a.astype(np.float64), b.astype(np.float64)
    g = (block * 256 + t) * 16
    return _random_half(g[:, None] + i[None, :]), _random_half(g[:, None] + 8 + i[None, :])


@pytest.mark.parametrize("kind", [2, 3, 4, 5])
@pytest.mark.parametrize("iters", [1, 3])
def test_peak_mfma_values(lib, cuda, kind, iters):
    # every accumulator of a lane receives the same MFMA each iteration, so lane t's output is
    # n_acc * iters * (its output register r of one MFMA), r = t % 16 (32x32x16) or t % 4
    # (16x16x32), summed over the accumulators
    blocks = 2
    out = torch.empty(blocks * 256, device=cuda)
    st = torch.cuda.current_stream(cuda).cuda_stream
    assert lib.g16_peak_run(kind, blocks, iters, out.data_ptr(), st) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(blocks, 256)
    n_acc, regs, nreg = (8, _mfma32_regs, 16) if kind in (2, 4) else (16, _mfma16_regs, 4)
    for blk in range(blocks):
        a, b = _probe_operands(kind, blk)
        want, scale = np.zeros(256), np.zeros(256)
        for w in range(4):
            lanes = slice(64 * w, 64 * w + 64)
            r = regs(a[lanes], b[lanes])
            ra = regs(np.abs(a[lanes]), np.abs(b[lanes]))
            sel = (np.arange(64) % nreg)
            want[lanes] = n_acc * iters * r[np.arange(64), sel]
            scale[lanes] = n_acc * iters * ra[np.arange(64), sel]
        err = np.abs(got[blk] - want)
        assert (err <= 1e-5 * scale + 1e-30).all(), (blk, float(np.max(err / np.maximum(scale, 1e-30))))


def _c4_operands(ngroups: int, seed: int) -> np.ndarray:
    """Kind 8's operands: fp16 of N(0,1) for the 8 A fragments and of N(0, 0.02^2) for the 4 B
    fragments of both sets, for every lane of `ngroups` workgroups ([ngroups, 256, 2, 12, 8])."""
    rng = np.random.default_rng(seed)
    ops = np.empty((ngroups, 256, 2, 12, 8), dtype=np.float16)
    ops[..., :8, :] = rng.standard_normal((ngroups, 256, 2, 8, 8)).astype(np.float16)
    ops[..., 8:, :] = (0.02 * rng.standard_normal((ngroups, 256, 2, 4, 8))).astype(np.float16)
    return ops


@pytest.mark.parametrize("iters", [1, 2])
def test_peak_mfma_gemm_order_values(lib, cuda, iters):
    # kind 8: acc[i][j] of a lane = iters * (A0_i B0_j + A1_i B1_j) over its wavefront, every
    # accumulator stored; workgroups 0 and 2 share operand group 0 (ngroups = 2)
    blocks, ngroups = 3, 2
    ops = _c4_operands(ngroups, seed=11)
    dops = torch.from_numpy(ops.view(np.uint16).astype(np.int16)).to(cuda)
    out = torch.full((blocks * 256 * 128,), float("nan"), device=cuda)
    st = torch.cuda.current_stream(cuda).cuda_stream
    assert lib.g16_peak_mfma_data(blocks, iters, dops.data_ptr(), ngroups, out.data_ptr(), None, st) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(blocks, 256, 8, 4, 4)
    o = ops.astype(np.float64)
    for blk in range(blocks):
        g = blk % ngroups
        for w in range(4):
            lanes = slice(64 * w, 64 * w + 64)
            for i in range(8):
                for j in range(4):
                    want = sum(_mfma16_regs(o[g, lanes, s, i], o[g, lanes, s, 8 + j]) for s in range(2)) * iters
                    scale = sum(_mfma16_regs(np.abs(o[g, lanes, s, i]), np.abs(o[g, lanes, s, 8 + j]))
                                for s in range(2)) * iters
                    err = np.abs(got[blk, lanes, i, j] - want)
                    assert (err <= 1e-5 * scale + 1e-30).all(), (blk, w, i, j)


def test_peak_mfma_gemm_order_rejects(lib, cuda):
    out = torch.empty(256 * 128, device=cuda)
    ops = torch.zeros(256 * 24 * 8, dtype=torch.int16, device=cuda)
    st = torch.cuda.current_stream(cuda).cuda_stream
    assert lib.g16_peak_mfma_data(1, 1, ops.data_ptr(), 0, out.data_ptr(), None, st) == -1
    assert lib.g16_peak_mfma_data(1, 1, None, 1, out.data_ptr(), None, st) == -3
    assert lib.g16_peak_mfma_data(1, 1, ops.data_ptr() + 2, 1, out.data_ptr(), None, st) == -2
    assert lib.g16_peak_flops_per_lane_iter(8) == 64 * 16 * 16 * 32 * 2 / 64
