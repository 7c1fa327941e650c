"""GPU parity: the gfx950 kernels (through the C ABI of libg16.so) against the fp64 oracle.

Bars (per the north star): rowscale exponents and fp16 casts bit-exact; relative Frobenius error
<= 1e-3 on the GEMM paths (fp32 and fp16 output) and <= 1e-5 on the skinny fp32-accumulate path;
split reductions bitwise repeatable. Inputs are seeded on the CPU and copied to the device, so
the oracle sees the same bits. Shapes follow the reference's acceptance sweep
(tests/test_correctness.py:14-18) plus the BASELINE configurations.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _inputs import outlier_rows, randn
from _plan import tile as planned_tile

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-3
SKINNY_TOL = 1e-5


@pytest.fixture(scope="module")
def g(cuda):
    import gtx16_fp16

    return gtx16_fp16


@pytest.fixture(scope="module")
def lib(cuda):
    from gtx16_fp16 import _clib

    return _clib.load()


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def _stream(dev) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _split_bufs(partial_bytes: int, counter_bytes: int, dev):
    ws = torch.empty(max(partial_bytes, 16), dtype=torch.uint8, device=dev)
    cnt = torch.zeros(max(counter_bytes, 16), dtype=torch.uint8, device=dev)
    return ws, cnt


# ---------------------------------------------------------------------------------------------
# rowscale cast: exponents and fp16 values bit-exact
# ---------------------------------------------------------------------------------------------

def _rowscale_gpu(lib, x: torch.Tensor):
    M, K = x.shape
    y = torch.empty(M, K, dtype=torch.float16, device=x.device)
    s = torch.empty(M, dtype=torch.float32, device=x.device)
    fn = lib.g16_rowscale_f32 if x.dtype == torch.float32 else lib.g16_rowscale_f16
    st = fn(x.data_ptr(), y.data_ptr(), s.data_ptr(), M, K, 1024.0, _stream(x.device))
    assert st == 0, st
    torch.cuda.synchronize()
    return y, s


KAT_AMAX = [0.0, 1.0, 1023.9999, 1024.0, float(np.nextafter(np.float32(1024), np.float32(2048))), 2048.0,
            float(np.nextafter(np.float32(2048), np.float32(4096))), 65504.0, 179940.0, 2e5, 3.0e38]


@pytest.mark.parametrize("K", [8, 136, 1032, 3072, 4096, 8200])
@pytest.mark.parametrize("extra", [20, 21])
def test_rowscale_f32_bitexact(lib, cuda, K, extra):
    # 31 or 32 rows: at K = 4096 with a multiple of 8 rows the cast takes its two-row form
    M = len(KAT_AMAX) + extra
    x = randn((M, K), seed=K)
    for i, a in enumerate(KAT_AMAX):  # row i has |max| exactly a (at a column that depends on i)
        x[i] = x[i].clamp(-0.5, 0.5)
        x[i, (7 * i) % K] = -a if i % 2 else a
    x[len(KAT_AMAX) + 1, 3 % K] = float("nan")  # NaN is ignored by the max
    x[len(KAT_AMAX) + 2, 0] = -0.0  # signed zeros keep their sign through the scaling
    x[len(KAT_AMAX) + 2, K - 1] = 5000.0
    x[5, (K // 2) & ~1] = -0.0
    y, s = _rowscale_gpu(lib, x.to(cuda))
    y_ref, s_ref, e_ref = oracle.rowscale(_np(x))
    _assert_bits_equal(_np(s).view(np.uint32), s_ref.view(np.uint32), _np(x), "S")
    _assert_bits_equal(_np(y).view(np.uint16), y_ref.view(np.uint16), _np(x), "Y")


def _assert_bits_equal(got: np.ndarray, ref: np.ndarray, x: np.ndarray, what: str) -> None:
    bad = np.argwhere(got != ref)
    if bad.size:
        show = []
        for idx in bad[:8]:
            idx = tuple(int(i) for i in idx)
            xin = x[idx] if x.ndim == len(idx) else x[idx[0]]
            show.append(f"{idx}: got {got[idx]:#x} ref {ref[idx]:#x} x={xin!r}")
        raise AssertionError(f"{what}: {len(bad)} bit mismatches; first: " + "; ".join(show))


@pytest.mark.parametrize("K", [64, 1032, 4096, 6144])
def test_rowscale_f16_bitexact(lib, cuda, K):
    M = 40
    x = randn((M, K), seed=K + 1)
    x[:, 5] = 60000.0
    x[3, 9] = -50000.0
    x[7] = x[7] * 1e-6  # values that go subnormal in fp16 after scaling
    x[7, 0] = 2000.0
    x16 = x.half()
    x16[9, 3] = -0.0
    assert (x16 == 0).any()  # row 7 holds fp16 zeros of both signs and subnormals
    y, s = _rowscale_gpu(lib, x16.to(cuda))
    y_ref, s_ref, _ = oracle.rowscale(_np(x16))
    _assert_bits_equal(_np(s).view(np.uint32), s_ref.view(np.uint32), _np(x16), "S")
    _assert_bits_equal(_np(y).view(np.uint16), y_ref.view(np.uint16), _np(x16), "Y")


def test_rowscale_infinite_row_is_nonfinite(g, cuda):
    x = randn((16, 256), seed=5)
    x[2, 10] = float("inf")
    w = randn((256, 64), seed=6, scale=0.1, dtype=torch.float16)
    y = g.mm_t(x.to(cuda), w.to(cuda), None, torch.float32)
    torch.cuda.synchronize()
    assert not torch.isfinite(y[2]).any()
    assert torch.isfinite(torch.cat([y[:2], y[3:]])).all()


# ---------------------------------------------------------------------------------------------
# GEMM path (M > 8) through mm_t: plain tiles and split-K
# ---------------------------------------------------------------------------------------------

SHAPES = [  # (M, K, N) -- reference sweep, tests/test_correctness.py:14-18
    (128, 128, 128), (256, 512, 384), (1000, 1032, 776), (129, 136, 8), (3, 4096, 4096),
    (1, 1024, 3072), (8, 2048, 520), (9, 64, 64), (4096, 4096, 1024), (17, 8, 4104),
    (64, 1024, 1024), (33, 4096, 768), (200, 1032, 136),
]


# Medium shapes run on the 4-wavefront tiles (here 64x64 and 64x128), unsplit or split, as the
# planner's model picks them (all within one round of the CUs); bitwise repeatable either way.
@pytest.mark.parametrize("M,K,N", [(256, 3072, 1024), (1024, 3072, 1024), (520, 2056, 3072), (1024, 1024, 1024)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_short_k_small_tiles_match_oracle(g, cuda, M, K, N, out_dtype):
    x = randn((M, K), seed=M + 5 * K, scale=0.5)
    w = randn((K, N), seed=N + 3 * K, scale=0.5, dtype=torch.float16)
    b = randn((N,), seed=N + 1)
    xd, wd, bd = x.to(cuda), w.to(cuda), b.to(cuda)
    y = g.mm_t(xd, wd, bd, out_dtype)
    y2 = g.mm_t(xd, wd, bd, out_dtype)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16) if out_dtype == torch.float16 else y.view(torch.int32),
                       y2.view(torch.int16) if out_dtype == torch.float16 else y2.view(torch.int32))
    ref = oracle.mm_t(_np(x), _np(w), _np(b), "float32")
    assert oracle.rel_err(_np(y.float()), ref) <= GEMM_TOL


@pytest.mark.parametrize("M,K,N", SHAPES)
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("with_bias", [False, True])
def test_mm_t_matches_oracle(g, cuda, M, K, N, out_dtype, with_bias):
    x = randn((M, K), seed=M * 7 + K * 3 + N, scale=0.5, dtype=torch.float16)
    w = randn((K, N), seed=M + K + N, scale=0.5, dtype=torch.float16)
    b = randn((N,), seed=N + 11) if with_bias else None
    xd, wd = x.to(cuda), w.to(cuda)
    bd = b.to(cuda) if b is not None else None
    assert g.supported(xd, wd)
    y = g.mm_t(xd, wd, bd, out_dtype)
    torch.cuda.synchronize()
    assert y.dtype == out_dtype and y.shape == (M, N)
    assert torch.isfinite(y).all()
    ref = oracle.mm_t(_np(x), _np(w), None if b is None else _np(b), "float32")
    tol = SKINNY_TOL if (M <= 8 and out_dtype == torch.float32) else GEMM_TOL
    assert oracle.rel_err(_np(y.float()), ref) <= tol


@pytest.mark.parametrize("M,K,N", [(4096, 4096, 4096), (1024, 1024, 1024), (65536 // 64, 768, 3072)])
def test_large_gemm_fp32_activations_with_outliers(g, cuda, M, K, N):
    # C4: fp32 activations, 1% of rows with |max| ~ U[2e3, 2e5], fp16 weights ~ N(0, 0.02^2)
    x = outlier_rows(randn((M, K), seed=0), 0.01, 2e3, 2e5, seed=3)
    w = randn((K, N), seed=1, scale=0.02, dtype=torch.float16)
    y = g.mm_t(x.to(cuda), w.to(cuda), None, torch.float32)
    torch.cuda.synchronize()
    xs = _np(x)
    y16, S, e = oracle.rowscale(xs)
    assert (e > 0).sum() == int(round(0.01 * M))
    ref = oracle.gemm(y16, S, _np(w), None, "float32")
    assert oracle.rel_err(_np(y), ref) <= GEMM_TOL


def test_constant_16_known_answer(g, cuda):
    # tests/test_correctness.py:103-109: 16*16 summed over K = 4096 is exactly 1,048,576.
    x = torch.full((128, 4096), 16.0, device=cuda).half()
    w = torch.full((4096, 128), 16.0, device=cuda).half()
    y = g.mm_t(x, w, None, torch.float32)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    assert torch.equal(y, torch.full_like(y, 16 * 16 * 4096))


@pytest.mark.parametrize("M", [1, 5, 64, 300])
@pytest.mark.parametrize("in_dtype", [torch.float32, torch.float16])
def test_massive_activations(g, cuda, M, in_dtype):
    # tests/test_correctness.py:112-126
    K, N = 3072, 1024
    x = randn((M, K), seed=1)
    x[:, 7] = 179940.0 if in_dtype == torch.float32 else 60000.0
    x[0, 100] = -120000.0 if in_dtype == torch.float32 else -50000.0
    x = x.to(in_dtype)
    w = randn((K, N), seed=2, scale=0.3, dtype=torch.float16)
    y = g.mm_t(x.to(cuda), w.to(cuda), None, torch.float32)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    ref = oracle.mm_t(_np(x), _np(w), None, "float32")
    tol = SKINNY_TOL if M <= 8 else GEMM_TOL
    assert oracle.rel_err(_np(y), ref) <= tol


# (M, K, N, num_cus, tile): the launch plans its tile for the CU count it is given, so a small count
# forces the larger tiles onto shapes the device's own count would give smaller ones
SPLIT_CASES = [(64, 1024, 1024, 256, (32, 128)), (64, 4096, 1024, 256, (32, 128)),
               (1024, 1024, 1024, 256, (64, 64)), (33, 4096, 768, 256, (32, 128)),
               (64, 1024, 1024, 16, (64, 128)), (300, 1024, 264, 8, (128, 128)),
               (1024, 1024, 8192, 256, (256, 128)), (1024, 1024, 8192, 128, (256, 256))]


@pytest.mark.parametrize("M,K,N,num_cus,tile", SPLIT_CASES)
def test_splitk_deterministic_and_matches_plain(lib, cuda, M, K, N, num_cus, tile):
    assert planned_tile(lib, M, N, K, num_cus) == tile
    a = randn((M, K), seed=0, dtype=torch.float16).to(cuda)
    b = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).to(cuda)
    bias = randn((N,), seed=2, scale=0.02).to(cuda)
    s = torch.ones(M, device=cuda)
    st = _stream(cuda)
    plain = torch.empty(M, N, device=cuda)
    assert lib.g16_hgemm_splitk(a.data_ptr(), b.data_ptr(), plain.data_ptr(), 0, bias.data_ptr(), s.data_ptr(),
                                M, N, K, 1, num_cus, None, 0, None, 0, st) == 0
    ref = oracle.gemm(_np(a), _np(s), _np(b), _np(bias), "float32")
    for ksplit in (2, 3, 8, 16):
        ws, cnt = _split_bufs(lib.g16_hgemm_splitk_workspace_bytes(M, N, K, ksplit, num_cus),
                              lib.g16_hgemm_splitk_counter_bytes(M, N, K, ksplit, num_cus), cuda)
        outs = []
        for _ in range(10):
            c = torch.empty(M, N, device=cuda)
            assert lib.g16_hgemm_splitk(a.data_ptr(), b.data_ptr(), c.data_ptr(), 0, bias.data_ptr(), s.data_ptr(),
                                        M, N, K, ksplit, num_cus, ws.data_ptr(), ws.numel(), cnt.data_ptr(),
                                        cnt.numel(), st) == 0
            outs.append(c)
        torch.cuda.synchronize()
        for o in outs[1:]:
            assert torch.equal(o, outs[0])
        # (the ten calls share one counter buffer: each relies on the previous one leaving it zero,
        # or no slice would see itself arrive last and C would stay unwritten)
        assert oracle.rel_err(_np(outs[0]), ref) <= GEMM_TOL
        assert int(cnt.view(torch.int32).abs().sum().item()) == 0
    assert oracle.rel_err(_np(plain), ref) <= GEMM_TOL


def test_splitk_fp16_output(lib, cuda):
    M, K, N = 64, 4096, 1024
    a = randn((M, K), seed=0, dtype=torch.float16).to(cuda)
    b = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).to(cuda)
    bias = randn((N,), seed=2, scale=0.02).to(cuda)
    s = torch.ones(M, device=cuda)
    ws, cnt = _split_bufs(lib.g16_hgemm_splitk_workspace_bytes(M, N, K, 8, 0),
                          lib.g16_hgemm_splitk_counter_bytes(M, N, K, 8, 0), cuda)
    c = torch.empty(M, N, dtype=torch.float16, device=cuda)
    assert lib.g16_hgemm_splitk(a.data_ptr(), b.data_ptr(), c.data_ptr(), 1, bias.data_ptr(), s.data_ptr(),
                                M, N, K, 8, 0, ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(),
                                _stream(cuda)) == 0
    torch.cuda.synchronize()
    ref = oracle.gemm(_np(a), _np(s), _np(b), _np(bias), "float32")
    assert oracle.rel_err(_np(c.float()), ref) <= GEMM_TOL


# (M, N, K step, num_cus, tile): the 128x128 (BK 32), 64x128, 64x64 and 32x128 (BK 64) tiles, each
# forced by the CU count the launch is planned for (the 64x64 case with ragged M and N)
SMALL_TILES = [(300, 264, 32, 8, (128, 128)), (64, 1024, 64, 12, (64, 128)), (100, 200, 64, 16, (64, 64)),
               (20, 200, 64, 256, (32, 128))]


@pytest.mark.parametrize("M,N,bk,num_cus,tile", SMALL_TILES)
@pytest.mark.parametrize("steps", [1, 2, 3, 5])
def test_small_tiles_odd_and_even_step_counts(lib, cuda, M, N, bk, num_cus, tile, steps):
    # The 4-wavefront tiles run their K loop in step pairs plus a tail step for an odd count: whole
    # and ragged last steps, unsplit and in two slices (each slice has its own step count).
    st = _stream(cuda)
    for K in (bk * steps, bk * steps - 8):
        assert planned_tile(lib, M, N, K, num_cus) == tile
        a = randn((M, K), seed=steps, dtype=torch.float16).to(cuda)
        b = randn((K, N), seed=steps + 1, scale=0.05, dtype=torch.float16).to(cuda)
        bias = randn((N,), seed=2, scale=0.02).to(cuda)
        s = torch.ones(M, device=cuda)
        ref = oracle.gemm(_np(a), _np(s), _np(b), _np(bias), "float32")
        c = torch.empty(M, N, device=cuda)
        assert lib.g16_hgemm_splitk(a.data_ptr(), b.data_ptr(), c.data_ptr(), 0, bias.data_ptr(), s.data_ptr(),
                                    M, N, K, 1, num_cus, None, 0, None, 0, st) == 0
        ws, cnt = _split_bufs(lib.g16_hgemm_splitk_workspace_bytes(M, N, K, 2, num_cus),
                              lib.g16_hgemm_splitk_counter_bytes(M, N, K, 2, num_cus), cuda)
        c2 = torch.empty(M, N, device=cuda)
        assert lib.g16_hgemm_splitk(a.data_ptr(), b.data_ptr(), c2.data_ptr(), 0, bias.data_ptr(), s.data_ptr(),
                                    M, N, K, 2, num_cus, ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(),
                                    st) == 0
        torch.cuda.synchronize()
        assert oracle.rel_err(_np(c), ref) <= GEMM_TOL, K
        assert oracle.rel_err(_np(c2), ref) <= GEMM_TOL, K


# ---------------------------------------------------------------------------------------------
# skinny path (M <= 8)
# ---------------------------------------------------------------------------------------------

# 256-column strips up to N = 8192, 512-column strips above (8200: one 8-column group past 16
# strips; 11008 and 14336: the LLM MLP widths)
SKINNY_SHAPES = [(1, 4096, 4096), (4, 4096, 4096), (1, 1024, 3072), (8, 2048, 520), (3, 4096, 4096),
                 (2, 8, 8), (5, 200, 72), (7, 1032, 776), (6, 64, 4104), (1, 1000, 8192), (2, 520, 8200),
                 (1, 4096, 11008), (8, 1024, 14336), (4, 4096, 14336), (6, 136, 9000)]


@pytest.mark.parametrize("M,K,N", SKINNY_SHAPES)
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("with_bias", [False, True])
def test_skinny_matches_oracle(g, cuda, M, K, N, x_dtype, with_bias):
    x = randn((M, K), seed=M + K, dtype=x_dtype)
    w = randn((K, N), seed=K + N, scale=0.02, dtype=torch.float16)
    b = randn((N,), seed=N, scale=0.02) if with_bias else None
    y = g.mm_t(x.to(cuda), w.to(cuda), None if b is None else b.to(cuda), torch.float32)
    torch.cuda.synchronize()
    ref = oracle.skinny(_np(x), _np(w), None if b is None else _np(b))
    assert oracle.rel_err(_np(y), ref) <= SKINNY_TOL


# M = 1 and 3 reduce single columns, M >= 4 four-column groups (two per thread at M = 8, a partial
# second round of groups at M = 5)
@pytest.mark.parametrize("M,ksplit", [(4, 1), (4, 2), (4, 5), (4, 16), (4, 64), (1, 32), (3, 7), (5, 16),
                                      (8, 32), (8, 3)])
def test_skinny_explicit_splits_deterministic(lib, cuda, M, ksplit):
    K, N = 4096, 4096
    x = randn((M, K), seed=0).to(cuda)
    w = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).to(cuda)
    b = randn((N,), seed=2, scale=0.02).to(cuda)
    ws, cnt = _split_bufs(lib.g16_skinny_workspace_bytes(M, N, K, ksplit),
                          lib.g16_skinny_counter_bytes(M, N, K, ksplit), cuda)
    outs = []
    for _ in range(5):
        c = torch.full((M, N), float("nan"), device=cuda)
        assert lib.g16_skinny_f32in(x.data_ptr(), w.data_ptr(), c.data_ptr(), b.data_ptr(), M, N, K, ksplit,
                                    ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(), _stream(cuda)) == 0
        outs.append(c)
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    ref = oracle.skinny(_np(x), _np(w), _np(b))
    assert oracle.rel_err(_np(outs[0]), ref) <= SKINNY_TOL


def test_skinny_M1_4096_cache_rotation_parity(g, cuda):
    # The benchmark rotates distinct weight copies; every copy must give the oracle's answer.
    K = N = 4096
    x = randn((1, K), seed=0)
    b = randn((N,), seed=2, scale=0.02)
    for seed in (1, 101):
        w = randn((K, N), seed=seed, scale=0.02, dtype=torch.float16)
        y = g.mm_t(x.to(cuda), w.to(cuda), b.to(cuda), torch.float32)
        torch.cuda.synchronize()
        assert oracle.rel_err(_np(y), oracle.skinny(_np(x), _np(w), _np(b))) <= SKINNY_TOL


# ---------------------------------------------------------------------------------------------
# C ABI argument checks (rejected before any launch)
# ---------------------------------------------------------------------------------------------

def test_abi_rejects_bad_arguments(lib, cuda):
    a = torch.zeros(64, 64, dtype=torch.float16, device=cuda)
    c = torch.zeros(64, 64, device=cuda)
    st = _stream(cuda)
    assert lib.g16_hgemm_f32out(a.data_ptr(), a.data_ptr(), c.data_ptr(), None, None, 64, 64, 60, st) == -1
    assert lib.g16_hgemm_f32out(a.data_ptr() + 2, a.data_ptr(), c.data_ptr(), None, None, 64, 64, 64, st) == -2
    assert lib.g16_hgemm_f32out(None, a.data_ptr(), c.data_ptr(), None, None, 64, 64, 64, st) == -3
    assert lib.g16_hgemm_splitk(a.data_ptr(), a.data_ptr(), c.data_ptr(), 0, None, None, 64, 64, 1024, 4, 0,
                                None, 0, None, 0, st) == -4
    assert lib.g16_hgemm_splitk(a.data_ptr(), a.data_ptr(), c.data_ptr(), 0, None, None, 64, 64, 1024, 4, 0,
                                c.data_ptr(), c.numel() * 4, None, 0, st) == -4
    assert lib.g16_hgemm_splitk(a.data_ptr(), a.data_ptr(), c.data_ptr(), 0, None, None, 64, 64, 64, 0, 0,
                                None, 0, None, 0, st) == -5
    assert lib.g16_skinny_f32in(a.data_ptr(), a.data_ptr(), c.data_ptr(), None, 9, 64, 64, 1, None, 0, None, 0,
                                st) == -1
    assert lib.g16_rowscale_f32(a.data_ptr(), a.data_ptr(), c.data_ptr(), 4, 64, 1000.0, st) == -1
    assert lib.g16_hgemm_f32out(a.data_ptr(), a.data_ptr(), c.data_ptr(), None, None, 0, 64, 64, st) == 0
    assert b"workspace" in lib.g16_strerror(-4)


def test_mixed_shapes_share_split_buffers(g, cuda):
    # Skinny and split-K calls of different shapes on one stream share the cached partial and
    # counter buffers; every result must still match the oracle (regression: counters once lived
    # inside the partials buffer, where another shape's partial sums could land on them).
    shapes = [(1, 4096, 4096), (64, 1024, 1024), (4, 1024, 3072), (64, 4096, 1024), (8, 2048, 520),
              (33, 4096, 768), (1, 4096, 4096)]
    for i, (M, K, N) in enumerate(shapes * 2):
        x = randn((M, K), seed=100 + i)
        w = randn((K, N), seed=200 + i, scale=0.05, dtype=torch.float16)
        y = g.mm_t(x.to(cuda), w.to(cuda), None, torch.float32)
        torch.cuda.synchronize()
        ref = oracle.mm_t(_np(x), _np(w), None, "float32")
        assert oracle.rel_err(_np(y), ref) <= (SKINNY_TOL if M <= 8 else GEMM_TOL), (M, K, N)


# ---------------------------------------------------------------------------------------------
# committed golden fixtures (hand-derived exponents, exact rational results)
# ---------------------------------------------------------------------------------------------

GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def test_golden_rowscale_known_answers(lib, cuda):
    kat = np.load(GOLDEN / "rowscale_kat.npz")
    x = torch.from_numpy(kat["x"]).to(cuda)
    y, s = _rowscale_gpu(lib, x)
    assert np.array_equal(_np(s).view(np.uint32), kat["S"].view(np.uint32))
    y_ref, _, _ = oracle.rowscale(kat["x"])
    _assert_bits_equal(_np(y).view(np.uint16), y_ref.view(np.uint16), kat["x"], "Y")


@pytest.mark.parametrize("name", ["skinny_m3", "skinny_m8", "gemm_m12", "gemm_m9"])
def test_golden_mm_t_exact(g, cuda, name):
    d = np.load(GOLDEN / "mm_t_exact.npz")
    x, w = d[f"{name}_x"], d[f"{name}_w"]
    b = d[f"{name}_b"] if f"{name}_b" in d.files else None
    y = g.mm_t(torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda),
               None if b is None else torch.from_numpy(b).to(cuda), torch.float32)
    torch.cuda.synchronize()
    tol = SKINNY_TOL if x.shape[0] <= 8 else GEMM_TOL
    assert oracle.rel_err(_np(y), d[f"{name}_out"]) <= tol


# ---------------------------------------------------------------------------------------------
# tile-packed route: packed rowscale bit-exact against the oracle's cast laid out by the numpy
# model of the layout; packed GEMM bitwise equal to the row-major GEMM on the same data
# ---------------------------------------------------------------------------------------------

def _rowscale_pack_gpu(lib, x: torch.Tensor):
    M, K = x.shape
    yp = torch.full((lib.g16_packed_a_bytes(M, K) // 2,), float("nan"), dtype=torch.float16, device=x.device)
    s = torch.empty(M, dtype=torch.float32, device=x.device)
    fn = lib.g16_rowscale_pack_f32 if x.dtype == torch.float32 else lib.g16_rowscale_pack_f16
    st = fn(x.data_ptr(), yp.data_ptr(), s.data_ptr(), M, K, 1024.0, _stream(x.device))
    assert st == 0, st
    torch.cuda.synchronize()
    return yp, s


@pytest.mark.parametrize("M,K", [(1, 8), (255, 136), (300, 4096), (512, 40), (512, 4096)])
@pytest.mark.parametrize("in_dtype", [torch.float32, torch.float16])
def test_rowscale_pack_bitexact(lib, cuda, M, K, in_dtype):
    from _packing import pack_a

    x = randn((M, K), seed=M + K)
    x[0, 0] = -0.0
    if M > 3:
        x[1] *= 3000.0                      # pow2 rescale
        x[2, K // 2] = float("nan")         # ignored by the max
        x[3, K - 1] = 65504.0 if in_dtype == torch.float16 else 179940.0
    x = x.to(in_dtype)
    yp, s = _rowscale_pack_gpu(lib, x.to(cuda))
    y16, S, _ = oracle.rowscale(_np(x.float()) if in_dtype == torch.float32 else _np(x))
    expect = pack_a(y16)
    got = _np(yp)
    assert got.shape == expect.shape
    assert np.array_equal(got.view(np.uint16), expect.view(np.uint16)), "packed fp16 bits differ"
    assert np.array_equal(_np(s).view(np.uint32), S.view(np.uint32))


# (2048, 512, 4096) and the ragged (1800, 136, 3896) give 128 tiles of 256x256: they run 256x128 tiles
@pytest.mark.parametrize("M,K,N", [(300, 136, 264), (2300, 264, 4096), (4096, 4096, 4096), (4100, 1000, 2056),
                                   (2048, 512, 4096), (1800, 136, 3896)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_packed_gemm_bitwise_equals_rowmajor(lib, cuda, M, K, N, out_dtype):
    # outlier rows still need the pow2 rescale, but stay small enough that an fp16 output is finite
    hi = 2e5 if out_dtype == torch.float32 else 1e4
    x = outlier_rows(randn((M, K), seed=0), 0.01, 2e3, hi, seed=3).to(cuda)
    w = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).to(cuda)
    bias = randn((N,), seed=2, scale=0.02).to(cuda)
    st = _stream(cuda)
    y16 = torch.empty(M, K, dtype=torch.float16, device=cuda)
    s = torch.empty(M, dtype=torch.float32, device=cuda)
    assert lib.g16_rowscale_f32(x.data_ptr(), y16.data_ptr(), s.data_ptr(), M, K, 1024.0, st) == 0
    yp, sp = _rowscale_pack_gpu(lib, x)
    f16 = out_dtype == torch.float16
    c_row = torch.empty(M, N, dtype=out_dtype, device=cuda)
    c_pk = torch.empty(M, N, dtype=out_dtype, device=cuda)
    fn_row = lib.g16_hgemm_f16out if f16 else lib.g16_hgemm_f32out
    fn_pk = lib.g16_hgemm_packed_f16out if f16 else lib.g16_hgemm_packed_f32out
    # both on the same 256-row tile where the plain plan picks one; elsewhere the row-major GEMM
    # uses a smaller tile and only the oracle bar applies
    assert fn_row(y16.data_ptr(), w.data_ptr(), c_row.data_ptr(), bias.data_ptr(), s.data_ptr(), M, N, K, st) == 0
    assert fn_pk(yp.data_ptr(), w.data_ptr(), c_pk.data_ptr(), bias.data_ptr(), sp.data_ptr(), M, N, K, st) == 0
    torch.cuda.synchronize()
    if lib.g16_hgemm_use_packed(M, N, K, torch.cuda.get_device_properties(cuda).multi_processor_count):
        assert torch.equal(c_pk, c_row)
    ref = oracle.gemm(_np(y16), _np(s), _np(w), _np(bias), "float16" if f16 else "float32")
    assert oracle.rel_err(_np(c_pk.float()), ref.astype(np.float64)) <= GEMM_TOL


# (M, K, N, ksplit, rows per wavefront), each with fewer rows per wavefront than its batch: 256-column
# strips (two rows per load instruction; 8-row batches for M = 1 and 4, 16-row ones for M = 5) and
# the 512-column strips of N > 8192 (8-row batches for M = 1, 16-row ones for M = 8)
@pytest.mark.parametrize("M,K,N,ksplit,rpw", [(1, 1024, 1024, 32, 4), (4, 1024, 1024, 32, 4),
                                              (5, 1024, 1024, 16, 8), (1, 1024, 8704, 32, 4),
                                              (8, 1024, 8704, 16, 8)])
def test_skinny_partial_block_ignores_rows_past_the_slice(lib, cuda, M, K, N, ksplit, rpw):
    # A wavefront with fewer rows than its batch loads: the last batch re-reads the slice's last row
    # for the missing ones and must not use them. A +inf in that last row must therefore reach the
    # output as +inf (a 0 * inf from a reused row would make it NaN).
    x = randn((M, K), seed=21).abs() + 0.5          # positive activations
    w = randn((K, N), seed=22, scale=0.02, dtype=torch.float16)
    w[rpw - 1, 5] = float("inf")                    # last row of wavefront 0 of slice 0
    w[K - 1, 9] = float("inf")                      # last row of the last slice
    xd, wd = x.to(cuda), w.to(cuda)
    out = torch.empty(M, N, device=cuda)
    st = _stream(cuda)
    ws, cnt = _split_bufs(lib.g16_skinny_workspace_bytes(M, N, K, ksplit), lib.g16_skinny_counter_bytes(M, N, K, ksplit), cuda)
    assert lib.g16_skinny_f32in(xd.data_ptr(), wd.data_ptr(), out.data_ptr(), None, M, N, K, ksplit,
                                ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(), st) == 0
    torch.cuda.synchronize()
    y = _np(out)
    assert np.isposinf(y[:, 5]).all() and np.isposinf(y[:, 9]).all()
    finite = np.ones(N, dtype=bool)
    finite[[5, 9]] = False
    ref = oracle.skinny(_np(x), _np(w), None, "float32")
    assert np.isfinite(y[:, finite]).all()
    assert oracle.rel_err(y[:, finite], ref[:, finite]) <= SKINNY_TOL


# One shape per route of the GEMM path: plain 32x128 tiles, split-K, tile-packed 256x256, tile-packed
# 256x128 (128 tiles of 256^2 would leave half the CUs idle)
@pytest.mark.parametrize("M,K,N", [(300, 136, 264), (64, 1024, 1024), (4100, 264, 2056), (2048, 264, 4096)])
@pytest.mark.parametrize("in_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_mm_t_one_call_equals_separate_launches(lib, g, cuda, M, K, N, in_dtype, out_dtype):
    # mm_t runs g16_mm_t_gemm; the same rowscale cast and GEMM launched one by one must give the
    # same bits
    # outlier rows stay finite in the input dtype (fp16 tops out at 65504)
    hi = 2e5 if out_dtype == torch.float32 and in_dtype == torch.float32 else 1e4
    x = outlier_rows(randn((M, K), seed=0), 0.01, 2e3, hi, seed=3).to(in_dtype).to(cuda)
    w = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).to(cuda)
    bias = randn((N,), seed=2, scale=0.02).to(cuda)
    y = g.mm_t(x, w, bias, out_dtype)
    st = _stream(cuda)
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    f32in, f16out = in_dtype == torch.float32, out_dtype == torch.float16
    s = torch.empty(M, dtype=torch.float32, device=cuda)
    ref = torch.empty(M, N, dtype=out_dtype, device=cuda)
    if lib.g16_hgemm_use_packed(M, N, K, cus):
        yp = torch.empty(lib.g16_packed_a_bytes(M, K) // 2, dtype=torch.float16, device=cuda)
        rs = lib.g16_rowscale_pack_f32 if f32in else lib.g16_rowscale_pack_f16
        assert rs(x.data_ptr(), yp.data_ptr(), s.data_ptr(), M, K, 1024.0, st) == 0
        fn = lib.g16_hgemm_packed_f16out if f16out else lib.g16_hgemm_packed_f32out
        assert fn(yp.data_ptr(), w.data_ptr(), ref.data_ptr(), bias.data_ptr(), s.data_ptr(), M, N, K, st) == 0
    else:
        y16 = torch.empty(M, K, dtype=torch.float16, device=cuda)
        rs = lib.g16_rowscale_f32 if f32in else lib.g16_rowscale_f16
        assert rs(x.data_ptr(), y16.data_ptr(), s.data_ptr(), M, K, 1024.0, st) == 0
        ks = lib.g16_hgemm_plan(M, N, K, cus)
        if ks > 1:
            ws, cnt = _split_bufs(lib.g16_hgemm_splitk_workspace_bytes(M, N, K, ks, 0),
                                  lib.g16_hgemm_splitk_counter_bytes(M, N, K, ks, 0), cuda)
            assert lib.g16_hgemm_splitk(y16.data_ptr(), w.data_ptr(), ref.data_ptr(), 1 if f16out else 0,
                                        bias.data_ptr(), s.data_ptr(), M, N, K, ks, 0, ws.data_ptr(), ws.numel(),
                                        cnt.data_ptr(), cnt.numel(), st) == 0
        else:
            fn = lib.g16_hgemm_f16out if f16out else lib.g16_hgemm_f32out
            assert fn(y16.data_ptr(), w.data_ptr(), ref.data_ptr(), bias.data_ptr(), s.data_ptr(), M, N, K, st) == 0
    torch.cuda.synchronize()
    bits = torch.int32 if out_dtype == torch.float32 else torch.int16
    assert torch.isfinite(y).all()
    assert torch.equal(y.view(bits), ref.view(bits))


def _same_nonfinite_pattern(got, want):
    # NaN positions, infinity positions and signs equal; finite entries within the skinny bar
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isposinf(got), np.isposinf(want))
    assert np.array_equal(np.isneginf(got), np.isneginf(want))
    fin = np.isfinite(want)
    if fin.any():
        assert oracle.rel_err(got[fin], want[fin]) <= SKINNY_TOL


@pytest.mark.parametrize("M", [1, 2, 4, 8])
@pytest.mark.parametrize("K,N", [(3072, 1024), (11008, 1024), (1024, 8704)])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.float16])
def test_skinny_nonfinite_activations_at_slice_edges(g, lib, cuda, M, K, N, x_dtype):
    # mm_t's skinny path (M <= 8) on the split kernel: +-inf activations at the first and last row of
    # the planned K slices and at K - 1 reach the output as the oracle's +-inf (NaN only where the
    # weight is zero or both signs meet), not as a NaN from rows a lane re-reads and skips
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    ks = lib.g16_skinny_plan(M, N, K, cus)
    slice_rows = -(-K // ks)
    x = randn((M, K), seed=K + M, dtype=x_dtype)
    edges = sorted({0, slice_rows - 1, slice_rows, min(K - 1, 2 * slice_rows - 1), K - 1})
    for m in range(M):
        x[m, edges[m % len(edges)]] = float("inf") if m % 2 == 0 else float("-inf")
    w = randn((K, N), seed=K, scale=0.02, dtype=torch.float16)
    b = randn((N,), seed=N, scale=0.02)
    y = g.mm_t(x.to(cuda), w.to(cuda), b.to(cuda), torch.float32)
    torch.cuda.synchronize()
    want = oracle.skinny(_np(x), _np(w), _np(b))
    assert not np.isfinite(want).any()
    _same_nonfinite_pattern(_np(y).astype(np.float64), want)
