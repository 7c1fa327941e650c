"""GPU parity of the public API on the routes the planner picks, and on the BASELINE configurations
exactly as configured.

* C1: ``matmul(a16, b16)`` at 1024^3 on N(0,1) fp16 from seeds 0 and 1, fp16 out (ops.py:111-119).
* C3: ``mm_t`` at 64x1024x1024 and 64x4096x1024 (fp16 A, fp32 bias and out) at the split the
  library plans for this GPU, ten calls bitwise equal (the reference's split-K is not
  deterministic, README.md:79; tests/test_correctness.py:52-59 checks repeatability).
* Each split-K tile through ``mm_t``: the 128x128 tile split twice, the 64x128 tile split twice
  and 4 ways, the square 64x64 tile unsplit and split 2 and 3 ways, the 128x128 tile unsplit and
  split with an odd number of K steps and a ragged last step, and the 32x128 tile of C3 and at
  M > 64. The packed-weight 256x256 and 256x128 tiles the planner falls back to when no
  4-wavefront grid fits one round (M >= 512, long K, large N) run unsplit; past 256 tiles their
  grid is persistent (one workgroup per CU walking several tiles), here with ragged tile counts and
  at the BERT-base linear shapes (sampled rows). The tile
  each case runs on is the library's own report (g16_hgemm_tile), so a plan change that moves a
  case to another tile fails here instead of silently dropping that tile from the tests.
* Rows holding +-inf or NaN (at tile-row edges and at K - 1), an all-zero row and rescaled rows
  through the tile-packed route (both 256-row tiles, one round and persistent) and through every
  4-wavefront route (split and unsplit, the resident cast), fp32 and fp16 x and out; likewise weight
  columns holding +-inf and NaN (at k = 0, mid-K and K - 1) against exact-zero activations: exactly
  the oracle's non-finite pattern, every other row and column within the GEMM bar.
* The fp16-output golden fixtures (exact rational results, tests/golden/make_golden.py).

Every result is checked against the fp64 oracle: relative Frobenius error <= 1e-3 on the GEMM
paths, <= 1e-5 on the skinny path, fp16 outputs within one fp16 ulp of the exact fixture.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from _inputs import randn
from _plan import tile as planned_tile

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-3
SKINNY_TOL = 1e-5
GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def g(cuda):
    import gtx16_fp16

    return gtx16_fp16


@pytest.fixture(scope="module")
def lib(cuda):
    from gtx16_fp16 import _clib

    return _clib.load()


@pytest.fixture(scope="module")
def cus(cuda):
    return torch.cuda.get_device_properties(cuda).multi_processor_count


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def test_c1_matmul_exactly_as_configured(g, cuda):
    a = randn((1024, 1024), seed=0, dtype=torch.float16)
    b = randn((1024, 1024), seed=1, dtype=torch.float16)
    y = g.matmul(a.to(cuda), b.to(cuda))
    torch.cuda.synchronize()
    assert y.dtype == torch.float16 and y.shape == (1024, 1024)
    ref = oracle.mm_t(_np(a), _np(b), None, "float16")
    assert np.isfinite(_np(y).astype(np.float64)).all()
    assert oracle.rel_err(_np(y), ref) <= GEMM_TOL
    # the C1 ids are fp16 and at most ~5 in magnitude: no row is rescaled
    assert (oracle.row_exponent(oracle.row_amax(_np(a))) == 0).all()


# (M, K, N, tile the planner picks on 256 CUs, ksplit it plans)
ROUTES = [
    (64, 1024, 1024, (32, 128), 4),      # C3
    (64, 4096, 1024, (32, 128), 8),      # C3
    (1024, 1024, 1024, (64, 64), 1),     # C1's shape: the square tile, unsplit
    (100, 2048, 3072, (64, 64), 2),      # the square tile split twice, ragged M
    (320, 4056, 1024, (64, 64), 3),      # ... 3 ways: slices of 22, 22 and 20 K steps, the last ragged
    (320, 8192, 4096, (128, 128), 2),    # 128x128 split twice
    (64, 4096, 11008, (64, 128), 2),     # 64x128 split twice
    (128, 8192, 4096, (64, 128), 4),     # 64x128 split 4 ways at M > 64
    (256, 11008, 264, (32, 128), 8),     # 32x128 split 8 ways at M > 64
    (768, 4056, 4096, (128, 128), 1),    # 128x128 unsplit: 127 K steps, the last one ragged
    (384, 4056, 3072, (128, 128), 3),    # split: slices of 44, 44 and 39 K steps, the last one ragged
    (768, 4096, 11008, (256, 256), 1),   # no 4-wavefront grid fits one round: packed 256x256 tiles
    (512, 4096, 11008, (256, 128), 1),   # ... packed 256x128 tiles where their grid fits one round
    (2560, 512, 8192, (256, 256), 1),    # 320 tiles: a persistent grid of 256 workgroups, 64 take two
    (3000, 264, 5800, (256, 256), 1),    # 276 ragged tiles (not a multiple of 8), persistent grid
]


@pytest.mark.parametrize("M,K,N,tile,ks", ROUTES)
def test_planned_route_matches_oracle_and_repeats_bitwise(g, lib, cus, cuda, M, K, N, tile, ks):
    if cus != 256:
        pytest.skip(f"the route table is for 256 CUs (this device has {cus})")
    assert planned_tile(lib, M, N, K, cus) == tile
    assert lib.g16_hgemm_plan(M, N, K, cus) == ks
    x = randn((M, K), seed=0, dtype=torch.float16).to(cuda)
    w = randn((K, N), seed=1, scale=0.02, dtype=torch.float16).to(cuda)
    bias = randn((N,), seed=2, scale=0.02).to(cuda)
    outs = [g.mm_t(x, w, bias, torch.float32) for _ in range(10)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    ref = oracle.mm_t(_np(x), _np(w), _np(bias), "float32")
    assert oracle.rel_err(_np(outs[0]), ref) <= GEMM_TOL
    # fp16 output on the same route: the split reduction casts in its epilogue
    y16 = g.mm_t(x, w, bias, torch.float16)
    torch.cuda.synchronize()
    assert oracle.rel_err(_np(y16), oracle.mm_t(_np(x), _np(w), _np(bias), "float16")) <= GEMM_TOL


@pytest.mark.parametrize("M,K,N", [(65536, 768, 768), (65536, 768, 3072), (65536, 3072, 768)])
def test_persistent_grid_at_bert_shapes(g, cuda, M, K, N):
    # The BERT-base linears at 256 x 256 tokens: 768 to 3072 tiles of 256x256, walked by a
    # persistent grid of one workgroup per CU. Rows are independent, so sampled rows of the result
    # are checked against the oracle on those rows alone; every tile is checked for repeatability.
    x = randn((M, K), seed=5).to(cuda)
    x[123] *= 4000.0  # a rescaled row
    w = randn((K, N), seed=6, scale=0.02, dtype=torch.float16).to(cuda)
    b = randn((N,), seed=7, scale=0.02).to(cuda)
    y = g.mm_t(x, w, b, torch.float32)
    y2 = g.mm_t(x, w, b, torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    rows = np.sort(np.random.default_rng(M + N).choice(M, 384, replace=False))
    rows = np.unique(np.concatenate([rows, [0, 123, 255, 256, M - 1]]))
    ref = oracle.mm_t(_np(x)[rows], _np(w), _np(b), "float32")
    assert oracle.rel_err(_np(y)[rows], ref) <= GEMM_TOL


@pytest.mark.parametrize("M,K,N", [(65636, 768, 776), (40000, 1032, 1288)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_persistent_grid_partial_tiles(g, lib, cuda, M, K, N, out_dtype):
    # A persistent grid (more 256x256 tiles than CUs) whose last tile row and column are partial and
    # whose last K step is partial (K = 1032): its C stores are the non-temporal buffer stores (16
    # bytes for fp32 out, 8 for fp16), bounds-guarded per row and 4-column chunk like the plain ones.
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    assert lib.g16_hgemm_use_packed(M, N, K, cus) == 1
    tiles = -(-M // 256) * -(-N // 256)
    assert tiles > cus
    x = randn((M, K), seed=11).to(cuda)
    x[M - 1] *= 4000.0  # a rescaled row in the partial tile row
    w = randn((K, N), seed=12, scale=0.02, dtype=torch.float16).to(cuda)
    b = randn((N,), seed=13, scale=0.02).to(cuda)
    y = g.mm_t(x, w, b, out_dtype)
    y2 = g.mm_t(x, w, b, out_dtype)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    rows = np.sort(np.random.default_rng(M + K).choice(M, 256, replace=False))
    rows = np.unique(np.concatenate([rows, [0, 255, 256, M - 257, M - 256, M - 2, M - 1]]))
    want = oracle.mm_t(_np(x)[rows], _np(w), _np(b), "float16" if out_dtype == torch.float16 else "float32")
    assert np.isfinite(_np(y)[rows]).all()
    assert oracle.rel_err(_np(y)[rows], want) <= GEMM_TOL


@pytest.mark.parametrize("M,K,N,tile", [(2600, 2056, 2824, (256, 256)), (4096, 1032, 4104, (256, 256)),
                                        (2048, 2056, 3080, (256, 128))])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.float16])
def test_packed_route_nonfinite_zero_and_rescaled_rows(g, lib, cus, cuda, M, K, N, tile, x_dtype):
    # The tile-packed route (rowscale_pack cast, then the 256-row GEMM; past one round a persistent
    # grid) with rows holding +inf, -inf or NaN, at tile-row edges and at K - 1, next to an all-zero
    # row and rescaled rows. An infinite row's scale is +inf and its cast 0 * inf = NaN, so its
    # output row is NaN; a NaN row's |max| ignores the NaN and its output row is NaN too. The
    # non-finite pattern must be the oracle's exactly, and no other row may be touched by it.
    if cus != 256:
        pytest.skip(f"the route table is for 256 CUs (this device has {cus})")
    assert lib.g16_hgemm_use_packed(M, N, K, cus) == 1
    assert planned_tile(lib, M, N, K, cus) == tile
    x = randn((M, K), seed=31)
    special = {5: ("inf", 7), 255: ("nan", 100), 256: ("inf", K - 1), 300: ("nan", 0), 301: ("-inf", K - 1),
               M - 1: ("-inf", K // 2)}
    for r, (v, k) in special.items():
        x[r, k] = float(v)
    x[777 % M] = 0.0           # an all-zero row
    x[1000 % M, 3] = 3.0e4     # rescaled rows (exponent 5), fp16-representable
    x[257, K - 1] = -2.5e4
    x = x.to(x_dtype)
    w = randn((K, N), seed=32, scale=0.02, dtype=torch.float16)
    b = randn((N,), seed=33, scale=0.02)
    for out_dtype, name in ((torch.float32, "float32"), (torch.float16, "float16")):
        y = g.mm_t(x.to(cuda), w.to(cuda), b.to(cuda), out_dtype)
        torch.cuda.synchronize()
        rows = np.sort(np.random.default_rng(M + N).choice(M, 192, replace=False))
        rows = np.unique(np.concatenate([rows, list(special), [777 % M, 1000 % M, 257, 0, 254, 302, M - 2]]))
        got = _np(y)[rows].astype(np.float64)
        want = oracle.mm_t(_np(x)[rows], _np(w), _np(b), name).astype(np.float64)
        assert np.array_equal(np.isnan(got), np.isnan(want))
        assert np.array_equal(np.isposinf(got), np.isposinf(want))
        assert np.array_equal(np.isneginf(got), np.isneginf(want))
        bad = np.isin(rows, list(special))
        assert np.isnan(want[bad]).all() and np.isfinite(want[~bad]).all()
        assert oracle.rel_err(got[~bad], want[~bad]) <= GEMM_TOL


# (M, K, N, tile, ksplit, resident): the 4-wavefront routes. With fp32 x the cast is its own launch,
# or, on the unsplit 32x128 tile with K <= 1280, the GEMM casts its rows into LDS (resident); with
# fp16 x the GEMM streams x itself and recomputes the tiles whose rows exceed the threshold.
SMALL_ROUTES = [
    (48, 768, 1024, (32, 128), 1, True),
    (64, 1024, 1024, (32, 128), 4, False),
    (64, 4096, 1024, (32, 128), 8, False),
    (1024, 1024, 1024, (64, 64), 1, False),
    (320, 4056, 1024, (64, 64), 3, False),
    (128, 8192, 4096, (64, 128), 4, False),
    (768, 4056, 4096, (128, 128), 1, False),
    (384, 4056, 3072, (128, 128), 3, False),
]


@pytest.mark.parametrize("M,K,N,tile,ks,resident", SMALL_ROUTES)
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.float16])
def test_small_tile_routes_nonfinite_zero_and_rescaled_rows(g, lib, cus, cuda, M, K, N, tile, ks, resident, x_dtype):
    # The same rows as on the packed route, on every 4-wavefront route: the split reduction adds
    # the slices' NaN rows like any other, and no slice's non-finite row reaches another row.
    if cus != 256:
        pytest.skip(f"the route table is for 256 CUs (this device has {cus})")
    assert planned_tile(lib, M, N, K, cus) == tile
    assert lib.g16_hgemm_plan(M, N, K, cus) == ks
    assert (lib.g16_mm_t_scratch_bytes(M, N, K, cus) == 0) == resident
    x = randn((M, K), seed=41)
    special = {1: ("inf", 7), 31: ("nan", 100), 32: ("inf", K - 1), M - 3: ("nan", 0), M - 2: ("-inf", K - 1),
               M - 1: ("-inf", K // 2)}
    assert len(special) == 6 and not {3, 10, 33} & set(special)
    for r, (v, k) in special.items():
        x[r, k] = float(v)
    x[3] = 0.0           # an all-zero row
    x[10, 3] = 3.0e4     # rescaled rows (exponent 5), fp16-representable
    x[33, K - 1] = -2.5e4
    x = x.to(x_dtype)
    w = randn((K, N), seed=42, scale=0.02, dtype=torch.float16)
    b = randn((N,), seed=43, scale=0.02)
    for out_dtype, name in ((torch.float32, "float32"), (torch.float16, "float16")):
        y = g.mm_t(x.to(cuda), w.to(cuda), b.to(cuda), out_dtype)
        torch.cuda.synchronize()
        got = _np(y).astype(np.float64)
        want = oracle.mm_t(_np(x), _np(w), _np(b), name).astype(np.float64)
        assert np.array_equal(np.isnan(got), np.isnan(want))
        assert np.array_equal(np.isposinf(got), np.isposinf(want))
        assert np.array_equal(np.isneginf(got), np.isneginf(want))
        bad = np.isin(np.arange(M), list(special))
        assert np.isnan(want[bad]).all() and np.isfinite(want[~bad]).all()
        assert oracle.rel_err(got[~bad], want[~bad]) <= GEMM_TOL


WEIGHT_ROUTES = [(M, K, N) for (M, K, N, *_r) in SMALL_ROUTES] + [
    (2600, 2056, 2824),   # packed 256x256, one round
    (4096, 1032, 4104),   # packed 256x256, persistent grid
    (2048, 2056, 3080),   # packed 256x128
]


@pytest.mark.parametrize("M,K,N", WEIGHT_ROUTES)
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.float16])
def test_nonfinite_weights_on_every_route(g, lib, cus, cuda, M, K, N, x_dtype):
    # Weight columns holding +inf (at k = 0), -inf (at K - 1, in the last K step and slice) and NaN
    # (mid-K), and a column holding +inf and -inf: each output entry is +-inf by the sign of the
    # activation it meets, NaN where that activation is exactly zero or the column's infinities
    # cancel, the oracle's pattern exactly; the other columns are untouched.
    if cus != 256:
        pytest.skip(f"the route table is for 256 CUs (this device has {cus})")
    x = randn((M, K), seed=51)
    x[5, 0] = 0.0          # inf * 0 -> NaN in row 5 of the +inf column
    x[9, K - 1] = 0.0
    x[12, 3] = 4.0e4       # a rescaled row
    x = x.to(x_dtype)
    w = randn((K, N), seed=52, scale=0.02, dtype=torch.float16)
    cols = {3: (0, "inf"), N // 2: (K - 1, "-inf"), N - 1: (K // 2, "nan")}
    for c, (k, v) in cols.items():
        w[k, c] = float(v)
    w[1, 7], w[K - 2, 7] = float("inf"), float("-inf")
    b = randn((N,), seed=53, scale=0.02)
    for out_dtype, name in ((torch.float32, "float32"), (torch.float16, "float16")):
        y = g.mm_t(x.to(cuda), w.to(cuda), b.to(cuda), out_dtype)
        torch.cuda.synchronize()
        got = _np(y).astype(np.float64)
        want = oracle.mm_t(_np(x), _np(w), _np(b), name).astype(np.float64)
        assert np.array_equal(np.isnan(got), np.isnan(want))
        assert np.array_equal(np.isposinf(got), np.isposinf(want))
        assert np.array_equal(np.isneginf(got), np.isneginf(want))
        special = np.isin(np.arange(N), list(cols) + [7])
        assert not np.isfinite(want[:, special]).any() and np.isnan(want[5, 3]) and np.isnan(want[9, N // 2])
        assert oracle.rel_err(got[:, ~special], want[:, ~special]) <= GEMM_TOL


CASES16 = ("skinny_m3", "skinny_m8", "gemm_m12", "gemm_m9", "skinny_tie16", "gemm_tie16")


@pytest.mark.parametrize("name", CASES16)
def test_golden_fp16_output(g, cuda, name):
    d = np.load(GOLDEN / "mm_t_exact.npz")
    x, w = d[f"{name}_x"], d[f"{name}_w"]
    b = d[f"{name}_b"] if f"{name}_b" in d.files else None
    y = g.mm_t(torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda),
               None if b is None else torch.from_numpy(b).to(cuda), torch.float16)
    torch.cuda.synchronize()
    got = _np(y).view(np.uint16).astype(np.int32)
    want = d[f"{name}_out16"].astype(np.int32)
    # same sign, at most one fp16 ulp apart (the kernels accumulate in fp32 in their own order)
    assert ((got & 0x8000) == (want & 0x8000)).all() or np.all(np.abs(_np(y)) < 2.0 ** -14)
    assert np.abs(got - want).max() <= 1, name
    if name == "skinny_tie16":
        # fp32 result 1 + 2^-11 exactly (the fixture's tie), cast like out.to(fp16): even, 1.0
        assert int(got[0, 0]) == 0x3C00
    tol = SKINNY_TOL if x.shape[0] <= 8 else GEMM_TOL
    y32 = g.mm_t(torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda),
                 None if b is None else torch.from_numpy(b).to(cuda), torch.float32)
    torch.cuda.synchronize()
    assert oracle.rel_err(_np(y32), d[f"{name}_out"]) <= tol
