"""CPU tests pinning the fp64 oracle (oracle/semantics.py) to facts other than its own formulas.

Each check is also run against a deliberately broken copy of the oracle function (a planted mistake
of the kind that could slip in: floor instead of ceil, a non-strict threshold, a dropped bias term,
a transposed operand, quantised skinny activations) and must reject it.
"""
from __future__ import annotations

from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

import oracle
from oracle import semantics as S

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------------------------------------
# checks (take the function under test)
# ---------------------------------------------------------------------------------------------

def check_exponent_kats(row_exponent) -> None:
    kat = np.load(GOLDEN / "rowscale_kat.npz")
    got = row_exponent(kat["amax"])
    assert np.array_equal(got, kat["e"]), (got, kat["e"])


def check_exponent_minimal(row_exponent) -> None:
    # e is the smallest e >= 0 with amax / 2^e <= 1024 (searched exactly with rationals)
    rng = np.random.default_rng(3)
    amax = np.concatenate([rng.uniform(0, 3000, 300), np.exp(rng.uniform(np.log(1024), np.log(3e38), 300)),
                           [1024.0, 2048.0, 4096.0, 1025.0]]).astype(np.float32)
    got = row_exponent(amax)
    for a, e in zip(amax.tolist(), got.tolist()):
        q = Fraction(a)
        want = 0
        while q / Fraction(2) ** want > 1024:
            want += 1
        assert e == want, (a, e, want)


def check_rowscale_fixture(rowscale) -> None:
    kat = np.load(GOLDEN / "rowscale_kat.npz")
    y16, Sv, e = rowscale(kat["x"])
    assert np.array_equal(e, kat["e"])
    assert np.array_equal(Sv.view(np.uint32), kat["S"].view(np.uint32))
    # the scaled row fits under the threshold and scaling back recovers x to fp16 precision
    y = y16.astype(np.float64)
    assert (np.abs(y).max(axis=1) <= 1024).all()
    back = y * Sv[:, None].astype(np.float64)
    x = kat["x"].astype(np.float64)
    assert np.all(np.abs(back - x) <= np.abs(x) * 2.0 ** -11 + Sv[:, None] * 2.0 ** -25)


def check_mm_t_exact(mm_t) -> None:
    d = np.load(GOLDEN / "mm_t_exact.npz")
    for name in ("skinny_m3", "skinny_m8", "gemm_m12", "gemm_m9"):
        b = d[f"{name}_b"] if f"{name}_b" in d.files else None
        got = mm_t(d[f"{name}_x"], d[f"{name}_w"], b, "float32").astype(np.float64)
        want = d[f"{name}_out"].astype(np.float32).astype(np.float64)  # the exact result in fp32
        np.testing.assert_allclose(got, want, rtol=2 ** -22, atol=1e-30, err_msg=name)


CASES16 = ("skinny_m3", "skinny_m8", "gemm_m12", "gemm_m9", "skinny_tie16", "gemm_tie16")


def check_mm_t_exact16(mm_t) -> None:
    # fp16 output, bit for bit: the GEMM path's single rounding of the exact result, the skinny
    # path's fp32-then-fp16 rounding (the *_tie16 cases tell the two apart)
    d = np.load(GOLDEN / "mm_t_exact.npz")
    for name in CASES16:
        b = d[f"{name}_b"] if f"{name}_b" in d.files else None
        got = np.asarray(mm_t(d[f"{name}_x"], d[f"{name}_w"], b, "float16")).astype(np.float16).view(np.uint16)
        want = d[f"{name}_out16"]
        assert np.array_equal(got, want), (name, np.argwhere(got != want)[:4].tolist())


def check_identity_and_permutation(gemm) -> None:
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((16, 8))).astype(np.float16)
    eye = np.eye(16, dtype=np.float16)
    assert np.array_equal(gemm(eye, np.ones(16, np.float32), w, None, "float32"), w.astype(np.float32))
    perm = rng.permutation(16)
    P = eye[perm]
    assert np.array_equal(gemm(P, np.ones(16, np.float32), w, None, "float32"), w[perm].astype(np.float32))
    # a row scale of 2^e multiplies the row exactly
    Sv = np.ldexp(np.float32(1), np.arange(16) % 5).astype(np.float32)
    got = gemm(eye, Sv, w, None, "float32")
    assert np.array_equal(got, (w.astype(np.float64) * Sv[:, None]).astype(np.float32))


def check_constant16(mm_t) -> None:
    # tests/test_correctness.py:103-109: every output is 16 * 16 * 4096 = 1,048,576 exactly
    x = np.full((128, 4096), 16.0, dtype=np.float16)
    w = np.full((4096, 128), 16.0, dtype=np.float16)
    y = mm_t(x, w, None, "float32")
    assert np.all(y == np.float32(1048576.0))


def check_skinny_unquantised(mm_t) -> None:
    # M <= 8 uses fp32 activations as is; M > 8 quantises them to fp16 (kernels.py:176-191 vs 243-244)
    v = np.float32(1 + 2.0 ** -20)
    w = np.ones((8, 8), dtype=np.float16)
    x8 = np.zeros((8, 8), dtype=np.float32)
    x8[:, 0] = v
    x9 = np.zeros((9, 8), dtype=np.float32)
    x9[:, 0] = v
    assert np.all(mm_t(x8, w, None, "float32") == v)
    assert np.all(mm_t(x9, w, None, "float32") == np.float32(1.0))


# ---------------------------------------------------------------------------------------------
# the oracle passes every check
# ---------------------------------------------------------------------------------------------

def test_exponent_known_answers():
    check_exponent_kats(oracle.row_exponent)


def test_exponent_is_smallest_power_of_two():
    check_exponent_minimal(oracle.row_exponent)


def test_rowscale_fixture_and_invariants():
    check_rowscale_fixture(oracle.rowscale)


def test_mm_t_matches_exact_rational_results():
    check_mm_t_exact(oracle.mm_t)


def test_mm_t_fp16_output_matches_exact_rational_results():
    check_mm_t_exact16(oracle.mm_t)


def test_identity_permutation_and_scale():
    check_identity_and_permutation(oracle.gemm)


def test_constant_16_known_answer():
    check_constant16(oracle.mm_t)


def test_skinny_path_does_not_quantise():
    check_skinny_unquantised(oracle.mm_t)


@pytest.mark.parametrize("value,bits", [
    (1.0, 0x3C00), (1 + 2.0 ** -11, 0x3C00), (1 + 3 * 2.0 ** -11, 0x3C02),   # ties to even
    (65504.0, 0x7BFF), (65519.99, 0x7BFF), (65520.0, 0x7C00), (-70000.0, 0xFC00),  # overflow at the tie
    (2.0 ** -24, 0x0001), (2.0 ** -25, 0x0000), (3 * 2.0 ** -26, 0x0001),      # smallest subnormal
    (1.5 * 2.0 ** -24, 0x0002), (2.5 * 2.0 ** -24, 0x0002), (2.0 ** -14, 0x0400),
    (-0.0, 0x8000), (-(2.0 ** -26), 0x8000),
])
def test_fp16_rounding_known_answers(value, bits):
    assert int(oracle.fp16_rne(np.float64(value)).view(np.uint16)) == bits


def test_row_amax_ignores_nan_and_starts_at_zero():
    x = np.array([[np.nan, -3.0, 2.0], [np.nan, np.nan, np.nan], [-0.0, 0.0, -0.0]], dtype=np.float32)
    assert oracle.row_amax(x).tolist() == [3.0, 0.0, 0.0]


def test_infinite_row_gets_infinite_scale():
    x = np.array([[1.0, np.inf, 2.0], [1.0, 2.0, 3.0]], dtype=np.float32)
    y16, Sv, e = oracle.rowscale(x)
    assert np.isinf(Sv[0]) and Sv[1] == 1.0 and e[0] == oracle.semantics.INF_EXPONENT
    assert y16[1].tolist() == [1.0, 2.0, 3.0]


def test_rel_err_known_answer():
    assert oracle.rel_err([1.0, 0.0], [1.0, 1.0]) == pytest.approx(2 ** -0.5)
    assert oracle.rel_err([0.0], [0.0]) == 0.0


def test_fixture_generator_rounding_agrees_with_known_answers():
    # the bit-by-bit fp16 rounding used to build mm_t_exact.npz, on the known answers above
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    for value, bits in [(1 + 2.0 ** -11, 0x3C00), (65520.0, 0x7C00), (3 * 2.0 ** -26, 0x0001),
                        (1.5 * 2.0 ** -24, 0x0002), (-(2.0 ** -26), 0x8000), (2.0 ** -14 - 2.0 ** -25, 0x0400)]:
        assert mg.fp16_bits_exact(Fraction(value)) == bits
    rng = np.random.default_rng(1)
    for v in rng.standard_normal(2000) * np.exp(rng.uniform(-20, 12, 2000)):
        with np.errstate(over="ignore"):
            want = int(np.float64(v).astype(np.float16).view(np.uint16))
        assert mg.fp16_bits_exact(Fraction(float(v))) == want
    # its fp32 rounding: ties to even at 1 + 2^-24, subnormals, and numpy's fp64 -> fp32 on random values
    assert mg.fp32_round_exact(1 + Fraction(1, 2 ** 24)) == 1
    assert mg.fp32_round_exact(1 + Fraction(3, 2 ** 24)) == 1 + Fraction(1, 2 ** 22)
    assert mg.fp32_round_exact(Fraction(3, 2 ** 151)) == Fraction(1, 2 ** 149)
    for v in rng.standard_normal(2000) * np.exp(rng.uniform(-100, 80, 2000)):
        assert float(mg.fp32_round_exact(Fraction(float(v)))) == float(np.float32(v))


# ---------------------------------------------------------------------------------------------
# planted mistakes are caught
# ---------------------------------------------------------------------------------------------

def _floor_exponent(amax, thresh=1024.0):
    amax = np.asarray(amax, dtype=np.float64)
    r = np.where(amax > thresh, amax / thresh, 1.0)
    return np.where(amax > thresh, np.floor(np.log2(r)), 0).astype(np.int32)


def _non_strict_exponent(amax, thresh=1024.0):
    e = S.row_exponent(amax, thresh)
    return np.where(np.asarray(amax) == thresh, 1, e).astype(np.int32)


def _mm_t_without_bias(x, w, bias=None, out_dtype="float32"):
    return S.mm_t(x, w, None, out_dtype)


def _gemm_transposed(y16, Sv, w16, bias=None, out_dtype="float32"):
    return S.gemm(y16, Sv, np.ascontiguousarray(np.asarray(w16).T) if w16.shape[0] == w16.shape[1] else w16[::-1],
                  bias, out_dtype)


def _mm_t_quantised_skinny(x, w, bias=None, out_dtype="float32"):
    x = np.asarray(x)
    if x.shape[0] <= 8:
        return S.skinny(x.astype(np.float16), w, bias, out_dtype)
    return S.mm_t(x, w, bias, out_dtype)


def _gemm_fp16_via_fp32(x, w, bias=None, out_dtype="float32"):
    # the GEMM path's fp16 output rounded to fp32 first (two roundings instead of one)
    x = np.asarray(x)
    if x.shape[0] <= 8 or out_dtype != "float16":
        return S.mm_t(x, w, bias, out_dtype)
    return S.fp16_rne(S.mm_t(x, w, bias, "float32"))


def _skinny_fp16_single_rounding(x, w, bias=None, out_dtype="float32"):
    # the skinny path's fp16 output rounded once from the exact sum (no fp32 step)
    x = np.asarray(x)
    if x.shape[0] > 8 or out_dtype != "float16":
        return S.mm_t(x, w, bias, out_dtype)
    out = np.asarray(x, dtype=np.float64) @ np.asarray(w, dtype=np.float64)
    if bias is not None:
        out = out + np.asarray(bias, dtype=np.float64)[None, :]
    return S.fp16_rne(out)


@pytest.mark.parametrize("broken,check", [
    (_gemm_fp16_via_fp32, check_mm_t_exact16),
    (_skinny_fp16_single_rounding, check_mm_t_exact16),
    (_mm_t_without_bias, check_mm_t_exact16),
    (_floor_exponent, check_exponent_kats),
    (_floor_exponent, check_exponent_minimal),
    (_non_strict_exponent, check_exponent_kats),
    (_mm_t_without_bias, check_mm_t_exact),
    (_mm_t_quantised_skinny, check_mm_t_exact),
    (_mm_t_quantised_skinny, check_skinny_unquantised),
    (_gemm_transposed, check_identity_and_permutation),
])
def test_planted_mistake_is_rejected(broken, check):
    with pytest.raises(AssertionError):
        check(broken)
