"""Write the golden fixtures under tests/golden/ (run from the repository root):

    python tests/golden/make_golden.py

The reference ships no stored vectors (its tests compare against torch fp32 on the GPU at run time,
tests/test_correctness.py:29), so the expected outputs here are computed independently of the
oracle's numpy path:

* ``rowscale_kat.npz`` -- rows whose |max| is a hand-picked value, with the exponent written down by
  hand from e = ceil(log2(amax/1024)) (strict threshold), and S = 2^e.
* ``mm_t_exact.npz`` -- small seeded mm_t cases (skinny M <= 8 and quantised GEMM M > 8, with
  and without bias, with an outlier row) whose expected outputs are the EXACT rational results
  (fractions.Fraction over the fp16/fp32 input values, the row scale applied exactly) rounded once
  to fp64; the fp16 quantisation of the GEMM path is done bit by bit (round-half-even on the
  exact rational), not with numpy's converter. ``{case}_out16`` holds the fp16 output bits: on the
  GEMM path the exact result rounded once to fp16 (the epilogue's cast, kernels.py:133), on the
  skinny path the exact result rounded to fp32 and that fp32 value to fp16 (the fp32 kernel output
  cast by ``.to(fp16)``, ops.py:84). The two ``*_tie16`` cases put an exact result just above an
  fp16 rounding tie by less than half an fp32 ulp, where one rounding and two roundings differ.
"""
from __future__ import annotations

from fractions import Fraction
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

# (amax, e) -- e written down by hand: ceil(log2(amax / 1024)) for amax > 1024, else 0.
ROWSCALE_KAT = [
    (0.0, 0),
    (1.0, 0),
    (1023.5, 0),
    (1024.0, 0),                    # strict threshold: equal is not scaled
    (1024.0001220703125, 1),        # nextafter(1024, inf) in fp32
    (1536.0, 1),
    (2048.0, 1),                    # exactly 2 * 1024
    (2048.000244140625, 2),         # nextafter(2048, inf) in fp32
    (4096.0, 2),
    (65504.0, 6),                   # fp16 max: 63.97 * 1024
    (179940.0, 8),                  # the Qwen3-TTS activation of tests/test_correctness.py:119
    (200000.0, 8),
    (262144.0, 8),                  # exactly 256 * 1024
    (262144.03125, 9),              # nextafter(262144, inf) in fp32
    (1.5 * 2.0 ** 127, 118),        # 1.5 * 2^117 * 1024: near the top of the fp32 range
]


def fp32_round_exact(q: Fraction) -> Fraction:
    """The rational q rounded once to the nearest fp32 value, ties to even (subnormals included;
    the cases here never come near fp32 overflow, which raises)."""
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    a = -q if q < 0 else q
    E = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** E > a:
        E -= 1
    E = max(E, -126)                      # subnormal range shares the 2^-126 exponent
    ulp = Fraction(2) ** (E - 23)
    m = a / ulp
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    r = n * ulp
    if r >= Fraction(2) ** 128:
        raise OverflowError("fp32 overflow")
    return sign * r


def fp16_bits_exact(q: Fraction) -> int:
    """IEEE binary16 bits of the rational q, rounded once to nearest-even (subnormals, overflow)."""
    sign = 0x8000 if q < 0 else 0
    a = -q if q < 0 else q
    if a == 0:
        return sign
    # exponent of a: 2^E <= a < 2^(E+1)
    E = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** E > a:
        E -= 1
    E = max(E, -14)                       # subnormal range shares the 2^-14 exponent
    ulp = Fraction(2) ** (E - 10)
    m = a / ulp                            # significand in units of the ulp
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    if n == 2048:                          # carried into the next binade
        n, E = 1024, E + 1
    if E > 15:
        return sign | 0x7C00
    if n < 1024:                           # subnormal
        return sign | n
    return sign | ((E + 15) << 10) | (n - 1024)


def fp16_from_bits(b: int) -> Fraction:
    s = -1 if b & 0x8000 else 1
    e = (b >> 10) & 0x1F
    f = b & 0x3FF
    if e == 0:
        return s * Fraction(f, 1 << 24)
    return s * Fraction(1024 + f, 1 << 10) * Fraction(2) ** (e - 15)


def exact_mm_t_fracs(x: np.ndarray, w16: np.ndarray, bias: np.ndarray | None) -> list:
    """Exact rational restatement of mm_t (ops.py:65-108): the [M][N] results as Fractions."""
    M, K = x.shape
    N = w16.shape[1]
    W = [[fp16_from_bits(int(b)) for b in row] for row in w16.view(np.uint16)]
    X = [[Fraction(float(v)) for v in row] for row in x.astype(np.float64)]
    out = [[Fraction(0)] * N for _ in range(M)]
    for i in range(M):
        if M <= 8:
            row, scale = X[i], Fraction(1)
        else:
            amax = max((abs(v) for v in X[i]), default=Fraction(0))
            e = 0
            while amax / Fraction(2) ** e > 1024:   # smallest e with amax / 2^e <= 1024
                e += 1
            scale = Fraction(2) ** e
            row = [fp16_from_bits(fp16_bits_exact(v / scale)) for v in X[i]]
        for j in range(N):
            acc = sum((row[k] * W[k][j] for k in range(K)), Fraction(0)) * scale
            if bias is not None:
                acc += Fraction(float(bias[j]))
            out[i][j] = acc
    return out


def exact_mm_t(x: np.ndarray, w16: np.ndarray, bias: np.ndarray | None) -> np.ndarray:
    """The exact mm_t results rounded once to fp64."""
    return np.array([[float(q) for q in row] for row in exact_mm_t_fracs(x, w16, bias)], dtype=np.float64)


def exact_out16(fracs: list, skinny: bool) -> np.ndarray:
    """fp16 output bits of mm_t(..., out_dtype=fp16) from the exact results: one rounding on the
    GEMM path, fp32 then fp16 on the skinny path."""
    if skinny:
        return np.array([[fp16_bits_exact(fp32_round_exact(q)) for q in row] for row in fracs], dtype=np.uint16)
    return np.array([[fp16_bits_exact(q) for q in row] for row in fracs], dtype=np.uint16)


def tie16_case(M: int, rng) -> tuple:
    """Inputs whose output [0, 0] is exactly 1 + 2^-11 + 2^-30: 2^-30 above the fp16 tie between
    1 and 1 + 2^-10, and less than half an fp32 ulp (2^-24) above it. Rounded once to fp16 it is
    1 + 2^-10 (bits 0x3C01); rounded to fp32 first it is the tie itself, which goes to even, 1.0
    (0x3C00). K = N = 8; the other entries are small seeded values, column 0 of w has no other
    nonzero entry, and row 0 of x has |max| <= 1024 (no rescale on the GEMM path)."""
    K = N = 8
    x = (0.01 * rng.standard_normal((M, K))).astype(np.float32)
    w = (0.25 * rng.standard_normal((K, N))).astype(np.float16)
    w[:, 0] = 0
    x[0, :] = 0
    if M > 8:   # GEMM path: the operands are fp16 values, product 2^-15 * 2^-15 = 2^-30
        x[0, 0], x[0, 1], x[0, 2] = 1.0, 2.0 ** -11, 2.0 ** -15
        w[0, 0], w[1, 0], w[2, 0] = 1.0, 1.0, 2.0 ** -15
    else:       # skinny path: fp32 activations used as they are
        x[0, 0], x[0, 1] = np.float32(1 + 2.0 ** -11), np.float32(2.0 ** -30)
        w[0, 0], w[1, 0] = 1.0, 1.0
    return x, w


def make_rowscale_kat() -> dict:
    K = 24
    rng = np.random.default_rng(7)
    x = (rng.random((len(ROWSCALE_KAT), K)) - 0.5).astype(np.float32)  # |x| < 0.5
    for i, (a, _) in enumerate(ROWSCALE_KAT):
        x[i, (5 * i) % K] = np.float32(-a if i % 3 == 1 else a)
        assert float(np.float32(a)) == a, a
    e = np.array([e for _, e in ROWSCALE_KAT], dtype=np.int32)
    return {"x": x, "amax": np.array([a for a, _ in ROWSCALE_KAT], dtype=np.float32), "e": e,
            "S": np.ldexp(np.float32(1), e).astype(np.float32)}


def make_mm_t_exact() -> dict:
    rng = np.random.default_rng(11)
    cases = {}
    for name, (M, K, N, bias) in {"skinny_m3": (3, 16, 8, True), "skinny_m8": (8, 24, 16, False),
                                  "gemm_m12": (12, 16, 8, True), "gemm_m9": (9, 32, 24, False)}.items():
        x = rng.standard_normal((M, K)).astype(np.float32)
        x[1, 3] = np.float32(1 + 2.0 ** -20)    # not representable in fp16
        if M > 8:
            x[2] *= np.float32(3000.0)          # outlier row: pow2 rescale e >= 1
            x[4, 0] = np.float32(7e-6)          # goes subnormal in fp16
        w = (0.25 * rng.standard_normal((K, N))).astype(np.float16)
        b = rng.standard_normal(N).astype(np.float32) if bias else None
        cases[f"{name}_x"] = x
        cases[f"{name}_w"] = w
        if b is not None:
            cases[f"{name}_b"] = b
        fr = exact_mm_t_fracs(x, w, b)
        cases[f"{name}_out"] = np.array([[float(q) for q in row] for row in fr], dtype=np.float64)
        cases[f"{name}_out16"] = exact_out16(fr, M <= 8)
    for name, M in (("skinny_tie16", 2), ("gemm_tie16", 9)):
        x, w = tie16_case(M, rng)
        fr = exact_mm_t_fracs(x, w, None)
        assert fr[0][0] == 1 + Fraction(1, 2 ** 11) + Fraction(1, 2 ** 30)
        cases[f"{name}_x"] = x
        cases[f"{name}_w"] = w
        cases[f"{name}_out"] = np.array([[float(q) for q in row] for row in fr], dtype=np.float64)
        cases[f"{name}_out16"] = exact_out16(fr, M <= 8)
        assert int(cases[f"{name}_out16"][0, 0]) == (0x3C00 if M <= 8 else 0x3C01)
    return cases


def main() -> None:
    np.savez(HERE / "rowscale_kat.npz", **make_rowscale_kat())
    np.savez(HERE / "mm_t_exact.npz", **make_mm_t_exact())
    print("wrote", HERE / "rowscale_kat.npz", HERE / "mm_t_exact.npz")


if __name__ == "__main__":
    main()
