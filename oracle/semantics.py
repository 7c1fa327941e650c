"""fp64 restatement of the reference semantics of ``gtx16_fp16.mm_t`` (numpy, CPU).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, never by the product package.

Every function names the reference lines it restates (paths relative to the reference checkout,
package files under ``src/gtx16_fp16/``). Pinning, i.e. what checks each function against something
other than its own formula, lives in ``tests/test_oracle.py``:

* ``row_amax`` / ``row_exponent`` / ``rowscale``: hand-derived known answers (strict threshold,
  powers of two and their fp32 neighbours, the 179,940 activation of the reference's test), a
  brute-force search for the smallest power of two, and the fp16 rounding known answers (ties to
  even, subnormals, overflow to inf).
* ``gemm`` / ``skinny`` / ``mm_t``: exact rational (``fractions.Fraction``) brute force on tiny
  shapes, identity and permutation matrices, and the constant-16 known answer 16*16*4096 of
  ``tests/test_correctness.py:103-109``.

There are no golden vectors in the reference (its tests compare against torch fp32 on the GPU at run
time), so the fixtures under ``tests/golden/`` hold hand-derived exponents and exact rational
results written by ``tests/golden/make_golden.py``, independently of this module.
"""
from __future__ import annotations

import numpy as np

# ops.py:14-16 -- rows whose |max| exceeds this are scaled by a power of two before the fp16 cast.
ROW_SCALE_THRESHOLD = 1024.0
# kernels.py:253 -- M <= 8 takes the fp32-math skinny path on the unquantised activations.
SKINNY_MAX_M = 8

# Exponent reported for a row whose |max| is +inf (its scale is +inf, its output non-finite).
INF_EXPONENT = 255


def fp16_rne(a) -> np.ndarray:
    """Round to fp16, nearest-even, subnormals kept, overflow to inf (``__float2half_rn``,
    kernels.py:133,244). numpy converts float64 -> float16 with a single correct rounding."""
    with np.errstate(over="ignore"):
        return np.asarray(a, dtype=np.float64).astype(np.float16)


def row_amax(x) -> np.ndarray:
    """``amax = max_k |x[i,k]|`` starting from 0, NaN ignored (``fmaxf``), kernels.py:233-241.

    Returns float32 (the max of fp32/fp16 magnitudes is exact in fp32)."""
    a = np.abs(np.asarray(x).astype(np.float32))
    a = np.where(np.isnan(a), np.float32(0), a)
    if a.shape[1] == 0:
        return np.zeros(a.shape[0], dtype=np.float32)
    return np.maximum(a.max(axis=1), np.float32(0)).astype(np.float32)


def row_exponent(amax, thresh: float = ROW_SCALE_THRESHOLD) -> np.ndarray:
    """``e = ceil(log2(amax / thresh))`` when ``amax > thresh`` (strict), else 0; kernels.py:242.

    Exact: ``r = amax/thresh`` is formed in fp64 (exact for a power-of-two threshold), written as
    ``r = m * 2**E`` with ``m`` in [0.5, 1) by ``frexp``; then ``ceil(log2 r)`` is ``E - 1`` when
    ``m == 0.5`` (``r`` a power of two) and ``E`` otherwise. ``amax = +inf`` gives
    ``INF_EXPONENT``."""
    amax = np.asarray(amax, dtype=np.float64)
    e = np.zeros(amax.shape, dtype=np.int32)
    big = amax > thresh
    fin = np.isfinite(amax)
    r = np.where(big & fin, amax / thresh, 1.0)
    m, E = np.frexp(r)
    e = np.where(big & fin, np.where(m == 0.5, E - 1, E), e)
    e = np.where(big & ~fin, INF_EXPONENT, e)
    return e.astype(np.int32)


def rowscale(x, thresh: float = ROW_SCALE_THRESHOLD):
    """The rowscale cast of kernels.py:227-250 (launched at ops.py:86-90).

    Returns ``(y16, S, e)``: ``y16 = fp16_rne(x * 2**-e)`` per row, ``S = 2**e`` (float32, +inf for
    an infinite row) and the integer exponents. For fp32 ``x`` the multiply by ``2**-e`` is exact
    before the single fp16 rounding."""
    x = np.asarray(x)
    amax = row_amax(x)
    e = row_exponent(amax, thresh)
    inf_row = e == INF_EXPONENT
    inv = np.where(inf_row, 0.0, np.ldexp(1.0, -np.where(inf_row, 0, e)))
    S = np.where(inf_row, np.inf, np.ldexp(1.0, np.where(inf_row, 0, e))).astype(np.float32)
    with np.errstate(invalid="ignore"):
        y16 = fp16_rne(x.astype(np.float64) * inv[:, None])
    return y16, S, e


def _out_cast(acc64: np.ndarray, out_dtype: str) -> np.ndarray:
    if out_dtype in ("float32", "f32", np.float32):
        return acc64.astype(np.float32)
    if out_dtype in ("float16", "f16", np.float16):
        return fp16_rne(acc64)
    raise ValueError(f"out_dtype must be float32 or float16, got {out_dtype}")


def gemm(y16, S, w16, bias=None, out_dtype: str = "float32") -> np.ndarray:
    """Quantised GEMM of kernels.py:35-151 with the epilogue order of kernels.py:106-135:
    ``out = S[row] * (y16 @ w16) + bias`` in fp64, then cast (fp32, or fp16 nearest-even).

    The products of fp16 values are exact in fp64; the fp64 sum is the reference's ideal (its own
    hybrid fp16/fp32 accumulation is an approximation of it)."""
    S = np.asarray(S, dtype=np.float64)
    with np.errstate(invalid="ignore", over="ignore"):  # inf * 0 and inf - inf are NaN, as on the GPU
        acc = np.asarray(y16, dtype=np.float64) @ np.asarray(w16, dtype=np.float64)
        out = acc * S[:, None]
        if bias is not None:
            out = out + np.asarray(bias, dtype=np.float64)[None, :]
    return _out_cast(out, out_dtype)


def skinny(x, w16, bias=None, out_dtype: str = "float32") -> np.ndarray:
    """Skinny path (M <= 8) of kernels.py:160-219, ops.py:78-84: fp32 math on the UNQUANTISED
    activations (fp32 or fp16 used as is), fp16 weights, bias added once; fp32 out, or its
    nearest-even fp16 (``out.to(fp16)``, ops.py:84)."""
    with np.errstate(invalid="ignore", over="ignore"):
        out = np.asarray(x, dtype=np.float64) @ np.asarray(w16, dtype=np.float64)
        if bias is not None:
            out = out + np.asarray(bias, dtype=np.float64)[None, :]
    if out_dtype in ("float16", "f16", np.float16):
        return fp16_rne(out.astype(np.float32))
    return _out_cast(out, out_dtype)


def mm_t(x, w16, bias=None, out_dtype: str = "float32", thresh: float = ROW_SCALE_THRESHOLD):
    """Dispatch of ops.py:65-108 as semantics: M <= SKINNY_MAX_M -> ``skinny``; otherwise
    ``rowscale`` then ``gemm``. (Whether the GEMM is split over K is a scheduling choice with the
    same ideal result.)"""
    x = np.asarray(x)
    if x.shape[0] <= SKINNY_MAX_M:
        return skinny(x, w16, bias, out_dtype)
    y16, S, _ = rowscale(x, thresh)
    return gemm(y16, S, w16, bias, out_dtype)


def rel_err(y, ref) -> float:
    """``||y - ref||_F / max(||ref||_F, 1e-12)`` in fp64 (tests/test_correctness.py:10-11)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-12))
