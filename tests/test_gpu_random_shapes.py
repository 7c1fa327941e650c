"""Seeded random shapes through every route of mm_t (skinny, split-K, plain, tile-packed) against the
fp64 oracle: ragged M, K and N (multiples of 8 as supported() requires), fp16 and fp32 activations,
fp32 and fp16 outputs, with and without bias, a few rows pushed over the rescale threshold. Each
result is also checked for bitwise repeatability."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _inputs import randn

pytestmark = pytest.mark.gpu


def _cases(n: int = 40):
    rng = np.random.default_rng(1234)
    out = []
    for i in range(n):
        M = int(rng.choice([1, 2, 3, 5, 8, 9, 17, 64, 100, 255, 256, 257, 300, 640, 1100]))
        K = int(rng.integers(1, 160)) * 8
        N = int(rng.integers(1, 130)) * 8
        out.append((i, M, K, N, bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), bool(rng.integers(0, 2))))
    # shapes that reach each route on 256 CUs (test_gpu_routes.py pins the tile of its own cases):
    # 100, 103: 32x128 tiles split 8 ways; 101, 102: 128x128 unsplit; 104, 106: tile-packed 256x128
    # (128 tiles of 256x256 would leave half the CUs idle); 105: 256 unsplit 32x128 tiles;
    # 107: tile-packed 256x256 (144 tiles); 108: 64x128 unsplit (32x128 would need 272 tiles)
    out += [(100, 64, 2048, 512, True, True, False), (101, 1100, 264, 4096, False, True, True),
            (102, 2300, 136, 2048, True, False, True), (103, 33, 4096, 256, False, False, False),
            (104, 2048, 136, 4096, False, False, True), (105, 512, 2048, 2048, True, True, True),
            (106, 1900, 264, 3896, True, False, False), (107, 2304, 264, 4096, False, True, True),
            (108, 520, 1024, 2048, True, False, True)]
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"{c[0]}-{c[1]}x{c[2]}x{c[3]}")
def test_random_shape_matches_oracle(cuda, case):
    import gtx16_fp16 as g

    seed, M, K, N, fp16_in, fp16_out, with_bias = case
    x = randn((M, K), seed=seed)
    if M > 3:
        x[seed % M] *= 2500.0                         # one row over the rescale threshold
    x = x.to(torch.float16 if fp16_in else torch.float32)
    w = randn((K, N), seed=seed + 1, scale=0.05, dtype=torch.float16)
    b = randn((N,), seed=seed + 2, scale=0.05) if with_bias else None
    out_dtype = torch.float16 if fp16_out else torch.float32
    xd, wd = x.to(cuda), w.to(cuda)
    bd = None if b is None else b.to(cuda)
    y = g.mm_t(xd, wd, bd, out_dtype)
    y2 = g.mm_t(xd, wd, bd, out_dtype)
    torch.cuda.synchronize()
    assert y.dtype == out_dtype and y.shape == (M, N)
    assert torch.equal(y, y2)
    ref = oracle.mm_t(x.numpy(), w.numpy(), None if b is None else b.numpy(), "float16" if fp16_out else "float32")
    got = y.float().cpu().numpy()
    assert np.isfinite(got).all() == np.isfinite(ref).all()
    tol = 1e-5 if (M <= 8 and not fp16_out) else 1e-3
    assert oracle.rel_err(got, ref.astype(np.float64)) <= tol
