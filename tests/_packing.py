"""numpy model of the tile-packed fp16 activation layout (g16_rowscale_pack_* / g16_hgemm_packed_*).

Blocks of 256 rows x 32 columns, block (tm, ks) at index tm * ceil(K/32) + ks, 16 KB each. Inside a
block, 16-byte chunk q*64 + i (q < 16, i < 64) holds columns 8*((i % 4) ^ ((r // 2) % 4)) .. +7 of
local row r = 16q + i//4. Rows >= M and columns >= K are zero.
"""
from __future__ import annotations

import numpy as np

ROWS, KSTEP = 256, 32


def packed_elems(M: int, K: int) -> int:
    if M <= 0 or K <= 0:
        return 0
    return -(-M // ROWS) * -(-K // KSTEP) * ROWS * KSTEP


def pack_a(y: np.ndarray) -> np.ndarray:
    """Row-major [M, K] fp16 -> the packed 1-D fp16 array (vectorised)."""
    M, K = y.shape
    ntm, nks = -(-M // ROWS), -(-K // KSTEP)
    padded = np.zeros((ntm * ROWS, nks * KSTEP), dtype=y.dtype)
    padded[:M, :K] = y
    q = np.arange(16)[:, None]
    i = np.arange(64)[None, :]
    r = 16 * q + i // 4                      # local row of chunk (q, i)
    c = (i % 4) ^ ((r // 2) % 4)             # logical 8-column group it holds
    blocks = padded.reshape(ntm, ROWS, nks, 4, 8)           # tm, r, ks, c, 8
    out = blocks.transpose(0, 2, 1, 3, 4)[:, :, r.reshape(-1), c.reshape(-1), :]  # tm, ks, 1024, 8
    return np.ascontiguousarray(out).reshape(-1)


def packed_index(row: int, col: int, K: int) -> int:
    """Element index of y[row, col] in the packed array (scalar restatement, for checking pack_a)."""
    nks = -(-K // KSTEP)
    tm, r = divmod(row, ROWS)
    ks, kk = divmod(col, KSTEP)
    cgroup, e = divmod(kk, 8)
    i = (r % 16) * 4 + (cgroup ^ ((r // 2) % 4))
    q = r // 16
    return (((tm * nks + ks) * 1024) + q * 64 + i) * 8 + e
