"""The GEMM tile the library plans for a shape, from its own query (g16_hgemm_tile)."""
from __future__ import annotations

import ctypes


def tile(lib, M: int, N: int, K: int, num_cus: int) -> tuple[int, int]:
    """(rows, columns) of the tile the GEMM entry points run (M, N, K) on for num_cus CUs."""
    rows, cols = ctypes.c_int(0), ctypes.c_int(0)
    status = lib.g16_hgemm_tile(M, N, K, num_cus, ctypes.byref(rows), ctypes.byref(cols))
    assert status == 0, status
    return rows.value, cols.value
