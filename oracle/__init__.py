"""CPU fp64 oracle for the gtx16_fp16 GEMM hot path.

TEST INFRASTRUCTURE ONLY. This package is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it. The
product path (``gtx16_fp16``) never routes through it and fails loudly when its HIP library is
missing.
"""
from .semantics import (  # noqa: F401
    ROW_SCALE_THRESHOLD,
    SKINNY_MAX_M,
    fp16_rne,
    gemm,
    mm_t,
    rel_err,
    row_amax,
    row_exponent,
    rowscale,
    skinny,
)
