"""Fast fp16 matmul for MI355X (gfx950): the gtx16_fp16 API on hand-written CDNA4 kernels.

    import gtx16_fp16
    n = gtx16_fp16.patch(model)          # swap nn.Linear -> FastLinear (on gfx950 devices)
    y = gtx16_fp16.matmul(a16, b16)      # fp16 matmul on the matrix cores, fp32 accumulation

Same exports and version as the reference package (src/gtx16_fp16/__init__.py:7-11).
"""
from .linear import FastLinear, patch
from .ops import is_affected, matmul, mm_t, supported

__all__ = ["FastLinear", "patch", "is_affected", "matmul", "mm_t", "supported"]
__version__ = "0.1.0"
