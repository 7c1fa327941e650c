"""Activation-range diagnostics for the fp16 GEMM path.

The reference's bench/diag_ranges.py:11-35 hooks every nn.Linear of a model, runs it, and lists the
layers whose inputs or weights leave the fp16-safe range (it also measures the 16-element partial
sums its hybrid fp16 accumulation sees). This module does the same for this package's numerics:
the GEMM path accumulates in fp32, so the quantities that matter are

* how often the per-row power-of-two rescale fires (rows with |max| > ROW_SCALE_THRESHOLD, the
  rule of the reference's ops.py:14-16, kernels.py:242) and the largest exponent it needs;
* whether the fp16 weight copy overflows (|w| > 65504 becomes inf, linear.py:33-37);
* whether an fp16 output would overflow (|y| > 65504).

    stats, handles = range_hooks(model)        # nn.Linear and FastLinear layers
    model(inputs)
    print(report(stats)); [h.remove() for h in handles]

Everything is computed with torch on the layer's own device; nothing here launches a kernel of the
library.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from .kernels import SKINNY_MAX_M
from .linear import FastLinear
from .ops import ROW_SCALE_THRESHOLD

FP16_MAX = 65504.0


def _weight_amax(mod: nn.Module) -> float:
    w = mod.weight_t if isinstance(mod, FastLinear) else mod.weight
    return float(w.detach().float().abs().max().item()) if w.numel() else 0.0


def range_hooks(model: nn.Module, min_features: int = 256, thresh: float = ROW_SCALE_THRESHOLD):
    """Register forward hooks on every nn.Linear / FastLinear with min(in, out) >= min_features.
    Returns (stats, handles); stats[name] is updated on every forward:

    K, N, w_amax, x_amax, y_amax, rows (rows seen), rows_rescaled (|max| > thresh), max_exponent
    (largest ceil(log2(|max| / thresh)) seen), nonfinite_rows (rows containing inf or NaN).

    rows_rescaled and max_exponent follow mm_t's dispatch (ops.py:78): a call with at most
    SKINNY_MAX_M rows takes the skinny path, which multiplies the unquantised activations and never
    rescales, so its rows are counted in ``rows`` (and x_amax) but not as rescaled."""
    stats: dict[str, dict] = {}
    handles = []

    def hook(name):
        def f(mod, inp, out):
            x = inp[0].detach()
            x2 = x.reshape(-1, x.shape[-1]).float()
            s = stats.setdefault(name, {"K": mod.in_features, "N": mod.out_features, "w_amax": _weight_amax(mod),
                                        "x_amax": 0.0, "y_amax": 0.0, "rows": 0, "rows_rescaled": 0,
                                        "max_exponent": 0, "nonfinite_rows": 0})
            if x2.numel():
                finite = torch.isfinite(x2).all(dim=1)
                # NaN is ignored by the kernels' row max (fmaxf); inf rows get an infinite scale
                amax = torch.nan_to_num(x2.abs(), nan=0.0).max(dim=1).values
                s["rows"] += x2.shape[0]
                s["nonfinite_rows"] += int((~finite).sum().item())
                top = float(amax.max().item())
                s["x_amax"] = max(s["x_amax"], top)
                quantised = x2.shape[0] > SKINNY_MAX_M  # the GEMM path, where the rescale applies
                if quantised:
                    s["rows_rescaled"] += int((amax > thresh).sum().item())
                if quantised and math.isfinite(top) and top > thresh:
                    # smallest e with top / 2^e <= thresh
                    m, e = math.frexp(top / thresh)
                    s["max_exponent"] = max(s["max_exponent"], e - 1 if m == 0.5 else e)
            y = out.detach()
            if y.numel():
                s["y_amax"] = max(s["y_amax"], float(torch.nan_to_num(y.float().abs(), nan=0.0).max().item()))
        return f

    for name, mod in model.named_modules():
        if isinstance(mod, (nn.Linear, FastLinear)) and min(mod.in_features, mod.out_features) >= min_features:
            handles.append(mod.register_forward_hook(hook(name)))
    return stats, handles


def risky(stats: dict) -> dict:
    """Layers where the fp16 path needs care: rows rescaled, an fp16 weight or output overflow, or
    non-finite inputs."""
    return {n: s for n, s in stats.items()
            if s["rows_rescaled"] or s["w_amax"] > FP16_MAX or s["y_amax"] > FP16_MAX or s["nonfinite_rows"]}


def report(stats: dict, top: int = 15) -> str:
    """A short text table: the layers with the largest inputs first."""
    bad = risky(stats)
    lines = [f"layers checked: {len(stats)}; needing care (rescaled rows, fp16 weight/output overflow, "
             f"non-finite inputs): {len(bad)}"]
    for n, s in sorted(stats.items(), key=lambda kv: -kv[1]["x_amax"])[:top]:
        frac = s["rows_rescaled"] / s["rows"] if s["rows"] else 0.0
        lines.append(f"{n:60} K={s['K']:5} N={s['N']:5} x_amax={s['x_amax']:12.1f} w_amax={s['w_amax']:8.3f} "
                     f"y_amax={s['y_amax']:12.1f} rescaled={frac:7.2%} max_e={s['max_exponent']}")
    return "\n".join(lines)
