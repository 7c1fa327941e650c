"""CPU tests of the activation-range diagnostics (the analogue of the reference's
bench/diag_ranges.py): counts and exponents against the oracle's rescale rule."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn

import oracle
from gtx16_fp16 import FastLinear
from gtx16_fp16.diag import range_hooks, report, risky


def test_range_hooks_count_rescaled_rows_and_exponents():
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(256, 512), nn.ReLU(), nn.Linear(512, 256), nn.Linear(256, 64))
    x = torch.randn(3, 40, 256)
    x[0, 5] *= 3000.0                 # |max| ~ 1e4: exponent 4 or so
    x[2, 7, 3] = 179940.0             # the reference test's activation: exponent 8
    x[1, 1, 1] = float("nan")         # ignored by the max
    stats, handles = range_hooks(model)
    with torch.no_grad():
        model(x)
    for h in handles:
        h.remove()
    assert set(stats) == {"0", "2"}   # the 256 -> 64 layer is below min_features
    s = stats["0"]
    x2 = x.reshape(-1, 256).numpy()
    amax = oracle.row_amax(x2)
    e = oracle.row_exponent(amax)
    assert s["rows"] == 120
    assert s["rows_rescaled"] == int((amax > 1024).sum()) == 2
    assert s["max_exponent"] == int(e.max()) == 8
    assert s["nonfinite_rows"] == 1
    assert np.isclose(s["x_amax"], float(amax.max()))
    assert np.isclose(s["w_amax"], model[0].weight.abs().max().item())
    assert "0" in risky(stats)
    assert "layers checked: 2" in report(stats)


def test_range_hooks_cover_fast_linear_and_accumulate_calls():
    torch.manual_seed(1)
    fl = FastLinear.from_linear(nn.Linear(256, 256))
    stats, handles = range_hooks(nn.Sequential(fl))
    with torch.no_grad():
        fl(torch.randn(4, 256))
        fl(torch.randn(6, 256))
    for h in handles:
        h.remove()
    s = stats["0"]
    assert s["rows"] == 10 and s["rows_rescaled"] == 0 and s["max_exponent"] == 0
    assert np.isclose(s["w_amax"], fl.weight_t.float().abs().max().item())
    assert risky(stats) == {}


def test_range_hooks_do_not_count_rescales_on_the_skinny_path():
    # mm_t sends calls with <= 8 rows to the skinny path, which never rescales (ops.py:78): their
    # rows are seen and their max recorded, but nothing is counted as rescaled
    lin = nn.Linear(256, 256)
    stats, handles = range_hooks(nn.Sequential(lin))
    x = torch.randn(8, 256)
    x[3, 9] = 5.0e4
    with torch.no_grad():
        lin(x)
    s = stats["0"]
    assert s["rows"] == 8 and s["rows_rescaled"] == 0 and s["max_exponent"] == 0
    assert np.isclose(s["x_amax"], 5.0e4)
    x9 = torch.cat([x, torch.randn(1, 256)])  # 9 rows: the GEMM path
    with torch.no_grad():
        lin(x9)
    for h in handles:
        h.remove()
    assert s["rows"] == 17 and s["rows_rescaled"] == 1
    assert s["max_exponent"] == int(oracle.row_exponent(oracle.row_amax(x9.numpy())).max()) == 6
