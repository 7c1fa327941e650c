"""BERT-base through ``patch``: the fifth benchmark configuration as a parity test.

Random-init BERT-base (transformers ``BertConfig()`` defaults), batch 256 x 256 token ids uniform
over the vocabulary, fp32. The fp32 model runs first, then ``patch`` swaps every ``nn.Linear``
(73 of them) for ``FastLinear`` and the same ids run again. The bar is a cosine of at least
0.99999 between the mean-pooled embeddings, and the same for the CLS-token embeddings that the
reference's end-to-end script compares (bench/e2e_embeddings.py:21-40). One patched layer is also
checked against the fp64 oracle on the activations it really sees.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from _models import BERT_LINEARS, bert_base, embeddings, token_ids

pytestmark = pytest.mark.gpu

COSINE_MIN = 0.99999


@pytest.fixture(scope="module")
def bert(cuda):
    pytest.importorskip("transformers")
    import gtx16_fp16 as g

    torch.backends.cuda.matmul.allow_tf32 = False
    model = bert_base(seed=0).to(cuda)
    ids = token_ids(256, 256, seed=0).to(cuda)
    ref_mean, ref_cls = embeddings(model, ids)
    n = g.patch(model)
    mean, cls = embeddings(model, ids)
    torch.cuda.synchronize()
    return {"g": g, "model": model, "ids": ids, "n": n, "ref": (ref_mean, ref_cls), "out": (mean, cls)}


def test_patch_replaces_every_linear(bert):
    g = bert["g"]
    assert bert["n"] == BERT_LINEARS
    fast = [m for m in bert["model"].modules() if isinstance(m, g.FastLinear)]
    assert len(fast) == BERT_LINEARS
    assert not any(type(m) is torch.nn.Linear for m in bert["model"].modules())


@pytest.mark.parametrize("which", [0, 1], ids=["mean_pooled", "cls"])
def test_embedding_cosine(bert, which):
    ref, out = bert["ref"][which], bert["out"][which]
    assert torch.isfinite(out).all()
    cos = F.cosine_similarity(out.double(), ref.double(), dim=1)
    assert cos.shape == (256,)
    assert cos.min().item() >= COSINE_MIN, f"min cosine {cos.min().item():.8f}"


def test_ffn_layer_matches_oracle_on_real_activations(bert, cuda):
    # The FFN-out projection (K=3072, N=768) of the last layer, on the first 512 token rows of its
    # real input: the quantised GEMM path (M > 8) against the fp64 oracle.
    layer = bert["model"].encoder.layer[-1].output.dense
    seen = {}

    def keep_input(module, inp, out):  # returns None: the layer's output is left as it is
        seen.setdefault("x", inp[0].detach())

    hook = layer.register_forward_hook(keep_input)
    try:
        embeddings(bert["model"], bert["ids"][:2])
    finally:
        hook.remove()
    x = seen["x"].reshape(-1, layer.in_features)[:512].contiguous()
    with torch.no_grad():
        y = layer(x)
    torch.cuda.synchronize()
    ref = oracle.mm_t(x.cpu().numpy(), layer.weight_t.cpu().numpy(), layer.bias.cpu().numpy(), "float32")
    assert oracle.rel_err(y.cpu().numpy(), ref) <= 1e-3
    assert np.isfinite(y.cpu().numpy()).all()


def test_range_hooks_on_the_patched_model(bert):
    # The activation-range hooks (bench/diag_ranges.py:11-35 of the reference) on the 73 patched
    # FastLinear layers running on the GPU: every layer's row count, rescaled-row count, largest
    # exponent and input max against the oracle's rescale rule on the inputs the layer really saw
    # (rescales count on the GEMM path only: the pooler sees 4 CLS rows, the skinny path).
    from gtx16_fp16.diag import range_hooks

    g, model = bert["g"], bert["model"]
    seen: dict[str, list] = {}

    def keep(name):
        def f(mod, inp, out):  # returns None: the output is left as it is
            seen.setdefault(name, []).append(inp[0].detach().reshape(-1, mod.in_features).float().cpu())
        return f

    stats, handles = range_hooks(model)
    handles += [m.register_forward_hook(keep(n)) for n, m in model.named_modules() if isinstance(m, g.FastLinear)]
    try:
        embeddings(model, bert["ids"][:4])
    finally:
        for h in handles:
            h.remove()
    assert len(stats) == BERT_LINEARS
    for name, s in stats.items():
        calls = seen[name]
        rows = sum(c.shape[0] for c in calls)
        assert s["rows"] == rows, name
        rescaled, top_e = 0, 0
        for c in calls:
            amax = oracle.row_amax(c.numpy())
            if c.shape[0] > 8:
                rescaled += int((amax > 1024).sum())
                top_e = max(top_e, int(oracle.row_exponent(amax).max()))
        assert s["rows_rescaled"] == rescaled, name
        assert s["max_exponent"] == top_e, name
        assert np.isclose(s["x_amax"], max(float(oracle.row_amax(c.numpy()).max()) for c in calls)), name
    assert stats["pooler.dense"]["rows"] == 4


def test_range_hooks_on_gpu_layers_with_outlier_rows(cuda):
    # The same hooks on two patched GPU layers fed rows that do need the rescale (5 % of 300 rows at
    # |max| in [2e3, 2e5]), plus a 4-row decode call whose large entry must not count (skinny path).
    import torch.nn as nn

    import gtx16_fp16 as g
    from _inputs import outlier_rows, randn
    from gtx16_fp16.diag import range_hooks

    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(512, 768), nn.Linear(768, 256)).to(cuda)
    assert g.patch(model, force=True) == 2
    seen: dict[str, list] = {}

    def keep(name):
        def f(mod, inp, out):
            seen.setdefault(name, []).append(inp[0].detach().float().cpu())
        return f

    stats, handles = range_hooks(model)
    handles += [model[i].register_forward_hook(keep(str(i))) for i in range(2)]
    x = outlier_rows(randn((300, 512), seed=0), 0.05, 2e3, 2e5, seed=3)
    dec = randn((4, 512), seed=5)
    dec[1, 7] = 3.0e4
    try:
        with torch.no_grad():
            model(x.to(cuda))
            model(dec.to(cuda))
    finally:
        for h in handles:
            h.remove()
    torch.cuda.synchronize()
    amax0 = oracle.row_amax(x.numpy())
    s0 = stats["0"]
    assert s0["rows"] == 304
    assert s0["rows_rescaled"] == int((amax0 > 1024).sum()) == 15
    assert s0["max_exponent"] == int(oracle.row_exponent(amax0).max())
    assert np.isclose(s0["x_amax"], max(float(amax0.max()), 3.0e4))
    big = seen["1"][0].numpy()  # the second layer's GEMM-path input, as computed on the GPU
    amax1 = oracle.row_amax(big)
    assert stats["1"]["rows_rescaled"] == int((amax1 > 1024).sum())
    assert stats["1"]["max_exponent"] == int(oracle.row_exponent(amax1).max())

