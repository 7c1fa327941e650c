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
