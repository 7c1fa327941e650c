"""The BERT-base encoder of the fifth benchmark configuration: random init, token ids uniform over
the vocabulary, mean-pooled embeddings.

The reference's end-to-end check (bench/e2e_embeddings.py:10-40) loads BAAI/bge-base-en-v1.5, a
BERT-base encoder, runs 256 texts x 256 tokens in fp32, patches it and compares the normalised
CLS-token embeddings by cosine with the fp32 run. With no network the weights cannot be fetched, so
the same architecture (transformers' ``BertConfig()`` defaults: 12 layers, hidden 768, 12 heads,
FFN 3072 GELU, vocab 30522) is built locally with seeded random weights, and both the mean-pooled
embedding and the CLS token are compared.
"""
from __future__ import annotations

import torch

from _inputs import gen

BERT_LINEARS = 12 * 6 + 1  # per layer Q, K, V, attention output, FFN in, FFN out; plus the pooler


def bert_base(seed: int = 0, layers: int | None = None):
    """BERT-base (``BertConfig()`` defaults), weights from ``torch.manual_seed(seed)``, fp32, eval."""
    from transformers import BertConfig, BertModel

    cfg = BertConfig() if layers is None else BertConfig(num_hidden_layers=layers)
    cfg.attn_implementation = "sdpa"
    state = torch.random.get_rng_state()
    try:
        torch.manual_seed(seed)
        model = BertModel(cfg)
    finally:
        torch.random.set_rng_state(state)
    return model.float().eval()


def token_ids(batch: int, seq: int, vocab: int = 30522, seed: int = 0) -> torch.Tensor:
    return torch.randint(0, vocab, (batch, seq), generator=gen(seed))


def embeddings(model, ids: torch.Tensor, chunk: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(mean of ``last_hidden_state`` over the sequence, its CLS row), both fp32 [batch, hidden],
    attention mask all ones; ``chunk`` splits the batch to bound activation memory."""
    means, cls = [], []
    step = chunk or ids.shape[0]
    with torch.no_grad():
        for i in range(0, ids.shape[0], step):
            part = ids[i:i + step]
            h = model(input_ids=part, attention_mask=torch.ones_like(part)).last_hidden_state.float()
            means.append(h.mean(dim=1))
            cls.append(h[:, 0])
    return torch.cat(means), torch.cat(cls)
