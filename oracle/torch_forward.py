"""The reference's torch CPU fp32 forward, for the CPU baseline.

TEST INFRASTRUCTURE ONLY, like ``bert_oracle``: only ``tests/`` and
``bench.py``'s ``cpu_baseline`` leg import it; the product never does.

The reference's ``cpu_fp32`` measurement (scripts/benchmark.py:64-86,110-111)
times sentence-transformers' ``encode`` of all-MiniLM-L6-v2 in fp32 on the
CPU: transformers' ``BertModel`` forward, then masked mean pooling and L2
normalisation (scripts/dump_weights.py:108-120).  The hub model cannot be
fetched here, so this builds the same ``BertModel`` from a local
``BertConfig`` with the MiniLM-L6 shape and loads the seeded fp32 weights the
GPU run uses.  Tokenization is excluded: the ids are pre-generated.

Pinned by tests/test_oracle.py: its embeddings equal ``bert_oracle.bert_embed``
(the numpy restatement) and the committed transformers golden vectors on the
same inputs.
"""

from __future__ import annotations

import numpy as np

HIDDEN, LAYERS, HEADS, FFN, VOCAB, MAX_POS, TYPES = 384, 6, 12, 1536, 30522, 512, 2


def build(weights: dict, attn_implementation: str = "sdpa"):
    """transformers BertModel (no pooler) with `weights` (state_dict names ->
    fp32 arrays) loaded, in eval mode on the CPU."""
    import torch
    from transformers import BertConfig, BertModel

    cfg = BertConfig(vocab_size=VOCAB, hidden_size=HIDDEN, num_hidden_layers=LAYERS,
                     num_attention_heads=HEADS, intermediate_size=FFN,
                     max_position_embeddings=MAX_POS, type_vocab_size=TYPES,
                     layer_norm_eps=1e-12, hidden_act="gelu",
                     attn_implementation=attn_implementation)
    model = BertModel(cfg, add_pooling_layer=False).eval()
    model.load_state_dict({k: torch.from_numpy(np.asarray(v, np.float32)) for k, v in weights.items()},
                          strict=True)
    return model


def embed(model, ids, types, mask):
    """(B, 384) float32: BertModel -> masked mean pool (count clamped at 1e-9)
    -> x / max(||x||, 1e-12), as scripts/dump_weights.py:111-120."""
    import torch

    t = lambda a: torch.as_tensor(np.asarray(a, np.int64))  # noqa: E731
    with torch.inference_mode():
        hidden = model(input_ids=t(ids), attention_mask=t(mask), token_type_ids=t(types)).last_hidden_state
        m = t(mask).unsqueeze(-1).to(hidden.dtype)
        pooled = (hidden * m).sum(dim=1) / m.sum(dim=1).clamp(min=1e-9)
        out = pooled / pooled.norm(dim=-1, keepdim=True).clamp(min=1e-12)
    return out.numpy()
