"""Write the committed golden fixtures under tests/golden/.

Run in the build container only (needs torch + transformers on the CPU; no
network, no hub fetch):

    python tests/golden/make_golden.py

1. ``kats.npz`` - the reference's kernel known-answer tests, regenerated from
   the recipes in scripts/dump_weights.py (the dumped files themselves are
   gitignored upstream and absent):
     * matmul  :195-208  default_rng(0), shapes small 4x16x8 and real
                128x384x384, A,B ~ 0.1*N(0,1); C = A @ B^T (numpy fp32)
     * layernorm :211-232 default_rng(1), 128x384, gamma ~ 1+0.1N, beta ~ 0.1N,
                fp16-rounded inputs; y = torch.nn.functional.layer_norm
     * gelu    :235-243  default_rng(2), n = 128*1536, x ~ 1.5N, fp16-rounded;
                y = torch.nn.functional.gelu (exact erf)
     * softmax :246-254  default_rng(3), 128x128, x ~ 2N, fp16-rounded;
                y = torch.nn.functional.softmax
2. ``model_seed0.npz`` - model-level vectors from transformers' own
   ``BertModel`` (the library the reference's oracle calls,
   scripts/dump_weights.py:108-120,146,165-166,186), built from a local
   ``BertConfig`` with the MiniLM-L6 shape and loaded with the seeded fp32
   weights of ``bbh.synth.make_weights(0)``.  Same quantities the reference
   dumps: emb_out (:136-150), attn0_out with the (1-m)*finfo.min extended mask
   (:153-170), layer0_out (:173-192), and the mean-pooled L2-normalised
   embedding (:111-120), for the 9-token configs[0] row at seq 16 and at
   seq 128, plus a ragged six-sentence batch with token types 0/1 at seq 32.
"""

import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "bert-by-hand_amd"))

from bbh import synth  # noqa: E402


def make_kats():
    out = {}
    rng = np.random.default_rng(0)
    for tag, M, N, K in [("small", 4, 16, 8), ("real", 128, 384, 384)]:
        A = rng.standard_normal((M, K)).astype(np.float32) * 0.1
        B = rng.standard_normal((N, K)).astype(np.float32) * 0.1
        C = A @ B.T
        out[f"matmul_{tag}_A"] = A.astype(np.float16)
        out[f"matmul_{tag}_B"] = B.astype(np.float16)
        out[f"matmul_{tag}_C"] = C.astype(np.float32)

    M, D = 128, 384
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((M, D)) * 1.0).astype(np.float16).astype(np.float32)
    g = (rng.standard_normal((D,)) * 0.1 + 1.0).astype(np.float16).astype(np.float32)
    b = (rng.standard_normal((D,)) * 0.1).astype(np.float16).astype(np.float32)
    y = F.layer_norm(torch.from_numpy(x), (D,), weight=torch.from_numpy(g),
                     bias=torch.from_numpy(b), eps=1e-12).numpy()
    out.update(ln_x=x.astype(np.float16), ln_gamma=g.astype(np.float16),
               ln_beta=b.astype(np.float16), ln_y=y.astype(np.float32))

    n = 128 * 1536
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(n) * 1.5).astype(np.float16).astype(np.float32)
    out.update(gelu_x=x.astype(np.float16),
               gelu_y=F.gelu(torch.from_numpy(x)).numpy().astype(np.float32))

    rng = np.random.default_rng(3)
    x = (rng.standard_normal((128, 128)) * 2.0).astype(np.float16).astype(np.float32)
    out.update(softmax_x=x.astype(np.float16),
               softmax_y=F.softmax(torch.from_numpy(x), dim=-1).numpy().astype(np.float32))
    np.savez_compressed(os.path.join(HERE, "kats.npz"), **out)


def build_model(weights):
    from transformers import BertConfig, BertModel

    cfg = BertConfig(vocab_size=synth.VOCAB_SIZE, hidden_size=synth.HIDDEN,
                     num_hidden_layers=synth.NUM_LAYERS, num_attention_heads=synth.NUM_HEADS,
                     intermediate_size=synth.FFN_DIM, max_position_embeddings=synth.MAX_POSITION,
                     type_vocab_size=synth.TYPE_VOCAB_SIZE, layer_norm_eps=synth.LAYER_NORM_EPS,
                     hidden_act="gelu", attn_implementation="eager")
    model = BertModel(cfg, add_pooling_layer=False).eval()
    model.load_state_dict({k: torch.from_numpy(v) for k, v in weights.items()}, strict=True)
    return model


def run_model(model, ids, types, mask):
    t = lambda a: torch.from_numpy(np.asarray(a, np.int64))  # noqa: E731
    with torch.no_grad():
        hidden = model(input_ids=t(ids), attention_mask=t(mask),
                       token_type_ids=t(types)).last_hidden_state
        m = t(mask).unsqueeze(-1).float()
        pooled = (hidden * m).sum(dim=1) / m.sum(dim=1).clamp(min=1e-9)
        emb = pooled / pooled.norm(dim=-1, keepdim=True).clamp(min=1e-12)
        e_out = model.embeddings(input_ids=t(ids), token_type_ids=t(types))
        ext = (1.0 - t(mask)[:, None, None, :].float()) * torch.finfo(torch.float32).min
        a0 = model.encoder.layer[0].attention(e_out, attention_mask=ext)[0]
        l0 = model.encoder.layer[0](e_out, attention_mask=ext)
        if isinstance(l0, tuple):
            l0 = l0[0]
    f = lambda x: x.numpy().astype(np.float32)  # noqa: E731
    return dict(hidden=f(hidden), embedding=f(emb), emb_out=f(e_out), attn0_out=f(a0),
                layer0_out=f(l0))


def make_model_vectors():
    weights = synth.make_weights(0)
    model = build_model(weights)
    out = {}
    for tag, seq in (("s16", 16), ("s128", 128)):
        ids, types, mask = synth.cfg_fixed(1, seq)
        res = run_model(model, ids, types, mask)
        out[f"{tag}_ids"], out[f"{tag}_types"], out[f"{tag}_mask"] = ids, types, mask
        for k, v in res.items():
            if tag == "s128" and k not in ("embedding",):
                continue
            out[f"{tag}_{k}"] = v

    rng = np.random.default_rng(7)
    lengths = [5, 9, 17, 23, 31, 32]
    rows = [synth.sentence(rng, L) for L in lengths]
    ids, types, mask = synth.pack(rows, 32)
    types[1, 3:7] = 1
    types[4, :] = 1
    res = run_model(model, ids, types, mask)
    out.update(rag_ids=ids, rag_types=types, rag_mask=mask, rag_hidden=res["hidden"],
               rag_embedding=res["embedding"], rag_layer0_out=res["layer0_out"])

    import transformers

    out["versions"] = np.array([torch.__version__, transformers.__version__, np.__version__])
    np.savez_compressed(os.path.join(HERE, "model_seed0.npz"), **out)


if __name__ == "__main__":
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    make_kats()
    make_model_vectors()
    print("wrote", sorted(os.listdir(HERE)))
