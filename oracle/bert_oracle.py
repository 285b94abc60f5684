"""CPU oracle for the MiniLM-L6 ``bert_embed`` path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker (or the timed CPU baseline), never as the thing measured or shipped.
The product path (``bert-by-hand_amd``) never imports it and fails loudly when
its HIP library is missing.

This is a plain numpy restatement of the reference's forward.  The reference's
own ground truth is the HF ``BertModel`` fp32 CPU forward reached through
sentence-transformers (scripts/dump_weights.py:97-192); its CUDA engine spells
the same math out kernel by kernel.  Each function cites the lines it follows.
All arithmetic is float32 (as the reference's torch oracle) unless a caller
passes float64 arrays.

How each function is pinned (tests/test_oracle.py):

* ``linear``      - the reference matmul KATs regenerated from their recipe
                    (default_rng(0), shapes 4x16x8 and 128x384x384) vs numpy
                    float64 A @ B^T; brute-force triple loop on a tiny shape.
* ``gelu``        - the reference GELU KAT recipe (default_rng(2)) vs
                    torch.nn.functional.gelu; GELU(0) = 0, tails -> x and 0.
* ``layer_norm``  - the reference LN KAT recipe (default_rng(1)) vs
                    torch.nn.functional.layer_norm; mean 0 / var 1 invariants.
* ``masked_softmax`` - the reference softmax KAT recipe (default_rng(3)) vs
                    torch.softmax; rows sum to 1, masked columns exactly 0,
                    shift invariance.
* ``embedding_sum`` - brute-force index arithmetic on a tiny table.
* ``attention`` / ``attention_block`` / ``encoder_layer`` / ``bert_embed`` -
                    golden fixtures written by transformers' own BertModel
                    (tests/golden/make_golden.py) built from a local
                    BertConfig with the same seeded weights, plus
                    torch.nn.functional.scaled_dot_product_attention for the
                    attention core; effective-length invariance and unit norm.
* ``mean_pool`` / ``l2_normalize`` - closed forms vs the golden fixtures'
                    pooled embeddings; count-0 rows give 0.
"""

from __future__ import annotations

import numpy as np

HIDDEN = 384
NUM_LAYERS = 6
NUM_HEADS = 12
HEAD_DIM = 32
FFN_DIM = 1536
LAYER_NORM_EPS = 1e-12
NORM_FLOOR = 1e-12


def _erf(x):
    from scipy.special import erf

    return erf(x)


def gelu(x):
    """Exact-erf GELU: x * 0.5 * (1 + erf(x / sqrt(2))).
    src/kernels/matmul.cu:27-28, src/kernels/gelu.cu:14."""
    x = np.asarray(x)
    return (x * 0.5 * (1.0 + _erf(x / np.sqrt(2.0).astype(x.dtype)))).astype(x.dtype)


def linear(x, w, b=None, act_gelu=False):
    """out = x @ w^T (+ b) (+ GELU); w is the torch Linear (out, in) layout.
    src/kernels/matmul.h:1-13, epilogue src/kernels/matmul.cu:23-30."""
    y = x @ w.T
    if b is not None:
        y = y + b
    if act_gelu:
        y = gelu(y)
    return y


def layer_norm(x, gamma, beta, eps=LAYER_NORM_EPS, residual=None):
    """Row LayerNorm of (x + residual): two-pass mean / variance, rsqrt.
    src/kernels/layernorm.cu:17-59 (residual prologue :29-36)."""
    v = x if residual is None else x + residual
    mean = v.mean(axis=-1, keepdims=True)
    d = v - mean
    var = (d * d).mean(axis=-1, keepdims=True)
    return d / np.sqrt(var + np.asarray(eps, v.dtype)) * gamma + beta


def masked_softmax(x, key_mask=None):
    """Softmax over the last axis; keys with mask 0 are dropped (-> 0), and a
    row with every key masked is all zeros.
    src/kernels/softmax.cu:26-63 (mask :37-44, zeroing :57-62)."""
    x = np.asarray(x)
    if key_mask is None:
        keep = np.ones(x.shape, bool)
    else:
        keep = np.broadcast_to(np.asarray(key_mask) != 0, x.shape)
    neg = np.where(keep, x, -np.inf)
    m = neg.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    e = np.where(keep, np.exp(neg - m), 0.0)
    s = e.sum(axis=-1, keepdims=True)
    out = np.where(s > 0, e / np.where(s > 0, s, 1.0), 0.0)
    return out.astype(x.dtype)


def embedding_sum(ids, types, word, pos, typ):
    """h[b, s] = word[ids[b, s]] + pos[s] + type[types[b, s]]; the position id
    is the index within the sequence.  src/kernels/embedding.cu:20-30."""
    ids = np.asarray(ids)
    seq = ids.shape[-1]
    return word[ids] + pos[np.arange(seq)] + typ[np.asarray(types)]


def attention(qkv, mask, heads=NUM_HEADS, head_dim=HEAD_DIM):
    """Masked scaled-dot-product attention read straight from the fused QKV
    activations.  qkv is (B, S, 3*H) with Q | K | V column blocks
    (src/model/weights.h:38-54); head h uses columns h*32..h*32+31 of each
    block (src/kernels/attention.cu:25-28,74-75); scale 1/sqrt(32)
    (src/model/encoder.cu:28) applied to Q K^T (attention.cu:57); masked keys
    dropped (softmax.cu:35-44); context written merged (attention.cu:87-92).
    Returns (B, S, H)."""
    b, s, three_h = qkv.shape
    hid = three_h // 3
    scale = np.asarray(1.0 / np.sqrt(head_dim), qkv.dtype)
    q = qkv[:, :, 0:hid].reshape(b, s, heads, head_dim).transpose(0, 2, 1, 3)
    k = qkv[:, :, hid:2 * hid].reshape(b, s, heads, head_dim).transpose(0, 2, 1, 3)
    v = qkv[:, :, 2 * hid:].reshape(b, s, heads, head_dim).transpose(0, 2, 1, 3)
    out = np.empty((b, s, hid), qkv.dtype)
    step = max(1, (1 << 22) // max(1, heads * s * s))
    for b0 in range(0, b, step):
        sl = slice(b0, b0 + step)
        sc = (q[sl] @ k[sl].transpose(0, 1, 3, 2)) * scale
        km = np.asarray(mask)[sl][:, None, None, :]
        p = masked_softmax(sc, km)
        ctx = p @ v[sl]
        out[sl] = ctx.transpose(0, 2, 1, 3).reshape(-1, s, hid)
    return out


def _layer(w, i):
    p = f"encoder.layer.{i}."
    g = lambda n: w[p + n]  # noqa: E731
    qkv_w = np.concatenate([g("attention.self.query.weight"), g("attention.self.key.weight"),
                            g("attention.self.value.weight")], axis=0)
    qkv_b = np.concatenate([g("attention.self.query.bias"), g("attention.self.key.bias"),
                            g("attention.self.value.bias")], axis=0)
    return dict(
        qkv_w=qkv_w, qkv_b=qkv_b,
        o_w=g("attention.output.dense.weight"), o_b=g("attention.output.dense.bias"),
        ln1_g=g("attention.output.LayerNorm.weight"), ln1_b=g("attention.output.LayerNorm.bias"),
        f1_w=g("intermediate.dense.weight"), f1_b=g("intermediate.dense.bias"),
        f2_w=g("output.dense.weight"), f2_b=g("output.dense.bias"),
        ln2_g=g("output.LayerNorm.weight"), ln2_b=g("output.LayerNorm.bias"),
    )


def attention_block(hidden, lw, mask):
    """Fused-QKV projection -> masked attention -> output dense -> residual
    LayerNorm.  src/model/encoder.cu:25-51; hidden is (B, S, 384)."""
    qkv = linear(hidden, lw["qkv_w"], lw["qkv_b"])
    ctx = attention(qkv, mask)
    proj = linear(ctx, lw["o_w"], lw["o_b"])
    return layer_norm(proj, lw["ln1_g"], lw["ln1_b"], residual=hidden)


def ffn_block(hidden, lw):
    """Intermediate dense + GELU -> output dense -> residual LayerNorm.
    src/model/encoder.cu:53-65."""
    inter = linear(hidden, lw["f1_w"], lw["f1_b"], act_gelu=True)
    proj = linear(inter, lw["f2_w"], lw["f2_b"])
    return layer_norm(proj, lw["ln2_g"], lw["ln2_b"], residual=hidden)


def encoder_layer(hidden, lw, mask):
    """src/model/encoder.cu:67-71."""
    return ffn_block(attention_block(hidden, lw, mask), lw)


def embeddings(w, ids, types):
    """Embedding sum then the embedding LayerNorm (src/model/forward.cu:28-31)."""
    h = embedding_sum(ids, types, w["embeddings.word_embeddings.weight"],
                      w["embeddings.position_embeddings.weight"],
                      w["embeddings.token_type_embeddings.weight"])
    return layer_norm(h, w["embeddings.LayerNorm.weight"], w["embeddings.LayerNorm.bias"])


def bert_encode(w, ids, types, mask, layers=NUM_LAYERS, collect=False):
    """Embeddings then every encoder layer (src/model/forward.cu:20-42).
    Returns the final hidden state (B, S, 384), and with collect=True also the
    list [emb_ln_out, layer0_out, ...]."""
    h = embeddings(w, ids, types)
    trace = [h]
    for i in range(layers):
        h = encoder_layer(h, _layer(w, i), mask)
        trace.append(h)
    return (h, trace) if collect else h


def mean_pool(hidden, mask):
    """out[b] = sum_s mask*h / max(sum_s mask, 1).  src/kernels/pooling.cu:21-31
    (sentence-transformers clamps the count at 1e-9, scripts/dump_weights.py:119,
    which is the same for integer counts)."""
    m = np.asarray(mask).astype(hidden.dtype)[..., None]
    cnt = m.sum(axis=-2)
    return (hidden * m).sum(axis=-2) / np.maximum(cnt, 1.0)


def l2_normalize(x):
    """x / max(||x||_2, 1e-12).  src/kernels/normalize.cu:7,29-30,
    scripts/dump_weights.py:120."""
    n = np.sqrt((x * x).sum(axis=-1, keepdims=True))
    return x / np.maximum(n, NORM_FLOOR)


def bert_embed(w, ids, types, mask):
    """encode -> masked mean pool -> L2 normalize (src/model/forward.cu:44-53).
    Returns (B, 384)."""
    h = bert_encode(w, ids, types, mask)
    return l2_normalize(mean_pool(h, mask))


def as_dtype(weights: dict, dtype=np.float32) -> dict:
    return {k: np.asarray(v).astype(dtype) for k, v in weights.items()}
