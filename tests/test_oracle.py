"""Pins the CPU oracle (oracle/bert_oracle.py) before anything is checked
against it.  Each check is independent of the oracle's own formula: the
reference's known-answer recipes (regenerated, tests/golden/kats.npz), the
transformers BertModel golden vectors (tests/golden/model_seed0.npz), torch
library routines, brute force on tiny inputs, and invariants that a dropped
term, a wrong index or a transposed operand would break."""

import numpy as np
import pytest

from conftest import cosine_rows
from oracle import bert_oracle as O


# ---- Linear ----------------------------------------------------------------

@pytest.mark.parametrize("tag", ["small", "real"])
def test_linear_matches_reference_matmul_kat(kats, tag):
    # tests/test_matmul.cu:17-54 feeds fp16 A, B and compares to fp32 C (cos >= 0.9995)
    A = kats[f"matmul_{tag}_A"].astype(np.float32)
    B = kats[f"matmul_{tag}_B"].astype(np.float32)
    C = kats[f"matmul_{tag}_C"]
    got = O.linear(A, B)
    assert cosine_rows(got.ravel(), C.ravel()) >= 0.9999
    assert np.abs(got - C).max() < 2e-3  # fp16 rounding of the inputs only


def test_linear_bruteforce_bias_gelu():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((3, 5))
    w = rng.standard_normal((4, 5))
    b = rng.standard_normal(4)
    want = np.zeros((3, 4))
    for i in range(3):
        for j in range(4):
            v = b[j] + sum(x[i, k] * w[j, k] for k in range(5))
            want[i, j] = v * 0.5 * (1.0 + __import__("math").erf(v / 2 ** 0.5))
    np.testing.assert_allclose(O.linear(x, w, b, act_gelu=True), want, rtol=1e-12, atol=1e-12)


def test_linear_is_not_transposed():
    # A non-square weight catches an (in, out) vs (out, in) mix-up.
    x = np.arange(6, dtype=np.float64).reshape(2, 3)
    w = np.array([[1.0, 0.0, 0.0], [0.0, 0.0, 2.0]])
    np.testing.assert_array_equal(O.linear(x, w), [[0.0, 4.0], [3.0, 10.0]])


# ---- GELU ------------------------------------------------------------------

def test_gelu_matches_reference_kat(kats):
    x = kats["gelu_x"].astype(np.float32)
    y = kats["gelu_y"]
    got = O.gelu(x)
    assert np.abs(got - y).max() < 1e-6
    assert cosine_rows(got, y) >= 0.999999


def test_gelu_special_points():
    assert O.gelu(np.array([0.0]))[0] == 0.0
    big = np.array([10.0, -10.0])
    np.testing.assert_allclose(O.gelu(big), [10.0, 0.0], atol=1e-12)
    # Phi(1) = 0.8413447460685429 (standard normal CDF)
    np.testing.assert_allclose(O.gelu(np.array([1.0]))[0], 0.8413447460685429, rtol=1e-12)


# ---- LayerNorm ---------------------------------------------------------------

def test_layernorm_matches_reference_kat(kats):
    x = kats["ln_x"].astype(np.float32)
    g = kats["ln_gamma"].astype(np.float32)
    b = kats["ln_beta"].astype(np.float32)
    got = O.layer_norm(x, g, b, eps=1e-12)
    assert np.abs(got - kats["ln_y"]).max() < 1e-5


def test_layernorm_residual_and_invariants():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((7, 384))
    r = rng.standard_normal((7, 384))
    y = O.layer_norm(x, np.ones(384), np.zeros(384), residual=r)
    np.testing.assert_allclose(y.mean(-1), 0.0, atol=1e-12)
    np.testing.assert_allclose(y.var(-1), 1.0, rtol=1e-9)
    # residual enters as a plain sum: LN(x + r) == LN(r + x) == LN(x + r, no residual)
    np.testing.assert_allclose(y, O.layer_norm(x + r, np.ones(384), np.zeros(384)), atol=1e-12)
    # gamma / beta are an affine map per column
    g, b = rng.standard_normal(384), rng.standard_normal(384)
    np.testing.assert_allclose(O.layer_norm(x, g, b, residual=r), y * g + b, atol=1e-12)


# ---- softmax -----------------------------------------------------------------

def test_softmax_matches_reference_kat(kats):
    x = kats["softmax_x"].astype(np.float32)
    got = O.masked_softmax(x)
    assert np.abs(got - kats["softmax_y"]).max() < 1e-6


def test_masked_softmax_invariants():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((5, 40)) * 3
    mask = (rng.random(40) > 0.4).astype(np.int32)
    p = O.masked_softmax(x, mask)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-12)
    assert np.all(p[:, mask == 0] == 0.0)
    np.testing.assert_allclose(O.masked_softmax(x + 7.5, mask), p, atol=1e-12)
    # all keys masked -> all zeros (src/kernels/softmax.cu: sum 0 -> every entry zeroed)
    assert np.all(O.masked_softmax(x, np.zeros(40, np.int32)) == 0.0)


# ---- embedding gather --------------------------------------------------------

def test_embedding_sum_bruteforce():
    rng = np.random.default_rng(8)
    word, pos, typ = rng.standard_normal((50, 6)), rng.standard_normal((9, 6)), rng.standard_normal((2, 6))
    ids = rng.integers(0, 50, (2, 4))
    types = rng.integers(0, 2, (2, 4))
    got = O.embedding_sum(ids, types, word, pos, typ)
    for b in range(2):
        for s in range(4):
            np.testing.assert_array_equal(got[b, s], word[ids[b, s]] + pos[s] + typ[types[b, s]])


# ---- attention core vs torch SDPA -------------------------------------------

def test_attention_matches_torch_sdpa():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(9)
    B, S = 3, 20
    qkv = rng.standard_normal((B, S, 3 * 384)).astype(np.float64)
    mask = np.ones((B, S), np.int32)
    mask[0, 13:] = 0
    mask[2, [1, 4, 5, 17]] = 0
    got = O.attention(qkv, mask)
    t = torch.from_numpy(qkv)
    q, k, v = (t[..., i * 384:(i + 1) * 384].reshape(B, S, 12, 32).transpose(1, 2) for i in range(3))
    add = torch.zeros((B, 1, 1, S), dtype=torch.float64)
    add[torch.from_numpy(mask)[:, None, None, :] == 0] = float("-inf")
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=add)
    ref = ref.transpose(1, 2).reshape(B, S, 384).numpy()
    np.testing.assert_allclose(got, ref, atol=1e-10)


def test_attention_heads_are_not_mixed():
    # Put information only in head 3's V; other heads' outputs must be zero.
    rng = np.random.default_rng(10)
    qkv = rng.standard_normal((1, 16, 1152))
    qkv[..., 768:] = 0.0
    qkv[..., 768 + 3 * 32:768 + 4 * 32] = 1.0
    out = O.attention(qkv, np.ones((1, 16), np.int32))
    np.testing.assert_allclose(out[..., 3 * 32:4 * 32], 1.0, atol=1e-12)
    assert np.all(out[..., :3 * 32] == 0.0) and np.all(out[..., 4 * 32:] == 0.0)


# ---- full model vs transformers' BertModel ----------------------------------

def test_embeddings_and_layer0_match_transformers(weights32, golden_model):
    g = golden_model
    ids, types, mask = g["s16_ids"], g["s16_types"], g["s16_mask"]
    e = O.embeddings(weights32, ids, types)
    assert np.abs(e - g["s16_emb_out"]).max() < 1e-5
    lw = O._layer(weights32, 0)
    assert np.abs(O.attention_block(e, lw, mask) - g["s16_attn0_out"]).max() < 1e-5
    assert np.abs(O.encoder_layer(e, lw, mask) - g["s16_layer0_out"]).max() < 1e-5


@pytest.mark.parametrize("tag", ["s16", "rag"])
def test_bert_embed_matches_transformers(weights32, golden_model, tag):
    g = golden_model
    ids, types, mask = g[f"{tag}_ids"], g[f"{tag}_types"], g[f"{tag}_mask"]
    h = O.bert_encode(weights32, ids, types, mask)
    assert np.abs(h - g[f"{tag}_hidden"]).max() < 2e-5
    e = O.l2_normalize(O.mean_pool(h, mask))
    assert np.abs(e - g[f"{tag}_embedding"]).max() < 1e-6
    np.testing.assert_allclose(np.linalg.norm(e, axis=-1), 1.0, rtol=1e-5)


def test_effective_length_invariance(weights32, golden_model):
    # The s16 and s128 goldens are the same 9-token sentence (README.md:80-83).
    from bbh import synth

    ids, types, mask = synth.cfg_fixed(1, 128)
    e128 = O.bert_embed(weights32, ids, types, mask)
    assert np.abs(e128 - golden_model["s128_embedding"]).max() < 1e-6
    assert np.abs(e128 - golden_model["s16_embedding"]).max() < 1e-6


def test_pool_normalize_closed_forms():
    h = np.array([[[1.0, 2.0], [3.0, 4.0], [100.0, 100.0]]])
    m = np.array([[1, 1, 0]])
    np.testing.assert_allclose(O.mean_pool(h, m), [[2.0, 3.0]])
    np.testing.assert_allclose(O.l2_normalize(np.array([[3.0, 4.0]])), [[0.6, 0.8]])
    # count 0 -> 0 (pooling.cu:30 divides by max(count, 1)), floor keeps 0 at 0
    z = O.l2_normalize(O.mean_pool(h, np.zeros((1, 3), np.int32)))
    assert np.all(z == 0.0)


def test_synthetic_inputs_match_recorded_statistics():
    # BASELINE configs[3] statistics recorded for numpy default_rng(0)
    from bbh import synth

    lengths = synth.varlen_lengths()
    assert abs(lengths.mean() - 13.4285) < 1e-3
    batches = synth.varlen_mix()
    effs = [b[3] for b in batches]
    assert {e: effs.count(e) for e in set(effs)} == {32: 8, 48: 21, 64: 3}
    assert sum(b[0].shape[0] * b[3] for b in batches) == 91648
    # FLOPs(B, s) = B*s*21,233,664 + B*9,216*s^2: 21.89 G at B64 s16, 3,401.6 G at B256 s512
    assert synth.flops_per_forward(64, 16) == 21_894_266_880
    assert abs(synth.flops_per_forward(256, 512) / 1e9 - 3401.6) < 0.1


@pytest.mark.parametrize("tag", ["s16", "rag"])
def test_torch_cpu_forward_matches_golden_and_oracle(weights32, golden_model, tag):
    # The CPU baseline's forward (transformers BertModel, sdpa attention) on
    # the seeded weights gives the committed golden embeddings (written by the
    # eager BertModel) and the numpy oracle's.
    from oracle import torch_forward as T

    g = golden_model
    ids, types, mask = g[f"{tag}_ids"], g[f"{tag}_types"], g[f"{tag}_mask"]
    got = T.embed(T.build(weights32), ids, types, mask)
    assert np.abs(got - g[f"{tag}_embedding"]).max() < 1e-5
    assert np.abs(got - O.bert_embed(weights32, ids, types, mask)).max() < 1e-5


def test_corpus_modes_follow_reference_batching():
    # bench/corpus.cu:64-77 (every batch at seq 128) and :79-118 (length-sorted,
    # each batch at max(16, round16(longest))) on the configs[3] sentences.
    from bbh import synth

    rows = synth.varlen_rows()
    lens = np.array([len(r) for r in rows])
    sorted_b, order = synth.varlen_sorted()
    assert sorted(order.tolist()) == list(range(2000))
    assert np.all(np.diff(lens[order]) >= 0)
    got = [row for b in sorted_b for row in b[0]]
    assert all(np.array_equal(got[k][:lens[i]], rows[i]) and not got[k][lens[i]:].any()
               for k, i in enumerate(order))
    effs = [b[3] for b in sorted_b]
    assert effs == [max(16, -(-int(lens[order[s:s + 64]].max()) // 16) * 16)
                    for s in range(0, 2000, 64)]
    assert sum(b[0].shape[0] * b[3] for b in sorted_b) == 41984
    padded = synth.varlen_padded()
    assert all(b[3] == 128 and b[0].shape[1] == 128 for b in padded)
    assert np.array_equal(np.concatenate([b[2].sum(1) for b in padded]), lens)
