"""Direct oracle parity of every path bench.py times, called exactly as
bench.py calls it: per-sentence embedding cosine >= 0.9999 against the fp32
oracle (the reference's fp32 torch forward, restated) over all 2000 sentences
of the varlen mix, as the reference's corpus benchmark compares every corpus
sentence with its torch embedding (bench/corpus.cu:135-151)."""

import numpy as np
import pytest

from conftest import cosine_rows
from oracle import bert_oracle as O

pytestmark = pytest.mark.gpu

COS = 0.9999


def _np(t):
    return t.float().cpu().numpy()


@pytest.fixture(scope="module")
def mix():
    from bbh import synth

    return synth.varlen_mix()


@pytest.fixture(scope="module")
def mix_oracle(weights32, mix):
    """fp32 oracle embeddings of the 2000 sentences, batch by batch."""
    return np.concatenate([O.bert_embed(weights32, *b[:3]) for b in mix])


def _check(got, want):
    assert got.shape == want.shape == (2000, 384)
    assert np.isfinite(got).all()
    cos = cosine_rows(got, want)
    assert cos.min() >= COS, (int(cos.argmin()), float(cos.min()))
    np.testing.assert_allclose(np.linalg.norm(got, axis=-1), 1.0, atol=2e-3)


def test_headline_per_batch_pass_matches_oracle(torch_cuda, model, mix, mix_oracle):
    # bench.py's value: bbh_embed_each over the 32 consecutive batches on
    # EACH_STREAMS streams.  Every sentence against the oracle; every batch
    # bit for bit against bert_embed on that batch alone; one stream and
    # EACH_STREAMS streams give the same bits.
    import bench
    from bbh import engine

    torch = torch_cuda
    pk = engine.PackedBatches([b[:3] for b in mix])
    pool = engine.Pool(bench.EACH_STREAMS, 64, 64)
    got = _np(engine.embed_each(pool, model, pk))
    pool1 = engine.Pool(1, 64, 64)
    got1 = _np(engine.embed_each(pool1, model, pk))
    ws = engine.Workspace(64, 64)
    dev = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
    alone = np.concatenate([_np(engine.bert_embed(ws, model, *(dev(a) for a in b[:3]))) for b in mix])
    torch.cuda.synchronize()
    for p in (pool, pool1, ws):
        p.close()
    _check(got, mix_oracle)
    assert np.array_equal(got, got1)
    assert np.array_equal(got, alone)


def test_packed_pass_matches_oracle(torch_cuda, model, mix, mix_oracle):
    # bench.py's varlen_packed: embed_packed on the equal-seq-grouped batches
    # through Pool(1, POOL_BATCH, 64), as bench.py calls it.
    import bench
    from bbh import engine

    torch = torch_cuda
    pk = engine.PackedBatches([b[:3] for b in mix], group_by_seq=True)
    pool = engine.Pool(1, bench.POOL_BATCH, 64)
    got = _np(pk.unpermute(engine.embed_packed(pool, model, pk)))
    merged = _np(pk.unpermute(engine.embed_batches(pool, model, pk)))
    torch.cuda.synchronize()
    pool.close()
    _check(got, mix_oracle)
    _check(merged, mix_oracle)


def test_corpus_sorted_dynamic_matches_oracle(torch_cuda, model, mix_oracle):
    # The reference corpus benchmark's dynamic mode (bench/corpus.cu:79-132):
    # length-sorted batches, each at max(16, round16(longest)); embeddings
    # gathered back to input order as corpus.cu:140-146 does.
    import bench
    from bbh import engine, synth

    torch = torch_cuda
    sb, order = synth.varlen_sorted()
    pk = engine.PackedBatches([b[:3] for b in sb])
    pool = engine.Pool(bench.EACH_STREAMS, 64, 64)
    emb = _np(engine.embed_each(pool, model, pk))
    torch.cuda.synchronize()
    pool.close()
    got = np.empty_like(emb)
    got[order] = emb
    _check(got, mix_oracle)


def test_corpus_padded_128_matches_oracle(torch_cuda, model, mix_oracle):
    # The padded mode (bench/corpus.cu:64-77): every batch at seq 128, so
    # 70-123 masked positions per sentence (effective-length invariance).
    import bench
    from bbh import engine, synth

    torch = torch_cuda
    pk = engine.PackedBatches([b[:3] for b in synth.varlen_padded()])
    pool = engine.Pool(bench.EACH_STREAMS, 64, 128)
    got = _np(engine.embed_each(pool, model, pk))
    torch.cuda.synchronize()
    pool.close()
    _check(got, mix_oracle)


def test_cfg5_packed_matches_oracle(torch_cuda, model, cfg5_oracle):
    # bench.py's cfg5 packed figure: embed_packed over the 256 x 512 batch
    # (valid tokens only, ~98k rows, fused LayerNorm GEMMs).  32 sentences
    # spread over lengths 256-512 against the oracle.
    from bbh import engine, synth

    torch = torch_cuda
    ids, types, mask = synth.long_batch()
    pk = engine.PackedBatches([(ids, types, mask)])
    pool = engine.Pool(1, 256, 512)
    got = _np(engine.embed_packed(pool, model, pk))
    torch.cuda.synchronize()
    pool.close()
    picks, want = cfg5_oracle
    cos = cosine_rows(got[picks], want)
    assert cos.min() >= COS, (picks[np.argmin(cos)], cos.min())
    np.testing.assert_allclose(np.linalg.norm(got, axis=-1), 1.0, atol=2e-3)


def test_pool_capacity_errors_before_any_launch(torch_cuda, model):
    # A packed sentence longer than the pool workspace's rows, and a batch
    # whose seq exceeds the workspace's max_seq, are rejected with
    # BBH_ERR_CAPACITY before anything is enqueued.
    from bbh import capi, engine, synth

    rows = [synth.sentence(np.random.default_rng(0), L) for L in (20, 100)]
    ids, types, mask = synth.pack(rows, 128)
    pk = engine.PackedBatches([(ids, types, mask)])
    pool = engine.Pool(1, 1, 64)
    with pytest.raises(capi.BBHError) as e:
        engine.embed_packed(pool, model, pk)
    assert e.value.name == "BBH_ERR_CAPACITY" and "exceeds the pool workspace" in str(e.value)
    with pytest.raises(capi.BBHError) as e:
        engine.embed_each(pool, model, pk)
    assert e.value.name == "BBH_ERR_CAPACITY"
    pool.close()
