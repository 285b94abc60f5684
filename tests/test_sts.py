"""The STS evaluation harness (bbh.sts, after the reference's
scripts/benchmark.py:19-105): rank statistics against scipy.stats and closed
forms, corpus reading and deduplication, pair similarity.  Host-only."""

import gzip
import json

import numpy as np
import pytest
import scipy.stats as ss

from conftest import ROOT  # noqa: F401  (sets sys.path)


def _sts():
    from bbh import sts

    return sts


def test_rankdata_matches_scipy():
    sts = _sts()
    rng = np.random.default_rng(0)
    for x in (rng.integers(0, 5, 40), rng.standard_normal(33), np.array([3.0, 3.0, 3.0]),
              np.array([2.0]), np.zeros(0)):
        np.testing.assert_array_equal(sts.rankdata(x), ss.rankdata(x, method="average"))


def test_spearman_closed_forms():
    sts = _sts()
    # no ties: rho = 1 - 6 sum(d^2) / (n (n^2 - 1)); d = (-1, 1, -1, 1, 0) -> 1 - 24/120
    assert sts.spearman([1, 2, 3, 4, 5], [2, 1, 4, 3, 5]) == pytest.approx(0.8, abs=1e-15)
    x = np.linspace(-3, 3, 50)
    assert sts.spearman(x, np.exp(x)) == pytest.approx(1.0, abs=1e-15)  # any increasing map
    assert sts.spearman(x, -x ** 3) == pytest.approx(-1.0, abs=1e-15)
    # ties: x ranks (1, 2.5, 2.5, 4), y ranks (1, 2, 3, 4): centred (-1.5, 0, 0, 1.5) and
    # (-1.5, -0.5, 0.5, 1.5): 4.5 / sqrt(4.5 * 5)
    assert sts.spearman([1, 2, 2, 3], [10, 20, 30, 40]) == pytest.approx(4.5 / np.sqrt(22.5), abs=1e-15)
    assert np.isnan(sts.spearman([1, 1, 1], [1, 2, 3]))  # constant input
    with pytest.raises(ValueError):
        sts.spearman([1, 2], [1, 2, 3])
    with pytest.raises(ValueError):
        sts.spearman([1, np.nan], [1, 2])


def test_spearman_matches_scipy():
    sts = _sts()
    rng = np.random.default_rng(1)
    for _ in range(20):
        n = int(rng.integers(3, 300))
        a = rng.integers(0, 7, n) + 0.25 * rng.standard_normal(n).round(1)  # many ties
        b = a * rng.uniform(-1, 1) + rng.standard_normal(n)
        assert sts.spearman(a, b) == pytest.approx(ss.spearmanr(a, b)[0], abs=1e-12)


ROWS = [("A man plays.", "A man is playing.", 4.2), ("Cats sleep.", "A man plays.", 0.4),
        ("A man plays.", "A man plays.", 5.0), ("Tab\there", 'He said "hi"', 1.25)]


def test_load_corpus_dedup_first_seen():
    sts = _sts()
    sentences, pairs, scores = sts.load_corpus(ROWS)
    assert sentences == ["A man plays.", "A man is playing.", "Cats sleep.", "Tab\there",
                         'He said "hi"']
    assert pairs == [(0, 1), (2, 0), (0, 0), (3, 4)]
    assert scores == [4.2, 0.4, 5.0, 1.25]


def test_read_pairs_formats(tmp_path):
    sts = _sts()
    rows = [(a, b, s) for a, b, s in ROWS if "\t" not in a]  # a tab cannot sit in a TSV field
    js = "".join(json.dumps({"split": "test", "score": s, "sentence1": a, "sentence2": b}) + "\n"
                 for a, b, s in rows)
    (tmp_path / "p.jsonl").write_text(js, encoding="utf-8")
    with gzip.open(tmp_path / "p.jsonl.gz", "wt", encoding="utf-8") as f:
        f.write(js)
    # GLUE STS-B layout: unquoted fields, bare quotes inside sentences
    head = "index\tgenre\tfilename\tyear\told_index\tsource1\tsource2\tsentence1\tsentence2\tscore\n"
    tsv = head + "".join(f"{i}\tmain\tx\t2012\t{i}\tnone\tnone\t{a}\t{b}\t{s}\n"
                         for i, (a, b, s) in enumerate(rows))
    (tmp_path / "p.tsv").write_text(tsv, encoding="utf-8")
    import csv

    with open(tmp_path / "p.csv", "w", newline="", encoding="utf-8") as f:
        w = csv.writer(f)
        w.writerow(["sentence1", "sentence2", "label"])
        w.writerows(rows)
    import pyarrow as pa
    import pyarrow.parquet as pq

    pq.write_table(pa.table({"sentence1": [r[0] for r in rows], "sentence2": [r[1] for r in rows],
                             "score": [r[2] for r in rows]}), tmp_path / "p.parquet")
    for name in ("p.jsonl", "p.jsonl.gz", "p.tsv", "p.csv", "p.parquet"):
        assert sts.read_pairs(tmp_path / name) == rows, name
    (tmp_path / "bad.jsonl").write_text('{"sentence1": "a", "sentence2": "b"}\n', encoding="utf-8")
    with pytest.raises(ValueError, match="numeric score"):
        sts.read_pairs(tmp_path / "bad.jsonl")
    with pytest.raises(ValueError, match="unknown STS file type"):
        sts.read_pairs(tmp_path / "p.txt")


def test_pair_similarity_and_correlate():
    sts = _sts()
    t = np.linspace(0, np.pi, 7)
    emb = np.stack([np.cos(t), np.sin(t), np.zeros_like(t)], 1).astype(np.float16)  # unit rows
    pairs = [(0, i) for i in range(7)]
    sims = sts.pair_similarity(emb, pairs)
    np.testing.assert_allclose(sims, np.cos(t), atol=2e-3)  # cos of the angle to row 0
    assert sts.correlate(emb, pairs, 7 - np.arange(7)) == pytest.approx(1.0)
    assert sts.correlate(emb, pairs, np.arange(7)) == pytest.approx(-1.0)
