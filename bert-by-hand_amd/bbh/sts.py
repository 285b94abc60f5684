"""Semantic textual similarity (STS) evaluation of the embedding path.

Computes Spearman's rho between each sentence pair's embedding similarity and
its gold score, and times the encode.  Follows the reference's
scripts/benchmark.py:
- load_corpus (:85-98): sentences deduplicated in first-seen order, pairs as
  index tuples into that list, gold scores as floats;
- correlate (:54-61): the row-wise dot product of the two L2-normalized
  embeddings, then Spearman's rho (scipy.stats.spearmanr) against the gold
  scores;
- encode_and_time (:64-82): one untimed encode of the first batch, then the
  whole corpus timed, with the device synchronized on both sides;
- save_baseline (:19-43): the result fields.

The reference downloads mteb/stsbenchmark-sts.  Here the corpus is a local
file: JSON lines, CSV, or TSV with a header naming sentence1, sentence2 and
score (the mteb and GLUE STS-B layouts), optionally gzip-compressed, or
parquet.

Encoding is the library's own path end to end:
1. bbh_tokenize (WordPiece, [CLS] ... [SEP], truncated at max_seq).
2. Batches of batch_size consecutive sentences, each padded to round16 of
   its longest sentence, as the reference's corpus bench does.
3. bbh_embed_packed over all of them: valid tokens only.

The product path has no CPU fallback: without the HIP library it raises.
"""

import argparse
import csv
import gzip
import io
import json
import os
import sys
import time

import numpy as np


# ---- corpus -------------------------------------------------------------------

def _open_text(path):
    if str(path).endswith(".gz"):
        return io.TextIOWrapper(gzip.open(path, "rb"), encoding="utf-8", newline="")
    return open(path, encoding="utf-8", newline="")


def _row(d, where):
    try:
        s1, s2 = d["sentence1"], d["sentence2"]
        score = d["score"] if "score" in d else d["label"]
        return str(s1), str(s2), float(score)
    except (KeyError, TypeError, ValueError) as e:
        raise ValueError(f"{where}: needs sentence1, sentence2 and a numeric score ({e!r})")


def read_pairs(path):
    """(sentence1, sentence2, score) rows of a local STS file, in file order."""
    name = str(path)
    base = name[:-3] if name.endswith(".gz") else name
    ext = os.path.splitext(base)[1].lower()
    rows = []
    if ext == ".parquet":
        import pyarrow.parquet as pq

        for i, d in enumerate(pq.read_table(name).to_pylist()):
            rows.append(_row(d, f"{name} row {i}"))
    elif ext in (".jsonl", ".json"):
        with _open_text(name) as f:
            for i, line in enumerate(f):
                if line.strip():
                    rows.append(_row(json.loads(line), f"{name} line {i + 1}"))
    elif ext in (".tsv", ".csv"):
        with _open_text(name) as f:
            # GLUE STS-B's TSV has bare quotes inside sentences: no quoting there.
            rd = (csv.DictReader(f, delimiter="\t", quoting=csv.QUOTE_NONE) if ext == ".tsv"
                  else csv.DictReader(f))
            for i, d in enumerate(rd):
                rows.append(_row(d, f"{name} line {i + 2}"))
    else:
        raise ValueError(f"{name}: unknown STS file type (jsonl, json, csv, tsv, parquet, + .gz)")
    return rows


def load_corpus(rows):
    """Sentences deduplicated in first-seen order, the index pair of each row
    and its gold score (scripts/benchmark.py:85-98)."""
    seen = {}
    pairs, scores = [], []
    for s1, s2, score in rows:
        i1 = seen.setdefault(s1, len(seen))
        i2 = seen.setdefault(s2, len(seen))
        pairs.append((i1, i2))
        scores.append(float(score))
    return list(seen.keys()), pairs, scores


# ---- statistics ---------------------------------------------------------------

def rankdata(x):
    """1-based ranks with ties sharing their mean rank (scipy.stats.rankdata,
    method 'average')."""
    x = np.asarray(x, np.float64).ravel()
    n = x.size
    order = np.argsort(x, kind="mergesort")
    xs = x[order]
    starts = np.r_[0, np.flatnonzero(xs[1:] != xs[:-1]) + 1] if n else np.zeros(0, np.int64)
    ends = np.r_[starts[1:], n] if n else np.zeros(0, np.int64)
    r = np.empty(n, np.float64)
    r[order] = np.repeat((starts + ends + 1) / 2.0, ends - starts)
    return r


def spearman(a, b):
    """Spearman's rho: the Pearson correlation of the average ranks
    (scipy.stats.spearmanr's definition).  NaN when either input is constant."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    if a.size != b.size:
        raise ValueError(f"spearman: {a.size} vs {b.size} values")
    if not (np.all(np.isfinite(a)) and np.all(np.isfinite(b))):
        raise ValueError("spearman: non-finite input")
    ra, rb = rankdata(a), rankdata(b)
    ra -= ra.mean()
    rb -= rb.mean()
    den = np.sqrt((ra * ra).sum() * (rb * rb).sum())
    return float((ra * rb).sum() / den) if den > 0 else float("nan")


def pair_similarity(emb, pairs):
    """Row-wise dot product of the pairs' embeddings in fp32 (the embeddings
    are L2-normalized, so this is their cosine)."""
    e = np.asarray(emb, np.float32)
    idx = np.asarray(pairs, np.int64).reshape(-1, 2)
    return np.einsum("ij,ij->i", e[idx[:, 0]], e[idx[:, 1]])


def correlate(emb, pairs, gold):
    """Spearman's rho of the pair similarities against the gold scores
    (scripts/benchmark.py:54-61)."""
    return spearman(pair_similarity(emb, pairs), gold)


# ---- encode -------------------------------------------------------------------

def _round16(n):
    return (n + 15) // 16 * 16


def encode(tokenizer, model, pool, sentences, batch_size=32, max_seq=256):
    """Embeddings (n, 384) float32 of `sentences`, in input order."""
    from . import engine

    n = len(sentences)
    if n == 0:
        return np.zeros((0, engine.HIDDEN), np.float32)
    ids, types, mask, lengths = tokenizer(sentences, seq=max_seq)
    batches = []
    for s in range(0, n, batch_size):
        e = min(n, s + batch_size)
        seq = min(max_seq, _round16(int(lengths[s:e].max())))
        batches.append((ids[s:e, :seq], types[s:e, :seq], mask[s:e, :seq]))
    packed = engine.PackedBatches(batches, group_by_seq=True)
    emb = engine.embed_packed(pool, model, packed)
    return packed.unpermute(emb).float().cpu().numpy()


def evaluate(tokenizer, model, rows, batch_size=32, max_seq=256, pool=None):
    """Encode the corpus of `rows` (timed as scripts/benchmark.py:64-82) and
    correlate; returns the result fields of scripts/benchmark.py:19-43."""
    from . import engine

    torch = engine._torch()
    sentences, pairs, scores = load_corpus(rows)
    own = pool is None
    if own:
        pool = engine.Pool(1, 1024, 64)
    try:
        encode(tokenizer, model, pool, sentences[:batch_size], batch_size, max_seq)  # warm
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        emb = encode(tokenizer, model, pool, sentences, batch_size, max_seq)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3
    finally:
        if own:
            pool.close()
    n = len(sentences)
    return {
        "n_sentences": n,
        "n_pairs": len(pairs),
        "batch_size": batch_size,
        "max_seq": max_seq,
        "elapsed_ms": round(ms, 3),
        "ms_per_sentence": round(ms / n, 5) if n else None,
        "throughputs_sps": round(n / (ms / 1e3), 2) if n and ms > 0 else None,
        "spearman_rho": round(correlate(emb, pairs, scores), 6) if pairs else None,
    }, emb


def main(argv=None):
    from . import engine, synth

    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--pairs", required=True, help="local STS file (jsonl/csv/tsv/parquet[.gz])")
    ap.add_argument("--vocab", required=True, help="WordPiece vocab.txt")
    ap.add_argument("--weights", default=None,
                    help="directory of the reference's .bin files or a .safetensors file "
                         "(default: seeded random-init weights, which make rho meaningless)")
    ap.add_argument("--batch-size", type=int, default=32)
    ap.add_argument("--max-seq", type=int, default=256)
    ap.add_argument("--cased", action="store_true", help="do not lowercase")
    ap.add_argument("--out", default=None, help="write the result JSON here")
    args = ap.parse_args(argv)
    if not 1 <= args.max_seq <= synth.MAX_POSITION:
        ap.error(f"--max-seq must be in [1, {synth.MAX_POSITION}]")

    if args.weights is None:
        print("sts: no --weights given: seeded random-init weights", file=sys.stderr)
        model = engine.Model.from_weights(synth.make_weights(0))
        wdesc = "synthetic seed 0"
    elif args.weights.endswith(".safetensors"):
        model, wdesc = engine.Model.load_safetensors(args.weights), args.weights
    else:
        model, wdesc = engine.Model.load_dir(args.weights), args.weights
    tok = engine.Tokenizer(args.vocab, lowercase=not args.cased)
    try:
        res, _ = evaluate(tok, model, read_pairs(args.pairs), args.batch_size, args.max_seq)
    finally:
        tok.close()
        model.close()
    res = {"corpus": args.pairs, "weights": wdesc, **res}
    print(json.dumps(res), flush=True)
    if args.out:
        with open(args.out, "w") as f:
            json.dump(res, f, indent=2)
    return 0


if __name__ == "__main__":
    sys.exit(main())
