"""bbh_tokenize against the tokenizer the reference calls: transformers'
BertTokenizerFast (Hugging Face tokenizers 0.22.2, scripts/dump_weights.py:
100-106, scripts/dump_corpus.py:34-39) with padding="max_length",
truncation=True.  The real MiniLM vocab.txt is not available offline, so both
run on the same seeded synthetic vocabulary; the texts mix ASCII, accented
Latin, Greek, Cyrillic, CJK, Hangul, emoji, control / format characters,
Unicode whitespace, long words and unknown characters.  Host-only: runs on
the CPU."""

import ctypes
import os

import numpy as np
import pytest

from conftest import ROOT  # noqa: F401  (sets sys.path)

def _lib():
    from bbh import capi

    if not os.path.exists(capi.LIB_PATH):
        pytest.fail("libbbh.so not built (run __graft_entry__.build())")
    return capi.lib()


def make_vocab(seed=0):
    from bbh import synth

    return synth.text_vocab(seed)


def make_texts(seed=1, n=400):
    from bbh import synth

    return synth.texts(seed, n)


def _tokenize(L, path, texts, seq, lowercase=True):
    t = ctypes.c_void_p()
    assert L.bbh_tokenizer_load(path.encode(), int(lowercase), ctypes.byref(t)) == 0, L.bbh_last_error()
    n = len(texts)
    arr = (ctypes.c_char_p * n)(*[s.encode("utf-8") for s in texts])
    ids = np.zeros((n, seq), np.int32)
    types = np.ones((n, seq), np.int32)
    mask = np.zeros((n, seq), np.int32)
    lens = np.zeros(n, np.int32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    assert L.bbh_tokenize(t, arr, n, seq, p(ids), p(types), p(mask), p(lens)) == 0
    vs = L.bbh_tokenizer_vocab_size(t)
    L.bbh_tokenizer_free(t)
    return ids, types, mask, lens, vs


@pytest.mark.parametrize("seq,lowercase", [(128, True), (16, True), (64, False)])
def test_matches_bert_tokenizer_fast(tmp_path, seq, lowercase):
    transformers = pytest.importorskip("transformers")
    L = _lib()
    vocab = make_vocab()
    path = tmp_path / "vocab.txt"
    path.write_text("\n".join(vocab) + "\n", encoding="utf-8")
    texts = make_texts()
    ref = transformers.BertTokenizerFast.from_pretrained(str(tmp_path), do_lower_case=lowercase)
    enc = ref(texts, padding="max_length", truncation=True, max_length=seq, return_tensors="np")
    ids, types, mask, lens, vs = _tokenize(L, str(path), texts, seq, lowercase)
    assert vs == len(vocab)
    bad = [i for i in range(len(texts)) if not np.array_equal(ids[i], enc["input_ids"][i])]
    assert not bad, [(texts[i], ids[i][:12], enc["input_ids"][i][:12]) for i in bad[:3]]
    assert np.array_equal(mask, enc["attention_mask"])
    assert np.array_equal(types, enc["token_type_ids"])
    assert np.array_equal(lens, mask.sum(1))


def test_golden_fixture(tmp_path):
    # committed vectors written by tests/golden/make_tokenizer_golden.py with
    # BertTokenizerFast (for hosts without transformers)
    L = _lib()
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "tokenizer.npz"), allow_pickle=False)
    path = tmp_path / "vocab.txt"
    path.write_text("\n".join(g["vocab"].tolist()) + "\n", encoding="utf-8")
    texts = g["texts"].tolist()
    ids, types, mask, lens, _ = _tokenize(L, str(path), texts, int(g["seq"]))
    assert np.array_equal(ids, g["ids"]) and np.array_equal(mask, g["mask"])


def test_errors_and_malformed_utf8(tmp_path):
    L = _lib()
    t = ctypes.c_void_p()
    assert L.bbh_tokenizer_load(b"/nonexistent/vocab.txt", 1, ctypes.byref(t)) == 4
    bad = tmp_path / "v.txt"
    bad.write_text("a\nb\n[CLS]\n", encoding="utf-8")
    assert L.bbh_tokenizer_load(str(bad).encode(), 1, ctypes.byref(t)) == 4
    assert b"[UNK]" in L.bbh_last_error()
    good = tmp_path / "g.txt"
    good.write_text("[PAD]\n[UNK]\n[CLS]\n[SEP]\nab\r\n", encoding="utf-8")  # CRLF trimmed
    assert L.bbh_tokenizer_load(str(good).encode(), 1, ctypes.byref(t)) == 0
    arr = (ctypes.c_char_p * 2)(b"ab \xff\xfe ab", b"a\xc3")  # invalid bytes dropped
    ids = np.zeros((2, 8), np.int32)
    z = np.zeros((2, 8), np.int32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    assert L.bbh_tokenize(t, arr, 2, 8, p(ids), p(z), p(z.copy()), None) == 0
    assert ids[0].tolist() == [2, 4, 4, 3, 0, 0, 0, 0]
    assert ids[1].tolist() == [2, 1, 3, 0, 0, 0, 0, 0]  # "a" is not in the vocabulary
    assert L.bbh_tokenize(t, arr, 2, 1, p(ids), p(z), p(z), None) == 1  # seq < 2
    L.bbh_tokenizer_free(t)
