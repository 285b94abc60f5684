"""Write tests/golden/tokenizer.npz: a seeded synthetic vocabulary, texts and
the ids / mask transformers' BertTokenizerFast gives them (padding to
max_length 64, truncation), for hosts without transformers.

    python tests/golden/make_tokenizer_golden.py
"""

import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "bert-by-hand_amd"))

import transformers  # noqa: E402

from bbh import synth  # noqa: E402

vocab = synth.text_vocab()
texts = synth.texts(seed=7, n=120)
with tempfile.TemporaryDirectory() as d:
    path = os.path.join(d, "vocab.txt")
    with open(path, "w", encoding="utf-8") as f:
        f.write("\n".join(vocab) + "\n")
    tok = transformers.BertTokenizerFast.from_pretrained(d, do_lower_case=True)
    enc = tok(texts, padding="max_length", truncation=True, max_length=64, return_tensors="np")
np.savez_compressed(os.path.join(HERE, "tokenizer.npz"), vocab=np.array(vocab), texts=np.array(texts),
                    seq=np.int32(64), ids=enc["input_ids"].astype(np.int32),
                    mask=enc["attention_mask"].astype(np.int32),
                    versions=np.array([transformers.__version__]))
print("wrote", len(texts), "texts,", len(vocab), "vocab entries")
