"""Seeded synthetic weights and token batches for the MiniLM-L6 embedding path.

There is no network here, so neither the real all-MiniLM-L6-v2 checkpoint nor
the STS corpus the reference benchmarks on (scripts/dump_weights.py:14,265,
scripts/dump_corpus.py) can be fetched.  Everything below is a deterministic
stand-in of the same shape:

* weights: every embedding table, Linear weight and Linear bias ~ N(0, 0.02)
  (numpy PCG64 ``default_rng(seed)``, drawn in HF ``state_dict`` order, fp32
  masters); LayerNorm gamma = 1, beta = 0.  The engine gets the fp16
  round-to-nearest-even casts, exactly as the reference dumps fp16 files from
  fp32 tensors (scripts/dump_weights.py:80) while its oracle runs the fp32
  model (scripts/dump_weights.py:108).
* token rows: [CLS]=101, ids uniform in [1000, 30521], [SEP]=102, zero pad,
  attention mask 1 on real tokens, token types 0.

Tensor names and element counts follow the reference loader
(src/model/weights.h:56-107, src/core/model_config.h:7-17).
"""

from __future__ import annotations

import numpy as np

VOCAB_SIZE = 30522
HIDDEN = 384
NUM_LAYERS = 6
NUM_HEADS = 12
HEAD_DIM = 32
FFN_DIM = 1536
MAX_POSITION = 512
TYPE_VOCAB_SIZE = 2
LAYER_NORM_EPS = 1e-12

CLS_ID = 101
SEP_ID = 102
ID_LO, ID_HI = 1000, 30521  # inclusive range of synthetic word ids


def param_specs():
    """(name, shape) for the 101 tensors of BertModel without the pooler, in
    HF state_dict order (pooler skipped as in scripts/dump_weights.py:28,75-78)."""
    specs = [
        ("embeddings.word_embeddings.weight", (VOCAB_SIZE, HIDDEN)),
        ("embeddings.position_embeddings.weight", (MAX_POSITION, HIDDEN)),
        ("embeddings.token_type_embeddings.weight", (TYPE_VOCAB_SIZE, HIDDEN)),
        ("embeddings.LayerNorm.weight", (HIDDEN,)),
        ("embeddings.LayerNorm.bias", (HIDDEN,)),
    ]
    for i in range(NUM_LAYERS):
        p = f"encoder.layer.{i}."
        for part in ("query", "key", "value"):
            specs.append((p + f"attention.self.{part}.weight", (HIDDEN, HIDDEN)))
            specs.append((p + f"attention.self.{part}.bias", (HIDDEN,)))
        specs += [
            (p + "attention.output.dense.weight", (HIDDEN, HIDDEN)),
            (p + "attention.output.dense.bias", (HIDDEN,)),
            (p + "attention.output.LayerNorm.weight", (HIDDEN,)),
            (p + "attention.output.LayerNorm.bias", (HIDDEN,)),
            (p + "intermediate.dense.weight", (FFN_DIM, HIDDEN)),
            (p + "intermediate.dense.bias", (FFN_DIM,)),
            (p + "output.dense.weight", (HIDDEN, FFN_DIM)),
            (p + "output.dense.bias", (HIDDEN,)),
            (p + "output.LayerNorm.weight", (HIDDEN,)),
            (p + "output.LayerNorm.bias", (HIDDEN,)),
        ]
    return specs


def make_weights(seed: int = 0, std: float = 0.02) -> dict:
    """fp32 master weights, name -> array, in state_dict order."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in param_specs():
        if name.endswith("LayerNorm.weight"):
            out[name] = np.ones(shape, np.float32)
        elif name.endswith("LayerNorm.bias"):
            out[name] = np.zeros(shape, np.float32)
        else:
            out[name] = (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)
    return out


def to_fp16(weights: dict) -> dict:
    """Round-to-nearest-even fp16 copies (what the engine holds)."""
    return {k: v.astype(np.float16) for k, v in weights.items()}


def fp16_as_fp32(weights: dict) -> dict:
    """The fp16 weights widened back to fp32 (what the engine computes with)."""
    return {k: v.astype(np.float16).astype(np.float32) for k, v in weights.items()}


def write_weights_dir(weights: dict, directory) -> None:
    """Write the reference's on-disk layout: one raw little-endian fp16 file per
    tensor, ``<dir>/<state_dict name>.bin`` (scripts/dump_weights.py:75-83)."""
    import os

    os.makedirs(directory, exist_ok=True)
    for name, arr in weights.items():
        arr.astype(np.float16).tofile(os.path.join(directory, name + ".bin"))


# --------------------------------------------------------------------------
# token batches
# --------------------------------------------------------------------------

def round16(n: int) -> int:
    """Effective length: real length rounded up to 16, at least 16
    (bench/bench.cu:63, bench/corpus.cu:96)."""
    return max(16, (int(n) + 15) // 16 * 16)


def sentence(rng, length: int) -> np.ndarray:
    """[CLS] + (length-2) uniform ids + [SEP]; length counts CLS/SEP."""
    inner = rng.integers(ID_LO, ID_HI + 1, size=max(0, length - 2))
    return np.concatenate([[CLS_ID], inner, [SEP_ID]]).astype(np.int32)


def pack(rows, seq: int):
    """Pack sentences into (B, seq) int32 ids / types / mask, zero-padded."""
    b = len(rows)
    ids = np.zeros((b, seq), np.int32)
    mask = np.zeros((b, seq), np.int32)
    for i, r in enumerate(rows):
        n = len(r)
        assert n <= seq
        ids[i, :n] = r
        mask[i, :n] = 1
    types = np.zeros((b, seq), np.int32)
    return ids, types, mask


def cfg1_row(seed: int = 1) -> np.ndarray:
    """The 9-token sentence of BASELINE configs[0..2]: CLS, 7 ids, SEP."""
    return sentence(np.random.default_rng(seed), 9)


def cfg_fixed(batch: int, seq: int, seed: int = 1):
    """configs[0..2]: the same 9-token row repeated `batch` times at `seq`."""
    row = cfg1_row(seed)
    return pack([row] * batch, seq)


def varlen_lengths(n: int = 2000, seed: int = 0) -> np.ndarray:
    """Total token lengths (incl. CLS/SEP): lognormal(median 12, sigma 0.5),
    rounded, clipped to [5, 64]."""
    rng = np.random.default_rng(seed)
    return np.clip(np.round(rng.lognormal(np.log(12), 0.5, n)), 5, 64).astype(np.int64)


def varlen_rows(n: int = 2000, seed: int = 0) -> list:
    """The sentences of configs[3], in seeded order."""
    lengths = varlen_lengths(n, seed)
    rng = np.random.default_rng(seed + 1)
    return [sentence(rng, int(L)) for L in lengths]


def batches_of(rows, batch: int = 64, seq=None):
    """Consecutive batches of `batch` rows, each padded to round16(longest)
    or to a fixed `seq`.  Returns a list of (ids, types, mask, seq)."""
    out = []
    for s in range(0, len(rows), batch):
        chunk = rows[s:s + batch]
        sq = round16(max(len(r) for r in chunk)) if seq is None else seq
        ids, types, mask = pack(chunk, sq)
        out.append((ids, types, mask, sq))
    return out


def varlen_mix(n: int = 2000, seed: int = 0, batch: int = 64):
    """consecutive batches of `batch` in seeded order, each padded
    to round16(longest).  Returns a list of (ids, types, mask, seq)."""
    return batches_of(varlen_rows(n, seed), batch)


def varlen_sorted(n: int = 2000, seed: int = 0, batch: int = 64):
    """The reference corpus benchmark's dynamic mode on the configs[3]
    sentences (bench/corpus.cu:79-118): sentences stable-sorted by length,
    batches of `batch`, each padded to max(16, round16(longest)).  Returns
    (batches, order) with order[k] = the input index of sorted sentence k."""
    rows = varlen_rows(n, seed)
    order = np.argsort(np.asarray([len(r) for r in rows]), kind="stable")
    return batches_of([rows[i] for i in order], batch), order


def varlen_padded(n: int = 2000, seed: int = 0, batch: int = 64, seq: int = 128):
    """The reference corpus benchmark's padded mode on the configs[3]
    sentences (bench/corpus.cu:64-77): consecutive batches at seq 128."""
    return batches_of(varlen_rows(n, seed), batch, seq)


def long_batch(batch: int = 256, seq: int = 512, seed: int = 5, lo: int = 256):
    """batch 256 at seq 512, real lengths uniform in [lo, seq]."""
    rng = np.random.default_rng(seed)
    lengths = rng.integers(lo, seq + 1, size=batch)
    rows = [sentence(rng, int(L)) for L in lengths]
    return pack(rows, seq)


def flops_per_forward(batch: int, seq: int) -> int:
    """Algorithmic FLOPs of one forward at executed length `seq`: GEMMs
    6*2*(384*1152 + 384*384 + 384*1536 + 1536*384) per token plus QK^T and PV
    6*4*12*32*seq^2 per sequence."""
    gemm = NUM_LAYERS * 2 * (HIDDEN * 3 * HIDDEN + HIDDEN * HIDDEN + 2 * HIDDEN * FFN_DIM)
    attn = NUM_LAYERS * 4 * NUM_HEADS * HEAD_DIM
    return batch * seq * gemm + batch * attn * seq * seq


# --------------------------------------------------------------------------
# text (tokenizer tests and timing)
# --------------------------------------------------------------------------

TEXT_WORDS = ("the a of and to in is was for on with as by at from that this it be are "
         "hello world model token embed sentence vector gpu kernel matrix batch layer "
         "attention learning deep neural network fast slow big small red blue green "
         "café naïve résumé über straße mañana ελληνικά русский язык").split()


def text_vocab(seed: int = 0) -> list:
    """A seeded WordPiece vocabulary (specials, characters, ## pieces, the
    TEXT_WORDS and their subword pieces) for tokenizer tests and timing; the
    real MiniLM vocab.txt is not available offline."""
    rng = np.random.default_rng(seed)
    toks = ["[PAD]", "[UNK]", "[CLS]", "[SEP]", "[MASK]"]
    chars = [chr(c) for c in range(33, 127)] + list("αβγδεζηθλμπσςωабвгдежзиклмн中文字词语日本語한국어") \
        + ["ᄀ", "ᅡ", "ᆨ", "ᄒ", "ᅩ"]
    toks += [c.lower() for c in chars]
    toks += ["##" + c.lower() for c in chars if c.isalnum()]
    for w in TEXT_WORDS:
        w = w.lower()
        toks.append(w)
        for k in range(2, len(w)):  # subword pieces of every word
            if rng.random() < 0.5:
                toks.append("##" + w[k:])
            if rng.random() < 0.3:
                toks.append(w[:k])
    for _ in range(400):  # random pieces
        n = int(rng.integers(2, 6))
        s = "".join(rng.choice(list("abcdefghijklmnopqrstuvwxyz"), n))
        toks.append(("##" if rng.random() < 0.5 else "") + s)
    seen, vocab = set(), []
    for t in toks:
        if t not in seen:
            seen.add(t)
            vocab.append(t)
    return vocab


def texts(seed: int = 1, n: int = 400) -> list:
    """Seeded synthetic sentences over TEXT_WORDS, punctuation and a set of
    Unicode edge cases (each also appended alone)."""
    rng = np.random.default_rng(seed)
    extra = ["中文", "日本語です", "한국어", "Ωmega", "ÅNGSTRÖM", "Ǆ", "İstanbul", "ß", "ΣΑΣ",
             "emoji 🙂👍", "zero​width", "tab\there", "nl\nline", "nbsp x",
             "ideo　space", "ctl\x07bell", "\x0bvt", "soft­hyphen", "x" * 120,
             "unk§¶word", "dashes—and–more", "quote«»„“", "num3r1c 42 3.14", "a.b,c;d:e!f?g",
             "[cls] lower", "[CLS][SEP]x[MASK]y", "[UNK", "e\u0301te", "A\u030Angstrom",
             "1+1=2 <tag> a|b ~x ^y `z", "price 5€ ©2024 ™", "ｆｕｌｌｗｉｄｔｈ", "ﬁne ligature",
             "\u0915\u094D\u0937", "mixed中文and한글text"]
    texts = []
    for _ in range(n):
        k = int(rng.integers(1, 25))
        parts = []
        for _ in range(k):
            r = rng.random()
            if r < 0.6:
                w = rng.choice(TEXT_WORDS)
                parts.append(w.upper() if rng.random() < 0.2 else w.capitalize() if rng.random() < 0.3 else w)
            elif r < 0.8:
                parts.append(str(rng.choice(list(",.!?;:'\"()-"))))
            else:
                parts.append(str(rng.choice(extra)))
        sep = " " if rng.random() < 0.8 else "  \t"
        texts.append(sep.join(parts))
    texts += ["", "   ", "[CLS] literal", "Hello, World!"] + extra  # every case at least once
    return texts
