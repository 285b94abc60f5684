import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "bert-by-hand_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def weights32():
    """fp32 master weights, seed 0 (the oracle's model)."""
    from bbh import synth

    return synth.make_weights(0)


@pytest.fixture(scope="session")
def weights16(weights32):
    """The engine's fp16 weights widened to fp32 (isolates kernel error)."""
    from bbh import synth

    return synth.fp16_as_fp32(weights32)


@pytest.fixture(scope="session")
def golden_model():
    return np.load(os.path.join(GOLDEN, "model_seed0.npz"), allow_pickle=False)


@pytest.fixture(scope="session")
def kats():
    return np.load(os.path.join(GOLDEN, "kats.npz"), allow_pickle=False)


# ---- GPU fixtures -----------------------------------------------------------

@pytest.fixture(scope="session")
def torch_cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.fixture(scope="session")
def model(torch_cuda, weights32):
    from bbh import engine

    m = engine.Model.from_weights(weights32)
    yield m
    m.close()


@pytest.fixture(scope="session")
def ws(torch_cuda):
    """One workspace big enough for every config (256 x 512 rows)."""
    from bbh import engine

    w = engine.Workspace(256, 512)
    yield w
    w.close()


@pytest.fixture(scope="session")
def cfg5_oracle(weights32):
    """configs[4] (256 x 512, lengths 256-512): indices of 32 sentences spread
    over the lengths, shortest and longest included, and the fp32 oracle's
    embeddings of them, in four calls of 8 sentences each at the effective
    length (round16) of the longest of the 8."""
    from bbh import synth
    from oracle import bert_oracle as O

    ids, types, mask = synth.long_batch()
    lens = mask.sum(1)
    picks = sorted({int(np.argmin(np.abs(lens - t)))
                    for t in np.linspace(lens.min(), lens.max(), 32)})
    assert len(picks) >= 28 and lens[picks].min() == lens.min() and lens[picks].max() == lens.max()
    picks = np.asarray(picks)
    picks = picks[np.argsort(lens[picks], kind="stable")]
    want = []
    for grp in np.array_split(picks, 4):
        s = synth.round16(int(lens[grp].max()))
        want.append(O.bert_embed(weights32, ids[grp, :s], types[grp, :s], mask[grp, :s]))
    return picks, np.concatenate(want)


def cosine_rows(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    num = (a * b).sum(-1)
    den = np.sqrt((a * a).sum(-1)) * np.sqrt((b * b).sum(-1)) + 1e-30
    return num / den


def to_dev(torch, arr, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(arr))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()
