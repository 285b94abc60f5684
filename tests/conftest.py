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
