"""bbh_model_load_safetensors: the reader's checks, which all run before any
device allocation (so on the CPU), against files written by the safetensors
package itself."""

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


@pytest.fixture(scope="module")
def st():
    return pytest.importorskip("safetensors.numpy")


def _load(L, path):
    h = ctypes.c_void_p()
    st = L.bbh_model_load_safetensors(str(path).encode(), ctypes.byref(h))
    return st, L.bbh_last_error().decode()


def test_missing_and_malformed_files(tmp_path):
    L = _lib()
    st, msg = _load(L, tmp_path / "nope.safetensors")
    assert st == 4 and "cannot open" in msg
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes((10).to_bytes(8, "little") + b'{"a": [1, ')
    st, msg = _load(L, bad)
    assert st == 4 and "malformed" in msg
    short = tmp_path / "short.safetensors"
    short.write_bytes((1 << 20).to_bytes(8, "little") + b"{}")
    st, msg = _load(L, short)
    assert st == 4 and "header length" in msg


def test_tensor_checks(tmp_path, weights32, st):
    L = _lib()
    w = dict(weights32)
    # a missing tensor is named
    d = dict(w)
    del d["encoder.layer.4.output.dense.bias"]
    st.save_file(d, str(tmp_path / "a.safetensors"))
    code, msg = _load(L, tmp_path / "a.safetensors")
    assert code == 4 and "missing tensor encoder.layer.4.output.dense.bias" in msg
    # a transposed weight is a shape error
    d = dict(w)
    d["encoder.layer.0.output.dense.weight"] = np.ascontiguousarray(
        w["encoder.layer.0.output.dense.weight"].T)
    st.save_file(d, str(tmp_path / "b.safetensors"))
    code, msg = _load(L, tmp_path / "b.safetensors")
    assert code == 4 and "shape [1536,384]" in msg
    # an integer tensor is a dtype error
    d = dict(w)
    d["embeddings.LayerNorm.bias"] = np.zeros(384, np.int32)
    st.save_file(d, str(tmp_path / "c.safetensors"))
    code, msg = _load(L, tmp_path / "c.safetensors")
    assert code == 4 and "dtype I32" in msg


def test_data_offsets_checked(tmp_path, weights32, st):
    # a header whose byte range runs past the end of the file is rejected
    L = _lib()
    good = tmp_path / "g.safetensors"
    st.save_file({k: v.astype(np.float16) for k, v in weights32.items()}, str(good))
    raw = good.read_bytes()
    cut = tmp_path / "cut.safetensors"
    cut.write_bytes(raw[:-1000])
    code, msg = _load(L, cut)
    assert code == 4 and "data_offsets" in msg
