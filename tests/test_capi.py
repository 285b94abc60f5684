"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, and rejects bad arguments before touching the device.  No
compute entry point is called without a GPU."""

import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "bbh.h")


def _lib():
    from bbh import capi

    if not os.path.exists(capi.LIB_PATH):
        pytest.fail("libbbh.so not built (run __graft_entry__.build())")
    return capi.lib()


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(bbh_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_all_exported():
    L = _lib()
    from bbh import capi

    names = declared_symbols()
    assert len(names) == 55
    for n in names:
        assert hasattr(L, n), n
    # the Python binding types every declared entry point
    assert sorted(capi.SIGNATURES) == names


def test_param_table_matches_state_dict_order():
    L = _lib()
    from bbh import synth

    specs = synth.param_specs()
    assert L.bbh_param_count() == len(specs) == 101
    total = 0
    for i, (name, shape) in enumerate(specs):
        assert L.bbh_param_name(i).decode() == name
        assert L.bbh_param_numel(i) == int(np.prod(shape))
        total += int(np.prod(shape))
    assert total == 22_565_376  # BertModel without pooler
    assert L.bbh_param_name(101) is None and L.bbh_param_numel(-1) == 0


def test_status_strings():
    L = _lib()
    for s in range(8):
        assert L.bbh_status_string(s)
    assert b"gfx950" in L.bbh_version()


def test_workspace_bytes():
    L = _lib()
    rows = 64 * 128
    # QKV, FFN intermediate, four (rows, 384) buffers, the packed-forward
    # sentence table (24 bytes per possible sentence), and the carried
    # LayerNorm statistics of up to 8192 rows (two buffers of 6 float pairs
    # a row, two of one pair a row)
    rc = min(rows, 8192)
    want = sum((n + 255) // 256 * 256
               for n in [rows * 1152 * 2, rows * 1536 * 2] + [rows * 384 * 2] * 4 + [rows * 24]
               + [rc * 48] * 2 + [rc * 8] * 2)
    assert L.bbh_workspace_bytes(64, 128) == want
    assert L.bbh_workspace_bytes(0, 128) == 0


def test_null_arguments_rejected_without_device_work():
    L = _lib()
    from bbh import capi

    assert L.bbh_embed(None, None, None, None, None, None, 1, 16, None) == 1
    assert b"null" in L.bbh_last_error()
    assert L.bbh_linear(None, None, None, 1, 1, 1, None, 0, None) == 1
    assert L.bbh_layernorm(None, None, None, None, 1, 384, ctypes.c_float(1e-12), None, None) == 1
    assert L.bbh_attention(None, None, None, 1, 12, 16, 32, ctypes.c_float(0.1), None) == 1
    h = ctypes.c_void_p()
    assert L.bbh_workspace_create(0, 16, ctypes.byref(h)) == 1
    assert L.bbh_workspace_create(4, 24, ctypes.byref(h)) == 2  # seq % 16
    assert L.bbh_workspace_create(4, 528, ctypes.byref(h)) == 3  # > 512
    assert L.bbh_workspace_create(2049, 512, ctypes.byref(h)) == 3  # > 2^20 rows
    with pytest.raises(capi.BBHError) as e:
        capi.call("bbh_model_from_host", None, 101, ctypes.byref(h))
    assert e.value.name == "BBH_ERR_INVALID_ARG"


def test_shape_validation_order():
    # Fake (never dereferenced) handles: shape checks fire before any launch.
    L = _lib()
    fake = ctypes.c_void_p(1)
    st = L.bbh_attention(fake, fake, fake, 1, 12, 24, 32, ctypes.c_float(0.1), None)
    assert st == 2 and b"16" in L.bbh_last_error()
    st = L.bbh_attention(fake, fake, fake, 1, 12, 16, 64, ctypes.c_float(0.1), None)
    assert st == 7
    st = L.bbh_linear_residual_layernorm(fake, fake, fake, fake, fake, fake, fake, 4, 512, 384,
                                         ctypes.c_float(1e-12), None)
    assert st == 7


def test_load_dir_missing_and_truncated_files(tmp_path, weights32):
    L = _lib()
    from bbh import synth

    h = ctypes.c_void_p()
    assert L.bbh_model_load_dir(str(tmp_path / "nope").encode(), ctypes.byref(h)) == 4
    assert b"cannot open" in L.bbh_last_error()

    small = {k: v for k, v in weights32.items()}
    synth.write_weights_dir(small, str(tmp_path))
    # truncate one tensor: rejected with the file name, before any device allocation
    victim = tmp_path / "encoder.layer.3.output.dense.bias.bin"
    victim.write_bytes(victim.read_bytes()[:-2])
    assert L.bbh_model_load_dir(str(tmp_path).encode(), ctypes.byref(h)) == 4
    msg = L.bbh_last_error().decode()
    assert "encoder.layer.3.output.dense.bias" in msg and "768" in msg
    # an oversized file is rejected too (the reference only checks for short reads)
    victim.write_bytes(b"\0" * 770)
    assert L.bbh_model_load_dir(str(tmp_path).encode(), ctypes.byref(h)) == 4


def test_product_path_fails_loudly_without_library(tmp_path, monkeypatch):
    from bbh import capi

    monkeypatch.setattr(capi, "_lib", None)
    monkeypatch.setattr(capi, "LIB_PATH", str(tmp_path / "libbbh.so"))
    with pytest.raises(RuntimeError, match="not built"):
        capi.lib()


def test_weight_view_entry_points_validate_before_launch():
    L = _lib()
    from bbh import capi

    aw, fw = capi.AttnWeights(), capi.FfnWeights()
    assert L.bbh_model_layer(None, 0, ctypes.byref(aw), ctypes.byref(fw)) == 1
    # range is checked before the handle is read
    assert L.bbh_model_layer(ctypes.c_void_p(1), 6, None, None) == 1
    assert b"out of range" in L.bbh_last_error()
    fake = ctypes.c_void_p(256)
    assert L.bbh_attention_block_w(None, fake, ctypes.byref(aw), fake, fake, 1, 16, None) == 1
    assert L.bbh_ffn_block_w(None, fake, ctypes.byref(fw), fake, 1, 16, None) == 1
    assert L.bbh_encoder_layer_w(None, fake, ctypes.byref(aw), ctypes.byref(fw), fake, fake, 1, 16,
                                 None) == 1
    # launch_gelu: n == 0 is a no-op, negative n and a null buffer are errors
    assert L.bbh_gelu(None, 0, None) == 0
    assert L.bbh_gelu(None, 5, None) == 1
    assert L.bbh_gelu(fake, -1, None) == 1


def test_tile_names_and_timing_arguments():
    L = _lib()
    assert L.bbh_gemm_tile_name(26) == b"Cfg<64,64,2,2,2,4,2>"
    assert L.bbh_gemm_tile_name(0) == b"Cfg<64,64,2,2,4,0,2>"
    assert L.bbh_gemm_tile_name(33) == b"WRes<12x32,384>"
    # sweep-only configurations are not in the product build
    assert L.bbh_gemm_tile_name(23) == b"generic"
    assert L.bbh_gemm_tile_name(-1) == b"generic" and L.bbh_gemm_tile_name(999) == b"generic"
    cnt = ctypes.c_int(7)
    assert L.bbh_pool_timing(None, 16) == 1
    assert L.bbh_pool_timing_read(None, None, 0, ctypes.byref(cnt)) == 1


def test_graph_entry_points_validate_before_touching_hip():
    L = _lib()
    g = ctypes.c_void_p()
    fake = ctypes.c_void_p(256)
    assert L.bbh_embed_graph_create(None, fake, fake, fake, fake, fake, 1, 16, ctypes.byref(g)) == 1
    assert L.bbh_embed_graph_create(fake, fake, fake, fake, fake, ctypes.c_void_p(258), 1, 16,
                                    ctypes.byref(g)) == 1  # emb not 4-byte aligned
    assert L.bbh_graph_launch(None, None) == 1
    assert L.bbh_graph_free(None) == 0
