"""The reference's own test programs (tests/test_{matmul,gelu,layernorm,
softmax,embedding,attention,layer,embed,batch}.cu), restated in C++ against
the drop-in header bert-by-hand_amd/cpp/bert_by_hand.hpp and built as
bert-by-hand_amd/cpp/dropin_check, run on the GPU.

As in the reference, the program reads weights/ and ref/ from its working
directory.  This test writes them: the seeded model in the reference's
on-disk layout (one raw fp16 file per state_dict tensor), the regenerated
kernel KATs (tests/golden/kats.npz), the s128 sentence with the
transformers BertModel embedding as expected_embedding, and the oracle's
embedding-LayerNorm, attention-block and layer-0 outputs at seq 128."""

import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT
from oracle import bert_oracle as O

BIN = os.path.join(ROOT, "bert-by-hand_amd", "cpp", "dropin_check")
N_CASES = 20  # 2 matmul, gelu, layernorm, softmax, embedding, 4 block, embed, encode, 8 batch rows


def _write_ref(ref, weights32, kats, golden):
    def put(name, arr):
        np.ascontiguousarray(arr).tofile(os.path.join(ref, name + ".bin"))

    for k in kats.files:  # fp16 inputs, fp32 expected outputs, the reference's formats
        put(k, kats[k])
    ids, types, mask = golden["s128_ids"], golden["s128_types"], golden["s128_mask"]
    put("input_ids", ids.astype(np.int32))
    put("token_type_ids", types.astype(np.int32))
    put("attention_mask", mask.astype(np.int32))
    emb = O.embeddings(weights32, ids, types)
    put("emb_out", emb.astype(np.float32))
    # the program feeds emb_out to the blocks rounded to fp16
    h16 = emb.astype(np.float16).astype(np.float32)
    lw = O._layer(weights32, 0)
    put("attn0_out", O.attention_block(h16, lw, mask).astype(np.float32))
    put("layer0_out", O.encoder_layer(h16, lw, mask).astype(np.float32))
    put("expected_embedding", golden["s128_embedding"].astype(np.float32))


@pytest.mark.gpu
def test_reference_test_programs_through_cpp_dropin(torch_cuda, weights32, kats, golden_model,
                                                   tmp_path):
    from bbh import synth

    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built (run __graft_entry__.build())")
    synth.write_weights_dir(weights32, str(tmp_path / "weights"))
    ref = tmp_path / "ref"
    ref.mkdir()
    _write_ref(str(ref), weights32, kats, golden_model)
    r = subprocess.run([BIN], cwd=str(tmp_path), capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout
    assert r.stdout.count(" PASS") == N_CASES, r.stdout


def test_cpp_dropin_aborts_on_missing_ref_file(tmp_path):
    # The reference aborts with the path when an input file is missing
    # (src/core/file_io.h:12-15); so does the drop-in's read_bin.  The program
    # stops at its first file read, before any HIP call, so this runs on the CPU.
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built (run __graft_entry__.build())")
    (tmp_path / "ref").mkdir()
    r = subprocess.run([BIN], cwd=str(tmp_path), capture_output=True, text=True, timeout=60)
    assert r.returncode != 0
    assert "cannot open" in r.stderr
