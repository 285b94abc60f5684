"""bbh_embed_noalloc (the workspace-free entry point for callers that cannot
allocate) against bbh_embed on a workspace, through the C ABI: the same
kernels on the same inputs, so the embeddings must be equal bit for bit, on
consecutive calls with shrinking inputs (the library's device array keeps the
previous call's contents)."""

import ctypes

import numpy as np
import pytest

from conftest import to_dev

pytestmark = pytest.mark.gpu


def _ragged(rng, B, S):
    from bbh import synth

    lens = rng.integers(2, S + 1, size=B)
    lens[0] = S
    ids, types, mask = synth.pack([synth.sentence(rng, int(n)) for n in lens], S)
    types[1, : lens[1] // 2] = 1
    return ids, types, mask


def test_noalloc_equals_workspace_embed(torch_cuda, model):
    from bbh import capi, engine

    torch = torch_cuda
    L = capi.lib()
    ws = engine.Workspace(64, 128)
    rng = np.random.default_rng(11)
    for B, S in [(64, 128), (24, 48), (5, 16)]:  # the full capacity first, then smaller
        ids, types, mask = (to_dev(torch, a) for a in _ragged(rng, B, S))
        want = engine.bert_embed(ws, model, ids, types, mask)
        got = torch.full((B, 384), float("nan"), dtype=torch.float16, device="cuda")
        st = L.bbh_embed_noalloc(model.handle, ctypes.c_void_p(ids.data_ptr()),
                                 ctypes.c_void_p(types.data_ptr()), ctypes.c_void_p(mask.data_ptr()),
                                 ctypes.c_void_p(got.data_ptr()), B, S,
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert st == 0, L.bbh_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), (B, S)
        # the Python wrapper takes the same path
        assert torch.equal(engine.bert_embed_noalloc(model, ids, types, mask), want)
    ws.close()


def test_noalloc_rejects_sizes_beyond_its_array(torch_cuda, model):
    from bbh import capi, engine

    torch = torch_cuda
    L = capi.lib()
    ids = torch.zeros((65, 128), dtype=torch.int32, device="cuda")
    emb = torch.empty((65, 384), dtype=torch.float16, device="cuda")
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    # 65 x 128 rows > BBH_NOALLOC_MAX_ROWS = 8192: refused before any launch
    assert L.bbh_embed_noalloc(model.handle, p(ids), p(ids), p(ids), p(emb), 65, 128, None) == 3
    assert b"exceeds 8192 rows" in L.bbh_last_error()
    assert L.bbh_embed_noalloc(model.handle, p(ids), p(ids), p(ids), p(emb), 16, 520, None) == 2
    assert L.bbh_embed_noalloc(None, p(ids), p(ids), p(ids), p(emb), 1, 16, None) == 1
    with pytest.raises(capi.BBHError) as e:
        engine.bert_embed_noalloc(model, ids, ids, ids, emb)
    assert e.value.name == "BBH_ERR_CAPACITY"
