"""Host-side mirror of the reference's C++ API over the C ABI, for torch
device tensors (torch is used only for device memory and streams).

Reference names kept: ``load_model_weights`` (src/model/weights.h:88),
``make_workspace`` (src/model/workspace.h:20), ``bert_embed`` / ``bert_encode``
(src/model/forward.h:11-19), ``encoder_layer`` / ``attention_block`` /
``ffn_block`` (src/model/encoder.h:27-46) and the ``launch_*`` kernel
launchers (src/kernels/*.h).  Like the reference, every call only enqueues
work on the current stream; errors raise ``BBHError`` instead of aborting.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import capi
from .capi import call, lib

HIDDEN = 384
NUM_LAYERS = 6
NUM_HEADS = 12
HEAD_DIM = 32
FFN_DIM = 1536
LAYER_NORM_EPS = 1e-12


def _torch():
    import torch

    return torch


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _stream(stream=None):
    if stream is not None:
        return ctypes.c_void_p(stream)
    torch = _torch()
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class Model:
    """Device-resident weights (the reference's ModelWeights)."""

    def __init__(self, handle: ctypes.c_void_p):
        self.handle = handle

    @classmethod
    def from_weights(cls, weights: dict) -> "Model":
        """weights: state_dict name -> array (any float dtype; cast to fp16 RNE)."""
        L = lib()
        n = L.bbh_param_count()
        keep, ptrs = [], (ctypes.c_void_p * n)()
        for i in range(n):
            name = L.bbh_param_name(i).decode()
            arr = np.ascontiguousarray(np.asarray(weights[name]).astype(np.float16))
            if arr.size != L.bbh_param_numel(i):
                raise ValueError(f"{name}: expected {L.bbh_param_numel(i)} elements, got {arr.size}")
            keep.append(arr)
            ptrs[i] = arr.ctypes.data
        h = ctypes.c_void_p()
        call("bbh_model_from_host", ptrs, n, ctypes.byref(h))
        return cls(h)

    @classmethod
    def load_dir(cls, directory: str) -> "Model":
        h = ctypes.c_void_p()
        call("bbh_model_load_dir", directory.encode(), ctypes.byref(h))
        return cls(h)

    @classmethod
    def load_safetensors(cls, path: str) -> "Model":
        h = ctypes.c_void_p()
        call("bbh_model_load_safetensors", path.encode(), ctypes.byref(h))
        return cls(h)

    def close(self):
        if self.handle:
            call("bbh_model_free", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Workspace:
    """All scratch of a forward, allocated once (the reference's Workspace)."""

    def __init__(self, max_batch: int, max_seq: int = 128):
        self.max_batch, self.max_seq = max_batch, max_seq
        self.handle = ctypes.c_void_p()
        call("bbh_workspace_create", max_batch, max_seq, ctypes.byref(self.handle))

    def hidden(self, batch: int, seq: int):
        """Zero-copy (batch*seq, 384) fp16 view of the final-hidden buffer
        (ws.attn_out); holds the encoder output after bert_embed."""
        torch = _torch()
        if batch * seq > self.max_batch * self.max_seq:
            raise ValueError("view larger than the workspace")
        ptr = lib().bbh_workspace_hidden(self.handle)
        return torch.as_tensor(_DeviceArray(ptr, (batch * seq, HIDDEN), "<f2"), device="cuda")

    def close(self):
        if self.handle:
            call("bbh_workspace_free", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _DeviceArray:
    """Minimal __cuda_array_interface__ exporter for a device pointer the
    library owns (torch.as_tensor wraps it without copying)."""

    def __init__(self, ptr: int, shape, typestr: str):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": typestr,
                                         "data": (int(ptr), False), "version": 3,
                                         "strides": None}


class EmbedGraph:
    """bert_embed on fixed device buffers, captured once as a HIP graph and
    replayed with one launch (bbh_embed_graph_create / bbh_graph_launch)."""

    def __init__(self, ws: "Workspace", w: "Model", ids, types, mask, emb):
        _check_i32(ids, types, mask)
        B, S = ids.shape
        self.handle = ctypes.c_void_p()
        self.emb = emb
        self._keep = (ws, w, ids, types, mask, emb)  # the graph reads these buffers
        call("bbh_embed_graph_create", ws.handle, w.handle, _ptr(ids), _ptr(types), _ptr(mask),
             _ptr(emb), B, S, ctypes.byref(self.handle))

    def launch(self, stream=None):
        call("bbh_graph_launch", self.handle, _stream(stream))
        return self.emb

    def close(self):
        if self.handle:
            call("bbh_graph_free", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Pool:
    """n slots, each with its own workspace: slot n-1 runs on the caller's
    stream, the others on n-1 HIP streams of the pool; embed_batches overlaps
    independent batches across them (replaces a sequential batch loop)."""

    def __init__(self, n_streams: int, max_batch: int, max_seq: int):
        self.handle = ctypes.c_void_p()
        call("bbh_pool_create", n_streams, max_batch, max_seq, ctypes.byref(self.handle))

    def timing(self, capacity: int):
        """Start timing each op of later embed_batches calls (0 stops)."""
        call("bbh_pool_timing", self.handle, capacity)

    OPS = {1: "qkv", 2: "attention", 3: "o_proj_ln", 4: "ffn1_gelu", 5: "ffn2_ln", 6: "embed",
           7: "pool", 8: "layernorm", 9: "ffn"}

    def timing_read(self):
        """The recorded launches: dicts of op, tile, fused_ln, m, n, k, ms."""
        cnt = ctypes.c_int()
        call("bbh_pool_timing_read", self.handle, None, 0, ctypes.byref(cnt))
        buf = (capi.LaunchTime * max(cnt.value, 1))()
        call("bbh_pool_timing_read", self.handle, buf, cnt.value, ctypes.byref(cnt))
        return [dict(op=self.OPS[r.op], tile=r.tile, fused_ln=int(r.fused_ln), m=r.m, n=r.n,
                     k=r.k, ms=r.ms) for r in buf[:cnt.value]]

    def busy(self) -> int:
        """Pool streams and workspaces (on any stream) with work pending."""
        n = ctypes.c_int()
        call("bbh_pool_busy", self.handle, ctypes.byref(n))
        return n.value

    def fail_at(self, batch: int):
        """Test hook: later calls fail on reaching batch / group / forward `batch`."""
        call("bbh_pool_fail_at", self.handle, batch)

    def close(self):
        if self.handle:
            call("bbh_pool_free", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class PackedBatches:
    """Batches packed back to back in device memory for embed_batches:
    batch i = (ids, types, mask) of shape (B_i, S_i).

    With group_by_seq=True the batches are stable-sorted by S_i before
    packing, so equal-length batches are adjacent and embed_batches runs each
    such run as one larger forward; every batch keeps its own padding.
    `order` is the packed position -> input batch index map, and
    `unpermute(emb)` returns the embeddings in input sentence order."""

    def __init__(self, batches, group_by_seq: bool = False):
        torch = _torch()
        n = len(batches)
        seqs_in = [int(b[0].shape[1]) for b in batches]
        order = sorted(range(n), key=lambda i: seqs_in[i]) if group_by_seq else list(range(n))
        self.order = np.asarray(order, np.int64)
        batches = [batches[i] for i in order]
        sizes = [int(b[0].shape[0]) for b in batches]
        seqs = [int(b[0].shape[1]) for b in batches]
        toks = [b * s for b, s in zip(sizes, seqs)]
        self.tok_offsets = np.concatenate([[0], np.cumsum(toks)[:-1]]).astype(np.int64)
        self.emb_rows = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
        self.sizes = np.asarray(sizes, np.int32)
        self.seqs = np.asarray(seqs, np.int32)
        self.rows = int(sum(sizes))
        cat = lambda k: torch.from_numpy(np.concatenate([np.asarray(b[k]).reshape(-1) for b in batches]).astype(np.int32)).cuda()  # noqa: E731
        self.ids, self.types, self.mask = cat(0), cat(1), cat(2)
        self.n = n
        # per sentence (packed order): number of valid tokens, and whether
        # every mask is right-padding (ones then zeros), which embed_packed needs
        rows_mask = [np.asarray(b[2]).reshape(int(b[0].shape[0]), -1) != 0 for b in batches]
        self.lengths = (np.concatenate([m.sum(axis=1) for m in rows_mask]).astype(np.int32)
                        if n else np.zeros(0, np.int32))
        self.right_padded = all(
            bool(np.all(m == (np.arange(m.shape[1])[None, :] < m.sum(axis=1)[:, None])))
            for m in rows_mask)
        # packed sentence row -> input sentence row
        in_sizes = np.zeros(n, np.int64)
        in_sizes[self.order] = self.sizes
        in_start = np.concatenate([[0], np.cumsum(in_sizes)[:-1]])
        self._rows_src = np.concatenate(
            [in_start[i] + np.arange(in_sizes[i]) for i in self.order]).astype(np.int64) \
            if n else np.zeros(0, np.int64)

    def unpermute(self, emb):
        """Embeddings (rows, 384) in packed order -> input sentence order."""
        torch = _torch()
        out = torch.empty_like(emb)
        out[torch.from_numpy(self._rows_src).to(emb.device)] = emb
        return out


def embed_batches(pool: Pool, w: Model, packed: PackedBatches, emb=None, stream=None):
    """(rows, 384) fp16 embeddings of every packed batch, in batch order."""
    torch = _torch()
    if emb is None:
        emb = torch.empty((packed.rows, HIDDEN), dtype=torch.float16, device="cuda")
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    call("bbh_embed_batches", pool.handle, w.handle, _ptr(packed.ids), _ptr(packed.types),
         _ptr(packed.mask), p(packed.tok_offsets), p(packed.sizes), p(packed.seqs),
         p(packed.emb_rows), _ptr(emb), packed.n, _stream(stream))
    return emb


def embed_each(pool: Pool, w: Model, packed: PackedBatches, emb=None, stream=None):
    """One bert_embed per packed batch (the reference's corpus loop,
    bench/corpus.cu:120-132), the batches spread over the pool's streams;
    nothing is merged (bbh_embed_each).  (rows, 384) fp16, in batch order."""
    torch = _torch()
    if emb is None:
        emb = torch.empty((packed.rows, HIDDEN), dtype=torch.float16, device="cuda")
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    call("bbh_embed_each", pool.handle, w.handle, _ptr(packed.ids), _ptr(packed.types),
         _ptr(packed.mask), p(packed.tok_offsets), p(packed.sizes), p(packed.seqs),
         p(packed.emb_rows), _ptr(emb), packed.n, _stream(stream))
    return emb


def embed_packed(pool: Pool, w: Model, packed: PackedBatches, emb=None, stream=None):
    """embed_batches without the padding rows: only each sentence's valid
    tokens enter the forward (bbh_embed_packed).  Needs right-padded masks."""
    torch = _torch()
    if not packed.right_padded:
        raise ValueError("embed_packed needs right-padded masks (ones, then zeros)")
    if emb is None:
        emb = torch.empty((packed.rows, HIDDEN), dtype=torch.float16, device="cuda")
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    call("bbh_embed_packed", pool.handle, w.handle, _ptr(packed.ids), _ptr(packed.types),
         p(packed.tok_offsets), p(packed.sizes), p(packed.seqs), p(packed.lengths),
         p(packed.emb_rows), _ptr(emb), packed.n, _stream(stream))
    return emb


def load_model_weights(weights_or_dir) -> Model:
    if isinstance(weights_or_dir, (str, bytes)):
        return Model.load_dir(weights_or_dir)
    return Model.from_weights(weights_or_dir)


def make_workspace(batch: int = 1, max_seq: int = 128) -> Workspace:
    return Workspace(batch, max_seq)


def _check_i32(*ts):
    torch = _torch()
    for t in ts:
        if t.dtype != torch.int32 or not t.is_contiguous() or not t.is_cuda:
            raise TypeError("ids/types/mask must be contiguous int32 CUDA tensors")


def bert_embed(ws: Workspace, w: Model, ids, types, mask, emb=None, batch=None, seq=None,
               stream=None):
    """(batch, seq) int32 device tensors -> (batch, 384) fp16 embeddings."""
    torch = _torch()
    _check_i32(ids, types, mask)
    batch = ids.shape[0] if batch is None else batch
    seq = ids.shape[-1] if seq is None else seq
    if emb is None:
        emb = torch.empty((batch, HIDDEN), dtype=torch.float16, device=ids.device)
    call("bbh_embed", ws.handle, w.handle, _ptr(ids), _ptr(types), _ptr(mask), _ptr(emb), batch, seq,
         _stream(stream))
    return emb


NOALLOC_MAX_ROWS = 8192  # BBH_NOALLOC_MAX_ROWS


def bert_embed_noalloc(w: Model, ids, types, mask, emb=None, batch=None, seq=None, stream=None):
    """bert_embed without a workspace (bbh_embed_noalloc): the library's own
    device array holds the activations, so the call allocates nothing.  At
    most NOALLOC_MAX_ROWS = batch * seq rows; calls overlapping on one GPU race."""
    torch = _torch()
    _check_i32(ids, types, mask)
    batch = ids.shape[0] if batch is None else batch
    seq = ids.shape[-1] if seq is None else seq
    if emb is None:
        emb = torch.empty((batch, HIDDEN), dtype=torch.float16, device=ids.device)
    call("bbh_embed_noalloc", w.handle, _ptr(ids), _ptr(types), _ptr(mask), _ptr(emb), batch, seq,
         _stream(stream))
    return emb


def bert_encode(ws: Workspace, w: Model, ids, types, mask, out=None, batch=None, seq=None,
                stream=None):
    torch = _torch()
    _check_i32(ids, types, mask)
    batch = ids.shape[0] if batch is None else batch
    seq = ids.shape[-1] if seq is None else seq
    if out is None:
        out = torch.empty((batch * seq, HIDDEN), dtype=torch.float16, device=ids.device)
    call("bbh_encode", ws.handle, w.handle, _ptr(ids), _ptr(types), _ptr(mask), _ptr(out), batch,
         seq, _stream(stream))
    return out


def attention_block(ws, w, layer, hidden, mask, out, batch, seq, stream=None):
    call("bbh_attention_block", ws.handle, w.handle, layer, _ptr(hidden), _ptr(mask), _ptr(out),
         batch, seq, _stream(stream))
    return out


def ffn_block(ws, w, layer, hidden, out, batch, seq, stream=None):
    call("bbh_ffn_block", ws.handle, w.handle, layer, _ptr(hidden), _ptr(out), batch, seq,
         _stream(stream))
    return out


def encoder_layer(ws, w, layer, hidden, mask, out, batch, seq, stream=None):
    call("bbh_encoder_layer", ws.handle, w.handle, layer, _ptr(hidden), _ptr(mask), _ptr(out),
         batch, seq, _stream(stream))
    return out


# ---- kernel launchers (src/kernels/*.h) ------------------------------------

def launch_matmul(A, B, C, M, N, K, bias=None, gelu=False, stream=None):
    call("bbh_linear", _ptr(A), _ptr(B), _ptr(C), M, N, K, _ptr(bias), int(bool(gelu)),
         _stream(stream))
    return C


def launch_linear_residual_layernorm(A, B, bias, residual, gamma, beta, y, M, K,
                                     eps=LAYER_NORM_EPS, stream=None):
    call("bbh_linear_residual_layernorm", _ptr(A), _ptr(B), _ptr(bias), _ptr(residual),
         _ptr(gamma), _ptr(beta), _ptr(y), M, HIDDEN, K, ctypes.c_float(eps), _stream(stream))
    return y


def launch_layernorm(x, gamma, beta, y, M, D, eps=LAYER_NORM_EPS, residual=None, stream=None):
    call("bbh_layernorm", _ptr(x), _ptr(gamma), _ptr(beta), _ptr(y), M, D, ctypes.c_float(eps),
         _ptr(residual), _stream(stream))
    return y


def launch_embedding(ids, types, word, pos, typ, out, seq, hidden, batch=1, stream=None):
    call("bbh_embedding", _ptr(ids), _ptr(types), _ptr(word), _ptr(pos), _ptr(typ), _ptr(out), seq,
         hidden, batch, _stream(stream))
    return out


def launch_embedding_layernorm(ids, types, word, pos, typ, gamma, beta, out, seq, batch=1,
                               eps=LAYER_NORM_EPS, stream=None):
    call("bbh_embedding_layernorm", _ptr(ids), _ptr(types), _ptr(word), _ptr(pos), _ptr(typ),
         _ptr(gamma), _ptr(beta), _ptr(out), seq, HIDDEN, batch, ctypes.c_float(eps), _stream(stream))
    return out


def launch_attention(qkv, mask, merged, batch, seq, heads=NUM_HEADS, head_dim=HEAD_DIM,
                     scale=None, stream=None):
    scale = 1.0 / np.sqrt(head_dim) if scale is None else scale
    call("bbh_attention", _ptr(qkv), _ptr(mask), _ptr(merged), batch, heads, seq, head_dim,
         ctypes.c_float(scale), _stream(stream))
    return merged


def launch_attention_scores(qkv, scores, batch, heads, seq, head_dim, qkv_stride, q_off, k_off,
                            scale, stream=None):
    call("bbh_attention_scores", _ptr(qkv), _ptr(scores), batch, heads, seq, head_dim, qkv_stride,
         q_off, k_off, ctypes.c_float(scale), _stream(stream))
    return scores


def launch_softmax(x, M, N, mask=None, mask_stride=0, stream=None):
    call("bbh_softmax", _ptr(x), M, N, _ptr(mask), mask_stride, _stream(stream))
    return x


def launch_attention_context(probs, qkv, merged, batch, heads, seq, head_dim, qkv_stride, v_off,
                             stream=None):
    call("bbh_attention_context", _ptr(probs), _ptr(qkv), _ptr(merged), batch, heads, seq, head_dim,
         qkv_stride, v_off, _stream(stream))
    return merged


def launch_mean_pool(hidden, mask, out, seq, dim, batch=1, stream=None):
    call("bbh_mean_pool", _ptr(hidden), _ptr(mask), _ptr(out), seq, dim, batch, _stream(stream))
    return out


def launch_l2_normalize(x, n, batch=1, stream=None):
    call("bbh_l2_normalize", _ptr(x), n, batch, _stream(stream))
    return x


def launch_gelu(x, n, stream=None):
    call("bbh_gelu", _ptr(x), n, _stream(stream))
    return x


def launch_pool_normalize(hidden, mask, out, seq, batch=1, stream=None):
    call("bbh_pool_normalize", _ptr(hidden), _ptr(mask), _ptr(out), seq, HIDDEN, batch,
         _stream(stream))
    return out


class Tokenizer:
    """The uncased BERT WordPiece tokenizer (bbh_tokenizer_load / bbh_tokenize):
    texts -> host int32 (n, seq) ids, types, mask, as
    BertTokenizerFast(..., padding="max_length", truncation=True) gives."""

    def __init__(self, vocab_path: str, lowercase: bool = True):
        self.handle = ctypes.c_void_p()
        call("bbh_tokenizer_load", vocab_path.encode(), int(lowercase), ctypes.byref(self.handle))

    @property
    def vocab_size(self) -> int:
        return lib().bbh_tokenizer_vocab_size(self.handle)

    def __call__(self, texts, seq: int = 128):
        n = len(texts)
        arr = (ctypes.c_char_p * max(n, 1))(*[t.encode("utf-8") for t in texts])
        ids, types, mask = (np.zeros((n, seq), np.int32) for _ in range(3))
        lengths = np.zeros(n, np.int32)
        p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
        call("bbh_tokenize", self.handle, arr, n, seq, p(ids), p(types), p(mask), p(lengths))
        return ids, types, mask, lengths

    def close(self):
        if self.handle:
            call("bbh_tokenizer_free", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def gemm_tile_name(tile: int) -> str:
    """Template argument of the GEMM kernel symbol for a tile id."""
    return capi.lib().bbh_gemm_tile_name(tile).decode()


BBHError = capi.BBHError
