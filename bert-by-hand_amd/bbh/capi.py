"""ctypes binding of include/bbh.h (libbbh.so, built in-tree by the Makefile).

There is deliberately no fallback: if libbbh.so is missing or fails to load,
importing the product path raises.  Nothing here computes anything on the CPU.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libbbh.so")

c_int, c_float, c_size_t, c_void_p, c_char_p = (ctypes.c_int, ctypes.c_float, ctypes.c_size_t,
                                               ctypes.c_void_p, ctypes.c_char_p)
c_i32p = ctypes.POINTER(ctypes.c_int32)


class AttnWeights(ctypes.Structure):
    """bbh_attn_weights: device pointers of one layer's attention tensors."""
    _fields_ = [(n, c_void_p) for n in ("qkv_w", "qkv_b", "o_w", "o_b", "ln_w", "ln_b")]


class FfnWeights(ctypes.Structure):
    """bbh_ffn_weights: device pointers of one layer's feed-forward tensors."""
    _fields_ = [(n, c_void_p) for n in ("inter_w", "inter_b", "out_w", "out_b", "ln_w", "ln_b")]


class LaunchTime(ctypes.Structure):
    """bbh_launch_time: one timed op launch of a pool."""
    _fields_ = [("op", c_int), ("tile", c_int), ("fused_ln", c_int), ("m", c_int), ("n", c_int),
                ("k", c_int), ("ms", c_float)]


_AWp, _FWp = ctypes.POINTER(AttnWeights), ctypes.POINTER(FfnWeights)

# name -> (restype, argtypes); every symbol declared in include/bbh.h.
SIGNATURES = {
    "bbh_status_string": (c_char_p, [c_int]),
    "bbh_last_error": (c_char_p, []),
    "bbh_version": (c_char_p, []),
    "bbh_param_count": (c_int, []),
    "bbh_param_name": (c_char_p, [c_int]),
    "bbh_param_numel": (c_size_t, [c_int]),
    "bbh_model_load_dir": (c_int, [c_char_p, ctypes.POINTER(c_void_p)]),
    "bbh_model_load_safetensors": (c_int, [c_char_p, ctypes.POINTER(c_void_p)]),
    "bbh_model_from_host": (c_int, [ctypes.POINTER(c_void_p), c_int, ctypes.POINTER(c_void_p)]),
    "bbh_model_free": (c_int, [c_void_p]),
    "bbh_model_device_bytes": (c_size_t, [c_void_p]),
    "bbh_workspace_create": (c_int, [c_int, c_int, ctypes.POINTER(c_void_p)]),
    "bbh_workspace_free": (c_int, [c_void_p]),
    "bbh_workspace_bytes": (c_size_t, [c_int, c_int]),
    "bbh_workspace_hidden": (c_void_p, [c_void_p]),
    "bbh_embed": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                          c_void_p]),
    "bbh_embed_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                  c_void_p]),
    "bbh_encode": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                           c_void_p]),
    "bbh_embed_graph_create": (c_int, [c_void_p] * 6 + [c_int, c_int, ctypes.POINTER(c_void_p)]),
    "bbh_graph_launch": (c_int, [c_void_p, c_void_p]),
    "bbh_graph_free": (c_int, [c_void_p]),
    "bbh_pool_create": (c_int, [c_int, c_int, c_int, ctypes.POINTER(c_void_p)]),
    "bbh_pool_free": (c_int, [c_void_p]),
    "bbh_embed_batches": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "bbh_embed_each": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                               c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "bbh_embed_packed": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                 c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "bbh_pool_busy": (c_int, [c_void_p, ctypes.POINTER(c_int)]),
    "bbh_pool_fail_at": (c_int, [c_void_p, c_int]),
    "bbh_pool_timing": (c_int, [c_void_p, c_int]),
    "bbh_pool_timing_read": (c_int, [c_void_p, ctypes.POINTER(LaunchTime), c_int,
                                     ctypes.POINTER(c_int)]),
    "bbh_gemm_tile_name": (c_char_p, [c_int]),
    "bbh_model_layer": (c_int, [c_void_p, c_int, _AWp, _FWp]),
    "bbh_attention_block_w": (c_int, [c_void_p, c_void_p, _AWp, c_void_p, c_void_p, c_int, c_int,
                                      c_void_p]),
    "bbh_ffn_block_w": (c_int, [c_void_p, c_void_p, _FWp, c_void_p, c_int, c_int, c_void_p]),
    "bbh_encoder_layer_w": (c_int, [c_void_p, c_void_p, _AWp, _FWp, c_void_p, c_void_p, c_int, c_int,
                                    c_void_p]),
    "bbh_attention_block": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int,
                                    c_int, c_void_p]),
    "bbh_ffn_block": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "bbh_encoder_layer": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int,
                                  c_int, c_void_p]),
    "bbh_linear": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_int,
                           c_void_p]),
    "bbh_linear_residual_layernorm": (c_int, [c_void_p] * 7 + [c_int, c_int, c_int, c_float,
                                                                c_void_p]),
    "bbh_layernorm": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_float,
                              c_void_p, c_void_p]),
    "bbh_embedding": (c_int, [c_void_p] * 6 + [c_int, c_int, c_int, c_void_p]),
    "bbh_embedding_layernorm": (c_int, [c_void_p] * 8 + [c_int, c_int, c_int, c_float, c_void_p]),
    "bbh_attention": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_float,
                              c_void_p]),
    "bbh_attention_scores": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
                                     c_int, c_float, c_void_p]),
    "bbh_softmax": (c_int, [c_void_p, c_int, c_int, c_void_p, c_int, c_void_p]),
    "bbh_attention_context": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                      c_int, c_int, c_void_p]),
    "bbh_mean_pool": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "bbh_l2_normalize": (c_int, [c_void_p, c_int, c_int, c_void_p]),
    "bbh_pool_normalize": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "bbh_gelu": (c_int, [c_void_p, c_int, c_void_p]),
    "bbh_tokenizer_load": (c_int, [c_char_p, c_int, ctypes.POINTER(c_void_p)]),
    "bbh_tokenizer_free": (c_int, [c_void_p]),
    "bbh_tokenizer_vocab_size": (c_int, [c_void_p]),
    "bbh_tokenize": (c_int, [c_void_p, ctypes.POINTER(c_char_p), c_int, c_int, c_void_p, c_void_p,
                             c_void_p, c_void_p]),
}

STATUS = {
    0: "BBH_OK", 1: "BBH_ERR_INVALID_ARG", 2: "BBH_ERR_SEQ_ALIGN", 3: "BBH_ERR_CAPACITY",
    4: "BBH_ERR_IO", 5: "BBH_ERR_HIP", 6: "BBH_ERR_OOM", 7: "BBH_ERR_UNSUPPORTED",
}


class BBHError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status
        self.name = STATUS.get(status, str(status))


_lib = None


def lib():
    """The loaded libbbh.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `make -C bert-by-hand_amd` "
                               "or __graft_entry__.build()")
        # torch first: its HIP runtime (linked as libamdhip64.so, soname
        # libamdhip64.so.7) then also serves this library's libamdhip64.so.7
        # dependency.  Loaded the other way round, the process ends up with
        # two HIP runtimes and torch finds no GPU.
        import torch  # noqa: F401

        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int):
    if status != 0:
        raise BBHError(status, lib().bbh_last_error().decode())


def call(name: str, *args):
    """Call an entry point and raise BBHError on a non-OK status."""
    check(getattr(lib(), name)(*args))
