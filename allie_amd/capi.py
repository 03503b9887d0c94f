"""ctypes binding of ``liballie_amd.so`` (the C ABI in include/allie_amd.h).

The library is built in-tree by ``allie_amd/build.py``.  There is no fallback:
if it is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liballie_amd.so")

ALLIE_OK = 0
MODE_FP32, MODE_BF16, MODE_FP8W = 0, 1, 2
MODE_IDS = {"float32": MODE_FP32, "bfloat16": MODE_BF16, "fp8w": MODE_FP8W}

W_WTE, W_WPE, W_CTRL, W_LNF_G, W_LNF_B, W_VALUE_W, W_VALUE_B, W_TIME_W, W_TIME_B = range(9)
(W_LN1_G, W_LN1_B, W_QKV_W, W_QKV_B, W_O_W, W_O_B, W_LN2_G, W_LN2_B, W_FC_W, W_FC_B, W_PR_W,
 W_PR_B) = range(16, 28)

EPI_STORE, EPI_GELU, EPI_RESID = 0, 1, 2
PROBE_QKV, PROBE_PROJ, PROBE_FC, PROBE_FC2, PROBE_ATTN, PROBE_DECODE = range(6)
WT_BF16, WT_F32, WT_FP8 = 0, 1, 2


class AllieConfig(C.Structure):
    _fields_ = [
        ("n_layer", C.c_int32), ("d_model", C.c_int32), ("n_head", C.c_int32),
        ("vocab_size", C.c_int32), ("n_positions", C.c_int32), ("max_length", C.c_int32),
        ("eps", C.c_float), ("mode", C.c_int32),
    ]


class AllieOutputs(C.Structure):
    _fields_ = [
        ("logits", C.c_void_p), ("value", C.c_void_p), ("time", C.c_void_p),
        ("top1", C.c_void_p), ("max_logit", C.c_void_p), ("lse", C.c_void_p),
        ("logits_raw", C.c_void_p),
    ]


# (name, restype, argtypes)
_SIGS = [
    ("allie_last_error", C.c_char_p, []),
    ("allie_abi_version", C.c_int, []),
    ("allie_model_create", C.c_int, [C.POINTER(AllieConfig), C.POINTER(C.c_void_p)]),
    ("allie_model_destroy", None, [C.c_void_p]),
    ("allie_model_set_weight", C.c_int,
     [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p]),
    ("allie_model_set_weight_fp8", C.c_int,
     [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p]),
    ("allie_model_finalize", C.c_int, [C.c_void_p]),
    ("allie_model_set_split_tokens", C.c_int, [C.c_void_p, C.c_int64, C.c_int64]),
    ("allie_model_set_tree_heads", C.c_int, [C.c_void_p, C.c_int]),
    ("allie_pack_ragged", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
      C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
      C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]),
    ("allie_prefill_workspace_bytes", C.c_size_t, [C.c_void_p, C.c_int, C.c_int]),
    ("allie_kv_block_bytes", C.c_size_t, [C.c_void_p]),
    ("allie_prefill", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_float, C.c_void_p, C.c_int,
      C.POINTER(AllieOutputs), C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p,
      C.c_void_p, C.c_size_t, C.c_void_p]),
    ("allie_extend_workspace_bytes", C.c_size_t, [C.c_void_p, C.c_int, C.c_int]),
    ("allie_extend", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,            # model, ids, pos, n_tok
      C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int,   # groups, prefix_len/blocks, max_blocks
      C.c_void_p, C.c_void_p, C.c_int,                        # extra_slot, n_extra, max_extra
      C.c_float, C.c_void_p, C.c_int, C.POINTER(AllieOutputs),  # temperature, legal, words, out
      C.c_void_p, C.c_int, C.c_void_p,                        # kv_pool, pool blocks, status
      C.c_void_p, C.c_size_t, C.c_void_p]),                   # workspace, bytes, stream
    ("allie_extend_noalloc", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,            # model, ids, pos, n_tok
      C.c_void_p, C.c_void_p, C.c_int,                        # group starts (host, device), n_groups
      C.c_void_p, C.c_void_p, C.c_int,                        # prefix_len/blocks, max_blocks
      C.c_void_p, C.c_void_p, C.c_int,                        # extra_slot, n_extra, max_extra
      C.c_float, C.c_void_p, C.c_int, C.POINTER(AllieOutputs),  # temperature, legal, words, out
      C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]),          # kv_pool, pool blocks, status, stream
    ("allie_probe_begin", C.c_int, [C.c_int, C.c_int]),
    ("allie_probe_span", C.c_int, [C.POINTER(C.c_float)]),
    ("allie_probe_end", C.c_int, [C.POINTER(C.c_float), C.POINTER(C.c_int)]),
    ("allie_gemm", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
      C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    ("allie_gemm_splitk", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
      C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_size_t, C.c_void_p]),
    ("allie_gemm_split_factor", C.c_int, [C.c_int, C.c_int, C.c_int]),
    ("allie_attn_varlen", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
      C.c_float, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]),
    ("allie_layernorm", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_float,
      C.c_void_p, C.c_int, C.c_void_p]),
]

EXPORTED = [name for name, _, _ in _SIGS]

_lib = None


class AllieError(RuntimeError):
    pass


def lib() -> C.CDLL:
    """Load the engine library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise AllieError(
                f"{LIB_PATH} is missing: build it with `python -m allie_amd.build` "
                "(there is no CPU fallback)"
            )
        L = C.CDLL(LIB_PATH)
        for name, res, args in _SIGS:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != ALLIE_OK:
        msg = lib().allie_last_error().decode(errors="replace")
        raise AllieError(f"{what or 'allie call'} failed ({rc}): {msg}")


def stream_ptr(stream=None):
    """hipStream_t of a torch stream (default: the current stream)."""
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def ptr(t) -> C.c_void_p:
    """Device (or host) address of a torch tensor / numpy array, or NULL."""
    if t is None:
        return C.c_void_p(0)
    if hasattr(t, "data_ptr"):
        return C.c_void_p(t.data_ptr())
    return C.c_void_p(t.ctypes.data)
