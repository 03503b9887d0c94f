"""ctypes front of ``pack_ref.c`` (the packing oracle) -- TEST INFRASTRUCTURE."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None
PAD_ID = 1996


def build() -> str:
    subprocess.check_call(["make", "-s", "-C", _HERE])
    return _LIB


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        _lib = ctypes.CDLL(_LIB)
        _lib.oracle_pack.restype = ctypes.c_int
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def pack(words: np.ndarray, lens: np.ndarray, max_len: int = 512, block: int = 16,
         first_block: int = 0, max_blocks: int | None = None, pad_id: int = PAD_ID) -> dict:
    """Packed layout of ``words``/``lens``; ``out["status"]`` has the engine's
    status bits (1 empty game, 4 table too small, 8 PAD id inside a game)."""
    lib = _load()
    words = np.ascontiguousarray(words, dtype=np.uint32)
    lens = np.ascontiguousarray(lens, dtype=np.int32)
    B = len(lens)
    n = np.clip(lens, 0, max_len)
    T = int(n.sum())
    if max_blocks is None:
        max_blocks = (max_len + block - 1) // block
    out = {
        "cu_seqlens": np.zeros(B + 1, np.int32),
        "ids": np.zeros(T, np.int32),
        "pos": np.zeros(T, np.int32),
        "seq_of": np.zeros(T, np.int32),
        "last_idx": np.zeros(B, np.int32),
        "blk_off": np.zeros(B + 1, np.int32),
        "block_table": np.zeros((B, max_blocks), np.int32),
        "slot": np.zeros(T, np.int32),
    }
    out["status"] = lib.oracle_pack(
        _p(words), _p(lens), ctypes.c_int(B), ctypes.c_int(max_len), ctypes.c_int(block),
        ctypes.c_int(first_block), ctypes.c_int(max_blocks), ctypes.c_int(pad_id),
        _p(out["cu_seqlens"]), _p(out["ids"]), _p(out["pos"]), _p(out["seq_of"]),
        _p(out["last_idx"]), _p(out["blk_off"]), _p(out["block_table"]), _p(out["slot"]))
    return out
