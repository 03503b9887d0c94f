"""Native host chess rules (``liballie_chess.so``, csrc/chess.cpp) for Game.

The search asks, per node, for the position after one more move, its legal
moves in python-chess order and whether the game is over (the reference:
src/modeling/data.py:51-61 and src/evaluation/decode.py:345-353, via
python-chess).  ``NativeBoard`` answers these in C++ with the methods
``Game`` and the strategies use (``push_uci``, ``legal_uci``, ``outcome``,
``is_check``, ``is_game_over``); the tests compare it, move list for move
list, with a Python restatement of the rules (oracle/movegen.py).  The
library is built by ``allie_amd.build`` (``build()``), or on first use when
it is missing or older than its sources; there is no switch to another
implementation.
"""
from __future__ import annotations

import ctypes as C
import glob
import os
import threading
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liballie_chess.so")
_lib = None
_lock = threading.Lock()

TERMINATIONS = {1: "checkmate", 2: "insufficient_material", 3: "stalemate", 4: "seventyfive_moves",
                5: "fivefold_repetition"}
_WINNER = {0: None, 1: True, 2: False}


def _stale() -> bool:
    """The library is missing or older than one of its sources."""
    if not os.path.exists(LIB_PATH):
        return True
    built = os.path.getmtime(LIB_PATH)
    srcs = glob.glob(os.path.join(_HERE, "csrc", "*.cpp")) + [os.path.join(_HERE, "..", "include", "allie_chess.h")]
    return any(os.path.exists(f) and os.path.getmtime(f) > built for f in srcs)


def lib():
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if _stale():
                    # host C++ only: built here on first use, or again when a
                    # source is newer than the library (g++, about two
                    # seconds); a failed build raises
                    from .build import build_chess

                    build_chess()
                L = C.CDLL(LIB_PATH)
                vp = C.c_void_p
                for name, res, args in (
                    ("allie_chess_start", vp, []),
                    ("allie_chess_from_fen", vp, [C.c_char_p]),
                    ("allie_chess_free", None, [vp]),
                    ("allie_chess_push_uci", vp, [vp, C.c_char_p]),
                    ("allie_chess_legal_uci", C.c_int, [vp, C.c_char_p, C.c_int]),
                    ("allie_chess_outcome", C.c_int, [vp]),
                    ("allie_chess_is_check", C.c_int, [vp]),
                    ("allie_chess_white_to_move", C.c_int, [vp]),
                    ("allie_chess_perft", C.c_longlong, [vp, C.c_int]),
                ):
                    f = getattr(L, name)
                    f.restype = res
                    f.argtypes = args
                _lib = L
    return _lib


class NativeBoard:
    """An immutable position (with its repetition history) in C++."""

    __slots__ = ("_h", "_lib", "_legal", "__weakref__")

    def __init__(self, handle: int):
        if not handle:
            raise MemoryError("allie_chess: position allocation failed")
        self._lib = lib()
        self._h = C.c_void_p(handle)
        self._legal: Optional[list] = None

    @classmethod
    def start(cls) -> "NativeBoard":
        return cls(lib().allie_chess_start())

    @classmethod
    def from_fen(cls, fen: str) -> "NativeBoard":
        h = lib().allie_chess_from_fen(fen.encode())
        if not h:
            raise ValueError(f"bad FEN {fen!r}")
        return cls(h)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.allie_chess_free(h)
            self._h = None

    def push_uci(self, uci: str) -> "NativeBoard":
        h = self._lib.allie_chess_push_uci(self._h, uci.encode())
        if not h:
            raise ValueError(f"illegal move {uci}")
        return NativeBoard(h)

    def legal_uci(self) -> list:
        if self._legal is None:
            buf = C.create_string_buffer(2048)
            n = self._lib.allie_chess_legal_uci(self._h, buf, 2048)
            if n < 0:
                raise RuntimeError("allie_chess_legal_uci: buffer too small")
            self._legal = buf.value.decode().split() if n else []
        return list(self._legal)

    def outcome(self) -> Optional[tuple]:
        """None while the game goes on, else (termination, winner) with
        winner True (white), False (black) or None (draw)."""
        code = self._lib.allie_chess_outcome(self._h)
        if code == 0:
            return None
        return TERMINATIONS[code >> 2], _WINNER[code & 3]

    def is_game_over(self) -> bool:
        return self.outcome() is not None

    def is_check(self) -> bool:
        return bool(self._lib.allie_chess_is_check(self._h))

    @property
    def white(self) -> bool:
        return bool(self._lib.allie_chess_white_to_move(self._h))

    def perft(self, depth: int) -> int:
        return int(self._lib.allie_chess_perft(self._h, depth))


def board_after(moves: list) -> NativeBoard:
    b = NativeBoard.start()
    for m in moves:
        b = b.push_uci(m)
    return b
