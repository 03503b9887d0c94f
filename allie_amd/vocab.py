"""Token table of the Allie chess language model.

Token ids follow the reference tokenizer (src/modeling/data.py:187-213):

* 0..1967      UCI move strings, in the order of ``CHESS_MOVES``
                (src/modeling/moves.py:3-1972, ``NUM_CHESS_MOVES`` at :1974)
* 1968..1991   blitz time-control tokens (data.py:117-142)
* 1992         ``<RESIGNED-OR-CHECKMATED>`` (data.py:144)
* 1993..1996   ``<BOS> <EOS> <UNK> <PAD>`` (data.py:197-198, default names :179-183)

An Elo rating ``e`` is carried as the out-of-vocabulary id ``e + 1997``
(data.py:228).

The move list is *generated* here rather than stored.  The reference list
(taken from a public gist, moves.py:1) enumerates, square by square with the
file as the outer loop and the rank as the inner loop (a1, a2, ..., a8, b1, ...):

1. every queen-line destination (rook + bishop rays) of the square,
2. then, in a second pass over the squares, every knight destination,
3. then, file by file, the pawn promotions: from rank 7 to rank 8 and from
   rank 2 to rank 1, capture to the right, capture to the left, straight push,
   each with the pieces ``q r b n``.

Within a square, destinations are ordered by rank descending and then by file
descending.  ``tests/test_vocab.py`` checks the generated list against a
SHA-256 of the reference list committed under ``tests/golden/``.
"""
from __future__ import annotations

import hashlib

FILES = "abcdefgh"
RANKS = "12345678"


def _square(f: int, r: int) -> str:
    return FILES[f] + RANKS[r]


def _ordered(dests: set[tuple[int, int]]) -> list[tuple[int, int]]:
    # rank descending, then file descending
    return sorted(dests, key=lambda fr: (-fr[1], -fr[0]))


def _queen_dests(f: int, r: int) -> set[tuple[int, int]]:
    out = set()
    for df, dr in ((1, 0), (-1, 0), (0, 1), (0, -1), (1, 1), (1, -1), (-1, 1), (-1, -1)):
        nf, nr = f + df, r + dr
        while 0 <= nf < 8 and 0 <= nr < 8:
            out.add((nf, nr))
            nf += df
            nr += dr
    return out


def _knight_dests(f: int, r: int) -> set[tuple[int, int]]:
    out = set()
    for df, dr in ((1, 2), (2, 1), (2, -1), (1, -2), (-1, -2), (-2, -1), (-2, 1), (-1, 2)):
        nf, nr = f + df, r + dr
        if 0 <= nf < 8 and 0 <= nr < 8:
            out.add((nf, nr))
    return out


def generate_moves() -> list[str]:
    moves: list[str] = []
    for gen in (_queen_dests, _knight_dests):
        for f in range(8):
            for r in range(8):
                src = _square(f, r)
                for nf, nr in _ordered(gen(f, r)):
                    moves.append(src + _square(nf, nr))
    for f in range(8):
        for src_r, dst_r in ((6, 7), (1, 0)):
            for df in (1, -1, 0):
                nf = f + df
                if not 0 <= nf < 8:
                    continue
                for piece in "qrbn":
                    moves.append(_square(f, src_r) + _square(nf, dst_r) + piece)
    return moves


CHESS_MOVES: list[str] = generate_moves()
NUM_CHESS_MOVES = len(CHESS_MOVES)  # 1968

BLITZ_TIME_CONTROLS_TOKENS = [
    "180+0", "300+0", "180+2", "300+3", "300+2", "420+0", "240+0", "180+1",
    "180+3", "300+1", "360+0", "300+4", "420+1", "240+2", "180+5", "120+2",
    "120+3", "240+3", "240+1", "360+2", "60+3", "60+5", "240+4", "240+5",
]
NORMAL_TERMINATION_TOKEN = "<RESIGNED-OR-CHECKMATED>"
SPECIAL_TOKENS = ["<BOS>", "<EOS>", "<UNK>", "<PAD>"]

TOKENS: list[str] = CHESS_MOVES + BLITZ_TIME_CONTROLS_TOKENS + [NORMAL_TERMINATION_TOKEN] + SPECIAL_TOKENS
VOCAB_SIZE = len(TOKENS)  # 1997
TOKEN_TO_ID = {t: i for i, t in enumerate(TOKENS)}

RESIGN_ID = TOKEN_TO_ID[NORMAL_TERMINATION_TOKEN]  # 1992
BOS_ID = TOKEN_TO_ID["<BOS>"]  # 1993
EOS_ID = TOKEN_TO_ID["<EOS>"]  # 1994
UNK_ID = TOKEN_TO_ID["<UNK>"]  # 1995
PAD_ID = TOKEN_TO_ID["<PAD>"]  # 1996

# word format of the tokenizer (data.py:246-268, unpacked at data.py:310-320)
ID_MASK = 0x3FFF
OUTCOME_SHIFT = 14
TIME_SHIFT = 16

ELO_MIN, ELO_MAX = 500, 3000  # model.py:26

# empirical move-time statistics (data.py:156-157)
TIME_MEAN = 4.64001
TIME_STDEV = 6.16533

MAX_LENGTH = 512  # pretrain_config/medium.yaml:18


def moves_sha256(moves: list[str] | None = None) -> str:
    moves = CHESS_MOVES if moves is None else moves
    return hashlib.sha256("\n".join(moves).encode()).hexdigest()
