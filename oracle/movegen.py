"""Python restatement of the rules of chess -- TEST INFRASTRUCTURE ONLY.

Only tests import it: it is the comparator of the native rules library
(``allie_amd.rules``, csrc/chess.cpp) that ``Game`` uses.

The reference gets these from python-chess (``Game.board`` replays the game
with ``chess.Board().push_uci``, ``Game.legal_moves`` lists
``board.legal_moves`` as UCI, src/modeling/data.py:51-61; ``MCTS`` asks
``board.is_game_over()`` / ``board.outcome()``, src/evaluation/decode.py:
345-353).  python-chess is not installed in this image, so this module
restates the rules of chess for games that start from the initial position.
The native library must give the same moves in the same order; the tests
compare them move list for move list (tests/test_rules.py).

Move ORDER matters to the reference: ``decode_full`` breaks argmax ties by
the order of ``legal_moves`` (decode.py:112) and MCTS expands children in
that order (decode.py:375-377).  The order here follows python-chess's
published generation order (python-chess 1.x ``generate_legal_moves``):
  * not in check: pieces other than pawns by from-square descending (a1 = 0
    ... h8 = 63), each with its targets by square descending; then castling,
    king side before queen side; then pawn captures by from-square
    descending, targets descending; then single pushes and then double
    pushes, by target square descending; then en passant captures by
    capturer square descending; promotions come as q, r, b, n;
  * in check: king moves first (targets descending), then, against a single
    checker, the moves of the other pieces (in the order above) that capture
    it or block its line, then an en passant capture of a checking pawn.
That order cannot be pinned without importing python-chess ("parity
unpinned"); legality itself is pinned by perft known answers in
tests/test_movegen.py.

Game over (python-chess ``is_game_over(claim_draw=False)`` / ``outcome()``):
checkmate (the side to move loses), insufficient material, stalemate, the
seventy-five-move rule (150 half-moves without capture or pawn move, unless
mate) and fivefold repetition are terminal; all but checkmate are draws.
"""
from __future__ import annotations

from typing import Optional

EMPTY, PAWN, KNIGHT, BISHOP, ROOK, QUEEN, KING = 0, 1, 2, 3, 4, 5, 6
BLACK_BIT = 8
PROMO = "qrbn"
PROMO_TYPE = {"q": QUEEN, "r": ROOK, "b": BISHOP, "n": KNIGHT}
FILES = "abcdefgh"


def sq_name(s: int) -> str:
    return FILES[s & 7] + str((s >> 3) + 1)


def parse_sq(t: str) -> int:
    return FILES.index(t[0]) + 8 * (int(t[1]) - 1)


def _steps(deltas):
    out = []
    for s in range(64):
        f, r = s & 7, s >> 3
        out.append([(r + dr) * 8 + f + df for df, dr in deltas if 0 <= f + df < 8 and 0 <= r + dr < 8])
    return out


_KNIGHT = _steps([(1, 2), (2, 1), (2, -1), (1, -2), (-1, -2), (-2, -1), (-2, 1), (-1, 2)])
_KING = _steps([(1, 0), (1, 1), (0, 1), (-1, 1), (-1, 0), (-1, -1), (0, -1), (1, -1)])
_ORTH = [(1, 0), (-1, 0), (0, 1), (0, -1)]
_DIAG = [(1, 1), (1, -1), (-1, 1), (-1, -1)]


def _rays(dirs):
    out = []
    for s in range(64):
        f, r = s & 7, s >> 3
        rs = []
        for df, dr in dirs:
            ray, nf, nr = [], f + df, r + dr
            while 0 <= nf < 8 and 0 <= nr < 8:
                ray.append(nr * 8 + nf)
                nf += df
                nr += dr
            rs.append(ray)
        out.append(rs)
    return out


_ORTH_RAYS = _rays(_ORTH)
_DIAG_RAYS = _rays(_DIAG)
_SQ_COLOR = [((s & 7) + (s >> 3)) & 1 for s in range(64)]  # 0 dark (a1), 1 light


class Board:
    """Mailbox board: squares 0 (a1) .. 63 (h8); piece = type | 8 for black."""

    __slots__ = ("sq", "white", "castling", "ep", "halfmove", "keys")

    def __init__(self):
        back = [ROOK, KNIGHT, BISHOP, QUEEN, KING, BISHOP, KNIGHT, ROOK]
        self.sq = [EMPTY] * 64
        for f in range(8):
            self.sq[f] = back[f]
            self.sq[8 + f] = PAWN
            self.sq[48 + f] = PAWN | BLACK_BIT
            self.sq[56 + f] = back[f] | BLACK_BIT
        self.white = True
        self.castling = {"K", "Q", "k", "q"}
        self.ep: Optional[int] = None
        self.halfmove = 0
        self.keys: list = []
        self.keys.append(self._key())

    # ---------------------------------------------------------------- setup
    @classmethod
    def from_fen(cls, fen: str) -> "Board":
        """Test helper: a position from a FEN string (no history)."""
        b = cls.__new__(cls)
        parts = fen.split()
        b.sq = [EMPTY] * 64
        codes = {"p": PAWN, "n": KNIGHT, "b": BISHOP, "r": ROOK, "q": QUEEN, "k": KING}
        for ri, row in enumerate(parts[0].split("/")):
            f = 0
            for ch in row:
                if ch.isdigit():
                    f += int(ch)
                else:
                    p = codes[ch.lower()] | (0 if ch.isupper() else BLACK_BIT)
                    b.sq[(7 - ri) * 8 + f] = p
                    f += 1
        b.white = parts[1] == "w"
        b.castling = set(parts[2]) - {"-"} if len(parts) > 2 else set()
        b.ep = parse_sq(parts[3]) if len(parts) > 3 and parts[3] != "-" else None
        b.halfmove = int(parts[4]) if len(parts) > 4 else 0
        b.keys = [b._key()]
        return b

    def copy(self) -> "Board":
        b = Board.__new__(Board)
        b.sq = self.sq[:]
        b.white = self.white
        b.castling = set(self.castling)
        b.ep = self.ep
        b.halfmove = self.halfmove
        b.keys = self.keys[:]
        return b

    # ------------------------------------------------------------- attacks
    def _ours(self, p: int) -> bool:
        return p != EMPTY and ((p & BLACK_BIT) == 0) == self.white

    def attacked_by(self, s: int, by_white: bool) -> bool:
        """Is square s attacked by the given side (pieces as they stand)?"""
        c = 0 if by_white else BLACK_BIT
        sq = self.sq
        for t in _KNIGHT[s]:
            if sq[t] == KNIGHT | c:
                return True
        for t in _KING[s]:
            if sq[t] == KING | c:
                return True
        for rays, a, b_ in ((_ORTH_RAYS[s], ROOK, QUEEN), (_DIAG_RAYS[s], BISHOP, QUEEN)):
            for ray in rays:
                for t in ray:
                    p = sq[t]
                    if p != EMPTY:
                        if p == a | c or p == b_ | c:
                            return True
                        break
        f, r = s & 7, s >> 3
        pr = r - 1 if by_white else r + 1  # rank a pawn of that side attacks s from
        if 0 <= pr < 8:
            for df in (-1, 1):
                if 0 <= f + df < 8 and sq[pr * 8 + f + df] == PAWN | c:
                    return True
        return False

    def king_square(self, white: bool) -> int:
        k = KING | (0 if white else BLACK_BIT)
        return self.sq.index(k)

    def is_check(self) -> bool:
        return self.attacked_by(self.king_square(self.white), not self.white)

    def _checkers(self) -> list:
        """Squares of the opposing pieces giving check."""
        k = self.king_square(self.white)
        c = BLACK_BIT if self.white else 0
        sq = self.sq
        out = [t for t in _KNIGHT[k] if sq[t] == KNIGHT | c]
        for rays, a in ((_ORTH_RAYS[k], ROOK), (_DIAG_RAYS[k], BISHOP)):
            for ray in rays:
                for t in ray:
                    p = sq[t]
                    if p != EMPTY:
                        if p == a | c or p == QUEEN | c:
                            out.append(t)
                        break
        f, r = k & 7, k >> 3
        pr = r + 1 if self.white else r - 1
        if 0 <= pr < 8:
            for df in (-1, 1):
                if 0 <= f + df < 8 and sq[pr * 8 + f + df] == PAWN | c:
                    out.append(pr * 8 + f + df)
        return out

    # ------------------------------------------------- pseudo-legal moves
    def _piece_targets(self, s: int, t: int) -> list:
        sq = self.sq
        if t == KNIGHT:
            return _KNIGHT[s]
        if t == KING:
            return _KING[s]
        out = []
        rays = (_ORTH_RAYS[s] if t == ROOK else _DIAG_RAYS[s] if t == BISHOP else _ORTH_RAYS[s] + _DIAG_RAYS[s])
        for ray in rays:
            for u in ray:
                out.append(u)
                if sq[u] != EMPTY:
                    break
        return out

    def _pseudo(self, to_ok=None, kings=True) -> list:
        """Pseudo-legal moves (from, to, promo) in the generation order."""
        sq, white = self.sq, self.white
        moves = []
        for s in range(63, -1, -1):
            p = sq[s]
            if p == EMPTY or not self._ours(p) or (p & 7) == PAWN:
                continue
            if (p & 7) == KING and not kings:
                continue
            for u in sorted(self._piece_targets(s, p & 7), reverse=True):
                if not self._ours(sq[u]) and (to_ok is None or u in to_ok):
                    moves.append((s, u, None))
        if kings and to_ok is None:
            moves += self._castling()
        pawn = PAWN | (0 if white else BLACK_BIT)
        fwd = 8 if white else -8
        last = 7 if white else 0

        def add(s, u):
            if (u >> 3) == last:
                moves.extend((s, u, pc) for pc in PROMO)
            else:
                moves.append((s, u, None))

        for s in range(63, -1, -1):  # captures
            if sq[s] != pawn:
                continue
            f = s & 7
            tg = [s + fwd + df for df in (-1, 1) if 0 <= f + df < 8]
            for u in sorted(tg, reverse=True):
                if sq[u] != EMPTY and not self._ours(sq[u]) and (to_ok is None or u in to_ok):
                    add(s, u)
        singles = [s + fwd for s in range(64) if sq[s] == pawn and sq[s + fwd] == EMPTY]
        for u in sorted(singles, reverse=True):
            if to_ok is None or u in to_ok:
                add(u - fwd, u)
        start = 1 if white else 6
        doubles = [s + 2 * fwd for s in range(64)
                   if sq[s] == pawn and (s >> 3) == start and sq[s + fwd] == EMPTY and sq[s + 2 * fwd] == EMPTY]
        for u in sorted(doubles, reverse=True):
            if to_ok is None or u in to_ok:
                moves.append((u - 2 * fwd, u, None))
        if self.ep is not None and (to_ok is None or self.ep in to_ok):  # en passant (may block a check)
            moves += self._ep_moves()
        return moves

    def _ep_moves(self) -> list:
        if self.ep is None:
            return []
        pawn = PAWN | (0 if self.white else BLACK_BIT)
        e = self.ep
        f = e & 7
        r_from = (e >> 3) - 1 if self.white else (e >> 3) + 1
        cap = [r_from * 8 + f + df for df in (-1, 1) if 0 <= f + df < 8]
        return [(s, e, None) for s in sorted(cap, reverse=True) if self.sq[s] == pawn]

    def _castling(self) -> list:
        white = self.white
        rank = 0 if white else 56
        king = KING | (0 if white else BLACK_BIT)
        rook = ROOK | (0 if white else BLACK_BIT)
        if self.sq[rank + 4] != king:
            return []
        out = []
        for side, rook_sq, empty, safe, to in (
            ("K" if white else "k", rank + 7, (5, 6), (4, 5, 6), rank + 6),
            ("Q" if white else "q", rank + 0, (1, 2, 3), (4, 3, 2), rank + 2),
        ):
            if side not in self.castling or self.sq[rook_sq] != rook:
                continue
            if any(self.sq[rank + e] != EMPTY for e in empty):
                continue
            if any(self.attacked_by(rank + q, not white) for q in safe):
                continue
            out.append((rank + 4, to, None))
        return out

    # --------------------------------------------------------- legal moves
    def _leaves_king_safe(self, m) -> bool:
        b = self._make(m)
        return not b.attacked_by(b.king_square(self.white), not self.white)

    def legal_moves(self) -> list:
        """Legal moves as (from, to, promo) in the generation order."""
        if not self.is_check():
            return [m for m in self._pseudo() if self._leaves_king_safe(m)]
        k = self.king_square(self.white)
        checkers = self._checkers()
        moves = [(k, u, None) for u in sorted(_KING[k], reverse=True) if not self._ours(self.sq[u])]
        if len(checkers) == 1:
            c = checkers[0]
            target = {c} | set(_between(k, c))
            moves += self._pseudo(to_ok=target, kings=False)
            if self.ep is not None and self.ep not in target:
                last_double = self.ep + (-8 if self.white else 8)
                if last_double == c:
                    moves += self._ep_moves()
        return [m for m in moves if self._leaves_king_safe(m)]

    def legal_uci(self) -> list:
        return [sq_name(a) + sq_name(b) + (p or "") for a, b, p in self.legal_moves()]

    # -------------------------------------------------------------- moves
    def _make(self, m) -> "Board":
        """The position after move m (no history update)."""
        s, u, promo = m
        b = Board.__new__(Board)
        sq = self.sq[:]
        p = sq[s]
        t = p & 7
        cap = sq[u] != EMPTY
        sq[u] = p if promo is None else PROMO_TYPE[promo] | (p & BLACK_BIT)
        sq[s] = EMPTY
        if t == PAWN and u == self.ep:  # en passant: remove the passed pawn
            sq[u + (-8 if self.white else 8)] = EMPTY
            cap = True
        if t == KING and abs(u - s) == 2:  # castling: move the rook
            if u > s:
                sq[s + 1], sq[s + 3] = sq[s + 3], EMPTY
            else:
                sq[s - 1], sq[s - 4] = sq[s - 4], EMPTY
        b.sq = sq
        b.white = not self.white
        rights = set(self.castling)
        if t == KING:
            rights -= {"K", "Q"} if self.white else {"k", "q"}
        for corner, r in ((0, "Q"), (7, "K"), (56, "q"), (63, "k")):
            if s == corner or u == corner:
                rights.discard(r)
        b.castling = rights
        b.ep = (s + u) // 2 if t == PAWN and abs(u - s) == 16 else None
        b.halfmove = 0 if (t == PAWN or cap) else self.halfmove + 1
        b.keys = self.keys
        return b

    def push_uci(self, uci: str) -> "Board":
        """The position after a legal UCI move (raises for an illegal one);
        keeps the history of positions for repetition."""
        s, u = parse_sq(uci[:2]), parse_sq(uci[2:4])
        promo = uci[4] if len(uci) > 4 else None
        if (s, u, promo) not in self.legal_moves():
            raise ValueError(f"illegal move {uci}")
        b = self._make((s, u, promo))
        b.keys = self.keys + [b._key()]
        return b

    # ------------------------------------------------------------ outcome
    def _key(self):
        ep = self.ep if (self.ep is not None and any(self._leaves_king_safe(m) for m in self._ep_moves())) else None
        return (tuple(self.sq), self.white, frozenset(self.castling), ep)

    def _insufficient(self, white: bool) -> bool:
        c = 0 if white else BLACK_BIT
        ours = [s for s in range(64) if self.sq[s] != EMPTY and (self.sq[s] & BLACK_BIT) == c]
        theirs = [s for s in range(64) if self.sq[s] != EMPTY and (self.sq[s] & BLACK_BIT) != c]
        types = [self.sq[s] & 7 for s in ours]
        if any(t in (PAWN, ROOK, QUEEN) for t in types):
            return False
        if KNIGHT in types:
            # a lone knight, and the opponent has only king and queens
            return len(ours) <= 2 and all((self.sq[s] & 7) in (KING, QUEEN) for s in theirs)
        if BISHOP in types:
            # all bishops on the board on one square colour, no pawns or knights
            bishops = [s for s in range(64) if (self.sq[s] & 7) == BISHOP]
            same = len({_SQ_COLOR[s] for s in bishops}) == 1
            no_pn = not any((self.sq[s] & 7) in (PAWN, KNIGHT) for s in range(64) if self.sq[s] != EMPTY)
            return same and no_pn
        return True

    def outcome(self) -> Optional[tuple]:
        """None while the game goes on, else (termination, winner) with
        winner True (white), False (black) or None (draw)."""
        has_moves = bool(self.legal_moves())
        if not has_moves and self.is_check():
            return ("checkmate", not self.white)
        if self._insufficient(True) and self._insufficient(False):
            return ("insufficient_material", None)
        if not has_moves:
            return ("stalemate", None)
        if self.halfmove >= 150:
            return ("seventyfive_moves", None)
        if self.keys and self.keys.count(self.keys[-1]) >= 5:
            return ("fivefold_repetition", None)
        return None

    def is_game_over(self) -> bool:
        return self.outcome() is not None


def _between(a: int, b: int) -> list:
    """Squares strictly between a and b on a rank, file or diagonal."""
    fa, ra, fb, rb = a & 7, a >> 3, b & 7, b >> 3
    df, dr = fb - fa, rb - ra
    if not (df == 0 or dr == 0 or abs(df) == abs(dr)):
        return []
    sf = (df > 0) - (df < 0)
    sr = (dr > 0) - (dr < 0)
    out, f, r = [], fa + sf, ra + sr
    while (f, r) != (fb, rb):
        out.append(r * 8 + f)
        f += sf
        r += sr
    return out


def board_after(moves: list) -> Board:
    b = Board()
    for m in moves:
        b = b.push_uci(m)
    return b


def legal_moves(moves: list) -> list:
    """UCI legal moves after a game given as UCI moves from the start."""
    return board_after(moves).legal_uci()


def perft(b: Board, depth: int) -> int:
    if depth == 0:
        return 1
    ms = b.legal_moves()
    if depth == 1:
        return len(ms)
    return sum(perft(b._make(m), depth - 1) for m in ms)
