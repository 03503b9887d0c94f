"""Python chess rules restatement (oracle/movegen.py): legality pinned by perft known
answers (node counts of the legal-move tree; the standard test positions of
the chess-programming literature exercise castling through and out of check,
en passant with pins and discovered checks, and under-promotion), plus
game-over/outcome cases.  The ORDER of legal moves follows python-chess's
generation order, which only an import could pin (parity unpinned)."""
import time

import pytest

from oracle.movegen import Board, board_after, legal_moves, perft

KIWIPETE = "r3k2r/p1ppqpb1/bn2pnp1/3PN3/1p2P3/2N2Q1p/PPPBBPPP/R3K2R w KQkq - 0 1"
POS3 = "8/2p5/3p4/KP5r/1R3p1k/8/4P1P1/8 w - - 0 1"
POS4 = "r3k2r/Pppp1ppp/1b3nbN/nP6/BBP1P3/q4N2/Pp1P2PP/R2Q1RK1 w kq - 0 1"
POS5 = "rnbq1k1r/pp1Pbppp/2p5/8/2B5/8/PPP1NnPP/RNBQK2R w KQ - 1 8"


@pytest.mark.parametrize("fen,counts", [
    (None, [20, 400, 8902]),
    (KIWIPETE, [48, 2039]),
    (POS3, [14, 191, 2812]),
    (POS4, [6, 264, 9467]),
    (POS5, [44, 1486]),
])
def test_perft_known_answers(fen, counts):
    b = Board() if fen is None else Board.from_fen(fen)
    for d, n in enumerate(counts, start=1):
        assert perft(b, d) == n, (fen, d)


def test_start_position_order_and_uci():
    ms = legal_moves([])
    assert len(ms) == 20
    # knights first (g1 before b1, targets descending), then pawn pushes by
    # target square descending, single before double
    assert ms[:4] == ["g1h3", "g1f3", "b1c3", "b1a3"]
    assert ms[4:12] == ["h2h3", "g2g3", "f2f3", "e2e3", "d2d3", "c2c3", "b2b3", "a2a3"]
    assert ms[12:] == ["h2h4", "g2g4", "f2f4", "e2e4", "d2d4", "c2c4", "b2b4", "a2a4"]


def test_castling_en_passant_promotion_by_moves():
    b = board_after("e2e4 e7e5 g1f3 b8c6 f1c4 g8f6".split())
    assert "e1g1" in b.legal_uci()
    b = b.push_uci("e1g1")
    assert b.sq[6] == 6 and b.sq[5] == 4  # king g1, rook f1
    b = board_after("e2e4 a7a6 e4e5 d7d5".split())
    assert "e5d6" in b.legal_uci()
    b2 = b.push_uci("e5d6")
    assert b2.sq[35] == 0  # the d5 pawn is gone
    b = board_after("a2a4 b7b5 a4b5 a7a6 b5a6 c8b7 a6b7 e7e6".split())
    assert {"b7a8q", "b7a8r", "b7a8b", "b7a8n"} <= set(b.legal_uci())
    with pytest.raises(ValueError):
        b.push_uci("e1e3")


def test_outcomes():
    mate = board_after("f2f3 e7e5 g2g4 d8h4".split())  # fool's mate
    assert mate.is_game_over() and mate.outcome() == ("checkmate", False)
    assert board_after("e2e4".split()).outcome() is None
    stale = Board.from_fen("7k/5Q2/6K1/8/8/8/8/8 b - - 0 1")
    assert stale.outcome() == ("stalemate", None)
    assert Board.from_fen("8/8/4k3/8/8/3NK3/8/8 b - - 0 1").outcome() == ("insufficient_material", None)
    assert Board.from_fen("8/8/4k3/8/8/3BK3/8/8 b - - 0 1").outcome() == ("insufficient_material", None)
    assert Board.from_fen("8/8/4k3/8/8/3RK3/8/8 b - - 0 1").outcome() is None
    assert Board.from_fen("8/8/4k3/8/8/3RK3/8/8 b - - 150 90").outcome() == ("seventyfive_moves", None)
    # knights shuffle back and forth: the start position occurs a fifth time
    shuffle = "g1f3 g8f6 f3g1 f6g8 " * 4
    rep = board_after(shuffle.split())
    assert rep.outcome() == ("fivefold_repetition", None)
    assert board_after(shuffle.split()[:-1]).outcome() is None


def test_evasion_order():
    # white in check from the bishop on b4; the king cannot move (d2 is on the
    # bishop's line), so the blocks come in piece order: queen d1, bishop c1,
    # knight b1 (targets descending), then the pawn push
    b = board_after("d2d4 e7e5 d4e5 f8b4".split())
    assert b.is_check()
    assert b.legal_uci() == ["d1d2", "c1d2", "b1c3", "b1d2", "c2c3"]
    # black in check from the queen on a4: king moves come first
    b = board_after("e2e4 d7d6 d1h5 e7e6 h5b5".split())
    ms = b.legal_uci()
    assert ms[0] == "e8e7" and ms[1:] == sorted(ms[1:], key=ms[1:].index)
    assert set(ms) == {"e8e7", "d8d7", "c8d7", "b8d7", "b8c6", "c7c6"}
