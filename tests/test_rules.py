"""Native host chess rules (allie_amd/rules.py over csrc/chess.cpp).

* Legality: perft known answers of the standard test positions (deeper than
  the Python restatement's test can afford).
* Order and game over: the same legal-move lists, in the same order, and the
  same outcomes as oracle/movegen.py on every position of seeded random
  games and of the test positions' subtrees (the order itself follows
  python-chess's generation order, unpinned without python-chess).
* Outcome known answers: mate, stalemate, insufficient material, the
  75-move rule and fivefold repetition.
"""
import numpy as np
import pytest

from oracle import movegen
from allie_amd.rules import NativeBoard, board_after

KIWIPETE = "r3k2r/p1ppqpb1/bn2pnp1/3PN3/1p2P3/2N2Q1p/PPPBBPPP/R3K2R w KQkq - 0 1"
POS3 = "8/2p5/3p4/KP5r/1R3p1k/8/4P1P1/8 w - - 0 1"
POS4 = "r3k2r/Pppp1ppp/1b3nbN/nP6/BBP1P3/q4N2/Pp1P2PP/R2Q1RK1 w kq - 0 1"
POS5 = "rnbq1k1r/pp1Pbppp/2p5/8/2B5/8/PPP1NnPP/RNBQK2R w KQ - 1 8"


@pytest.mark.parametrize("fen,counts", [
    (None, [20, 400, 8902, 197281]),
    (KIWIPETE, [48, 2039, 97862]),
    (POS3, [14, 191, 2812, 43238]),
    (POS4, [6, 264, 9467, 422333]),
    (POS5, [44, 1486, 62379]),
])
def test_perft_known_answers(fen, counts):
    b = NativeBoard.start() if fen is None else NativeBoard.from_fen(fen)
    for d, n in enumerate(counts, start=1):
        assert b.perft(d) == n, (fen, d)


def _same(nb, pb):
    assert nb.legal_uci() == pb.legal_uci()
    assert nb.outcome() == pb.outcome()
    assert nb.is_check() == pb.is_check()


def test_random_games_match_python_rules():
    rng = np.random.default_rng(17)
    n_pos = 0
    for _ in range(40):
        nb, pb = NativeBoard.start(), movegen.Board()
        for _ in range(160):
            _same(nb, pb)
            n_pos += 1
            legal = pb.legal_uci()
            if not legal or pb.outcome() is not None:
                break
            m = legal[int(rng.integers(len(legal)))]
            nb, pb = nb.push_uci(m), pb.push_uci(m)
    assert n_pos > 3000


@pytest.mark.parametrize("fen", [KIWIPETE, POS3, POS4, POS5])
def test_test_positions_subtrees_match_python_rules(fen):
    nb, pb = NativeBoard.from_fen(fen), movegen.Board.from_fen(fen)
    _same(nb, pb)
    for m in pb.legal_uci():
        n1, p1 = nb.push_uci(m), pb.push_uci(m)
        _same(n1, p1)
        for m2 in p1.legal_uci():
            _same(n1.push_uci(m2), p1.push_uci(m2))


def test_outcomes_and_errors():
    mate = board_after("f2f3 e7e5 g2g4 d8h4".split())
    assert mate.is_game_over() and mate.outcome() == ("checkmate", False)
    assert board_after("e2e4".split()).outcome() is None
    assert NativeBoard.from_fen("7k/5Q2/6K1/8/8/8/8/8 b - - 0 1").outcome() == ("stalemate", None)
    assert NativeBoard.from_fen("8/8/4k3/8/8/3NK3/8/8 b - - 0 1").outcome() == ("insufficient_material", None)
    assert NativeBoard.from_fen("8/8/4k3/8/8/3BK3/8/8 b - - 0 1").outcome() == ("insufficient_material", None)
    assert NativeBoard.from_fen("8/8/4k3/8/8/3RK3/8/8 b - - 0 1").outcome() is None
    assert NativeBoard.from_fen("8/8/4k3/8/8/3RK3/8/8 b - - 150 90").outcome() == ("seventyfive_moves", None)
    shuffle = "g1f3 g8f6 f3g1 f6g8 " * 4
    assert board_after(shuffle.split()).outcome() == ("fivefold_repetition", None)
    assert board_after(shuffle.split()[:-1]).outcome() is None
    # white mates: the winner is white
    scholar = board_after("e2e4 e7e5 f1c4 b8c6 d1h5 g8f6 h5f7".split())
    assert scholar.outcome() == ("checkmate", True)
    b = NativeBoard.start()
    for bad in ("e2e5", "e7e5", "e2", "e2e4x", "z9e4", "e7e8q"):
        with pytest.raises(ValueError):
            b.push_uci(bad)
    with pytest.raises(ValueError):
        NativeBoard.from_fen("8/8/8/8/8/8/8/8 w - - 0 1")  # no kings


def test_game_uses_native_rules():
    from allie_amd.tokenizer import Game

    g = Game("300+0", 1500, 1500, None, False, ["e2e4", "e7e5"], [1, 1], None)
    assert isinstance(g.board, NativeBoard)
    c = g.make_move("g1f3")
    assert c.legal_moves == movegen.legal_moves(["e2e4", "e7e5", "g1f3"])
