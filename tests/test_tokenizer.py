"""Host tokenizer: known answers for UCITokenizer.tokenize and
pad_and_collate (src/modeling/data.py:217-337), worked out by hand from the
code (the docstring at data.py:27-36 is wrong about the bit layout) on the
reference's own self-test game (src/server/test.py:9-32, read as text)."""
import numpy as np
import pytest
import torch

from allie_amd import vocab
from allie_amd.tokenizer import Game, UCITokenizer, apply_time_normalization, undo_time_normalization

DEEPBLUE = ("e2e4 e7e5 g1f3 b8c6 f1b5 a7a6 b5a4 g8f6 e1g1 f8e7 f1e1 b7b5 a4b3 d7d6 c2c3 e8g8 h2h3 h7h6 "
            "d2d4 f8e8").split()
ID = vocab.TOKEN_TO_ID


def partial(halfmove, secs=None):
    """json_to_partial_game (data.py:96-109) of the self-test game."""
    s = secs if secs is not None else [0] * 20
    return Game(time_control="5400+0", white_elo=2800, black_elo=2840, outcome=None,
                normal_termination=False, moves=DEEPBLUE[:halfmove], moves_seconds=s[:halfmove],
                next_move_seconds=s[halfmove] if halfmove < len(s) else None)


def test_tokenize_partial_game_known_answer():
    tok = UCITokenizer(max_length=512)
    assert len(tok) == 1997
    w = tok.tokenize(partial(4))
    # [w_elo + V, b_elo + V, tc | (t0+1)<<16, m0 | (t1+1)<<16, ..., m3 | 0]
    want = [2800 + 1997, 2840 + 1997, 1995 + (1 << 16), ID["e2e4"] + (1 << 16), ID["e7e5"] + (1 << 16),
            ID["g1f3"] + (1 << 16), ID["b8c6"]]
    assert w.dtype == np.uint32 and w.tolist() == want
    # halfmove 0: the time-control token carries no move time
    assert tok.tokenize(partial(0)).tolist() == [4797, 4837, 1995]


def test_tokenize_times_and_known_time_control():
    tok = UCITokenizer()
    g = Game("300+0", 1500, 1600, None, False, ["e2e4", "e7e5"], [7, 12])
    assert tok.tokenize(g).tolist() == [3497, 3597, 1969 + (8 << 16), ID["e2e4"] + (13 << 16), ID["e7e5"]]
    assert tok.tokenize(g, add_elo=False, add_time_control=False).tolist() == [
        1993, 1995 + (8 << 16), ID["e2e4"] + (13 << 16), ID["e7e5"]]
    with pytest.raises(AssertionError):
        tok.tokenize(Game("300+0", 1500, 1600, None, False, ["e2e4"], [0xFFFF]))


def test_tokenize_finished_game_outcome_bits():
    tok = UCITokenizer()
    g = Game("180+0", 2000, 2100, "0-1", True, ["e2e4", "e7e5"], [1, 2])
    want = [2000 + 1997, 2100 + 1997, 1968 + (2 << 16), ID["e2e4"] + (3 << 16), ID["e7e5"], 1992, 1994]
    assert tok.tokenize(g).tolist() == [x | 0x8000 for x in want]
    g2 = Game("180+0", 2000, 2100, "1/2-1/2", False, ["e2e4"], [1])
    assert tok.tokenize(g2).tolist() == [x | 0x4000 for x in [3997, 4097, 1968 + (2 << 16), ID["e2e4"], 1994]]
    assert tok.tokenize(g2, add_value=False).tolist() == [3997, 4097, 1968 + (2 << 16), ID["e2e4"], 1994]


def test_pad_and_collate_known_answer():
    tok = UCITokenizer(max_length=6)
    g1 = partial(2)  # 5 words
    g2 = partial(6, secs=[3] * 20)  # 9 words -> truncated to the first 6
    b = tok.pad_and_collate([g1, g2])
    assert b["input_ids"].tolist() == [
        [4797, 4837, 1995, ID["e2e4"], ID["e7e5"], 1996],
        [4797, 4837, 1995, ID["e2e4"], ID["e7e5"], ID["g1f3"]],
    ]
    assert b["attention_mask"].tolist() == [[1, 1, 1, 1, 1, 0], [1] * 6]
    assert b["position_ids"].tolist() == [[0, 1, 2, 3, 4, 4], [0, 1, 2, 3, 4, 5]]
    # Elo words are not LM targets; padding is -100
    assert b["labels"].tolist() == [[-100, -100, 1995, ID["e2e4"], ID["e7e5"], -100],
                                    [-100, -100, 1995, ID["e2e4"], ID["e7e5"], ID["g1f3"]]]
    t3 = (3 - 4.64001) / 6.16533
    t0 = (0 - 4.64001) / 6.16533
    tl = b["time_labels"]
    assert tl[0, :2].tolist() == [-100, -100] and tl[0, 4].item() == -100
    assert abs(tl[0, 2].item() - t0) < 1e-6 and abs(tl[1, 3].item() - t3) < 1e-6
    assert b["value_labels"].tolist() == [[1, 1, 1, 1, 1, -100], [1] * 6]


def test_time_normalisation_round_trip():
    assert abs(apply_time_normalization(100) - (60 - 4.64001) / 6.16533) < 1e-12
    assert abs(apply_time_normalization(-3) - (0 - 4.64001) / 6.16533) < 1e-12
    assert abs(undo_time_normalization(apply_time_normalization(17)) - 17) < 1e-9
    t = apply_time_normalization(torch.tensor([-1.0, 30.0, 99.0]))
    assert torch.allclose(t, (torch.tensor([0.0, 30.0, 60.0]) - 4.64001) / 6.16533)


def test_words_and_lens_and_side_to_move():
    tok = UCITokenizer()
    games = [partial(0), partial(3), partial(8)]
    words, lens = tok.words_and_lens(games)
    assert lens.tolist() == [3, 6, 11]
    assert words.tolist() == sum((tok.tokenize(g).tolist() for g in games), [])
    assert [g.white_to_move for g in games] == [True, False, True]
    child = games[1].make_move("f1b5")
    assert child.moves[-1] == "f1b5" and child.moves_seconds[-1] == 0 and child.next_move_seconds is None
