"""Host-side tokenizer and game record (the reference's L1 layer).

Mirrors ``Game`` (src/modeling/data.py:40-80) and ``UCITokenizer``
(data.py:175-337) of the reference, with one difference forced by the image:
python-chess is absent, so ``Game.legal_moves`` is taken from the caller
(``Game(..., legal=[...])``) or from the native host rules
(``allie_amd.rules``; the tests' Python restatement is ``oracle/movegen.py``).
The side to move is closed-form: white iff an even number of moves has been
played, because every game starts from the initial position
(data.py:51-56).

``UCITokenizer.tokenize`` produces the same uint32 words as data.py:217-270.
The GPU path consumes those words directly (``allie_amd.engine.Engine.prefill``
takes ``words`` + ``lens``); ``pad_and_collate`` exists for the drop-in model
call (data.py:281-337) and returns the same dict of padded tensors.
"""
# Portions of this file follow y0mingzhang/allie, src/modeling/data.py (the
# tokenizer's word format, padding and messages), distributed under this
# notice:
#
#   MIT License
#
#   Copyright (c) 2024 Yiming Zhang
#
#   Permission is hereby granted, free of charge, to any person obtaining a copy
#   of this software and associated documentation files (the "Software"), to deal
#   in the Software without restriction, including without limitation the rights
#   to use, copy, modify, merge, publish, distribute, sublicense, and/or sell
#   copies of the Software, and to permit persons to whom the Software is
#   furnished to do so, subject to the following conditions:
#
#   The above copyright notice and this permission notice shall be included in all
#   copies or substantial portions of the Software.
#
#   THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND, EXPRESS OR
#   IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF MERCHANTABILITY,
#   FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT. IN NO EVENT SHALL THE
#   AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM, DAMAGES OR OTHER
#   LIABILITY, WHETHER IN AN ACTION OF CONTRACT, TORT OR OTHERWISE, ARISING FROM,
#   OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE USE OR OTHER DEALINGS IN THE
#   SOFTWARE.

from __future__ import annotations

import logging
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from . import vocab

logger = logging.getLogger(__name__)

OUTCOME_MASKS = {"1-0": 0x0000, "1/2-1/2": 0x4000, "0-1": 0x8000}  # data.py:146-153


@dataclass
class Game:
    """Game record (data.py:40-49).  ``legal`` optionally carries the legal
    moves in the caller's order (python-chess order in the reference,
    data.py:58-61); argmax ties break by this order (decode.py:112)."""

    time_control: Optional[str]
    white_elo: Optional[int]
    black_elo: Optional[int]
    outcome: Optional[str]
    normal_termination: bool
    moves: list[str]
    moves_seconds: list[int]
    next_move_seconds: Optional[int] = None
    legal: Optional[list[str]] = field(default=None, repr=False, compare=False)
    _board: Optional[object] = field(default=None, repr=False, compare=False)
    _parent: Optional["Game"] = field(default=None, repr=False, compare=False)

    @property
    def white_to_move(self) -> bool:
        return len(self.moves) % 2 == 0

    @property
    def board(self):
        """The position after the game's moves (data.py:51-56), from the
        native host rules (``allie_amd.rules``); a child made by
        ``make_move`` extends its parent's cached board by one move."""
        if self._board is None:
            from . import rules

            p = self._parent
            if p is not None and p._board is not None:
                self._board = p._board.push_uci(self.moves[-1])
            else:
                self._board = rules.board_after(self.moves)
            self._parent = None
        return self._board

    @property
    def legal_moves(self) -> list[str]:
        """UCI legal moves (data.py:58-61); an explicit ``legal`` list from
        the caller takes precedence."""
        if self.legal is None:
            self.legal = self.board.legal_uci()
        return self.legal

    def make_move(self, move: str) -> "Game":
        """data.py:63-73: the child game has one more move, time 0, no
        next-move time, and the same metadata."""
        return Game(
            self.time_control,
            self.white_elo,
            self.black_elo,
            self.outcome,
            self.normal_termination,
            self.moves + [move],
            self.moves_seconds + [0],
            None,
            _parent=self,
        )


def apply_time_normalization(t):
    """data.py:160-168."""
    try:
        import torch

        if isinstance(t, torch.Tensor):
            t = t.clamp(0, 60)
            return (t - vocab.TIME_MEAN) / vocab.TIME_STDEV
    except ImportError:  # pragma: no cover
        pass
    t = min(max(t, 0), 60)
    return (t - vocab.TIME_MEAN) / vocab.TIME_STDEV


def undo_time_normalization(t_normed):
    """data.py:171-172."""
    return t_normed * vocab.TIME_STDEV + vocab.TIME_MEAN


class UCITokenizer:
    """Same constructor arguments and token ids as data.py:175-215."""

    def __init__(
        self,
        max_length: int = 128,
        vocab_size_multiple_of: int = 1,
        bos_token: str = "<BOS>",
        eos_token: str = "<EOS>",
        unk_token: str = "<UNK>",
        pad_token: str = "<PAD>",
        **kwargs,
    ):
        if kwargs:
            logger.warning(f"tokenizer got unrecognized arguments {kwargs}")
        specials = [bos_token, eos_token, unk_token, pad_token]
        self.tokens = (
            list(vocab.CHESS_MOVES)
            + list(vocab.BLITZ_TIME_CONTROLS_TOKENS)
            + [vocab.NORMAL_TERMINATION_TOKEN]
            + specials
        )
        i = 0
        while len(self.tokens) % vocab_size_multiple_of != 0:
            self.tokens.append(f"<UNUSED-{i}")
            i += 1
        self.max_length = max_length
        self.bos_token, self.eos_token = bos_token, eos_token
        self.unk_token, self.pad_token = unk_token, pad_token
        self.resigned_token = vocab.NORMAL_TERMINATION_TOKEN
        self.special_tokens = specials
        self.token_to_id = {t: i for i, t in enumerate(self.tokens)}
        self.special_token_ids = [self.token_to_id[t] for t in specials]
        self.bos_token_id = self.token_to_id[bos_token]
        self.eos_token_id = self.token_to_id[eos_token]
        self.unk_token_id = self.token_to_id[unk_token]
        self.pad_token_id = self.token_to_id[pad_token]
        self.resigned_token_id = self.token_to_id[self.resigned_token]

    def __len__(self) -> int:
        return len(self.tokens)

    def tokenize(
        self,
        game: Game,
        add_elo: bool = True,
        add_time_control: bool = True,
        add_termination: bool = True,
        add_value: bool = True,
    ) -> np.ndarray:
        """Game -> uint32 words (data.py:217-270).

        Word layout (the code, not the docstring at data.py:27-36, is
        authoritative): ``id | outcome << 14 | (secs + 1) << 16`` where the
        time paired with a token is the time of the *next* move.
        """
        V = len(self)
        if add_elo:
            assert isinstance(game.white_elo, int) and isinstance(game.black_elo, int)
            seq = [game.white_elo + V, game.black_elo + V]
        else:
            seq = [self.bos_token_id]
        moves = game.moves
        tc = game.time_control if add_time_control else self.unk_token
        assert isinstance(tc, str)
        secs = game.moves_seconds
        assert isinstance(secs, list) and len(moves) == len(secs)
        for tok, t in zip([tc] + moves, secs + [-1]):
            if t < 0:
                t = -1
            elif t >= 0xFFFF:
                raise AssertionError(f"move time {t}s overflows 16-bit repr")
            seq.append(self.token_to_id.get(tok, self.unk_token_id) + ((t + 1) << 16))
        if add_termination and game.normal_termination:
            seq.append(self.resigned_token_id)
        if game.outcome is not None:
            seq.append(self.eos_token_id)
        words = np.array(seq, dtype=np.uint32)
        if add_value and game.outcome is not None:
            words = words | np.uint32(OUTCOME_MASKS[game.outcome])
        return words

    def words_and_lens(self, games: list[Game]) -> tuple[np.ndarray, np.ndarray]:
        """Flat word stream + per-game word counts: the input of the GPU
        ragged packer (it truncates to ``max_length`` itself, data.py:290)."""
        seqs = [self.tokenize(g) for g in games]
        lens = np.array([len(s) for s in seqs], dtype=np.int32)
        words = np.concatenate(seqs).astype(np.uint32) if seqs else np.zeros(0, np.uint32)
        return words, lens

    def pad_and_collate(self, games, return_labels: bool = True) -> dict:
        """data.py:281-337: truncate to the first ``max_length`` words, right
        pad with PAD, unpack into the model's keyword arguments."""
        import torch

        if isinstance(games[0], np.ndarray):
            data = torch.from_numpy(np.array(games).astype(np.int64))
        else:
            seqs = [self.tokenize(g)[: self.max_length].astype(np.int64) for g in games]
            T = max(len(s) for s in seqs)
            data = torch.stack(
                [
                    torch.from_numpy(np.pad(s, (0, T - len(s)), "constant", constant_values=self.pad_token_id))
                    for s in seqs
                ]
            )
        enc = data >> 16
        time_labels = torch.where(enc == 0, -100, apply_time_normalization(enc - 1))
        outcomes = (data & 0xFFFF) >> 14
        assert outcomes.max() < 3
        input_ids = data & vocab.ID_MASK
        attention_mask = input_ids != self.pad_token_id
        labels = torch.where(attention_mask, input_ids, -100)
        labels[labels >= len(self)] = -100
        value_labels = torch.where(attention_mask, -outcomes.to(torch.float32) + 1, -100)
        position_ids = (attention_mask.long().cumsum(-1) - 1).clamp(0)
        out = {
            "input_ids": input_ids,
            "attention_mask": attention_mask.to(torch.float),
            "position_ids": position_ids,
            "value_labels": value_labels,
            "time_labels": time_labels,
        }
        if return_labels:
            out["labels"] = labels
        return out
