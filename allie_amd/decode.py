"""Decode strategies on the GPU engine: ``policy``, ``mcts``, ``adaptive-mcts``.

Same names, constructor arguments, results and search semantics as the
reference's ``DECODE_STRATEGIES`` (src/evaluation/decode.py:734-740):

* ``DecodeStrategy(model, tokenizer, sample=False, device=None,
  precision="float32", **init_kwargs)`` -> ``init(**kw)`` -> ``check()``
  (decode.py:58-81); ``decode_full(game) -> DecodeResult`` (:90-113);
  ``score_full(game, legal_moves) -> ScoreResult`` (:115-120).
* ``Policy`` (:185-238), ``MCTS`` (:309-470, PUCT selection, backup with
  alternating sign, KL-regularised final policy by bisection), and
  ``AdaptiveMCTS`` (:473-658, simulation budget from the time head).

``model`` is anything called as ``model(**tokenizer.pad_and_collate(games))``
returning ``logits`` / ``value_logits`` / ``time_logits`` whose ``[0, -1]``
entries belong to the last token; ``allie_amd.model.AllieModel`` is the GPU
engine behind that call.  The numeric precision is the engine's mode (fp32
check mode or bf16), chosen when the model is built; ``precision`` is kept
for signature compatibility (the reference wraps calls in torch autocast,
decode.py:74-78).

Game rules (legal moves in python-chess order, game over) come from the
native host rules (``allie_amd.rules``; the tests check them against a
Python restatement, oracle/movegen.py) because python-chess is absent from
this image.
The reference's quirks are kept: MCTS evaluates the root twice (:407, :410),
and the "rating-based" sampling rule reads the Elo of the side to move
(:97-107).

Beyond the reference, ``mcts`` and ``adaptive-mcts`` take ``kv_cache=True``:
the search keeps its root's keys and values in a paged pool and evaluates
each leaf as one new token over them (``allie_amd.search_kv``), with the same
sequential semantics and results up to summation order; the root is then
evaluated once.  ``leaf_batch=B`` (with ``kv_cache``) selects up to B leaves
per round under virtual loss and evaluates them in one call, which is a
different (batched) search.
"""
# Portions of this file follow y0mingzhang/allie, src/evaluation/decode.py (the
# decode strategies' API and search arithmetic), distributed under this
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

import math
from dataclasses import dataclass
from typing import Any, Optional

import torch
import torch.nn.functional as F

from .search_kv import KVSearchCache, NodeEval, pool_nodes_for, virtual_loss_apply
from .tokenizer import Game, UCITokenizer, apply_time_normalization, undo_time_normalization
from .vocab import NUM_CHESS_MOVES, TIME_MEAN, TIME_STDEV

PRECISIONS = ("bfloat16", "float16", "float32")


@dataclass(frozen=True)
class DecodeResult:
    move: str
    think_time: Optional[float]
    resigned: bool


@dataclass(frozen=True)
class ScoreResult:
    legal_move_probabilities: torch.Tensor
    think_time: Optional[float] = None
    resigned: Optional[bool] = None
    all_move_probabilities: Optional[torch.Tensor] = None
    top_move_legal: Optional[bool] = None
    sampled_move_legal: Optional[float] = None
    white_advantage: Optional[float] = None


class DecodeStrategy:
    def __init__(self, model, tokenizer: UCITokenizer, sample=False, device: Optional[str] = None,
                 precision: str = "float32", **kwargs: Any):
        if precision not in PRECISIONS:
            raise KeyError(precision)
        self.model = model
        self.tokenizer = tokenizer
        self.sample = sample
        self.device = device or ("cuda" if torch.cuda.is_available() else "cpu")
        self.precision = precision
        self.init(**kwargs)
        self.check()

    def init(self, *args, **kwargs) -> None: ...

    def check(self) -> None: ...

    def decode(self, game: Game) -> str:
        return self.decode_full(game).move

    def decode_full(self, game: Game) -> DecodeResult:
        legal_moves = game.legal_moves
        return self._choose(game, legal_moves, self.score_full(game, legal_moves))

    def _choose(self, game: Game, legal_moves: list[str], score: ScoreResult) -> DecodeResult:
        """decode.py:97-113: argmax or a sample of the legal-move
        probabilities, by ``sample`` (the "rating-based" rule included)."""
        probs = score.legal_move_probabilities
        if self.sample not in (True, False):
            assert self.sample == "rating-based"
            # decode.py:97-107 reads the Elo of the side to move
            opponent_elo = game.white_elo if game.white_to_move else game.black_elo
            sample = not (opponent_elo >= 2200 and len(game.moves) > 8)
        else:
            sample = self.sample
        if sample:
            choice = probs.multinomial(1)[0].item()
        else:
            choice = int(probs.argmax())  # the first maximum
        return DecodeResult(legal_moves[choice], score.think_time, score.resigned)

    def score_full(self, game: Game, legal_moves: list[str]) -> ScoreResult:
        raise NotImplementedError

    def run_stats(self) -> dict:
        return {}

    def cleanup(self) -> None: ...

    # the model call of the reference (decode.py:199-203, 356-360)
    def _forward(self, game: Game) -> dict:
        batch = self.tokenizer.pad_and_collate([game])
        with torch.no_grad():
            return self.model(**batch)


class Policy(DecodeStrategy):
    def init(self, temperature: float = 1.0, time_prediction: bool = True) -> None:
        self.temperature = max(temperature, 1e-5)
        self.time_prediction = time_prediction

    def score_full(self, game: Game, legal_moves: list[str]) -> ScoreResult:
        return self._score(game, legal_moves, self._full_eval(game))

    def _full_eval(self, game: Game) -> NodeEval:
        """The last token's outputs of the model call on the whole game."""
        outputs = self._forward(game)
        return NodeEval(outputs["logits"][0, -1].float().cpu(), float(outputs["value_logits"][0, -1].item()),
                        float(outputs["time_logits"][0, -1].item()))

    def _score(self, game: Game, legal_moves: list[str], ev: NodeEval) -> ScoreResult:
        """decode.py:204-238 on one evaluation of the game."""
        logits = ev.logits
        legal = torch.tensor([self.tokenizer.token_to_id[m] for m in legal_moves], dtype=torch.int64)
        move_logits = logits[legal]
        time_encoding = ev.time
        think_time = undo_time_normalization(time_encoding) if self.time_prediction else None
        pov = 1 if game.white_to_move else -1
        value = pov * ev.value
        resigned_logit = logits[self.tokenizer.resigned_token_id].item()
        resigned = resigned_logit > move_logits.max().item() and value < -0.9
        all_probs = F.softmax(logits[:NUM_CHESS_MOVES] / self.temperature, dim=0)
        top_move_idx = int(all_probs.argmax().item())
        return ScoreResult(
            F.softmax(move_logits / self.temperature, dim=0),
            think_time,
            resigned,
            all_probs,
            self.tokenizer.tokens[top_move_idx] in legal_moves,
            all_probs[legal].sum().item(),
            ev.value,
        )


class MCTSNode:
    """decode.py:273-306.  A child made at expansion holds its parent's game
    and its move, and builds its own game (``parent.make_move(move)``) the
    first time it is read: a node has about 30 children, of which a search
    reads few."""

    # the KV-cached search's per-node fields (allie_amd.search_kv) included
    __slots__ = ("prior", "children", "visit_count", "value_sum", "_game", "_from", "_kv_parent", "_kv_token",
                 "_kv_path", "_kv_eval", "__dict__")

    def __init__(self, prior: float, game: Optional[Game] = None, parent_game: Optional[Game] = None,
                 move: Optional[str] = None):
        self.prior = prior
        self.children: dict[str, "MCTSNode"] = {}
        self.visit_count = 0
        self.value_sum = 0.0
        self._game = game
        self._from = None if game is not None else (parent_game, move)

    @property
    def game(self) -> Game:
        if self._game is None:
            parent_game, move = self._from
            self._game = parent_game.make_move(move)
            self._from = None
        return self._game

    @property
    def board(self):
        return self.game.board

    @property
    def legal_moves(self) -> list[str]:
        return self.game.legal_moves

    def expanded(self) -> bool:
        return len(self.children) > 0

    def value(self) -> float:
        if self.visit_count == 0:
            return 0.0
        return self.value_sum / self.visit_count


def kl_regularised_policy(priors: torch.Tensor, values: torch.Tensor, visit_counts: torch.Tensor,
                          c_puct: float) -> torch.Tensor:
    """The search policy pi_bar = lambda_N * prior / (alpha - q) with
    lambda_N = c_puct * N / (|A| + N) and alpha found by bisection on
    [max(q + lambda_N * prior), max(q + lambda_N)] until sum(pi_bar) is within
    rtol 1e-3 of 1 (or the bracket is); the result is normalised
    (decode.py:438-467, float32 tensors as there)."""
    total_visits = visit_counts.sum().item()
    lambda_n = c_puct * total_visits / (len(visit_counts) + total_visits)
    alpha_min = (values + lambda_n * priors).max()
    alpha_max = (values + lambda_n).max()
    while True:
        alpha = (alpha_min + alpha_max) / 2
        pi_bar = lambda_n * priors / (alpha - values)
        if pi_bar.sum() > 1.0:
            alpha_min = alpha
        else:
            alpha_max = alpha
        if torch.isclose(pi_bar.sum(), torch.tensor(1.0), rtol=1e-3) or torch.isclose(alpha_min, alpha_max, rtol=1e-3):
            return pi_bar / pi_bar.sum()


class MCTS(Policy):
    def init(self, n_sims: int = 50, depth_limit: int = 100, c_puct: float = 1.25, c_base: float = 19652.0,
             dummy_value_function: bool = False, kl_reg_solution: bool = True, kv_cache: bool = False,
             leaf_batch: int = 1, kv_graph: bool = True, **kwargs) -> None:
        super().init(**kwargs)
        self.n_sims = n_sims
        self.depth_limit = depth_limit
        self.c_puct = c_puct
        self.c_base = c_base
        self.dummy_value_function = dummy_value_function
        self.kl_reg_solution = kl_reg_solution
        self.total_rollouts = 0
        self._init_kv(kv_cache, leaf_batch, kv_graph)

    def _init_kv(self, kv_cache: bool, leaf_batch: int, kv_graph: bool = True) -> None:
        """Opt-in search over a paged KV cache (``allie_amd.search_kv``):
        ``kv_cache=True`` evaluates each leaf as one new token over its
        root's and ancestors' cached keys, with the reference's sequential
        semantics; ``leaf_batch=B > 1`` also selects up to B leaves per round
        under virtual loss and evaluates them in one call (a different,
        batched search); ``kv_graph`` (default on) replays single leaves from
        a captured HIP graph, with identical results.  None of these exists
        in the reference."""
        if leaf_batch < 1:
            raise ValueError("leaf_batch must be >= 1")
        if leaf_batch > 1 and not kv_cache:
            raise ValueError("leaf_batch > 1 needs kv_cache=True")
        self.kv_cache = kv_cache
        self.leaf_batch = leaf_batch
        self.kv_graph = kv_graph
        self._kv: Optional[KVSearchCache] = None

    def check(self) -> None:
        assert callable(self.model), "model does not provide a value prediction"
        if self.kv_cache:
            assert hasattr(self.model, "engine"), "kv_cache needs the GPU model (allie_amd.model.AllieModel)"

    def _terminal_value(self, node: MCTSNode) -> Optional[float]:
        """decode.py:345-353: a draw is 0, a mate +1 for the side that moved."""
        oc = node.board.outcome()
        if oc is None:
            return None
        _, winner = oc
        if winner is None:
            return 0.0
        assert winner != node.game.white_to_move
        return 1.0

    def _node_eval(self, node: MCTSNode) -> NodeEval:
        kv = self._kv
        if kv is not None and kv.can_extend(node):
            return kv.evaluate([node])[0]
        return self._full_eval(node.game)

    def _evaluate(self, node: MCTSNode):
        """One model evaluation of a node: (priors over its legal moves, value
        from the parent's point of view, normalised time)."""
        ev = self._node_eval(node)
        legal = torch.tensor([self.tokenizer.token_to_id[m] for m in node.legal_moves], dtype=torch.int64)
        policy = F.softmax(ev.logits[legal], 0).tolist()
        pov = 1 if not node.game.white_to_move else -1  # black to move: the parent was white
        return policy, pov * ev.value, ev.time

    def _expand(self, node: MCTSNode, policy: list) -> None:
        kv = self._kv if self._kv is not None and self._kv.active else None
        game = node.game
        for action, prior in zip(node.legal_moves, policy):
            child = MCTSNode(prior, parent_game=game, move=action)
            if kv is not None:
                kv.attach(node, child, action)
            node.children[action] = child

    def evaluate_node(self, node: MCTSNode) -> float:
        tv = self._terminal_value(node)
        if tv is not None:
            return tv
        policy, value, _ = self._evaluate(node)
        self._expand(node, policy)
        return 0.0 if self.dummy_value_function else value

    def select_child(self, node: MCTSNode) -> MCTSNode:
        """The first child of maximal ``ucb_score`` (as max() picks it),
        with ucb_score's arithmetic in its order and the parent's terms
        computed once."""
        if type(self).ucb_score is not MCTS.ucb_score:
            return max(node.children.values(), key=lambda child: self.ucb_score(node, child))
        pb_base = math.log((node.visit_count + self.c_base + 1) / self.c_base) + self.c_puct
        sq = math.sqrt(node.visit_count)
        best, best_s = None, None
        for child in node.children.values():
            n = child.visit_count
            s = pb_base * (sq / (1 + n)) * child.prior + (child.value_sum / n if n else 0.0)
            if best is None or s > best_s:
                best, best_s = child, s
        return best

    def ucb_score(self, parent: MCTSNode, child: MCTSNode) -> float:
        pb_c = math.log((parent.visit_count + self.c_base + 1) / self.c_base) + self.c_puct
        pb_c *= math.sqrt(parent.visit_count) / (1 + child.visit_count)
        return pb_c * child.prior + child.value()

    def backup(self, search_path: list, value: float) -> None:
        for node in search_path[::-1]:
            node.value_sum += value
            node.visit_count += 1
            value = -value

    def _simulate(self, root: MCTSNode, n_sims: int) -> None:
        if self.leaf_batch > 1 and self._kv is not None and self._kv.active:
            return self._simulate_batched(root, n_sims)
        for _ in range(n_sims):
            node = root
            search_path = [node]
            while node.expanded() and len(search_path) <= self.depth_limit:
                node = self.select_child(node)
                search_path.append(node)
            value = self.evaluate_node(node)
            self.backup(search_path, value)

    def _simulate_batched(self, root: MCTSNode, n_sims: int) -> None:
        """Opt-in leaf batching: each round selects up to ``leaf_batch``
        paths, the later ones under the virtual loss of the earlier ones,
        evaluates the distinct leaves in one extend call, then backs every
        path up with its leaf's value (a leaf picked twice is evaluated once
        and backed up twice)."""
        done = 0
        while done < n_sims:
            b = min(self.leaf_batch, n_sims - done)
            paths = []
            for _ in range(b):
                node = root
                path = [node]
                while node.expanded() and len(path) <= self.depth_limit:
                    node = self.select_child(node)
                    path.append(node)
                virtual_loss_apply(path, +1)
                paths.append(path)
            for path in paths:
                virtual_loss_apply(path, -1)
            leaves = list({id(p[-1]): p[-1] for p in paths}.values())
            batch = [n for n in leaves if not n.expanded() and self._kv.can_extend(n)
                     and self._terminal_value(n) is None]
            if batch:
                self._kv.evaluate(batch)  # memoised; evaluate_node below reads the results
            values = {id(n): self.evaluate_node(n) for n in leaves}
            for path in paths:
                self.backup(path, values[id(path[-1])])
            done += b

    def _kv_begin(self, root: MCTSNode, game: Game, max_nodes: int) -> Optional[NodeEval]:
        if not self.kv_cache:
            return None
        if self._kv is None:
            self._kv = KVSearchCache(self.model.engine, self.tokenizer, graph=self.kv_graph)
        return self._kv.begin(root, game, max_nodes)

    def _kv_end(self) -> None:
        if self._kv is not None:
            self._kv.end()

    def _final_policy(self, root: MCTSNode, legal_moves: list, policy_score: ScoreResult) -> ScoreResult:
        visit_counts = torch.FloatTensor([root.children[m].visit_count for m in legal_moves])
        if not self.kl_reg_solution:
            return ScoreResult(visit_counts / visit_counts.sum(), policy_score.think_time, policy_score.resigned)
        priors = torch.FloatTensor([root.children[m].prior for m in legal_moves])
        values = torch.FloatTensor([root.children[m].value() for m in legal_moves])
        return ScoreResult(kl_regularised_policy(priors, values, visit_counts, self.c_puct),
                           policy_score.think_time, policy_score.resigned)

    def score_full(self, game: Game, legal_moves: list[str]) -> ScoreResult:
        root = MCTSNode(0.0, game)
        ev = self._kv_begin(root, game, pool_nodes_for(self.n_sims, self.leaf_batch))
        try:
            # with the KV cache the root's one evaluation serves both calls
            policy_score = self._score(game, legal_moves, ev) if ev is not None else super().score_full(game, legal_moves)
            self.evaluate_node(root)
            self._simulate(root, self.n_sims)
        finally:
            self._kv_end()
        self.total_rollouts += self.n_sims
        return self._final_policy(root, legal_moves, policy_score)

    def run_stats(self) -> dict:
        st = {"total_rollouts": self.total_rollouts}
        if self._kv is not None:
            st["kv_leaf_evaluations"] = self._kv.n_evals
            st["kv_graph_replays"] = self._kv.n_graph
        return st


class AdaptiveMCTS(MCTS):
    def init(self, mean_n_sims: int = 50, depth_limit: int = 100, scale_c_puct: bool = True, c_puct: float = 1.25,
             c_base: float = 19652.0, dummy_value_function: bool = False, kl_reg_solution: bool = True,
             use_human_move_time: bool = False, conversion_strategy: str = "linear", kv_cache: bool = False,
             leaf_batch: int = 1, kv_graph: bool = True, **kwargs) -> None:
        Policy.init(self, **kwargs)
        self.mean_n_sims = mean_n_sims
        self.depth_limit = depth_limit
        self.scale_c_puct = scale_c_puct
        self.unscaled_c_puct = c_puct
        self.c_puct = c_puct
        self.c_base = c_base
        self.dummy_value_function = dummy_value_function
        self.kl_reg_solution = kl_reg_solution
        self.use_human_move_time = use_human_move_time
        assert conversion_strategy in ["linear", "binary"]
        self.conversion_strategy = conversion_strategy
        self.total_rollouts = 0
        self._init_kv(kv_cache, leaf_batch, kv_graph)

    def convert_time_to_sims(self, time_encoding: float) -> int:
        """decode.py:503-516."""
        if self.conversion_strategy == "linear":
            scale = self.mean_n_sims * TIME_STDEV / TIME_MEAN
            n_sims = round(scale * time_encoding + self.mean_n_sims)
        else:
            n_sims = 0 if time_encoding < 0 else self.mean_n_sims
        return 0 if n_sims < 0 else (200 if n_sims > 200 else n_sims)

    def evaluate_root(self, node: MCTSNode):
        """decode.py:518-573: (value, n_sims, think_time)."""
        oc = node.board.outcome()
        if oc is not None:
            _, winner = oc
            if winner is None:
                return 0.0, 1, 0.0
            assert winner != node.game.white_to_move
            return 1.0, 1, 0.0
        policy, value, time_encoding = self._evaluate(node)
        think_time = undo_time_normalization(time_encoding)
        if self.use_human_move_time:
            assert node.game.next_move_seconds is not None, "missing human move seconds"
            time_encoding = apply_time_normalization(node.game.next_move_seconds)
        n_sims = self.convert_time_to_sims(time_encoding)
        self._expand(node, policy)
        return (0.0 if self.dummy_value_function else value), n_sims, think_time

    def score_full(self, game: Game, legal_moves: list[str]) -> ScoreResult:
        root = MCTSNode(0.0, game)
        ev = self._kv_begin(root, game, pool_nodes_for(200, self.leaf_batch))  # n_sims <= 200 (:516)
        try:
            policy_score = self._score(game, legal_moves, ev) if ev is not None else Policy.score_full(self, game, legal_moves)
            _, n_sims, _ = self.evaluate_root(root)
            self.total_rollouts += n_sims
            if n_sims == 0:
                return ScoreResult(torch.FloatTensor([root.children[m].prior for m in legal_moves]),
                                   policy_score.think_time, policy_score.resigned)
            if self.scale_c_puct:
                self.c_puct = self.unscaled_c_puct * math.sqrt(self.mean_n_sims) / math.sqrt(n_sims)
            self._simulate(root, n_sims)
        finally:
            self._kv_end()
        return self._final_policy(root, legal_moves, policy_score)


DECODE_STRATEGIES = {
    "policy": Policy,
    "mcts": MCTS,
    "adaptive-mcts": AdaptiveMCTS,
}
