"""KV-cached leaf evaluation for the MCTS strategies.

The reference evaluates every search node with a full-prefix forward at
batch 1 (``MCTS.evaluate_node``, src/evaluation/decode.py:356-360; the root
twice, :407 and :410).  Here one search keeps a paged KV pool:

* the root's game is prefilled once, its keys and values written to the
  pool's first blocks; the outputs serve both the root's policy score and its
  expansion (the duplicate root forward disappears, with identical results);
* a node is its parent's game plus one move token (``Game.make_move``,
  data.py:63-73), so its evaluation is ONE new token: ``Engine.extend`` with
  the root's blocks as the prefix and, as private keys, the pool slots of its
  evaluated ancestors below the root and its own new slot, which receives its
  keys and values for its descendants.

The results equal the full recompute up to floating-point summation order:
the same model, the same tokens, the same positions.  Where a node's game
does not tokenize as its parent's tokens plus one move (a root with a result
or termination token, data.py:262-268) or exceeds the 512-token window (the
reference keeps the first 512 tokens, data.py:290), evaluation falls back to
the full forward of the model call.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

KV_BLOCK = 16


@dataclass
class NodeEval:
    """What a search reads from one evaluation: the last token's logits
    (fp32, host), the raw value head output (tanh applied) and the time head."""
    logits: torch.Tensor
    value: float
    time: float


class KVSearchCache:
    """Paged KV state of one search at a time on one engine.  The pool is
    kept and reused across searches; it grows when a search needs more."""

    def __init__(self, engine, tokenizer):
        self.eng = engine
        self.tok = tokenizer
        self.max_length = engine.cfg.max_length
        self.pool: Optional[torch.Tensor] = None
        self.status: Optional[torch.Tensor] = None  # device int32 [1]: validation flags of the last call
        self.active = False
        self.n_evals = 0  # leaf evaluations made through extend (statistics)

    # ----------------------------------------------------------------- root
    def begin(self, root, game, max_nodes: int) -> Optional[NodeEval]:
        """Prefill the root's game into the pool and return its evaluation,
        or None (and stay inactive) when the game cannot be extended move by
        move (see the module docstring)."""
        self.active = False
        self.root = None
        if game.outcome is not None or game.normal_termination:
            return None
        words = self.tok.tokenize(game)
        P = len(words)
        if P >= self.max_length:
            return None
        dev = self.eng.device
        pb = (P + KV_BLOCK - 1) // KV_BLOCK
        need = pb + (max_nodes + KV_BLOCK - 1) // KV_BLOCK
        if self.pool is None or self.eng.pool_blocks(self.pool) < need:
            self.pool = None
            self.pool = self.eng.new_kv_pool(need)
        self.n_slots = self.eng.pool_blocks(self.pool) * KV_BLOCK
        self.prefix_len = P
        self.table = torch.arange(pb, dtype=torch.int32, device=dev)[None].contiguous()
        self.next_slot = pb * KV_BLOCK
        if self.status is None:
            self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        out = self.eng.prefill(words, np.array([P], np.int32), kv_pool=self.pool, kv_block_table=self.table,
                               status=self.status)
        ev = NodeEval(out.logits[0].float().cpu(), float(out.value[0].item()), float(out.time[0].item()))
        self._check_status("prefill")
        root._kv_path = []
        root._kv_eval = ev
        self.root = root
        self.active = True
        return ev

    def _check_status(self, what: str) -> None:
        """The device-side validation of the last call (read after its
        outputs were copied, so it costs no extra synchronisation): a slot
        or block outside the pool, a bad key count or position."""
        st = int(self.status.item())
        if st != 0:
            raise RuntimeError(f"KV search {what} rejected its inputs on the device (status {st})")

    def end(self) -> None:
        self.active = False
        self.root = None

    # ---------------------------------------------------------------- nodes
    def attach(self, parent, child, move: str) -> None:
        """Record, at expansion, what the child's evaluation needs."""
        child._kv_parent = parent
        child._kv_token = self.tok.token_to_id.get(move, self.tok.unk_token_id)

    def can_extend(self, node) -> bool:
        if not self.active:
            return False
        if getattr(node, "_kv_eval", None) is not None:
            return True
        parent = getattr(node, "_kv_parent", None)
        if parent is None or getattr(parent, "_kv_path", None) is None:
            return False
        return self.prefix_len + len(parent._kv_path) + 1 <= self.max_length

    def evaluate(self, nodes: list) -> list[NodeEval]:
        """Evaluate nodes that ``can_extend`` in one extend call (one token
        each, all sharing the root's prefix); memoised nodes are not redone."""
        todo = [n for n in nodes if getattr(n, "_kv_eval", None) is None]
        if todo:
            if self.next_slot + len(todo) > self.n_slots:
                raise RuntimeError("KV search pool exhausted (more evaluations than the search was sized for)")
            paths = []
            for n in todo:
                paths.append(n._kv_parent._kv_path + [self.next_slot])
                self.next_slot += 1
            k = np.array([len(p) for p in paths], np.int32)
            extras = np.zeros((len(todo), int(k.max())), np.int32)
            for i, p in enumerate(paths):
                extras[i, : len(p)] = p
            ids = np.array([n._kv_token for n in todo], np.int32)
            pos = (self.prefix_len + k - 1).astype(np.int32)
            out = self.eng.extend(ids, pos, [len(todo)], np.array([self.prefix_len], np.int32), self.table,
                                  extras, k, self.pool, status=self.status)
            logits = out.logits.float().cpu()
            value = out.value.cpu().tolist()
            time = out.time.cpu().tolist()
            self._check_status("extend")
            for i, n in enumerate(todo):
                n._kv_path = paths[i]
                n._kv_eval = NodeEval(logits[i], value[i], time[i])
            self.n_evals += len(todo)
        return [n._kv_eval for n in nodes]


def pool_nodes_for(n_sims: int, leaf_batch: int) -> int:
    """Upper bound of the evaluations one search makes: one per simulation
    (a batch evaluates each distinct leaf once)."""
    return max(1, n_sims) + max(0, leaf_batch - 1)


def virtual_loss_apply(path: list, sign: int) -> None:
    """Virtual loss on a selected path (opt-in leaf batching): each node
    below the root counts one more visit with value -1 from its parent's
    point of view, so later selections in the same batch prefer other
    paths; ``sign=-1`` removes it."""
    for node in path[1:]:
        node.visit_count += sign
        node.value_sum -= sign
