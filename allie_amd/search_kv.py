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

A single leaf (the sequential search's case) is evaluated by replaying a
HIP graph of the allocation-free extend (``allie_extend_noalloc``) captured
once per pool: its inputs -- the token, its position, its key count and
pool slots, the root's prefix length and block table -- sit in one device
buffer refreshed by one pinned copy, and its outputs come back in one copy.
The graph runs the same kernels with the same arguments as the eager call,
so its results are identical; it removes the per-kernel launch gaps and the
host's argument staging (about 170 launches per leaf).

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


class LeafGraph:
    """One-token leaf evaluation over a search's pool, replayed from a HIP
    graph.  Inputs live in one device int32 buffer ``[token, pos, n_keys,
    prefix_len, 0, 1 (group starts), slots[MAX_EXTRA], table[max_blocks]]``;
    outputs (logits, value, time, max logit, lse, top-1, status) in one fp32
    buffer.  Captured for one pool; ``eligible`` says whether a leaf fits
    (at most MAX_EXTRA private keys)."""

    MAX_EXTRA = 64

    def __init__(self, engine, pool: torch.Tensor, prefix_len: int, table: np.ndarray, slot: int):
        from .engine import PrefillResult

        self.eng, self.pool = engine, pool
        dev = engine.device
        V = engine.cfg.vocab_size
        self.mb = (engine.cfg.max_length + KV_BLOCK - 1) // KV_BLOCK
        E, MB = self.MAX_EXTRA, self.mb
        self.n_in = 6 + E + MB
        self.host = torch.zeros(self.n_in, dtype=torch.int32, pin_memory=True)
        self.h = self.host.numpy()
        self.inp = torch.zeros(self.n_in, dtype=torch.int32, device=dev)
        self.gs_host = np.array([0, 1], np.int32)
        self.outbuf = torch.zeros(V + 8, dtype=torch.float32, device=dev)
        self.out_host = torch.zeros(V + 8, dtype=torch.float32, pin_memory=True)
        ob = self.outbuf
        self.out = PrefillResult(logits=ob[:V].view(1, V), value=ob[V:V + 1], time=ob[V + 1:V + 2],
                                 top1=ob[V + 4:V + 5].view(torch.int32), max_logit=ob[V + 2:V + 3],
                                 lse=ob[V + 3:V + 4])
        self.status = ob[V + 5:V + 6].view(torch.int32)
        self.V = V
        # a valid leaf for the eager warm-up: the next free slot, overwritten by
        # the first real leaf
        self.set_root(prefix_len, table)
        self._fill(0, prefix_len, [slot])
        self.inp.copy_(self.host)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self._launch()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, capture_error_mode="thread_local"):
            self._launch()

    def _launch(self):
        E, MB, i = self.MAX_EXTRA, self.mb, self.inp
        self.eng.extend_noalloc_raw(i[0:1], i[1:2], self.gs_host, i[4:6], i[3:4], i[6 + E:6 + E + MB].view(1, MB),
                                    i[6:6 + E].view(1, E), i[2:3], self.pool, self.out, self.status)

    def set_root(self, prefix_len: int, table: np.ndarray) -> None:
        E = self.MAX_EXTRA
        self.h[3], self.h[4], self.h[5] = prefix_len, 0, 1
        self.h[6 + E:] = 0
        self.h[6 + E:6 + E + len(table)] = table

    def _fill(self, token: int, pos: int, slots: list) -> None:
        self.h[0], self.h[1], self.h[2] = token, pos, len(slots)
        self.h[6:6 + len(slots)] = slots

    def eligible(self, n_keys: int) -> bool:
        return n_keys <= self.MAX_EXTRA

    def run(self, token: int, pos: int, slots: list) -> "NodeEval":
        self._fill(token, pos, slots)
        self.inp.copy_(self.host, non_blocking=True)
        self.graph.replay()
        self.out_host.copy_(self.outbuf, non_blocking=True)
        torch.cuda.current_stream().synchronize()
        o = self.out_host
        st = int(o[self.V + 5:self.V + 6].view(torch.int32).item())
        if st != 0:
            raise RuntimeError(f"KV search leaf rejected its inputs on the device (status {st})")
        return NodeEval(o[:self.V].clone(), float(o[self.V]), float(o[self.V + 1]))


class KVSearchCache:
    """Paged KV state of one search at a time on one engine.  The pool is
    kept and reused across searches; it grows when a search needs more.
    ``graph`` (default on): single leaves replay a captured HIP graph
    (``LeafGraph``); off, every leaf is an eager ``Engine.extend``."""

    def __init__(self, engine, tokenizer, graph: bool = True):
        self.eng = engine
        self.tok = tokenizer
        self.max_length = engine.cfg.max_length
        self.pool: Optional[torch.Tensor] = None
        self.status: Optional[torch.Tensor] = None  # device int32 [1]: validation flags of the last call
        self.active = False
        self.n_evals = 0  # leaf evaluations made through extend (statistics)
        self.use_graph = graph
        self.leaf_graph: Optional[LeafGraph] = None
        self.n_graph = 0  # of which replayed from the graph

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
            self.leaf_graph = None  # captured for the old pool
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
        if self.use_graph:
            table = np.arange(pb, dtype=np.int32)
            if self.leaf_graph is None:
                self.leaf_graph = LeafGraph(self.eng, self.pool, P, table, self.next_slot)
            else:
                self.leaf_graph.set_root(P, table)
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
        lg = self.leaf_graph if self.use_graph else None
        if len(todo) == 1 and lg is not None and lg.eligible(len(todo[0]._kv_parent._kv_path) + 1):
            n = todo[0]
            if self.next_slot + 1 > self.n_slots:
                raise RuntimeError("KV search pool exhausted (more evaluations than the search was sized for)")
            path = n._kv_parent._kv_path + [self.next_slot]
            self.next_slot += 1
            n._kv_eval = lg.run(n._kv_token, self.prefix_len + len(path) - 1, path)
            n._kv_path = path
            self.n_evals += 1
            self.n_graph += 1
        elif todo:
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
