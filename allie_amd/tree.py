"""MCTS tree expansion over a prefix-shared paged KV cache.

The reference evaluates every search node with a full recompute of its game
at batch 1 (``MCTS.evaluate_node``, src/evaluation/decode.py:356-360).  Here a
whole tree level is one ``Engine.extend`` call: the roots' games are
prefilled into the pool once, and each node of level k is a single new token
that attends its root's cached prefix, its k-1 cached ancestors and itself.

``TreeLayout`` is the slot arithmetic of a complete tree (R roots, branching
b, depth D): level-k node j (root-major order, j < R b^k) has root j // b^k,
parent j // b at level k-1, and its keys/values in pool slot
``node_slot(k, j)``.  Root r's prefix occupies ``prefix_blocks`` consecutive
blocks from ``r * prefix_blocks``; node slots follow.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .vocab import NUM_CHESS_MOVES

KV_BLOCK = 16


@dataclass(frozen=True)
class TreeLayout:
    n_roots: int
    prefix_len: int
    branching: int
    depth: int

    @property
    def prefix_blocks(self) -> int:
        return (self.prefix_len + KV_BLOCK - 1) // KV_BLOCK

    def level_size(self, k: int) -> int:
        return self.n_roots * self.branching ** k

    @property
    def n_nodes(self) -> int:
        return sum(self.level_size(k) for k in range(1, self.depth + 1))

    @property
    def node_block0(self) -> int:
        return self.n_roots * self.prefix_blocks

    @property
    def n_blocks(self) -> int:
        return self.node_block0 + (self.n_nodes + KV_BLOCK - 1) // KV_BLOCK

    def level_slot0(self, k: int) -> int:
        return self.node_block0 * KV_BLOCK + sum(self.level_size(l) for l in range(1, k))

    def node_slot(self, k: int, j) -> np.ndarray:
        return self.level_slot0(k) + np.asarray(j, dtype=np.int64)

    def root_table(self) -> np.ndarray:
        """[R, prefix_blocks] block ids of each root's prefix."""
        return (np.arange(self.n_roots)[:, None] * self.prefix_blocks
                + np.arange(self.prefix_blocks)[None, :]).astype(np.int32)

    def level_extras(self, k: int) -> np.ndarray:
        """[R b^k, k] slots of each level-k node's ancestors (level 1 first)
        and of the node itself."""
        j = np.arange(self.level_size(k), dtype=np.int64)
        cols = [self.node_slot(l, j // self.branching ** (k - l)) for l in range(1, k + 1)]
        return np.stack(cols, axis=1).astype(np.int32)

    def level_positions(self, k: int) -> np.ndarray:
        return np.full(self.level_size(k), self.prefix_len + k - 1, dtype=np.int32)


def synthetic_tree(layout: TreeLayout, seed: int = 3):
    """Root games and child move ids drawn uniformly from the move vocabulary
    (the C3 workload): returns (prefix ids [R, P], [ids of level 1..D])."""
    rng = np.random.default_rng(seed)
    prefixes = rng.integers(0, NUM_CHESS_MOVES, (layout.n_roots, layout.prefix_len)).astype(np.int32)
    levels = [rng.integers(0, NUM_CHESS_MOVES, layout.level_size(k)).astype(np.int32)
              for k in range(1, layout.depth + 1)]
    return prefixes, levels


def node_path(layout: TreeLayout, prefixes, levels, k: int, j: int) -> list[int]:
    """Token ids of level-k node j's whole game (prefix, ancestors, itself):
    what the reference recomputes for this node."""
    root = j // layout.branching ** k
    path = list(prefixes[root])
    for l in range(1, k + 1):
        path.append(int(levels[l - 1][j // layout.branching ** (k - l)]))
    return path


class TreeExpansion:
    """Prefill the roots, then evaluate the tree level by level on the GPU."""

    def __init__(self, engine, layout: TreeLayout, seed: int = 3):
        import torch

        self.eng, self.layout = engine, layout
        self.prefixes, self.levels = synthetic_tree(layout, seed)
        dev = engine.device
        self.pool = engine.new_kv_pool(layout.n_blocks)
        self.table = torch.from_numpy(layout.root_table()).to(dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        # per-level device inputs, built once
        self.inputs = []
        for k in range(1, layout.depth + 1):
            n = layout.level_size(k)
            self.inputs.append(dict(
                ids=torch.from_numpy(self.levels[k - 1]).to(dev),
                pos=torch.from_numpy(layout.level_positions(k)).to(dev),
                extras=torch.from_numpy(layout.level_extras(k)).to(dev),
                n_extra=torch.full((n,), k, dtype=torch.int32, device=dev),
                prefix_len=torch.full((layout.n_roots,), layout.prefix_len, dtype=torch.int32, device=dev),
                sizes=[layout.branching ** k] * layout.n_roots,
            ))

    def prefill_roots(self):
        lay = self.layout
        words = self.prefixes.reshape(-1).astype(np.uint32)
        lens = np.full(lay.n_roots, lay.prefix_len, np.int32)
        import torch

        wd = torch.from_numpy(words.view(np.int32)).to(self.eng.device)
        return self.eng.prefill(wd, lens, kv_pool=self.pool, kv_block_table=self.table, want_logits=False)

    def expand_level(self, k: int, want_logits: bool = False, out=None, want_raw_logits: bool = False):
        x = self.inputs[k - 1]
        return self.eng.extend(x["ids"], x["pos"], x["sizes"], x["prefix_len"], self.table, x["extras"],
                               x["n_extra"], self.pool, want_logits=want_logits, status=self.status, out=out,
                               want_raw_logits=want_raw_logits)
