"""Continuous-batching self-play decode over the paged KV cache.

The reference plays one move per model call: ``Policy.score_full`` runs a
full forward of the whole game at batch 1 for every appended move
(src/evaluation/decode.py:199-226, argmax at decode.py:112).  Here S slots
each hold a game; one step appends the greedy move of every slot with a
single ``Engine.extend`` over cached keys and values, finished games are
evicted and their slots refilled (prefill of the new game's prefix into the
slot's blocks), with no host synchronisation in the loop: the host knows
every game's length in advance, and the moves themselves stay on the GPU.

KV layout: slot s owns the pool blocks [s * B, (s + 1) * B) with
B = max_len / 16, so a slot's block table never changes (1,024 slots of the
medium model at 512 positions take 48 GiB of the 288 GiB HBM).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .vocab import NUM_CHESS_MOVES

KV_BLOCK = 16


@dataclass
class GameQueue:
    """Seeded synthetic games (the C4 workload): prefix length U[1, 50], game
    length min(Geometric(1/80), cap), at least prefix + 1; prefix moves uniform
    over the move vocabulary."""

    seed: int = 4
    mean_len: float = 80.0
    cap: int = 512
    prefix_lo: int = 1
    prefix_hi: int = 50
    rng: np.random.Generator = field(init=False)

    def __post_init__(self):
        self.rng = np.random.default_rng(self.seed)

    def draw(self, n: int):
        """n games: (prefix ids list, prefix lengths [n], total lengths [n])."""
        P = self.rng.integers(self.prefix_lo, self.prefix_hi + 1, n)
        G = np.minimum(self.rng.geometric(1.0 / self.mean_len, n), self.cap)
        total = np.maximum(G, P + 1)
        total = np.minimum(total, self.cap)
        prefixes = [self.rng.integers(0, NUM_CHESS_MOVES, int(p)).astype(np.int32) for p in P]
        return prefixes, P.astype(np.int32), total.astype(np.int32)


class PinnedUploader:
    """Host -> device copies of small int32 arrays without a stream sync: each
    array goes through one of a ring of pinned buffers, reused only after the
    event recorded behind its last copy has completed."""

    def __init__(self, device, capacity: int, ring: int = 8):
        import torch

        self.torch = torch
        self.device = device
        self.host = [torch.empty(capacity, dtype=torch.int32, pin_memory=True) for _ in range(ring)]
        self.dev = [torch.empty(capacity, dtype=torch.int32, device=device) for _ in range(ring)]
        self.ev = [None] * ring
        self.i = 0

    def __call__(self, a: np.ndarray):
        torch = self.torch
        i = self.i
        self.i = (i + 1) % len(self.host)
        if self.ev[i] is not None:
            self.ev[i].synchronize()
        n = len(a)
        assert n <= self.host[i].numel()
        self.host[i][:n].copy_(torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)))
        d = self.dev[i][:n]
        d.copy_(self.host[i][:n], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.ev[i] = ev
        return d


class ContinuousBatcher:
    """``record=True`` (tests) keeps each slot's game on the host and every
    (game so far, greedy move predicted for it) pair in ``checks``; it reads
    the moves back every step, so it synchronises the stream."""

    def __init__(self, engine, n_slots: int = 1024, queue: GameQueue | None = None, record: bool = False):
        import torch

        self.torch = torch
        self.eng = engine
        self.S = n_slots
        self.max_len = engine.cfg.max_length
        self.bps = (self.max_len + KV_BLOCK - 1) // KV_BLOCK  # blocks per slot
        dev = engine.device
        self.pool = engine.new_kv_pool(n_slots * self.bps)
        self.table = (torch.arange(n_slots, dtype=torch.int32, device=dev)[:, None] * self.bps
                      + torch.arange(self.bps, dtype=torch.int32, device=dev)[None, :]).contiguous()
        self.queue = queue or GameQueue()
        self.up = PinnedUploader(dev, capacity=max(4096, n_slots * 64))
        # per-slot state: host knows lengths, the device holds the moves
        self.cur = np.zeros(n_slots, np.int32)    # tokens cached per slot
        self.total = np.zeros(n_slots, np.int32)  # game length to reach
        self.cur_dev = torch.zeros(n_slots, dtype=torch.int32, device=dev)
        self.next_tok = torch.zeros(n_slots, dtype=torch.int32, device=dev)
        self.ones = torch.ones(n_slots, dtype=torch.int32, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        self.games_started = 0
        self.tokens = 0
        self.record = record
        self.games = [[] for _ in range(n_slots)]
        self.checks = []  # (game so far, predicted next move) when recording
        self.refill(np.arange(n_slots))

    def refill(self, slots: np.ndarray) -> None:
        """Start new games in `slots`: prefill their prefixes into the slots'
        blocks; the prefill's greedy move is the first move to append."""
        if len(slots) == 0:
            return
        torch = self.torch
        prefixes, P, total = self.queue.draw(len(slots))
        words = self.up(np.concatenate(prefixes))
        idx = self.up(slots.astype(np.int32)).long()
        out = self.eng.prefill(words, P, kv_pool=self.pool, kv_block_table=self.table[idx].contiguous(),
                               want_logits=False)
        self.next_tok.index_copy_(0, idx, out.top1)
        self.cur_dev.index_copy_(0, idx, self.up(P))
        self.cur[slots] = P
        self.total[slots] = total
        self.games_started += len(slots)
        if self.record:
            top = out.top1.cpu().numpy()
            for k, s in enumerate(slots):
                self.games[s] = [int(x) for x in prefixes[k]]
                self.checks.append((list(self.games[s]), int(top[k])))

    def step(self) -> int:
        """Append one greedy move to every slot; evict and refill finished
        games.  Returns the number of moves appended."""
        torch = self.torch
        cur = self.cur_dev
        fed = self.next_tok.cpu().numpy() if self.record else None
        slot = torch.gather(self.table, 1, (cur // KV_BLOCK).long()[:, None])[:, 0] * KV_BLOCK + cur % KV_BLOCK
        out = self.eng.extend(self.next_tok, cur, [1] * self.S, cur, self.table, slot[:, None].contiguous(),
                              self.ones, self.pool, want_logits=False, status=self.status)
        if self.record:
            top = out.top1.cpu().numpy()
            for s in range(self.S):
                self.games[s].append(int(fed[s]))
                self.checks.append((list(self.games[s]), int(top[s])))
        self.next_tok.copy_(out.top1)
        self.cur_dev += 1
        self.cur += 1
        self.tokens += self.S
        done = np.nonzero(self.cur >= self.total)[0]
        self.refill(done)
        return self.S
