"""Continuous-batching self-play decode over the paged KV cache.

The reference plays one move per model call: ``Policy.score_full`` runs a
full forward of the whole game at batch 1 for every appended move
(src/evaluation/decode.py:199-226, argmax at decode.py:112).  Here S slots
each hold a game; one step appends the greedy move of every slot with a
single ``Engine.extend`` over cached keys and values, finished games are
evicted and their slots refilled (the new game's prefix joins the next
step's forward), with no host synchronisation in the loop: the host knows
every game's length in advance, and the moves themselves stay on the GPU.

KV layout: slot s owns the pool blocks [s * B, (s + 1) * B) with
B = max_len / 16, so a slot's block table never changes (1,024 slots of the
medium model at 512 positions take 48 GiB of the 288 GiB HBM).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Optional

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


@dataclass
class Check:
    """One recorded forward row: the first ``n`` tokens of ``game`` (a slot's
    game, appended to in place) and the greedy move predicted after them;
    ``out`` holds the row's logits, raw logits, value and time when the
    batcher was asked to keep them."""

    game: list
    n: int
    move: int
    out: Optional[dict] = None

    @property
    def ids(self) -> list:
        return self.game[: self.n]


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
    """S slots of self-play games over the paged KV cache.

    One ``step`` is one ``Engine.extend`` over every slot: a running game
    feeds its last greedy move (a one-token group over the slot's cached
    keys), a game started since the previous step feeds its whole prefix (a
    group whose prefix is the game's own P positions, written by the same
    forward; token t sees positions 0..t), so new games ride in the same
    forward as the decode steps instead of a separate prefill.  Finished games are evicted at the end of a step and their slots
    drawn anew for the next one.  All integer metadata is known on the host
    (lengths, positions, pool slots); only the moves live on the GPU, so the
    loop never synchronises.

    ``record=True`` (tests) keeps each slot's game on the host and every
    (game so far, greedy move predicted for it) pair in ``checks``; it reads
    the moves back every step, so it synchronises the stream.  ``keep``
    (with ``record``), given a row's context length and whether the row is a
    new game's first move, says whether to keep that row's logits, raw
    logits, value and time as well; a step with such a row computes the full
    logits."""

    def __init__(self, engine, n_slots: int = 1024, queue: GameQueue | None = None, record: bool = False,
                 keep: Optional[Callable[[int, bool], bool]] = None):
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
        self.up = PinnedUploader(dev, capacity=max(8192, n_slots * 512))
        self.cur = np.zeros(n_slots, np.int32)    # tokens cached per slot
        self.total = np.zeros(n_slots, np.int32)  # game length to reach
        self.next_tok = torch.zeros(n_slots, dtype=torch.int32, device=dev)
        self.ones = torch.ones(n_slots * 64, dtype=torch.int32, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        self.games_started = 0
        self.tokens = 0        # moves appended
        self.keys_read = 0     # keys attended per layer, summed over steps
        self.fed = 0           # tokens fed (moves and new games' prefixes)
        self.decode_keys = 0   # keys attended by the running games' one-token steps
        self.decoded = 0       # one-token steps (running games)
        self.record = record
        self.keep = keep if record else None
        self.games = [[] for _ in range(n_slots)]
        self.checks: list[Check] = []  # when recording
        self.pending = {}  # slot -> (prefix ids, total length) to start next step
        self._draw(np.arange(n_slots))

    def _draw(self, slots: np.ndarray) -> None:
        if len(slots) == 0:
            return
        prefixes, P, total = self.queue.draw(len(slots))
        for k, s in enumerate(slots):
            self.pending[int(s)] = (prefixes[k], int(total[k]))
        self.games_started += len(slots)

    def step(self) -> int:
        """Append one greedy move to every running game and start the pending
        ones; evict finished games.  Returns the number of moves appended."""
        torch = self.torch
        pend = sorted(self.pending)
        is_pend = np.zeros(self.S, bool)
        is_pend[pend] = True
        R = np.nonzero(~is_pend)[0].astype(np.int32)  # running slots, one token each
        nR = len(R)
        pre = [self.pending[s][0] for s in pend]
        Ps = np.array([len(p) for p in pre], np.int32)
        nP = int(Ps.sum())
        n = nR + nP
        G = nR + len(pend)
        slot_stride = self.bps * KV_BLOCK  # pool slots per game slot
        # host metadata: one pinned upload, sliced on the device
        pos_p = np.concatenate([np.arange(P, dtype=np.int32) for P in Ps]) if pend else np.zeros(0, np.int32)
        pos = np.concatenate([self.cur[R], pos_p])
        prefix_len = np.concatenate([self.cur[R], Ps])
        gslot = np.concatenate([R, np.array(pend, np.int32)])
        # each token's only extra is its own pool slot (its key's position)
        own = np.concatenate([R, np.repeat(np.array(pend, np.int32), Ps)]) * slot_stride + pos
        ids_p = np.concatenate(pre).astype(np.int32) if pend else np.zeros(0, np.int32)
        meta = self.up(np.concatenate([pos, prefix_len, gslot, own, ids_p]))
        o = np.cumsum([0, n, G, G, n, nP])
        pos_t, pl_t, gs_t, own_t, idsp_t = (meta[o[i]:o[i + 1]] for i in range(5))
        gs_l = gs_t.long()
        ids = torch.cat([self.next_tok.index_select(0, gs_l[:nR]), idsp_t])
        fed = ids[:nR].cpu().numpy() if self.record else None
        # outputs: running games' next moves, new games' first moves (last prefix token)
        last = np.concatenate([np.arange(nR), nR + np.cumsum(Ps) - 1]).astype(np.int32) if pend else None
        ctx = np.concatenate([self.cur[R] + 1, Ps]) if pend else self.cur[R] + 1  # context of each output row
        kept = [j for j, c in enumerate(ctx) if self.keep(int(c), j >= nR)] if self.keep else []
        out = self.eng.extend(ids, pos_t, [1] * nR + Ps.tolist(), pl_t, self.table.index_select(0, gs_l),
                              own_t[:, None], self.ones[:n] if n <= len(self.ones) else torch.ones(
                                  n, dtype=torch.int32, device=meta.device),
                              self.pool, want_logits=bool(kept), want_raw_logits=bool(kept), status=self.status)
        if pend:
            last_t = self.up(last).long()
            self.next_tok.index_copy_(0, gs_l, out.top1.index_select(0, last_t))
        else:
            self.next_tok.index_copy_(0, gs_l, out.top1)
        if self.record:
            top = out.top1.cpu().numpy()
            rows = {}
            if kept:
                sel = torch.as_tensor(last[kept] if pend else np.asarray(kept), device=out.top1.device).long()
                host = {k: getattr(out, k).index_select(0, sel).cpu().numpy()
                        for k in ("logits", "logits_raw", "value", "time")}
                rows = {j: {k: v[q] for k, v in host.items()} for q, j in enumerate(kept)}
            for k, s in enumerate(R):
                self.games[s].append(int(fed[k]))
                self.checks.append(Check(self.games[s], len(self.games[s]), int(top[k]), rows.get(k)))
            for k, s in enumerate(pend):
                self.games[s] = [int(x) for x in pre[k]]  # a new list: earlier checks keep the old game
                self.checks.append(Check(self.games[s], len(self.games[s]), int(top[last[nR + k]]), rows.get(nR + k)))
        self.keys_read += int(self.cur[R].sum()) + nR + int((Ps * (Ps + 1) // 2).sum())
        self.decode_keys += int(self.cur[R].sum()) + nR
        self.decoded += nR
        self.cur[R] += 1
        for k, s in enumerate(pend):
            self.cur[s] = Ps[k]
            self.total[s] = self.pending[s][1]
        self.pending = {}
        self.tokens += nR
        self.fed += n
        self._draw(np.nonzero(self.cur >= self.total)[0])
        return nR
