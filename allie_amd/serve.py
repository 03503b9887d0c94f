"""Batched serving of the policy systems.

The reference server (src/server/main.py:57-91) answers one connection at a
time: it reads a JSON ``Game`` (src/server/utils.py:8-23), sets the engine's
Elo for the side to move (the opponent's Elo when the system has none,
main.py:66-78), runs ``algorithm.decode_full(game)`` with a batch of one, and
sends ``{"move", "think_time", "resigned"}`` back.  Here concurrent requests
share forwards instead:

* ``PolicyBatcher`` wraps a ``policy`` strategy (``allie_amd.decode.Policy``).
  Callers ``submit(game)`` from any thread and get a future; one worker
  thread takes the pending games (up to ``max_batch``, after waiting at most
  ``max_wait_ms`` for more to arrive), runs ONE model call over them (the
  ragged prefill packs the games with no padding), and finishes each game
  exactly as ``Policy.decode_full`` would: the same scoring
  (decode.py:194-238) and the same argmax / sampling rule (decode.py:90-113).
* ``serve_socket`` speaks the reference server's protocol, one thread per
  connection, every connection feeding the same batcher.

Search systems (``mcts``, ``adaptive-mcts``) run one search per request; they
are not batched across requests here.
"""
from __future__ import annotations

import json
import queue
import socket
import threading
from concurrent.futures import Future
from dataclasses import dataclass
from typing import Optional

import torch

from .decode import DecodeResult, Policy
from .search_kv import NodeEval
from .tokenizer import Game


@dataclass
class _Request:
    game: Game
    legal: list
    future: Future


class PolicyBatcher:
    def __init__(self, strategy: Policy, max_batch: int = 64, max_wait_ms: float = 2.0):
        if not isinstance(strategy, Policy) or type(strategy).__name__ != "Policy":
            raise TypeError("PolicyBatcher batches the policy strategy only")
        if max_batch < 1:
            raise ValueError("max_batch must be >= 1")
        self.strategy = strategy
        self.max_batch = max_batch
        self.max_wait = max_wait_ms / 1000.0
        self._q: "queue.Queue[Optional[_Request]]" = queue.Queue()
        self._stop = False
        self._lock = threading.Lock()  # orders submit's check-and-enqueue against close
        self.batches = 0
        self.requests = 0
        self._worker = threading.Thread(target=self._run, name="policy-batcher", daemon=True)
        self._worker.start()

    # -------------------------------------------------------------- callers
    def submit(self, game: Game) -> Future:
        """Queue one game.  It is checked here, on the caller's thread, so a
        bad request (an illegal move in its list, a missing Elo) fails only
        its own future and never joins a shared forward."""
        f: Future = Future()
        try:
            legal = game.legal_moves
            self.strategy.tokenizer.tokenize(game)
        except Exception as e:
            f.set_exception(e)
            return f
        with self._lock:
            if self._stop:
                raise RuntimeError("batcher is closed")
            self._q.put(_Request(game, legal, f))
        return f

    def decode_full(self, game: Game, timeout: Optional[float] = None) -> DecodeResult:
        return self.submit(game).result(timeout)

    def close(self) -> None:
        with self._lock:
            if self._stop:
                return
            self._stop = True
            self._q.put(None)
        self._worker.join()

    # --------------------------------------------------------------- worker
    def _take(self) -> list:
        first = self._q.get()
        if first is None:
            return []
        batch = [first]
        while len(batch) < self.max_batch:
            try:
                r = self._q.get(timeout=self.max_wait)
            except queue.Empty:
                break
            if r is None:
                self._q.put(None)  # seen again by the loop, after this batch
                break
            batch.append(r)
        return batch

    def _run(self) -> None:
        while True:
            batch = self._take()
            if not batch:
                # closed: nothing can be queued after the sentinel, but fail
                # anything still waiting rather than leave it unresolved
                while True:
                    try:
                        r = self._q.get_nowait()
                    except queue.Empty:
                        return
                    if r is not None and not r.future.done():
                        r.future.set_exception(RuntimeError("batcher is closed"))
            try:
                self._serve(batch)
            except BaseException as e:  # every waiting caller sees the failure
                for r in batch:
                    if not r.future.done():
                        r.future.set_exception(e)

    def _serve(self, batch: list) -> None:
        st = self.strategy
        games = [r.game for r in batch]
        legal = [r.legal for r in batch]
        with torch.no_grad():
            out = st.model(**st.tokenizer.pad_and_collate(games))
        logits = out["logits"][:, -1].float().cpu()
        value = out["value_logits"][:, -1].float().cpu().tolist()
        tm = out["time_logits"][:, -1].float().cpu().tolist()
        self.batches += 1
        self.requests += len(batch)
        for i, r in enumerate(batch):
            try:
                ev = NodeEval(logits[i], value[i], tm[i])
                score = st._score(r.game, legal[i], ev)
                r.future.set_result(st._choose(r.game, legal[i], score))
            except BaseException as e:
                r.future.set_exception(e)


# ------------------------------------------------------------ socket server
def _recv_dict(conn: socket.socket) -> dict:
    """server/utils.py:12-23: read until the bytes parse as one JSON object."""
    chunks = []
    while True:
        chunk = conn.recv(8192)
        if chunk == b"":
            raise RuntimeError("socket connection broken")
        chunks.append(chunk)
        try:
            return json.loads(b"".join(chunks).decode("utf-8"))
        except json.JSONDecodeError:
            continue


def _send_dict(conn: socket.socket, d: dict) -> None:
    conn.sendall(json.dumps(d).encode("utf-8"))


def handle_request(batcher: PolicyBatcher, data: dict, system_elo: Optional[int]) -> dict:
    """main.py:64-86 for one request: the system's Elo (or the opponent's)
    on the side to move, then the batched decode."""
    game = Game(**data)
    elo = system_elo
    if elo is None:
        elo = game.black_elo if game.white_to_move else game.white_elo
    if elo is None:
        raise ValueError("no Elo for the side to move")
    if game.white_to_move:
        game.white_elo = elo
    else:
        game.black_elo = elo
    res = batcher.decode_full(game)
    return {"move": res.move, "think_time": res.think_time, "resigned": res.resigned}


def serve_socket(batcher: PolicyBatcher, port: int, host: str = "127.0.0.1", system_elo: Optional[int] = None,
                 ready: Optional[threading.Event] = None, stop: Optional[threading.Event] = None) -> None:
    """Accept connections until ``stop`` is set; each connection sends one
    JSON game and receives one JSON move (the reference protocol), handled
    on its own thread so that concurrent games share forwards."""
    srv = socket.socket(socket.AF_INET, socket.SOCK_STREAM)
    srv.setsockopt(socket.SOL_SOCKET, socket.SO_REUSEADDR, 1)
    srv.bind((host, port))
    srv.listen(64)
    srv.settimeout(0.2)
    if ready is not None:
        ready.set()

    def one(conn):
        with conn:
            try:
                _send_dict(conn, handle_request(batcher, _recv_dict(conn), system_elo))
            except Exception as e:  # the reference drops the connection on errors
                try:
                    _send_dict(conn, {"error": str(e)})
                except OSError:
                    pass

    try:
        while stop is None or not stop.is_set():
            try:
                conn, _ = srv.accept()
            except socket.timeout:
                continue
            threading.Thread(target=one, args=(conn,), daemon=True).start()
    finally:
        srv.close()
