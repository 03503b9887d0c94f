"""Batched policy serving (allie_amd/serve.py) on the CPU, with the oracle
model standing in for the engine (outputs at each game's last token, as the
GPU model returns them).

* Concurrent requests through ``PolicyBatcher`` get exactly the answers of
  sequential ``Policy.decode_full`` (decode.py:90-113, 194-238), and share
  forwards.
* The socket front end speaks the reference server's protocol
  (src/server/main.py:57-91, utils.py:8-23), including the Elo rule for the
  side to move (main.py:66-78).
* A failing model call reaches every waiting caller.
"""
import json
import socket
import threading

import pytest
import torch

from allie_amd import config, weights
from allie_amd.decode import DECODE_STRATEGIES
from allie_amd.serve import PolicyBatcher, handle_request, serve_socket
from allie_amd.tokenizer import Game, UCITokenizer
from oracle.model_ref import RefModel

MOVES = ("e2e4 e7e5 g1f3 b8c6 f1b5 a7a6 b5a4 g8f6 e1g1 f8e7 f1e1 b7b5 a4b3 d7d6 c2c3 e8g8 h2h3 h7h6").split()


class LastTokenOracle:
    """model(**batch) with outputs at each row's last real token ([B, 1, ...])."""

    def __init__(self, cfg, sd):
        self.ref = RefModel(cfg, sd, mode="float32")
        self.calls = 0

    def __call__(self, input_ids, attention_mask=None, position_ids=None, **kw):
        self.calls += 1
        o = self.ref.forward_padded(input_ids, attention_mask, position_ids, last_only=True)
        return {"logits": o["logits"][:, None], "value_logits": o["value_logits"][:, None],
                "time_logits": o["time_logits"][:, None]}


@pytest.fixture(scope="module")
def model():
    cfg = config.TINY
    return LastTokenOracle(cfg, weights.init_weights(cfg, seed=4, perturb=True))


def games():
    return [Game(["300+0", "180+2", "60+0"][i % 3], 1100 + 150 * i, 2500 - 120 * i, None, False,
                 MOVES[:n], [5] * n, None) for i, n in enumerate([0, 1, 4, 7, 9, 12, 15, 18])]


def test_batched_answers_equal_sequential(model):
    tok = UCITokenizer(max_length=512)
    pol = DECODE_STRATEGIES["policy"](model, tok, device="cpu", temperature=0.7)
    want = [pol.decode_full(g) for g in games()]
    calls0 = model.calls
    b = PolicyBatcher(DECODE_STRATEGIES["policy"](model, tok, device="cpu", temperature=0.7), max_batch=8,
                      max_wait_ms=200)
    try:
        futs = [None] * len(want)
        gs = games()

        def go(i):
            futs[i] = b.submit(gs[i])

        ts = [threading.Thread(target=go, args=(i,)) for i in range(len(gs))]
        for t in ts:
            t.start()
        for t in ts:
            t.join()
        got = [f.result(timeout=60) for f in futs]
    finally:
        b.close()
    for g, w in zip(got, want):
        assert g.move == w.move and g.resigned == w.resigned
        assert g.think_time == pytest.approx(w.think_time, abs=1e-5)
    assert b.requests == len(want) and b.batches < len(want)
    assert model.calls - calls0 == b.batches


def test_socket_protocol_and_elo_rule(model):
    tok = UCITokenizer(max_length=512)
    b = PolicyBatcher(DECODE_STRATEGIES["policy"](model, tok, device="cpu"), max_batch=4, max_wait_ms=50)
    seq = DECODE_STRATEGIES["policy"](model, tok, device="cpu")
    ready, stop = threading.Event(), threading.Event()
    s0 = socket.socket()
    s0.bind(("127.0.0.1", 0))
    port = s0.getsockname()[1]
    s0.close()
    th = threading.Thread(target=serve_socket, args=(b, port), kwargs=dict(ready=ready, stop=stop), daemon=True)
    th.start()
    assert ready.wait(10)
    try:
        reqs = [dict(time_control="300+0", white_elo=1500, black_elo=2100, outcome=None, normal_termination=False,
                     moves=MOVES[:n], moves_seconds=[3] * n) for n in (2, 5, 8)]
        answers = [None] * len(reqs)

        def client(i):
            with socket.create_connection(("127.0.0.1", port), timeout=30) as c:
                c.sendall(json.dumps(reqs[i]).encode())
                answers[i] = json.loads(c.recv(65536).decode())

        ts = [threading.Thread(target=client, args=(i,)) for i in range(len(reqs))]
        for t in ts:
            t.start()
        for t in ts:
            t.join()
        for r, a in zip(reqs, answers):
            g = Game(**r)
            # no system Elo: the side to move plays at the opponent's Elo
            if g.white_to_move:
                g.white_elo = g.black_elo
            else:
                g.black_elo = g.white_elo
            w = seq.decode_full(g)
            assert a == {"move": w.move, "think_time": pytest.approx(w.think_time, abs=1e-5),
                         "resigned": w.resigned}
        # a fixed system Elo goes to the side to move
        out = handle_request(b, dict(reqs[0]), system_elo=2500)
        g = Game(**reqs[0])
        g.white_elo = 2500
        assert out["move"] == seq.decode_full(g).move
    finally:
        stop.set()
        th.join(5)
        b.close()


def test_model_failure_reaches_every_caller():
    class Broken:
        def __call__(self, **kw):
            raise RuntimeError("device lost")

    tok = UCITokenizer(max_length=512)
    b = PolicyBatcher(DECODE_STRATEGIES["policy"](Broken(), tok, device="cpu"), max_batch=4, max_wait_ms=100)
    try:
        fs = [b.submit(g) for g in games()[:3]]
        for f in fs:
            with pytest.raises(RuntimeError, match="device lost"):
                f.result(timeout=30)
    finally:
        b.close()
    with pytest.raises(RuntimeError):
        b.submit(games()[0])
    with pytest.raises(TypeError):
        PolicyBatcher(DECODE_STRATEGIES["mcts"](Broken(), tok, device="cpu"))


def test_bad_request_fails_alone(model):
    """A request with an illegal move, or no Elo for the tokenizer, fails its
    own future on submit; the good requests around it are still answered
    from one shared forward."""
    tok = UCITokenizer(max_length=512)
    seq = DECODE_STRATEGIES["policy"](model, tok, device="cpu")
    b = PolicyBatcher(DECODE_STRATEGIES["policy"](model, tok, device="cpu"), max_batch=8, max_wait_ms=200)
    try:
        good = games()[1:5]
        illegal = Game("300+0", 1500, 1500, None, False, ["e2e4", "e2e4"], [3, 3], None)
        no_elo = Game("300+0", None, 1500, None, False, ["e2e4"], [3], None)
        fs = [b.submit(good[0]), b.submit(illegal), b.submit(good[1]), b.submit(no_elo),
              b.submit(good[2]), b.submit(good[3])]
        with pytest.raises(Exception):
            fs[1].result(timeout=30)
        with pytest.raises(Exception):
            fs[3].result(timeout=30)
        got = [fs[i].result(timeout=60) for i in (0, 2, 4, 5)]
    finally:
        b.close()
    assert [g.move for g in got] == [seq.decode_full(g).move for g in good]
    assert b.requests == 4


def test_close_resolves_every_future(model):
    """Submitting races close: every submit either raises or gets a future
    that resolves (no caller waits forever)."""
    tok = UCITokenizer(max_length=512)
    b = PolicyBatcher(DECODE_STRATEGIES["policy"](model, tok, device="cpu"), max_batch=4, max_wait_ms=1)
    futs, errors = [], []

    def spam():
        for g in games() * 3:
            try:
                futs.append(b.submit(g))
            except RuntimeError:
                errors.append(1)

    ts = [threading.Thread(target=spam) for _ in range(3)]
    for t in ts:
        t.start()
    b.close()
    for t in ts:
        t.join()
    for f in futs:
        try:
            f.result(timeout=60)
        except RuntimeError:
            pass
    assert all(f.done() for f in futs)
