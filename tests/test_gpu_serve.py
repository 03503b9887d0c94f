"""Batched policy serving on the GPU engine (fp32 check mode): concurrent
requests through PolicyBatcher get the answers of sequential
Policy.decode_full on the same model (src/evaluation/decode.py:90-113)."""
import threading

import pytest

from allie_amd import config, weights
from allie_amd.decode import DECODE_STRATEGIES
from allie_amd.model import AllieModel
from allie_amd.serve import PolicyBatcher
from allie_amd.tokenizer import Game, UCITokenizer

pytestmark = pytest.mark.gpu

MOVES = ("e2e4 e7e5 g1f3 b8c6 f1b5 a7a6 b5a4 g8f6 e1g1 f8e7 f1e1 b7b5 a4b3 d7d6 c2c3 e8g8 h2h3 h7h6").split()


def test_gpu_batched_policy_equals_sequential(cuda):
    cfg = config.TINY
    model = AllieModel.from_state_dict(cfg, weights.init_weights(cfg, seed=9, perturb=True), mode="float32")
    try:
        tok = UCITokenizer(max_length=512)
        gs = [Game("300+0", 1200 + 50 * i, 2000 - 40 * i, None, False, MOVES[:n], [4] * n, None)
              for i, n in enumerate([0, 2, 3, 6, 9, 11, 14, 17, 18, 5, 1, 8])]
        seq = DECODE_STRATEGIES["policy"](model, tok, device="cuda")
        want = [seq.decode_full(g) for g in gs]
        b = PolicyBatcher(DECODE_STRATEGIES["policy"](model, tok, device="cuda"), max_batch=16, max_wait_ms=100)
        try:
            futs = [None] * len(gs)

            def go(i):
                futs[i] = b.submit(gs[i])

            ts = [threading.Thread(target=go, args=(i,)) for i in range(len(gs))]
            for t in ts:
                t.start()
            for t in ts:
                t.join()
            got = [f.result(timeout=120) for f in futs]
        finally:
            b.close()
        assert [g.move for g in got] == [w.move for w in want]
        assert [g.resigned for g in got] == [w.resigned for w in want]
        for g, w in zip(got, want):
            assert g.think_time == pytest.approx(w.think_time, abs=1e-3)
        assert b.batches < len(gs)
    finally:
        model.close()
