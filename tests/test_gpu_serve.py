"""Batched policy serving on the GPU engine (fp32 check mode): concurrent
requests through PolicyBatcher get the answers of sequential
Policy.decode_full (src/evaluation/decode.py:90-113) over the CPU oracle
model -- the reference server's path, one request per forward
(src/server/main.py:57-91) -- and of sequential decode_full on the GPU."""
import threading

import pytest

from allie_amd import config, weights
from allie_amd.decode import DECODE_STRATEGIES
from allie_amd.model import AllieModel
from allie_amd.serve import PolicyBatcher
from allie_amd.tokenizer import Game, UCITokenizer
from oracle.model_ref import RefModel


class OracleModel:
    """The reference's model call: padded batch, outputs at every position."""

    def __init__(self, cfg, sd):
        self.ref = RefModel(cfg, sd, mode="float32")

    def __call__(self, input_ids, attention_mask=None, position_ids=None, **kw):
        return self.ref.forward_padded(input_ids, attention_mask, position_ids)

pytestmark = pytest.mark.gpu

MOVES = ("e2e4 e7e5 g1f3 b8c6 f1b5 a7a6 b5a4 g8f6 e1g1 f8e7 f1e1 b7b5 a4b3 d7d6 c2c3 e8g8 h2h3 h7h6").split()


def test_gpu_batched_policy_equals_sequential(cuda):
    cfg = config.TINY
    sd = weights.init_weights(cfg, seed=9, perturb=True)
    model = AllieModel.from_state_dict(cfg, sd, mode="float32")
    try:
        tok = UCITokenizer(max_length=512)
        gs = [Game("300+0", 1200 + 50 * i, 2000 - 40 * i, None, False, MOVES[:n], [4] * n, None)
              for i, n in enumerate([0, 2, 3, 6, 9, 11, 14, 17, 18, 5, 1, 8])]
        seq = DECODE_STRATEGIES["policy"](model, tok, device="cuda")
        want = [seq.decode_full(g) for g in gs]
        ora = DECODE_STRATEGIES["policy"](OracleModel(cfg, sd), tok, device="cpu")
        want_ref = [ora.decode_full(g) for g in gs]
        assert [w.move for w in want] == [w.move for w in want_ref]
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
        for ref in (want, want_ref):
            assert [g.move for g in got] == [w.move for w in ref]
            assert [g.resigned for g in got] == [w.resigned for w in ref]
            for g, w in zip(got, ref):
                assert g.think_time == pytest.approx(w.think_time, abs=1e-3)
        assert b.batches < len(gs)
    finally:
        model.close()
