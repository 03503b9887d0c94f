"""Decode strategies (allie_amd/decode.py) on the CPU, with the oracle as
the model (called like the reference's: ``model(**pad_and_collate(games))``
returning outputs at every position).

Pins: the KL-regularised policy against its closed form and a float64
bisection; the PUCT score against a hand-computed value; Policy against the
softmax/argmax of the oracle's logits over the legal moves; MCTS/AdaptiveMCTS
bookkeeping (visit counts, rollouts, simulation budget formula)."""
import math

import numpy as np
import pytest
import torch

from allie_amd import config, weights
from allie_amd.decode import (DECODE_STRATEGIES, AdaptiveMCTS, MCTS, MCTSNode, Policy,
                              kl_regularised_policy)
from allie_amd.tokenizer import Game, UCITokenizer
from oracle.model_ref import RefModel

DEEPBLUE = ("e2e4 e7e5 g1f3 b8c6 f1b5 a7a6 b5a4 g8f6 e1g1 f8e7 f1e1 b7b5 a4b3 d7d6 c2c3 e8g8").split()


class OracleModel:
    """model(**batch) -> dict over the oracle (fp32, every position)."""

    def __init__(self, cfg, sd):
        self.ref = RefModel(cfg, sd, mode="float32")
        self.calls = 0

    def __call__(self, input_ids, attention_mask=None, position_ids=None, **kw):
        self.calls += 1
        return self.ref.forward_padded(input_ids, attention_mask, position_ids)


@pytest.fixture(scope="module")
def model():
    cfg = config.ModelConfig(n_layer=2, d_model=64, n_head=2)
    return OracleModel(cfg, weights.init_weights(cfg, seed=5, perturb=True))


def game(n):
    return Game("300+0", 1800, 1900, None, False, DEEPBLUE[:n], [3] * n, None)


def test_kl_policy_closed_form():
    pri = torch.FloatTensor([0.5, 0.3, 0.2])
    # equal values: pi_bar is proportional to the priors
    out = kl_regularised_policy(pri, torch.zeros(3), torch.FloatTensor([5, 3, 2]), 1.25)
    torch.testing.assert_close(out, pri, rtol=1e-6, atol=1e-6)
    # general case: pi_bar = lam * prior / (alpha - q), sum 1 (float64 bisection)
    q = torch.FloatTensor([0.1, -0.2, 0.4])
    n = torch.FloatTensor([10, 4, 6])
    out = kl_regularised_policy(pri, q, n, 1.25).double()
    lam = 1.25 * 20 / (3 + 20)
    lo, hi = max(q.double() + lam * pri.double()), max(q.double() + lam)
    for _ in range(200):
        a = (lo + hi) / 2
        s = (lam * pri.double() / (a - q.double())).sum()
        lo, hi = (a, hi) if s > 1 else (lo, a)
    exact = lam * pri.double() / (a - q.double())
    assert abs(out.sum().item() - 1) < 1e-6
    assert (out - exact / exact.sum()).abs().max() < 2e-3


def test_ucb_score_known_answer(model):
    tok = UCITokenizer(max_length=512)
    m = MCTS(model, tok, device="cpu", n_sims=1)
    parent, child = MCTSNode(0.0, game(0)), MCTSNode(0.3, game(1))
    parent.visit_count, child.visit_count, child.value_sum = 10, 2, 0.2
    pb = (math.log((10 + 19652 + 1) / 19652) + 1.25) * math.sqrt(10) / 3
    assert abs(m.ucb_score(parent, child) - (pb * 0.3 + 0.1)) < 1e-12


def test_policy_matches_oracle_softmax(model):
    tok = UCITokenizer(max_length=512)
    pol = DECODE_STRATEGIES["policy"](model, tok, device="cpu", temperature=0.7)
    g = game(6)
    legal = g.legal_moves
    res = pol.score_full(g, legal)
    out = model(**tok.pad_and_collate([g]))
    lg = out["logits"][0, -1]
    ids = torch.tensor([tok.token_to_id[m] for m in legal])
    torch.testing.assert_close(res.legal_move_probabilities, torch.softmax(lg[ids] / 0.7, 0))
    assert abs(res.white_advantage - out["value_logits"][0, -1].item()) < 1e-7
    d = pol.decode_full(g)
    assert d.move == legal[int(torch.argmax(lg[ids]))]
    assert d.think_time == pytest.approx(out["time_logits"][0, -1].item() * 6.16533 + 4.64001, rel=1e-6)


def test_mcts_and_adaptive_run(model):
    tok = UCITokenizer(max_length=512)
    g = game(8)
    m = MCTS(model, tok, device="cpu", n_sims=12)
    calls0 = model.calls
    res = m.score_full(g, g.legal_moves)
    # one Policy forward + the root evaluation + one per simulation (leaves
    # that are not terminal)
    assert model.calls - calls0 == 2 + 12
    p = res.legal_move_probabilities
    assert len(p) == len(g.legal_moves) and abs(p.sum().item() - 1) < 1e-5
    assert m.run_stats() == {"total_rollouts": 12}
    m2 = MCTS(model, tok, device="cpu", n_sims=12, kl_reg_solution=False)
    res2 = m2.score_full(g, g.legal_moves)
    assert abs(res2.legal_move_probabilities.sum().item() - 1) < 1e-6
    assert (res2.legal_move_probabilities * 12).round().sum().item() == 12  # visit counts / 12
    a = AdaptiveMCTS(model, tok, device="cpu", mean_n_sims=8)
    assert a.convert_time_to_sims(0.0) == 8
    assert a.convert_time_to_sims(10.0) == 114 and a.convert_time_to_sims(30.0) == 200
    assert a.convert_time_to_sims(-10.0) == 0
    assert a.convert_time_to_sims(0.5) == round(8 * 6.16533 / 4.64001 * 0.5 + 8)
    r = a.score_full(g, g.legal_moves)
    assert abs(r.legal_move_probabilities.sum().item() - 1) < 1e-5


def test_mcts_terminal_values(model):
    tok = UCITokenizer(max_length=512)
    m = MCTS(model, tok, device="cpu", n_sims=1)
    mated = Game("300+0", 1500, 1500, None, False, "f2f3 e7e5 g2g4 d8h4".split(), [1] * 4, None)
    assert m.evaluate_node(MCTSNode(0.0, mated)) == 1.0  # the side that just moved mated
