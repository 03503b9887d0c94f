"""Drop-in boundary on the GPU: ``AllieModel`` as ``model(**batch)`` and the
``policy`` / ``mcts`` / ``adaptive-mcts`` strategies on it.

The oracle model is called exactly like the reference's model (padded
batch, outputs at every position, src/modeling/model.py:85-147 restated);
the GPU model must agree on what the callers read (``[:, -1]``), and the
strategies must reach the same decisions (fp32 check mode)."""
import numpy as np
import pytest
import torch

from allie_amd import config, weights
from allie_amd.decode import DECODE_STRATEGIES
from allie_amd.model import AllieModel
from allie_amd.tokenizer import Game, UCITokenizer
from oracle.model_ref import RefModel

pytestmark = pytest.mark.gpu

MOVES = ("e2e4 e7e5 g1f3 b8c6 f1b5 a7a6 b5a4 g8f6 e1g1 f8e7 f1e1 b7b5 a4b3 d7d6 c2c3 e8g8 h2h3 h7h6").split()


class OracleModel:
    def __init__(self, cfg, sd):
        self.ref = RefModel(cfg, sd, mode="float32")

    def __call__(self, input_ids, attention_mask=None, position_ids=None, **kw):
        return self.ref.forward_padded(input_ids, attention_mask, position_ids)


@pytest.fixture(scope="module")
def models(cuda):
    cfg = config.TINY
    sd = weights.init_weights(cfg, seed=21, perturb=True)
    gpu = AllieModel.from_state_dict(cfg, sd, mode="float32")
    yield gpu, OracleModel(cfg, sd), cfg, sd
    gpu.close()


def games():
    out = []
    for i, n in enumerate([0, 3, 8, 13, 18]):
        tc = ["300+0", "5400+0", "180+2"][i % 3]  # 5400+0 is not a known control: <UNK>
        out.append(Game(tc, 1200 + 300 * i, 2900 - 200 * i, None, False, MOVES[:n], list(range(n)), None))
    return out


def test_model_call_matches_reference_shape(models):
    gpu, ora, cfg, _ = models
    tok = UCITokenizer(max_length=512)
    batch = tok.pad_and_collate(games())
    got = gpu(**batch)
    ref = ora(**batch)
    last = batch["attention_mask"].sum(1).long() - 1
    ar = torch.arange(len(last))
    np.testing.assert_allclose(got["logits"][:, -1].cpu().numpy(), ref["logits"][ar, last].numpy(), atol=1e-4)
    np.testing.assert_allclose(got["value_logits"][:, -1].cpu().numpy(), ref["value_logits"][ar, last].numpy(), atol=1e-4)
    np.testing.assert_allclose(got["time_logits"][:, -1].cpu().numpy(), ref["time_logits"][ar, last].numpy(), atol=1e-4)
    assert got["logits"].shape == (5, 1, cfg.vocab_size) and got["value_logits"].shape == (5, 1)


# gpu_kw: options of the GPU strategy only.  kv_cache=True evaluates each
# search leaf as one token over the root's cached keys (sequential, root
# evaluated once); its decisions must equal the oracle-driven search that
# recomputes every leaf's whole game, as MCTS.evaluate_node does
# (src/evaluation/decode.py:356-373, 401-467, 575-658).
@pytest.mark.parametrize("name,kw,gpu_kw", [
    ("policy", {"temperature": 0.5}, {}),
    ("mcts", {"n_sims": 16}, {}),
    ("adaptive-mcts", {"mean_n_sims": 10}, {}),
    ("mcts", {"n_sims": 16}, {"kv_cache": True}),
    ("mcts", {"n_sims": 16}, {"kv_cache": True, "leaf_batch": 1}),
    ("adaptive-mcts", {"mean_n_sims": 10}, {"kv_cache": True}),
])
def test_strategies_same_decisions(models, name, kw, gpu_kw):
    gpu, ora, _, _ = models
    tok = UCITokenizer(max_length=512)
    for g in games()[1:4]:
        a = DECODE_STRATEGIES[name](gpu, tok, device="cuda", **kw, **gpu_kw)
        b = DECODE_STRATEGIES[name](ora, tok, device="cpu", **kw)
        ra = a.score_full(g, g.legal_moves)
        rb = b.score_full(g, g.legal_moves)
        np.testing.assert_allclose(ra.legal_move_probabilities.numpy(), rb.legal_move_probabilities.numpy(),
                                   atol=1e-3)
        assert a.decode_full(g).move == b.decode_full(g).move
        if name != "policy":
            sa, sb = a.run_stats(), b.run_stats()
            assert sa["total_rollouts"] == sb["total_rollouts"]
            if gpu_kw.get("kv_cache"):
                assert sa["kv_leaf_evaluations"] > 0


def test_bf16_model_plays(cuda):
    cfg = config.TINY
    sd = weights.init_weights(cfg, seed=2)
    gpu = AllieModel.from_state_dict(cfg, sd, mode="bfloat16")
    tok = UCITokenizer(max_length=512)
    pol = DECODE_STRATEGIES["policy"](gpu, tok, device="cuda", precision="bfloat16")
    g = games()[4]
    r = pol.decode_full(g)
    assert r.move in g.legal_moves and isinstance(r.resigned, bool)
    gpu.close()
