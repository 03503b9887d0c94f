"""The C3 and C4 drivers at reduced size against the reference's semantics.

* Tree expansion: every node's outputs equal a full recompute of its game
  (prefix + ancestors + node), as MCTS.evaluate_node computes it
  (src/evaluation/decode.py:356-373).
* Continuous batching (fp32 check mode): every move the batcher appends is
  the first argmax of a full recompute of the game so far, as greedy
  Policy.decode_full picks it (decode.py:109-113, 204-226); the first move of
  a game comes from the prefill of its prefix.
"""
import numpy as np
import pytest
import torch

from allie_amd import config, weights
from allie_amd.batcher import ContinuousBatcher, GameQueue
from allie_amd.engine import Engine
from allie_amd.tree import TreeExpansion, TreeLayout, node_path
from oracle.model_ref import RefModel, policy_summary

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny():
    cfg = config.TINY
    return cfg, weights.init_weights(cfg, seed=13, perturb=True)


@pytest.mark.parametrize("mode,tol", [("float32", 1e-4), ("bfloat16", 2e-2)])
def test_tree_expansion_matches_recompute(tiny, mode, tol, cuda):
    cfg, sd = tiny
    lay = TreeLayout(n_roots=3, prefix_len=45, branching=5, depth=3)
    eng = Engine(cfg, sd, mode=mode)
    tx = TreeExpansion(eng, lay, seed=3)
    tx.prefill_roots()
    oracle = RefModel(cfg, sd, mode=mode)
    rng = np.random.default_rng(0)
    for k in range(1, lay.depth + 1):
        out = tx.expand_level(k, want_logits=True)
        torch.cuda.synchronize()
        assert int(tx.status.item()) == 0
        n = lay.level_size(k)
        pick = sorted(set([0, n - 1] + list(rng.integers(0, n, 12))))
        ref = oracle.forward_last([np.asarray(node_path(lay, tx.prefixes, tx.levels, k, j), np.int64) for j in pick])
        lg = out.logits.cpu().numpy()[pick]
        dl = float(np.abs(lg - ref["logits"]).max())
        dv = float(np.abs(out.value.cpu().numpy()[pick] - ref["value_logits"]).max())
        assert dl <= tol and dv <= tol, (mode, k, dl, dv)
        ps = policy_summary(ref["logits"])
        need = ps["margin"] > max(2 * dl, 1e-6)
        assert (out.top1.cpu().numpy()[pick][need] == ps["top1"][need]).all()
    eng.close()


@pytest.mark.parametrize("mode,margin", [("float32", 1e-4), ("bfloat16", 0.1)])
def test_continuous_batching_greedy_moves(tiny, mode, margin, cuda):
    """Every recorded (game so far, greedy move) pair against the oracle's
    full recompute of that game: new games' prefixes ride in the same extend
    as the running games' decode steps (in bf16 that batch mixes the decode
    kernel and the tiled kernel)."""
    cfg, sd = tiny
    eng = Engine(cfg, sd, mode=mode)
    q = GameQueue(seed=4, mean_len=12, cap=64, prefix_lo=1, prefix_hi=9)
    cb = ContinuousBatcher(eng, n_slots=5, queue=q, record=True)
    for _ in range(40):
        cb.step()
    torch.cuda.synchronize()
    assert int(cb.status.item()) == 0
    assert cb.games_started > 5  # slots were evicted and refilled
    seqs = [np.asarray(c.ids, np.int64) for c in cb.checks]
    pred = np.array([c.move for c in cb.checks])
    assert max(len(g) for g in seqs) <= 64
    ref = RefModel(cfg, sd, mode=mode).forward_last(seqs)
    ps = policy_summary(ref["logits"])
    need = ps["margin"] > margin
    assert need.mean() > 0.5
    assert (pred[need] == ps["top1"][need]).all(), np.nonzero(pred != ps["top1"])
    eng.close()
