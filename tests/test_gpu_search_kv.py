"""KV-cached search (allie_amd/search_kv.py, the ``kv_cache`` / ``leaf_batch``
options of ``mcts`` and ``adaptive-mcts``) on the GPU, fp32 check mode.

* Every evaluation through the cache (the root's prefill, one-token extends
  over the root's blocks and the ancestors' slots, batches mixing depths and
  parents) equals the model call on the node's whole game (what the
  reference's ``MCTS.evaluate_node`` runs, src/evaluation/decode.py:356-360)
  within 1e-4.
* The searches with the cache reach the same results as without it, also
  when nodes pass the 512-token window (here a 40-token window) and fall back.
* Leaf batching keeps the search's bookkeeping: every simulation backs up
  one path, and virtual loss is removed again.
"""
import numpy as np
import pytest
import torch

from allie_amd import config, weights
from allie_amd.decode import DECODE_STRATEGIES, MCTSNode
from allie_amd.model import AllieModel
from allie_amd.search_kv import KVSearchCache
from allie_amd.tokenizer import Game, UCITokenizer

pytestmark = pytest.mark.gpu

MOVES = ("e2e4 e7e5 g1f3 b8c6 f1b5 a7a6 b5a4 g8f6 e1g1 f8e7 f1e1 b7b5 a4b3 d7d6 c2c3 e8g8 h2h3 h7h6").split()


def game(n, tc="300+0", seed=None, plies=None):
    moves = list(MOVES[:n])
    if plies is not None:  # a longer legal game: seeded random play from the opening
        rng = np.random.default_rng(seed)
        g = Game(tc, 1500, 1600, None, False, moves, [3] * len(moves), None)
        while len(g.moves) < plies:
            legal = g.legal_moves
            assert legal and g.board.outcome() is None
            g = g.make_move(legal[int(rng.integers(len(legal)))])
        moves = g.moves
    return Game(tc, 1500, 1600, None, False, moves, [3] * len(moves), None)


@pytest.fixture(scope="module")
def tiny(cuda):
    cfg = config.TINY
    sd = weights.init_weights(cfg, seed=21, perturb=True)
    gpu = AllieModel.from_state_dict(cfg, sd, mode="float32")
    yield gpu, cfg
    gpu.close()


def full_eval(model, tok, g):
    out = model(**tok.pad_and_collate([g]))
    return (out["logits"][0, -1].float().cpu().numpy(), float(out["value_logits"][0, -1]),
            float(out["time_logits"][0, -1]))


def check(ev, ref):
    np.testing.assert_allclose(ev.logits.numpy(), ref[0], atol=1e-4, rtol=0)
    assert abs(ev.value - ref[1]) < 1e-4 and abs(ev.time - ref[2]) < 1e-4


def test_cache_evaluations_equal_full_forward(tiny):
    gpu, _ = tiny
    tok = UCITokenizer(max_length=512)
    g = game(13)
    root = MCTSNode(0.0, g)
    kv = KVSearchCache(gpu.engine, tok)
    check(kv.begin(root, g, max_nodes=64), full_eval(gpu, tok, g))

    def kids(node, moves):
        out = []
        for m in moves:
            c = MCTSNode(0.0, node.game.make_move(m))
            kv.attach(node, c, m)
            out.append(c)
        return out

    level1 = kids(root, g.legal_moves[:6])
    for c, ev in zip(level1, kv.evaluate(level1)):
        check(ev, full_eval(gpu, tok, c.game))
    # a batch mixing parents and depths: grandchildren of two children, a
    # child not evaluated before, and a great-grandchild
    gc = kids(level1[0], level1[0].game.legal_moves[:3]) + kids(level1[4], level1[4].game.legal_moves[-2:])
    kv.evaluate(gc[:1])
    ggc = kids(gc[0], gc[0].game.legal_moves[:1])
    late = kids(root, g.legal_moves[6:7])
    batch = gc + ggc + late
    for c, ev in zip(batch, kv.evaluate(batch)):
        check(ev, full_eval(gpu, tok, c.game))
    assert [len(c._kv_path) for c in batch] == [2] * 5 + [3, 1]
    assert kv.n_evals == 6 + 5 + 1 + 1
    # memoised: a second request makes no new evaluation
    kv.evaluate(batch)
    assert kv.n_evals == 13
    kv.end()


@pytest.mark.parametrize("name,kw", [("mcts", {"n_sims": 24}), ("adaptive-mcts", {"mean_n_sims": 12})])
def test_search_with_cache_matches_without(tiny, name, kw):
    gpu, _ = tiny
    tok = UCITokenizer(max_length=512)
    for n in (1, 8, 13):
        g = game(n)
        a = DECODE_STRATEGIES[name](gpu, tok, device="cuda", kv_cache=True, **kw)
        b = DECODE_STRATEGIES[name](gpu, tok, device="cuda", **kw)
        ra = a.score_full(g, g.legal_moves)
        rb = b.score_full(g, g.legal_moves)
        np.testing.assert_allclose(ra.legal_move_probabilities.numpy(), rb.legal_move_probabilities.numpy(),
                                   atol=1e-4)
        assert ra.think_time == pytest.approx(rb.think_time, abs=1e-3)
        assert ra.resigned == rb.resigned
        assert a.run_stats()["total_rollouts"] == b.run_stats()["total_rollouts"]
        if name == "mcts":
            assert a.run_stats()["kv_leaf_evaluations"] > 0


def test_window_fallback_matches(cuda):
    """A 40-token window: nodes past it fall back to the model call (which
    keeps the first 40 tokens, as pad_and_collate keeps the first 512)."""
    cfg = config.TINY.with_(max_length=40)
    sd = weights.init_weights(cfg, seed=5, perturb=True)
    gpu = AllieModel.from_state_dict(cfg, sd, mode="float32")
    try:
        tok = UCITokenizer(max_length=40)
        for plies in (34, 37, 40):  # 37, 40 and 43 tokens: partly, just and wholly past the window
            g = game(18, seed=plies, plies=plies)
            a = DECODE_STRATEGIES["mcts"](gpu, tok, device="cuda", kv_cache=True, n_sims=20)
            b = DECODE_STRATEGIES["mcts"](gpu, tok, device="cuda", n_sims=20)
            ra, rb = a.score_full(g, g.legal_moves), b.score_full(g, g.legal_moves)
            np.testing.assert_allclose(ra.legal_move_probabilities.numpy(), rb.legal_move_probabilities.numpy(),
                                       atol=1e-4)
    finally:
        gpu.close()


def test_leaf_batching_bookkeeping(tiny):
    gpu, _ = tiny
    tok = UCITokenizer(max_length=512)
    g = game(8)
    s = DECODE_STRATEGIES["mcts"](gpu, tok, device="cuda", kv_cache=True, leaf_batch=8, n_sims=40)
    root = MCTSNode(0.0, g)
    assert s._kv_begin(root, g, 64) is not None
    s.evaluate_node(root)
    s._simulate(root, 40)
    s._kv_end()
    assert root.visit_count == 40
    assert sum(c.visit_count for c in root.children.values()) == 40

    def walk(n):
        assert abs(n.value_sum) <= n.visit_count + 1e-6
        if n.expanded() and n is not root:
            assert sum(c.visit_count for c in n.children.values()) <= n.visit_count
        for c in n.children.values():
            walk(c)

    walk(root)
    assert s._kv.n_evals <= 40
    r = s.score_full(g, g.legal_moves)
    p = r.legal_move_probabilities
    assert torch.isfinite(p).all() and abs(float(p.sum()) - 1) < 1e-5


@pytest.mark.parametrize("mode", ["float32", "bfloat16"])
def test_leaf_graph_replays_equal_eager(cuda, mode):
    """Single leaves replay a captured HIP graph of the allocation-free
    extend.  Over two searches on one cache (the graph captured once, the
    root's prefix length and table changed between them), every replay --
    with eager extends and synchronisations in between -- equals the eager
    allie_extend of the same leaf bit for bit, and the full forward of the
    leaf's game within the mode's bar."""
    cfg = config.TINY
    sd = weights.init_weights(cfg, seed=21, perturb=True)
    gpu = AllieModel.from_state_dict(cfg, sd, mode=mode)
    tol = 1e-4 if mode == "float32" else 2e-2
    try:
        tok = UCITokenizer(max_length=512)
        kv = KVSearchCache(gpu.engine, tok)
        rng = np.random.default_rng(3)
        for plies in (8, 13):
            g = game(plies)
            root = MCTSNode(0.0, g)
            kv.begin(root, g, max_nodes=64)
            graph = kv.leaf_graph
            node = root
            for depth in range(1, 7):
                moves = node.game.legal_moves
                m = moves[int(rng.integers(len(moves)))]
                c = MCTSNode(0.0, node.game.make_move(m))
                kv.attach(node, c, m)
                before = kv.n_graph
                ev = kv.evaluate([c])[0]
                assert kv.n_graph == before + 1 and kv.leaf_graph is graph
                path = c._kv_path
                eager = gpu.engine.extend([c._kv_token], [kv.prefix_len + len(path) - 1], [1], [kv.prefix_len],
                                          kv.table, np.asarray(path, np.int32)[None], [len(path)], kv.pool)
                assert torch.equal(ev.logits, eager.logits[0].cpu()), (mode, plies, depth)
                assert ev.value == float(eager.value[0]) and ev.time == float(eager.time[0])
                ref = full_eval(gpu, tok, c.game)
                assert np.abs(ev.logits.numpy() - ref[0]).max() <= tol
                assert abs(ev.value - ref[1]) <= tol and abs(ev.time - ref[2]) <= tol
                node = c
            kv.end()
    finally:
        gpu.close()
