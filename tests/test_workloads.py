"""Host-side bookkeeping of the C3 (tree expansion) and C4 (continuous
batching) drivers: slot arithmetic and the seeded game queue (no GPU)."""
import numpy as np

from allie_amd.batcher import GameQueue
from allie_amd.tree import TreeLayout, node_path, synthetic_tree


def test_tree_layout_slots_and_ancestors():
    lay = TreeLayout(n_roots=3, prefix_len=37, branching=4, depth=3)
    assert lay.prefix_blocks == 3 and lay.level_size(2) == 48 and lay.n_nodes == 12 + 48 + 192
    slots = np.concatenate([lay.node_slot(k, np.arange(lay.level_size(k))) for k in (1, 2, 3)])
    assert len(np.unique(slots)) == lay.n_nodes                      # one slot per node
    assert slots.min() >= lay.node_block0 * 16                       # after the roots' blocks
    assert slots.max() < lay.n_blocks * 16                           # inside the pool
    ex = lay.level_extras(3)
    assert ex.shape == (192, 3)
    for j in (0, 5, 191):
        # self, parent, grandparent: j, j // 4 at level 2, j // 16 at level 1
        assert ex[j, 2] == lay.node_slot(3, j) and ex[j, 1] == lay.node_slot(2, j // 4)
        assert ex[j, 0] == lay.node_slot(1, j // 16)
    assert (lay.level_positions(3) == 37 + 2).all()
    tab = lay.root_table()
    assert tab.shape == (3, 3) and tab[2, 0] == 6


def test_tree_paths_follow_parents():
    lay = TreeLayout(n_roots=2, prefix_len=5, branching=3, depth=2)
    prefixes, levels = synthetic_tree(lay, seed=1)
    p = node_path(lay, prefixes, levels, 2, 13)  # root 13 // 9 = 1, parent 13 // 3 = 4
    assert p[:5] == list(prefixes[1]) and p[5] == levels[0][4] and p[6] == levels[1][13]


def test_game_queue_bounds_and_seed():
    q1, q2 = GameQueue(seed=4), GameQueue(seed=4)
    pre, P, T = q1.draw(5000)
    pre2, P2, T2 = q2.draw(5000)
    assert (P == P2).all() and (T == T2).all() and all((a == b).all() for a, b in zip(pre, pre2))
    assert P.min() >= 1 and P.max() <= 50 and (T >= P + 1).all() and T.max() <= 512
    assert all(len(p) == n for p, n in zip(pre, P))
    assert 70 < T.mean() < 95  # geometric(1/80) with the floor at P + 1
    assert all((p >= 0).all() and (p < 1968).all() for p in pre)
