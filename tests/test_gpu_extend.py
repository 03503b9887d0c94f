"""Parity of the paged-KV extend path (decode steps and MCTS tree levels).

The reference evaluates every leaf and every appended move by a full
recompute of the game at batch 1 (src/evaluation/decode.py:356-360,
199-203); the oracle here is exactly that: ``RefModel.forward_last`` over each
token's whole sequence (game prefix + ancestors + the token).  The engine
instead prefills the prefixes into a paged KV pool once and evaluates new
tokens with ``Engine.extend`` over cached keys and values.  Bars as for the
prefill: 1e-4 in the fp32 check mode, 2e-2 in bf16, top-1 identical where the
oracle's top-2 margin exceeds twice the observed logit error.
"""
import numpy as np
import pytest
import torch

from allie_amd import capi, config, weights
from allie_amd.engine import Engine
from oracle.model_ref import RefModel, policy_summary

pytestmark = pytest.mark.gpu

BPG = 8  # pool blocks owned by each game / root in these tests (128 positions)


def nan_pool(eng, n_blocks):
    """A KV pool whose unwritten memory holds NaN patterns (0xff bytes): a
    slot that is not visible to a token must not reach its result."""
    return eng.new_kv_pool(n_blocks).fill_(255)


def check(got, ref, tol, what):
    lg = got.logits.cpu().numpy()
    dl = float(np.abs(lg - ref["logits"]).max())
    dv = float(np.abs(got.value.cpu().numpy() - ref["value_logits"]).max())
    dt = float(np.abs(got.time.cpu().numpy() - ref["time_logits"]).max())
    assert dl <= tol and dv <= tol and dt <= tol, (what, dl, dv, dt)
    ps = policy_summary(ref["logits"])
    need = ps["margin"] > max(2 * dl, 1e-6)
    top1 = got.top1.cpu().numpy()
    assert (top1[need] == ps["top1"][need]).all(), (what, np.nonzero(top1 != ps["top1"]))


@pytest.fixture(scope="module")
def tiny():
    cfg = config.TINY
    return cfg, weights.init_weights(cfg, seed=11, perturb=True)


@pytest.mark.parametrize("mode,tol,split", [("float32", 1e-4, False), ("bfloat16", 2e-2, False), ("bfloat16", 2e-2, True)])
def test_decode_steps_match_full_recompute(tiny, mode, tol, split, cuda):
    """Decode steps of 9 games; with split, the step's one-token groups run as
    two halves on the model's two streams (threshold lowered to 4 games)."""
    cfg, sd = tiny
    rng = np.random.default_rng(5)
    B = 9
    lens = rng.integers(1, 70, B).astype(np.int32)
    seqs = [list(rng.integers(0, 1968, n)) for n in lens]
    eng = Engine(cfg, sd, mode=mode)
    if split:
        eng.set_split_tokens(24576, 4)
    pool = nan_pool(eng, B * BPG + 3)
    # game b owns blocks 3 + b * BPG ...: a non-contiguous, non-zero layout
    table = torch.tensor([[3 + b * BPG + j for j in range(BPG)] for b in range(B)], dtype=torch.int32, device=cuda)
    words = np.concatenate([np.asarray(s, np.uint32) for s in seqs])
    eng.prefill(words, lens, kv_pool=pool, kv_block_table=table)
    oracle = RefModel(cfg, sd, mode=mode)
    status = torch.full((1,), -1, dtype=torch.int32, device=cuda)
    for step in range(3):
        new = rng.integers(0, 1968, B)
        cur = np.array([len(s) for s in seqs], np.int32)  # position of the new token
        slots = np.array([(3 + b * BPG + cur[b] // 16) * 16 + cur[b] % 16 for b in range(B)], np.int32)
        out = eng.extend(new, cur, [1] * B, cur, table, slots[:, None], np.ones(B, np.int32), pool, status=status)
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        for b in range(B):
            seqs[b].append(int(new[b]))
        ref = oracle.forward_last([np.asarray(s, np.int64) for s in seqs])
        check(out, ref, tol, f"{mode} decode step {step}")
    eng.close()


def test_decode_long_games(tiny, cuda):
    """Decode steps of games of up to 514 positions (33 pool blocks) beside
    short ones, ragged last blocks over NaN-filled unwritten slots, against
    the full recompute (bf16, 2e-2)."""
    cfg, sd = tiny
    rng = np.random.default_rng(8)
    lens = np.array([270, 271, 286, 300, 417, 5, 100, 511, 33], np.int32)
    B, bpg = len(lens), 33  # 528 positions per game
    seqs = [list(rng.integers(0, 1968, n)) for n in lens]
    eng = Engine(cfg, sd, mode="bfloat16")
    pool = nan_pool(eng, B * bpg + 2)
    table = torch.tensor([[2 + b * bpg + j for j in range(bpg)] for b in range(B)], dtype=torch.int32, device=cuda)
    words = np.concatenate([np.asarray(s, np.uint32) for s in seqs])
    eng.prefill(words, lens, kv_pool=pool, kv_block_table=table)
    oracle = RefModel(cfg, sd, mode="bfloat16")
    status = torch.full((1,), -1, dtype=torch.int32, device=cuda)
    for step in range(3):
        new = rng.integers(0, 1968, B)
        cur = np.array([len(s) for s in seqs], np.int32)
        slots = np.array([(2 + b * bpg + cur[b] // 16) * 16 + cur[b] % 16 for b in range(B)], np.int32)
        out = eng.extend(new, cur, [1] * B, cur, table, slots[:, None], np.ones(B, np.int32), pool, status=status)
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        for b in range(B):
            seqs[b].append(int(new[b]))
        ref = oracle.forward_last([np.asarray(s, np.int64) for s in seqs])
        check(out, ref, 2e-2, f"long decode step {step}")
    eng.close()


@pytest.mark.parametrize("mode", ["bfloat16", "fp8w"])
def test_single_token_chain_matches_full_recompute(tiny, mode, cuda):
    """An MCTS search path evaluated one leaf at a time (one token, one
    group: the QKV projection runs the token's attention in its tail): a
    root prefilled into the pool, then four tokens, each over the root's
    blocks plus its ancestors' scattered private slots and its own, against
    the full recompute of root + path (2e-2, top-1 rule)."""
    cfg, sd = tiny
    rng = np.random.default_rng(21)
    P = 45
    root = list(rng.integers(0, 1968, P))
    eng = Engine(cfg, sd, mode=mode)
    pool = nan_pool(eng, 3 + BPG + 24)
    table = torch.tensor([[3 + j for j in range(BPG)] for _ in range(1)], dtype=torch.int32, device=cuda)
    eng.prefill(np.asarray(root, np.uint32), np.array([P], np.int32), kv_pool=pool, kv_block_table=table)
    oracle = RefModel(cfg, sd, mode=mode)
    status = torch.full((1,), -1, dtype=torch.int32, device=cuda)
    path, slots = [], [20 * 16 + 5, 21 * 16 + 0, 20 * 16 + 9, 23 * 16 + 15]
    for j in range(4):
        tok = int(rng.integers(0, 1968))
        extras = np.array([slots[: j + 1]], np.int32)
        out = eng.extend(np.array([tok]), np.array([P + j], np.int32), [1], np.array([P], np.int32), table, extras,
                         np.array([j + 1], np.int32), pool, status=status)
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        path.append(tok)
        ref = oracle.forward_last([np.asarray(root + path, np.int64)])
        check(out, ref, 2e-2, f"{mode} leaf {j}")
    eng.close()


# (prefix lengths, level-1 children per root): one root of 70 children spans
# two 64-query tiles of the tree kernel; groups of at most 16 children over
# prefix tables of at most 8 chunks take the split-prefix kernels in bf16
# (level 1 of the second case: full, ragged and one-block prefixes, a group of
# one child after the others), and level 2 of that case (groups of up to 32)
# the tree kernel again; in the third case level 2 holds a group of 300 tokens
# (more than one 256-query tile), which takes the span kernel in bf16
TREES = [([37, 64, 100], [3, 70, 5]), ([37, 64, 100, 128, 5], [3, 16, 5, 1, 9]), ([37, 100], [150, 9])]


@pytest.mark.parametrize("prefix,kids", TREES)
@pytest.mark.parametrize("mode,tol", [("float32", 1e-4), ("bfloat16", 2e-2)])
def test_tree_levels_match_full_recompute(tiny, mode, tol, prefix, kids, cuda):
    """Roots with shared prefixes; level-1 children and level-2 grandchildren
    that see the prefix, their parent and themselves."""
    cfg, sd = tiny
    rng = np.random.default_rng(9)
    R = len(prefix)
    roots = [list(rng.integers(0, 1968, n)) for n in prefix]
    eng = Engine(cfg, sd, mode=mode)
    node_base = R * BPG  # node slots live in the blocks after the roots'
    n1 = sum(kids)
    pool = nan_pool(eng, node_base + (3 * n1 + 15) // 16 + 1)
    table = torch.tensor([[r * BPG + j for j in range(BPG)] for r in range(R)], dtype=torch.int32, device=cuda)
    eng.prefill(np.concatenate([np.asarray(s, np.uint32) for s in roots]), np.array(prefix, np.int32),
                kv_pool=pool, kv_block_table=table)
    oracle = RefModel(cfg, sd, mode=mode)
    status = torch.zeros(1, dtype=torch.int32, device=cuda)

    # level 1: one token per child, extras = [own slot]
    ids1 = rng.integers(0, 1968, n1)
    slot1 = node_base * 16 + np.arange(n1, dtype=np.int32)
    root_of1 = np.repeat(np.arange(R), kids)
    pos1 = np.array([prefix[r] for r in root_of1], np.int32)
    out1 = eng.extend(ids1, pos1, kids, prefix, table, slot1[:, None], np.ones(n1, np.int32), pool, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    paths1 = [roots[root_of1[i]] + [int(ids1[i])] for i in range(n1)]
    check(out1, oracle.forward_last([np.asarray(p, np.int64) for p in paths1]), tol, f"{mode} level 1")

    # level 2: two children for every level-1 node, extras = [parent, own slot]
    par = np.repeat(np.arange(n1), 2)
    n2 = len(par)
    ids2 = rng.integers(0, 1968, n2)
    slot2 = node_base * 16 + n1 + np.arange(n2, dtype=np.int32)
    extra = np.stack([slot1[par], slot2], axis=1).astype(np.int32)
    pos2 = pos1[par] + 1
    sizes2 = [2 * k for k in kids]  # grouped by root, in order
    out2 = eng.extend(ids2, pos2, sizes2, prefix, table, extra, np.full(n2, 2, np.int32), pool, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    paths2 = [paths1[par[i]] + [int(ids2[i])] for i in range(n2)]
    check(out2, oracle.forward_last([np.asarray(p, np.int64) for p in paths2]), tol, f"{mode} level 2")
    eng.close()


# level-1 children per root: level 2 then holds groups of 300 and 18 tokens
# (128-query tiles) or of 40 and 60 (64-query tiles)
@pytest.mark.parametrize("kids", [[150, 9], [20, 30]])
def test_tree_head_groups_same_bits(tiny, kids, cuda):
    """The tree kernel taking 1, 2 or 4 heads per workgroup gives the same
    bits at every level; level 2 also against the oracle.  A group of fresh
    one-token games (no prefix, no other private key) covers heads with no
    key chunks at all."""
    cfg, sd = tiny
    assert cfg.n_head == 4
    rng = np.random.default_rng(21)
    prefix = [37, 100]
    R = len(prefix)
    roots = [list(rng.integers(0, 1968, n)) for n in prefix]
    n1 = sum(kids)
    ids1 = rng.integers(0, 1968, n1)
    root_of1 = np.repeat(np.arange(R), kids)
    pos1 = np.array([prefix[r] for r in root_of1], np.int32)
    par = np.repeat(np.arange(n1), 2)
    n2 = len(par)
    ids2 = rng.integers(0, 1968, n2)
    pos2 = pos1[par] + 1
    sizes2 = [2 * k for k in kids]
    n3 = 20
    ids3 = rng.integers(0, 1968, n3)
    results = {}
    for hg in (1, 2, 4):
        eng = Engine(cfg, sd, mode="bfloat16")
        eng.set_tree_heads(hg)
        node_base = R * BPG
        pool = nan_pool(eng, node_base + (n1 + n2 + n3 + 15) // 16 + 1)
        table = torch.tensor([[r * BPG + j for j in range(BPG)] for r in range(R)], dtype=torch.int32, device=cuda)
        eng.prefill(np.concatenate([np.asarray(x, np.uint32) for x in roots]), np.array(prefix, np.int32),
                    kv_pool=pool, kv_block_table=table)
        status = torch.zeros(1, dtype=torch.int32, device=cuda)
        slot1 = node_base * 16 + np.arange(n1, dtype=np.int32)
        out1 = eng.extend(ids1, pos1, kids, prefix, table, slot1[:, None], np.ones(n1, np.int32), pool, status=status)
        slot2 = node_base * 16 + n1 + np.arange(n2, dtype=np.int32)
        extra = np.stack([slot1[par], slot2], axis=1).astype(np.int32)
        out2 = eng.extend(ids2, pos2, sizes2, prefix, table, extra, np.full(n2, 2, np.int32), pool, status=status)
        slot3 = node_base * 16 + n1 + n2 + np.arange(n3, dtype=np.int32)
        out3 = eng.extend(ids3, np.zeros(n3, np.int32), [n3], [0], table[:1], slot3[:, None], np.ones(n3, np.int32),
                          pool, status=status)
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        results[hg] = [{k: getattr(o, k).cpu().numpy().copy() for k in ("logits", "value", "time", "top1")}
                       for o in (out1, out2, out3)]
        if hg == 1:
            oracle = RefModel(cfg, sd, mode="bfloat16")
            paths1 = [roots[root_of1[i]] + [int(ids1[i])] for i in range(n1)]
            paths2 = [paths1[par[i]] + [int(ids2[i])] for i in range(n2)]
            check(out2, oracle.forward_last([np.asarray(p, np.int64) for p in paths2]), 2e-2, "level 2")
            check(out3, oracle.forward_last([np.asarray([t], np.int64) for t in ids3]), 2e-2, "fresh games")
        eng.close()
    for hg in (2, 4):
        for lvl, (a, b) in enumerate(zip(results[1], results[hg])):
            for k in a:
                assert np.array_equal(a[k], b[k]), (hg, lvl, k)


@pytest.mark.parametrize("depth", [8, 9])
def test_tree_head_groups_deep_private_keys(tiny, depth, cuda):
    """Tokens with `depth` private keys (ancestor slots shared by runs of 10
    siblings, then the token's own): with 8 the column build is one batch and
    1, 2 or 4 heads per workgroup give the same bits; with 9 it takes two
    batches and every setting runs one head per workgroup (same bits too).
    The ancestors' slots are read as written by nothing but the zeroed pool."""
    cfg, sd = tiny
    rng = np.random.default_rng(31)
    prefix = [50, 90]
    sizes = [70, 30]
    n = sum(sizes)
    roots = [rng.integers(0, 1968, p) for p in prefix]
    ids = rng.integers(0, 1968, n)
    node_base = len(prefix) * BPG
    anc = node_base * 16 + np.arange(n * depth, dtype=np.int32)  # fresh ancestor slots
    extra = np.zeros((n, depth), np.int32)
    for i in range(n):
        for e in range(depth - 1):
            extra[i, e] = anc[(i // 10) * depth + e]  # shared by runs of 10 tokens
        extra[i, depth - 1] = anc[-1 - i]  # own slot
    root_of = np.repeat(np.arange(len(prefix)), sizes)
    pos = np.array([prefix[r] + depth - 1 for r in root_of], np.int32)
    outs = {}
    for hg in (1, 2, 4):
        eng = Engine(cfg, sd, mode="bfloat16")
        eng.set_tree_heads(hg)
        pool = eng.new_kv_pool(node_base + (len(anc) + 15) // 16 + 1).zero_()
        table = torch.tensor([[r * BPG + j for j in range(BPG)] for r in range(len(prefix))],
                             dtype=torch.int32, device=cuda)
        eng.prefill(np.concatenate([np.asarray(x, np.uint32) for x in roots]), np.array(prefix, np.int32),
                    kv_pool=pool, kv_block_table=table)
        status = torch.zeros(1, dtype=torch.int32, device=cuda)
        out = eng.extend(ids, pos, sizes, prefix, table, extra, np.full(n, depth, np.int32), pool, status=status)
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        assert torch.isfinite(out.logits).all()
        outs[hg] = {k: getattr(out, k).cpu().numpy().copy() for k in ("logits", "value", "time", "top1")}
        eng.close()
    for hg in (2, 4):
        for k in outs[1]:
            assert np.array_equal(outs[1][k], outs[hg][k]), (depth, hg, k)


# (tokens of the two new games over extras, tokens of the new game over its own
# prefix): with 70 the batch takes the tree kernel, with groups of at most 16
# the split-prefix kernels (a group with an empty prefix among them)
@pytest.mark.parametrize("new_sizes", [(1, 70, 45), (1, 12, 14)])
@pytest.mark.parametrize("mode,tol", [("float32", 1e-4), ("bfloat16", 2e-2)])
def test_mixed_batch_matches_full_recompute(tiny, mode, tol, new_sizes, cuda):
    """One extend holding decode steps (one-token groups first), new games'
    whole prefixes and three children sharing a cached game as prefix: the
    batch a continuous batcher runs when games start between decode steps.
    A new game's token t attends tokens 0..t, given either as its extras
    (prefix_len 0) or as the group's own prefix limited by the token's
    position (prefix_len = its length, one extra: its own slot)."""
    cfg, sd = tiny
    rng = np.random.default_rng(13)
    B = 6
    lens = rng.integers(1, 60, B).astype(np.int32)
    seqs = [list(rng.integers(0, 1968, n)) for n in lens]
    eng = Engine(cfg, sd, mode=mode)
    n_games = B + 3
    pool = nan_pool(eng, n_games * BPG + 1)
    table = torch.tensor([[g * BPG + j for j in range(BPG)] for g in range(n_games)], dtype=torch.int32,
                         device=cuda)
    eng.prefill(np.concatenate([np.asarray(s, np.uint32) for s in seqs]), lens, kv_pool=pool,
                kv_block_table=table[:B].contiguous())
    oracle = RefModel(cfg, sd, mode=mode)
    status = torch.zeros(1, dtype=torch.int32, device=cuda)
    new_pre = [list(rng.integers(0, 1968, new_sizes[0])), list(rng.integers(0, 1968, new_sizes[1]))]
    causal_pre = list(rng.integers(0, 1968, new_sizes[2]))
    kid_ids = rng.integers(0, 1968, 3)
    dec = rng.integers(0, 1968, B)
    ids, pos, sizes, plen, pblk, extra_rows, n_extra, paths = [], [], [], [], [], [], [], []
    ME = 70
    for b in range(B):  # decode steps
        p = len(seqs[b])
        ids.append(dec[b]); pos.append(p); sizes.append(1); plen.append(p); pblk.append(b)
        extra_rows.append([b * BPG * 16 + p]); n_extra.append(1)
        paths.append(seqs[b] + [int(dec[b])])
    for k, pre in enumerate(new_pre):  # new games, own blocks B + k
        g = B + k
        sizes.append(len(pre)); plen.append(0); pblk.append(g)
        for t, tok in enumerate(pre):
            ids.append(tok); pos.append(t)
            extra_rows.append([g * BPG * 16 + e for e in range(t + 1)]); n_extra.append(t + 1)
            paths.append([int(x) for x in pre[: t + 1]])
    g = B + 2  # new game over its own prefix positions
    sizes.append(len(causal_pre)); plen.append(len(causal_pre)); pblk.append(g)
    for t, tok in enumerate(causal_pre):
        ids.append(tok); pos.append(t)
        extra_rows.append([g * BPG * 16 + t]); n_extra.append(1)
        paths.append([int(x) for x in causal_pre[: t + 1]])
    kid_slot0 = n_games * BPG * 16  # children's slots: the last block
    sizes.append(3); plen.append(len(seqs[0])); pblk.append(0)
    for c in range(3):  # children of game 0 (shared cached prefix)
        ids.append(kid_ids[c]); pos.append(len(seqs[0]))
        extra_rows.append([kid_slot0 + c]); n_extra.append(1)
        paths.append(seqs[0] + [int(kid_ids[c])])
    extra = np.full((len(ids), ME), -1, np.int32)
    for i, r in enumerate(extra_rows):
        extra[i, : len(r)] = r
    # the decode tokens write their keys into the games' next positions, which
    # the children do not read (they attend the cached prefix and themselves)
    out = eng.extend(np.array(ids), np.array(pos, np.int32), sizes, np.array(plen, np.int32),
                     table.index_select(0, torch.tensor(pblk, device=cuda)), extra,
                     np.array(n_extra, np.int32), pool, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    check(out, oracle.forward_last([np.asarray(p, np.int64) for p in paths]), tol, f"{mode} mixed batch")
    eng.close()


def test_extend_status_flags(tiny, cuda):
    """Bad slots, counts and positions are flagged and never dereferenced."""
    cfg, sd = tiny
    eng = Engine(cfg, sd, mode="bfloat16")
    pool = eng.new_kv_pool(4)
    status = torch.zeros(1, dtype=torch.int32, device=cuda)
    table = np.zeros((1, 2), np.int32)
    # slot in block 9 of a 4-block pool
    eng.extend([5], [3], [1], [3], table, [[9 * 16 + 2]], [1], pool, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) & 2
    # n_extra = 0
    eng.extend([5], [3], [1], [3], table, [[1]], [0], pool, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) & 1
    # position past the model's positions; prefix block id -1
    eng.extend([5], [5000], [1], [3], np.full((1, 2), -1, np.int32), [[1]], [1], pool, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) & 4 and int(status.item()) & 2
    # a group of 17 tokens (tree kernel) over a table wider than 256 blocks:
    # refused on the host before any launch
    n = 17
    with pytest.raises(capi.AllieError, match="block tables of at most 256"):
        eng.extend(np.full(n, 5), np.arange(n, dtype=np.int32), [n], [0], np.zeros((1, 257), np.int32),
                   np.arange(n, dtype=np.int32)[:, None], np.ones(n, np.int32), pool, status=status)
    eng.close()


def test_fp32_group_over_wide_table(tiny, cuda):
    """The fp32 check mode runs every group on the per-token wave kernel,
    which takes any block-table width: a group of 17 children over a
    600-block table row is accepted and matches a full recompute."""
    cfg, sd = tiny
    rng = np.random.default_rng(17)
    P, n = 40, 17
    prefix = rng.integers(0, 1968, P)
    eng = Engine(cfg, sd, mode="float32")
    pool = nan_pool(eng, 8)
    table = np.zeros((1, 600), np.int32)
    table[0, :3] = [0, 1, 2]
    eng.prefill(np.asarray(prefix, np.uint32), [P], kv_pool=pool,
                kv_block_table=torch.from_numpy(table).to(cuda))
    kids = rng.integers(0, 1968, n)
    status = torch.full((1,), -1, dtype=torch.int32, device=cuda)
    out = eng.extend(kids, np.full(n, P, np.int32), [n], [P], table, (3 * 16 + np.arange(n, dtype=np.int32))[:, None],
                     np.ones(n, np.int32), pool, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    paths = [np.concatenate([prefix, [k]]).astype(np.int64) for k in kids]
    check(out, RefModel(cfg, sd, mode="float32").forward_last(paths), 1e-4, "fp32 wide table")
    eng.close()
