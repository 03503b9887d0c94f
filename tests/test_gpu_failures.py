"""Failure and edge handling of the prefill, forced from the host.

* NaN logits: a NaN row of ``wte`` (set from the host) makes that move's
  logit NaN in every game.  The reference picks the top move as
  ``softmax(logits[:1968] / T).argmax()`` (src/evaluation/decode.py:223-226)
  and the legal move as ``softmax(legal logits / T).argmax()``
  (decode.py:112, 231): one NaN turns the whole softmax NaN and torch's
  argmax then returns the first element.  Over all moves the first element
  is move id 0, so the heads kernel must give the reference's top-1 there,
  with max_logit and lse NaN, and the usual answer when the NaN move is
  masked out.  With a legal mask that keeps the NaN move, the reference's
  first element is legal_moves[0] in python-chess generation order, which
  is not available here (parity unpinned); the heads kernel follows a
  stated convention instead: the smallest legal move id.
* A KV pool too small for the prefill is rejected before any launch.
* The packer's flags reach the caller through ``status``: the <PAD> id
  inside a game (8; the reference's padded batch would mask that token,
  data.py:321, here it is an ordinary token) and a game longer than its
  block-table row (4).
"""
import numpy as np
import pytest
import torch

from allie_amd import capi, config, weights
from allie_amd.engine import Engine, legal_mask
from oracle.model_ref import RefModel

pytestmark = pytest.mark.gpu

NAN_ID = 5


@pytest.fixture(scope="module")
def tiny():
    cfg = config.TINY
    return cfg, weights.init_weights(cfg, seed=11, perturb=True)


def games(seed, B, lo, hi, avoid=()):
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, B).astype(np.int32)
    seqs = []
    for n in lens:
        s = rng.integers(0, 1968, n)
        for a in avoid:
            s[s == a] = a + 1
        seqs.append(s.astype(np.uint32))
    return seqs, lens


@pytest.mark.parametrize("mode", ["float32", "bfloat16"])
def test_nan_logit_follows_torch_softmax_argmax(tiny, mode, cuda):
    cfg, sd = tiny
    sd = dict(sd)
    wte = np.array(sd[weights.GLOBAL_KEYS["wte"]], np.float32)
    wte[NAN_ID] = np.nan
    sd[weights.GLOBAL_KEYS["wte"]] = wte
    seqs, lens = games(3, 6, 4, 40, avoid=(NAN_ID,))  # no game feeds the NaN embedding
    eng = Engine(cfg, sd, mode=mode)
    words = np.concatenate(seqs)
    T = 0.7
    # all moves: the reference's top move is element 0 of an all-NaN softmax
    r = eng.prefill(words, lens, temperature=T)
    lg = r.logits.cpu()
    assert torch.isnan(lg[:, NAN_ID]).all() and torch.isfinite(r.value).all()
    for b in range(len(lens)):
        want = int(torch.softmax(lg[b, :1968] / T, dim=0).argmax())
        assert want == 0 and int(r.top1[b]) == want
    assert torch.isnan(r.lse.cpu()).all() and torch.isnan(r.max_logit.cpu()).all()
    # legal moves without the NaN one: the ordinary first argmax
    legal_ok = [[1, 2, 7, 100, 1500], [3, 4, 9], [0, 8], [6], [10, 11, 12, 13], [1967, 4, 44]]
    r2 = eng.prefill(words, lens, temperature=T, legal=legal_mask(legal_ok))
    for b, ids in enumerate(legal_ok):
        srt = sorted(ids)
        want = srt[int(torch.softmax(lg[b, srt] / T, dim=0).argmax())]
        assert int(r2.top1[b]) == want and np.isfinite(float(r2.lse[b]))
    # legal moves including it: the smallest legal id (this library's convention; the reference's pick,
    # legal_moves[0] in python-chess order, is unpinned)
    legal_nan = [[3, NAN_ID, 9], [NAN_ID, 700], [NAN_ID], [2, 4, NAN_ID], [6, NAN_ID, 1000], [NAN_ID, 1967]]
    r3 = eng.prefill(words, lens, temperature=T, legal=legal_mask(legal_nan))
    for b, ids in enumerate(legal_nan):
        srt = sorted(ids)
        want = srt[int(torch.softmax(lg[b, srt] / T, dim=0).argmax())]
        assert int(r3.top1[b]) == want == srt[0]
        assert np.isnan(float(r3.lse[b]))
    eng.close()


def test_prefill_kv_pool_too_small(tiny, cuda):
    cfg, sd = tiny
    seqs, lens = games(4, 3, 40, 60)  # 3 games of >= 40 tokens need >= 9 blocks
    eng = Engine(cfg, sd, mode="bfloat16")
    pool = eng.new_kv_pool(4)
    with pytest.raises(capi.AllieError, match="KV pool too small"):
        eng.prefill(np.concatenate(seqs), lens, kv_pool=pool)
    with pytest.raises(capi.AllieError, match="KV pool too small"):
        eng.prefill(np.concatenate(seqs), lens, kv_pool=pool, first_block=2)
    eng.close()


def test_tree_heads_knob_rejects_non_divisors(tiny, cuda):
    """allie_model_set_tree_heads takes 0 or a divisor of the head count up
    to 16 (the tiny model has 4 heads); anything else fails before any launch
    and leaves the setting as it was."""
    cfg, sd = tiny
    eng = Engine(cfg, sd, mode="bfloat16")
    for bad in (3, -1, 32):
        with pytest.raises(capi.AllieError, match="tree heads"):
            eng.set_tree_heads(bad)
    for ok in (0, 1, 2, 4):
        eng.set_tree_heads(ok)
    eng.close()


def test_packer_status_reaches_the_caller(tiny, cuda):
    cfg, sd = tiny
    seqs, lens = games(5, 4, 10, 30)
    seqs[2][3] = 1996  # <PAD> inside game 2
    eng = Engine(cfg, sd, mode="float32")
    st = torch.full((1,), -1, dtype=torch.int32, device=eng.device)
    r = eng.prefill(np.concatenate(seqs), lens, status=st)
    assert int(st.item()) == 8
    # the PAD id is an ordinary token here (its embedding row is wte[1996])
    ref = RefModel(cfg, sd).forward_last([s.astype(np.int64) for s in seqs])
    np.testing.assert_allclose(r.logits.cpu().numpy(), ref["logits"], atol=1e-4)
    # clean batch: status 0
    seqs[2][3] = 17
    eng.prefill(np.concatenate(seqs), lens, status=st)
    assert int(st.item()) == 0
    # a block-table row shorter than its game: flag 4, its tail is not cached
    pool = eng.new_kv_pool(16)
    table = torch.tensor([[0, 1], [2, 3], [4, 5], [6, 7]], dtype=torch.int32, device=eng.device)
    eng.prefill(np.concatenate(seqs), lens, kv_pool=pool, kv_block_table=table, status=st)
    assert int(st.item()) == (4 if (lens > 32).any() else 0)
    long = lens.copy()
    seqs2 = [np.resize(s, 40).astype(np.uint32) for s in seqs]
    long[:] = 40
    eng.prefill(np.concatenate(seqs2), long, kv_pool=pool, kv_block_table=table, status=st)
    assert int(st.item()) == 4
    eng.close()
