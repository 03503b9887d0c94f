"""Pins the packing oracle (oracle/pack_ref.c) against the reference's
padded formulation, restated independently in numpy:
pad_and_collate (src/modeling/data.py:281-337) builds a right-padded
[B, Tmax] batch of the first max_length words, ``input_ids = w & 0x3FFF``,
``attention_mask = ids != PAD`` and ``position_ids = (cumsum(mask)-1).clamp(0)``;
the real tokens of that batch, read row by row, must be the oracle's flat
stream, and ``[:, -1]`` of a B=1 batch must be ``last_idx``.
"""
import numpy as np
import pytest

from oracle import pack as opack

PAD = 1996


def padded_reference(words, lens, max_len):
    offs = np.concatenate([[0], np.cumsum(lens)])
    seqs = [words[offs[i]: offs[i + 1]][:max_len].astype(np.int64) for i in range(len(lens))]
    T = max(len(s) for s in seqs)
    data = np.stack([np.pad(s, (0, T - len(s)), constant_values=PAD) for s in seqs])
    ids = data & 0x3FFF
    mask = ids != PAD
    pos = np.maximum(np.cumsum(mask, axis=1) - 1, 0)
    return ids, mask, pos


def words_for(rng, lens):
    T = int(np.sum(lens))
    ids = rng.integers(0, 1996, T).astype(np.uint32)  # the tokenizer never writes PAD
    return ids | (rng.integers(0, 3, T).astype(np.uint32) << 14) | ((rng.integers(0, 61, T).astype(np.uint32) + 1) << 16)


@pytest.mark.parametrize("seed,B,lo,hi,max_len", [(0, 1, 1, 1, 512), (1, 7, 1, 40, 512), (2, 64, 8, 400, 512),
                                                  (3, 20, 500, 700, 512), (4, 30, 1, 60, 16)])
def test_pack_oracle_vs_padded_collate(seed, B, lo, hi, max_len):
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, B).astype(np.int32)
    words = words_for(rng, lens)
    o = opack.pack(words, lens, max_len=max_len, first_block=5)
    assert o["status"] == 0
    ids, mask, pos = padded_reference(words, lens, max_len)
    np.testing.assert_array_equal(o["ids"], ids[mask])
    np.testing.assert_array_equal(o["pos"], pos[mask])
    np.testing.assert_array_equal(o["seq_of"], np.nonzero(mask)[0])
    n = mask.sum(1)
    np.testing.assert_array_equal(o["cu_seqlens"], np.concatenate([[0], np.cumsum(n)]))
    np.testing.assert_array_equal(o["last_idx"], np.cumsum(n) - 1)
    # [0, -1] of each game's own B=1 batch (what Policy/MCTS read) is its last token
    for b in range(B):
        i1, m1, _ = padded_reference(words[sum(lens[:b]):sum(lens[:b + 1])], lens[b:b + 1], max_len)
        assert o["ids"][o["last_idx"][b]] == i1[0, -1]
    # block tables: contiguous blocks per game, slot = block * 16 + offset
    nb = (n + 15) // 16
    np.testing.assert_array_equal(o["blk_off"], np.concatenate([[0], np.cumsum(nb)]))
    for b in range(B):
        row = o["block_table"][b]
        np.testing.assert_array_equal(row[: nb[b]], 5 + o["blk_off"][b] + np.arange(nb[b]))
        assert (row[nb[b]:] == -1).all()
        sl = o["slot"][o["cu_seqlens"][b]: o["cu_seqlens"][b + 1]]
        np.testing.assert_array_equal(sl, row[np.arange(n[b]) // 16] * 16 + np.arange(n[b]) % 16)
    # slots are a permutation-free injection into the pool
    assert len(np.unique(o["slot"])) == len(o["slot"])


def test_pack_oracle_status_bits():
    lens = np.array([3, 0, 2], np.int32)
    words = np.array([1, 2, 3, 4, 5], np.uint32)
    assert opack.pack(words, lens)["status"] & 1
    lens = np.array([40], np.int32)
    words = np.arange(40, dtype=np.uint32)
    assert opack.pack(words, lens, max_blocks=2)["status"] == 4
    words[7] = PAD | (1 << 16)
    assert opack.pack(words, lens)["status"] == 8
    assert opack.pack(words, lens, pad_id=-1)["status"] == 0
