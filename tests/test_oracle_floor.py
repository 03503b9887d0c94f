"""The floor of bf16 parity at depth, measured with the oracle alone.

A bf16-autocast forward rounds every GEMM output to bf16, so any change of
summation order or of one rounding detail flips some roundings, and the
flips compound through the layers.  This measures how far equally valid
implementations of the medium model (24 layers) sit from the oracle on the
four longest C2 games: fp64 instead of fp32 summation, P rounded against a
running maximum (online softmax, as flash-attention kernels including the
GPU prefill kernel do), and the exp2 form of gelu_new.  Each alone moves the
logits before their final bf16 rounding by more than 1e-2 -- about the
contract bar of 2e-2 -- while on the 2-layer model the same changes stay
below 1e-2 (measured: 0.016-0.018 at 24 layers, 0.000-0.007 at 2).  The at-size GPU tests hold the GPU to 2e-2
against this backdrop (tests/parity_floor.py).

Reference: bf16 autocast around the model, src/evaluation/decode.py:74-78.
"""
import numpy as np
import pytest
import torch

from allie_amd import config, weights
from bf16_variants import Exp2Gelu, OnlineSoftmax
from oracle.model_ref import RefModel


def c2_games(n):
    rng = np.random.default_rng(2)
    lens = rng.integers(8, 401, 256).astype(np.int32)
    seqs = [rng.integers(0, 1968, k).astype(np.int64) for k in lens]
    return [seqs[i] for i in np.argsort(-lens, kind="stable")[:n]]


def spreads(cfg, sd, games):
    base = RefModel(cfg, sd, mode="bfloat16").forward_last(games, batch=4)["logits_raw"]
    out = {}
    for name, m in (("fp64 summation", RefModel(cfg, sd, mode="bfloat16", accumulate="fp64")),
                    ("online-softmax P", OnlineSoftmax(cfg, sd, mode="bfloat16")),
                    ("exp2 gelu", Exp2Gelu(cfg, sd, mode="bfloat16"))):
        out[name] = float(np.abs(m.forward_last(games, batch=4)["logits_raw"] - base).max())
    return out


def test_bf16_floor_at_depth():
    torch.set_num_threads(max(1, min(8, torch.get_num_threads())))
    cfg = config.MEDIUM
    s = spreads(cfg, weights.init_weights(cfg, seed=0), c2_games(4))
    print("medium (24 layers):", {k: round(v, 4) for k, v in s.items()}, flush=True)
    for name, v in s.items():
        assert 1e-2 < v < 5e-2, (name, v)


def test_bf16_floor_shallow():
    cfg = config.TINY
    s = spreads(cfg, weights.init_weights(cfg, seed=1, perturb=True), c2_games(4))
    print("tiny (2 layers):", {k: round(v, 5) for k, v in s.items()}, flush=True)
    for name, v in s.items():
        assert v < 1e-2, (name, v)
