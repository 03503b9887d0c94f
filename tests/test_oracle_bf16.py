"""The oracle's bf16 mode against torch autocast running transformers' GPT-2.

Known answers: tests/golden/model_tiny_bf16.npz (written by
make_bf16_golden.py with the installed transformers under
torch.autocast(bf16); ``cuda`` run = CUDA autocast's op list, ``cpu`` run =
stock CPU autocast).  The reference's bf16 mode is autocast around the model
(src/evaluation/decode.py:74-78) with SDPA attention (src/modeling/model.py:190).

The sharp check is the output of block 0 (fp32 residual stream after one
block): an emulation with the same rounding points as autocast reproduces
most of its values bit for bit, the rest differing by summation order.  Each
plausible mistake -- a GEMM output, input or bias left unrounded, q/k/v or
the softmax probabilities kept in fp32, a bf16 residual stream, the GELU in
bf16 arithmetic -- drops the bit-identical fraction well below what the
oracle reaches (planted here on the CPU, one at a time).
"""
import math
import os

import numpy as np
import pytest
import torch

import oracle.model_ref as MR
from allie_amd import config, weights
from oracle.model_ref import RefModel, layer_norm, rb

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "model_tiny_bf16.npz")
EQ_MIN = 0.5  # bit-identical share of block-0 outputs an emulation with autocast's rounding points reaches


@pytest.fixture(scope="module")
def fx():
    return dict(np.load(FIX))


@pytest.fixture(scope="module")
def tiny():
    cfg = config.TINY
    return cfg, weights.init_weights(cfg, seed=7, perturb=True)


def games(fx):
    lens = fx["lens"]
    off = np.concatenate([[0], np.cumsum(lens)])
    return [fx["ids"][off[i]:off[i + 1]].astype(np.int64) for i in range(len(lens))]


def block0(cfg, sd, seqs, stride):
    r = RefModel(cfg, sd, mode="bfloat16")
    out = []
    with torch.no_grad():
        for s in seqs:
            ids = torch.from_numpy(s)[None]
            h = r.embed(ids, torch.arange(len(s))[None])
            h = r.block(h, r.layers[0], torch.ones(1, len(s), dtype=torch.bool))
            out.append(h[0, ::stride].numpy())
    return np.concatenate(out)


def eq_share(a, b):
    return float((a == b).mean())


def gelu_bf16_ops(x):
    """gelu_new with every op in bf16 (stock CPU autocast leaves pow in bf16)."""
    x = rb(x)
    t = rb(torch.pow(x, 3.0))
    t = rb(x + rb(0.044715 * t))
    t = rb(torch.tanh(rb(math.sqrt(2.0 / math.pi) * t)))
    return rb(rb(0.5 * x) * rb(1.0 + t))


def test_bf16_oracle_matches_autocast_fixture(fx, tiny):
    cfg, sd = tiny
    seqs = games(fx)
    got = block0(cfg, sd, seqs, int(fx["row_stride"]))
    share = eq_share(got, fx["cuda_block0"])
    err = np.abs(got - fx["cuda_block0"])
    print(f"block 0: {share:.3f} bit-identical, max |d| {err.max():.3g}")
    assert share >= EQ_MIN and err.max() < 4e-3
    # last-token outputs of the whole model within the bf16 bar
    ref = RefModel(cfg, sd, mode="bfloat16").forward_last(seqs, batch=1)
    dl = np.abs(ref["logits"] - fx["cuda_logits"]).max()
    dv = np.abs(ref["value_logits"] - fx["cuda_value"]).max()
    dt = np.abs(ref["time_logits"] - fx["cuda_time"]).max()
    print(f"last token: max|dlogit| {dl:.3g} max|dvalue| {dv:.3g} max|dtime| {dt:.3g}")
    assert dl <= 2e-2 and dv <= 2e-2 and dt <= 2e-2


def test_fixture_tells_cpu_from_cuda_autocast(fx, tiny, monkeypatch):
    """The one op-list difference (pow: fp32 on CUDA, bf16 on CPU) is visible:
    the oracle matches the CUDA-list run and not the stock CPU run; with its
    GELU planted in bf16 arithmetic it matches the CPU run instead."""
    cfg, sd = tiny
    seqs = games(fx)
    st = int(fx["row_stride"])
    base = block0(cfg, sd, seqs, st)
    assert eq_share(base, fx["cpu_block0"]) < EQ_MIN
    monkeypatch.setattr(MR, "gelu_new", gelu_bf16_ops)
    planted = block0(cfg, sd, seqs, st)
    assert eq_share(planted, fx["cpu_block0"]) >= EQ_MIN
    assert eq_share(planted, fx["cuda_block0"]) < EQ_MIN


def _attention_fp32_probs(self, qkv, key_mask):
    """Planted mistake: softmax probabilities kept in fp32 for the PV product."""
    B, T, _ = qkv.shape
    H, hd, d = self.cfg.n_head, self.cfg.head_dim, self.cfg.d_model
    q, k, v = (t.view(B, T, H, hd).transpose(1, 2) for t in qkv.split(d, dim=-1))
    s = (q @ k.transpose(-1, -2)) / math.sqrt(hd)
    allowed = torch.ones(T, T, dtype=torch.bool).tril()[None, None] & key_mask[:, None, None, :]
    p = torch.softmax(s.masked_fill(~allowed, float("-inf")), dim=-1)
    return rb((p @ v).transpose(1, 2).reshape(B, T, d))


def _block_fp32_qkv(self, h, lw, key_mask):
    """Planted mistake: q/k/v not rounded to bf16 (only the next GEMM input is)."""
    a = layer_norm(h, lw["ln1_g"], lw["ln1_b"], self.cfg.eps)
    qkv = rb(a) @ rb(lw["w_qkv"]) + rb(lw["b_qkv"])
    h = h + self._lin(self.attention(qkv, key_mask), lw["w_o"], lw["b_o"])
    a = layer_norm(h, lw["ln2_g"], lw["ln2_b"], self.cfg.eps)
    f = MR.gelu_new(self._lin(a, lw["w_fc"], lw["b_fc"]))
    return h + self._lin(f, lw["w_pr"], lw["b_pr"])


_ORIG_BLOCK = RefModel.block

MISTAKES = {
    "gemm output unrounded": ("_lin", lambda self, x, w, b: rb(x) @ rb(w) + rb(b)),
    "gemm inputs unrounded": ("_lin", lambda self, x, w, b: rb(x @ w + b)),
    "bias unrounded": ("_lin", lambda self, x, w, b: rb(rb(x) @ rb(w) + b)),
    "probabilities fp32": ("attention", _attention_fp32_probs),
    "q/k/v fp32": ("block", _block_fp32_qkv),
    "residual bf16": ("block", lambda self, h, lw, km: rb(_ORIG_BLOCK(self, h, lw, km))),
}


@pytest.mark.parametrize("name", sorted(MISTAKES))
def test_fixture_rejects_planted_mistake(fx, tiny, monkeypatch, name):
    cfg, sd = tiny
    attr, fn = MISTAKES[name]
    monkeypatch.setattr(RefModel, attr, fn)
    got = block0(cfg, sd, games(fx), int(fx["row_stride"]))
    share = eq_share(got, fx["cuda_block0"])
    print(f"{name}: {share:.3f} bit-identical")
    assert share < EQ_MIN, name
