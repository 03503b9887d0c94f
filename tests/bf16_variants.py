"""Equally valid bf16 numerics, for measuring the floor of bf16 parity.

Each class changes one rounding detail of the oracle's bf16 emulation
(oracle/model_ref.py) in a way that a correct implementation of the same
model may choose, and that this repository's GPU kernels do choose:

* ``OnlineSoftmax``: the attention probabilities P = exp(s - m) enter the PV
  product rounded to bf16 relative to the running maximum m of the keys seen
  so far, in blocks of ``key_block`` keys (flash-attention style, as the GPU
  prefill kernel does with 32-key blocks and torch's CUDA flash kernels do
  with theirs), instead of relative to the row's final maximum;
* ``Exp2Gelu``: gelu_new evaluated as x * sigmoid(2u) through exp2, the
  algebraically equal form the GPU epilogue uses, instead of the tanh form;
* ``accumulate="fp64"`` of the oracle itself: GEMM sums in float64.

Test infrastructure only (tests/test_oracle_floor.py).
"""
from __future__ import annotations

import math

import torch

import oracle.model_ref as mr
from oracle.model_ref import RefModel, rb


class OnlineSoftmax(RefModel):
    key_block = 32

    def attention(self, qkv, key_mask):
        if self.mode == "float32":
            return super().attention(qkv, key_mask)
        B, T, _ = qkv.shape
        H, hd, d = self.cfg.n_head, self.cfg.head_dim, self.cfg.d_model
        q, k, v = (t.view(B, T, H, hd).transpose(1, 2) for t in qkv.split(d, dim=-1))
        s = self._mm(q, k.transpose(-1, -2)) * (1.0 / math.sqrt(hd))
        allowed = torch.ones(T, T, dtype=torch.bool).tril()[None, None] & key_mask[:, None, None, :]
        s = s.masked_fill(~allowed, float("-inf"))
        nb = -(-T // self.key_block)
        sp = torch.nn.functional.pad(s, (0, nb * self.key_block - T), value=float("-inf"))
        m_run = torch.cummax(sp.view(B, H, T, nb, self.key_block).amax(-1), dim=-1).values  # after each key block
        m_key = m_run.repeat_interleave(self.key_block, dim=-1)[..., :T]  # running max when each key is used
        m_fin = m_run[..., -1:]
        p = torch.where(torch.isfinite(m_key), torch.exp(s - m_key), torch.zeros_like(s))
        w = rb(p) * torch.exp(m_key - m_fin).nan_to_num(0.0)  # rounded, then rescaled to the final max
        o = self._mm(w, v) / torch.exp(s - m_fin).sum(-1, keepdim=True)
        return rb(o.transpose(1, 2).reshape(B, T, d))


def gelu_exp2(x: torch.Tensor) -> torch.Tensor:
    k2 = -2.0 * math.sqrt(2.0 / math.pi) * math.log2(math.e)
    t = x * (x * x * (k2 * 0.044715) + k2)
    return x / (1.0 + torch.exp2(t))


class Exp2Gelu(RefModel):
    def block(self, h, lw, key_mask):
        old = mr.gelu_new
        mr.gelu_new = gelu_exp2
        try:
            return super().block(h, lw, key_mask)
        finally:
            mr.gelu_new = old
