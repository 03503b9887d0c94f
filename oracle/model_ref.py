"""CPU restatement of the Allie model forward -- TEST INFRASTRUCTURE ONLY.

Follows, op for op:
  * CausalLMWithControlToken.forward (src/modeling/model.py:28-57): Elo ids
    (``id >= V``) embed as ``[e, 1-e] @ control_embeds`` with
    ``e = (clamp(id - V, 500, 3000) - 500) / 2500``; other ids look up ``wte``.
  * [lib transformers==4.39.3 GPT2Model] ``h = inputs_embeds + wpe[pos]``;
    per block: ``h += c_proj(attn(ln_1(h)))``, ``h += mlp(ln_2(h))`` with
    Conv1D ``y = x @ W[in,out] + b``, q/k/v taken as column blocks of
    ``c_attn``, heads as 64-column groups, scale 1/sqrt(head_dim), causal
    softmax, and ``gelu_new(x) = 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3)))``;
    then ``ln_f`` and the tied ``lm_head`` (no bias).
  * [lib optimum==1.18 BetterTransformer GPT-2] at B>1 the additive mask is
    causal plus key padding (model.py:190); real queries of a right-padded
    batch therefore see keys 0..i of their own game only.
  * CausalLMWithRegressionHead.forward (model.py:85-110): value =
    ``tanh(h_L @ w_v + b_v)``, time = ``h_L @ w_t + b_t`` on the post-``ln_f``
    hidden state, at every position.

Modes:
  * ``float32``  -- plain fp32 (the reference's evaluation precision,
    evaluate.py:249; the fp32 check mode).
  * ``bfloat16`` -- emulation of torch CUDA autocast(bf16) (decode.py:74-78):
    GEMM operands and biases rounded to bf16, output of each GEMM rounded to
    bf16 (``addmm``), LayerNorm/residual in fp32, ``gelu_new`` computed in
    fp32 from the bf16 GEMM output (CUDA autocast casts ``pow`` to fp32; CPU
    autocast does not), the Elo ``[e, 1-e] @ Wc`` matmul in bf16, heads
    rounded to bf16.  Attention follows torch's bf16
    ``scaled_dot_product_attention`` kernels (autocast runs SDPA in bf16 on
    the bf16 q/k/v): scores and softmax statistics in fp32, the
    probabilities ``P = exp(s - rowmax)`` rounded to bf16 for the product
    with V (fp32 accumulation), normalised by the fp32 row sum, output
    rounded to bf16.  Pinned by tests/golden/model_tiny_bf16.npz (the
    installed transformers GPT-2 under torch.autocast; tests/test_oracle_bf16.py).
    Summation order is not pinnable: at 24 layers two orders differ by about
    one bf16 ulp of the largest logits.
  * ``fp8w`` -- as ``bfloat16`` but the four block GEMMs use fp8 e4m3 weights
    with a per-output-channel fp32 scale applied to the fp32 accumulator (the
    weight itself is not rounded to bf16).
"""
from __future__ import annotations

import math

import numpy as np
import torch

from allie_amd import weights as W
from allie_amd.config import ModelConfig


def rb(x: torch.Tensor) -> torch.Tensor:
    """Round fp32 -> bf16 -> fp32 (round to nearest even)."""
    return x.to(torch.bfloat16).to(torch.float32)


def gelu_new(x: torch.Tensor) -> torch.Tensor:
    return (0.5 * x) * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * torch.pow(x, 3.0))))


def layer_norm(x: torch.Tensor, g: torch.Tensor, b: torch.Tensor, eps: float) -> torch.Tensor:
    return torch.nn.functional.layer_norm(x, (x.shape[-1],), g, b, eps)


class RefModel:
    """accumulate: "fp32", or "fp64" to sum every GEMM in float64 (rounding
    points unchanged) -- an equally valid summation order, used to measure
    how far two faithful bf16 implementations drift apart."""

    def __init__(self, cfg: ModelConfig, sd: dict, mode: str = "float32", accumulate: str = "fp32"):
        assert mode in ("float32", "bfloat16", "fp8w")
        assert accumulate in ("fp32", "fp64")
        self.cfg, self.mode, self.acc64 = cfg, mode, accumulate == "fp64"
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
        g = W.GLOBAL_KEYS
        self.wte, self.wpe, self.ctrl = t(sd[g["wte"]]), t(sd[g["wpe"]]), t(sd[g["ctrl"]])
        self.lnf_g, self.lnf_b = t(sd[g["lnf_g"]]), t(sd[g["lnf_b"]])
        self.w_value, self.b_value = t(sd[g["w_value"]]), t(sd[g["b_value"]])
        self.w_time, self.b_time = t(sd[g["w_time"]]), t(sd[g["b_time"]])
        self.layers = []
        for i in range(cfg.n_layer):
            k = W.layer_keys(i)
            lw = {n: t(sd[key]) for n, key in k.items()}
            if mode == "fp8w":
                for n in ("w_qkv", "w_o", "w_fc", "w_pr"):
                    q, s = W.quantize_fp8_per_channel(sd[k[n]])
                    lw[n] = t(W.dequantize_fp8(q, s))
            self.layers.append(lw)

    # ---- numeric helpers -------------------------------------------------
    def _mm(self, x, w):
        if self.acc64:
            return (x.double() @ w.double()).float()
        return x @ w

    def _lin(self, x, w, b):
        """Conv1D / addmm (model weights are [in, out])."""
        if self.mode == "float32":
            return self._mm(x, w) + b
        wq = w if self.mode == "fp8w" else rb(w)
        return rb(self._mm(rb(x), wq) + rb(b))

    def _lin_bf16(self, x, w, b, round_out=True):
        """Linear layers outside the blocks (heads): bf16 weights in both
        reduced-precision modes; round_out=False gives the fp32 result before
        the output's bf16 rounding."""
        if self.mode == "float32":
            return self._mm(x, w) + (b if b is not None else 0.0)
        y = self._mm(rb(x), rb(w))
        if b is not None:
            y = y + rb(b)
        return rb(y) if round_out else y

    # ---- pieces ------------------------------------------------------------
    def embed(self, ids: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        V = self.cfg.vocab_size
        elo = ids >= V
        e = ((ids - V).clamp(500, 3000) - 500) / (3000 - 500)
        cv = torch.stack((e, 1 - e), dim=-1).to(torch.float32)
        if self.mode == "float32":
            ce = cv @ self.ctrl
        else:
            ce = rb(rb(cv) @ rb(self.ctrl))
        te = self.wte[ids.clamp(0, V - 1)]
        x = torch.where(elo.unsqueeze(-1), ce, te)
        return x + self.wpe[pos]

    def attention(self, qkv: torch.Tensor, key_mask: torch.Tensor) -> torch.Tensor:
        """qkv [B,T,3d], key_mask [B,T] bool -> [B,T,d]; causal."""
        B, T, _ = qkv.shape
        H, hd, d = self.cfg.n_head, self.cfg.head_dim, self.cfg.d_model
        q, k, v = qkv.split(d, dim=-1)
        q = q.view(B, T, H, hd).transpose(1, 2)
        k = k.view(B, T, H, hd).transpose(1, 2)
        v = v.view(B, T, H, hd).transpose(1, 2)
        s = self._mm(q, k.transpose(-1, -2)) * (1.0 / math.sqrt(hd))
        causal = torch.ones(T, T, dtype=torch.bool).tril()
        allowed = causal[None, None] & key_mask[:, None, None, :]
        s = s.masked_fill(~allowed, float("-inf"))
        if self.mode == "float32":
            p = torch.softmax(s, dim=-1)
            return self._mm(p, v).transpose(1, 2).reshape(B, T, d)
        # bf16 SDPA: P = exp(s - rowmax) enters the PV product as bf16; the
        # row sum and the accumulation stay fp32
        p = torch.exp(s - s.max(dim=-1, keepdim=True).values)
        o = self._mm(rb(p), v) / p.sum(dim=-1, keepdim=True)
        return rb(o.transpose(1, 2).reshape(B, T, d))

    def block(self, h: torch.Tensor, lw: dict, key_mask: torch.Tensor) -> torch.Tensor:
        eps = self.cfg.eps
        a = layer_norm(h, lw["ln1_g"], lw["ln1_b"], eps)
        qkv = self._lin(a, lw["w_qkv"], lw["b_qkv"])
        o = self.attention(qkv, key_mask)
        h = h + self._lin(o, lw["w_o"], lw["b_o"])
        a = layer_norm(h, lw["ln2_g"], lw["ln2_b"], eps)
        f = gelu_new(self._lin(a, lw["w_fc"], lw["b_fc"]))
        return h + self._lin(f, lw["w_pr"], lw["b_pr"])

    def heads(self, hL: torch.Tensor) -> dict:
        """hL: post-ln_f hidden state [..., d]."""
        raw = self._lin_bf16(hL, self.wte.T, None, round_out=False)
        logits = raw if self.mode == "float32" else rb(raw)
        v = self._lin_bf16(hL, self.w_value.T, self.b_value)[..., 0]
        value = torch.tanh(v) if self.mode == "float32" else rb(torch.tanh(v))
        time = self._lin_bf16(hL, self.w_time.T, self.b_time)[..., 0]
        return {"logits": logits, "value_logits": value, "time_logits": time, "logits_raw": raw}

    # ---- forwards ----------------------------------------------------------
    @torch.no_grad()
    def forward_padded(self, input_ids, attention_mask=None, position_ids=None, last_only=False):
        """The reference's execution shape: a right-padded [B, T] batch,
        outputs at every position (model.py:85-110, data.py:328-337)."""
        input_ids = torch.as_tensor(input_ids, dtype=torch.int64)
        B, T = input_ids.shape
        if attention_mask is None:
            attention_mask = torch.ones(B, T)
        key_mask = torch.as_tensor(attention_mask) > 0
        if position_ids is None:
            position_ids = (key_mask.long().cumsum(-1) - 1).clamp(0)
        h = self.embed(input_ids, torch.as_tensor(position_ids, dtype=torch.int64))
        for lw in self.layers:
            h = self.block(h, lw, key_mask)
        if last_only:
            n = key_mask.long().sum(-1)
            h = h[torch.arange(B), n - 1]
        hL = layer_norm(h, self.lnf_g, self.lnf_b, self.cfg.eps)
        return self.heads(hL)

    @torch.no_grad()
    def forward_last(self, seqs: list[np.ndarray], batch: int = 8) -> dict:
        """Last-token outputs of each id sequence (what Policy/MCTS read),
        computed over right-padded sub-batches; ``logits_raw`` holds the
        logits before their final bf16 rounding."""
        outs = {"logits": [], "value_logits": [], "time_logits": [], "logits_raw": []}
        for i in range(0, len(seqs), batch):
            chunk = seqs[i : i + batch]
            T = max(len(s) for s in chunk)
            ids = torch.full((len(chunk), T), 1996, dtype=torch.int64)
            m = torch.zeros(len(chunk), T)
            for j, s in enumerate(chunk):
                ids[j, : len(s)] = torch.as_tensor(np.asarray(s, dtype=np.int64))
                m[j, : len(s)] = 1
            o = self.forward_padded(ids, m, last_only=True)
            for k in outs:
                outs[k].append(o[k])
        return {k: torch.cat(v).numpy() for k, v in outs.items()}


def policy_summary(logits: np.ndarray, n_moves: int = 1968, temperature: float = 1.0) -> dict:
    """Per row: first-max argmax over the move logits and the logsumexp of
    ``logits[:n_moves] / T`` (decode.py:223-226; torch.argmax returns the
    first maximal index)."""
    l = np.asarray(logits, dtype=np.float64)[:, :n_moves] / max(temperature, 1e-5)
    top1 = l.argmax(axis=1)
    m = l.max(axis=1)
    lse = m + np.log(np.exp(l - m[:, None]).sum(axis=1))
    srt = np.sort(l, axis=1)
    margin = srt[:, -1] - srt[:, -2]
    return {"top1": top1.astype(np.int32), "lse": lse, "margin": margin}
