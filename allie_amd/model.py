"""Drop-in model call: ``model(**batch) -> dict`` on the GPU engine.

Stands in for ``CausalLMWithRegressionHead`` (src/modeling/model.py:85-147,
wrapping ``CausalLMWithControlToken`` :28-57 and the GPT-2 LM) as the decode
strategies call it: ``outputs = self.model(**tokenizer.pad_and_collate(...))``
(src/evaluation/decode.py:199-203, 356-360, 541-542).

Keyword arguments are those of ``pad_and_collate`` (data.py:328-337):
``input_ids`` [B, T] (right padded), ``attention_mask`` [B, T],
``position_ids``, ``labels``, ``value_labels``, ``time_labels``.  The real
tokens of each row (mask != 0) are packed into one ragged stream on the GPU
and evaluated in one forward; positions count the real tokens, which is what
``(cumsum(mask) - 1).clamp(0)`` gives them (data.py:327).

Returned keys, each at the LAST real token of every row (the only position
any caller reads: ``[0, -1]`` and ``[:, -1]``, decode.py:204,211,218,366-373):
``logits`` [B, 1, vocab] (fp32 values; bf16-rounded in bf16 mode),
``value_logits`` [B, 1] (tanh value head), ``time_logits`` [B, 1].  The
losses (model.py:112-146) and ``hidden_states`` are not computed: no caller
of the inference path reads them.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from .config import BF16, ModelConfig
from .engine import Engine


class AllieModel:
    def __init__(self, engine: Engine):
        self.engine = engine
        self.config = engine.cfg

    @classmethod
    def from_state_dict(cls, cfg: ModelConfig, state_dict: dict, mode: str = BF16,
                        device: str = "cuda:0") -> "AllieModel":
        """Weights in the reference checkpoint's key layout (``best.pt["model"]``,
        trainer.py:400-408)."""
        return cls(Engine(cfg, state_dict, mode=mode, device=device))

    @classmethod
    def from_checkpoint(cls, path: str, mode: str = BF16, device: str = "cuda:0",
                        n_head: Optional[int] = None) -> "AllieModel":
        """A reference ``best.pt`` (trainer.py:397-408), read as
        evaluate.py:240-243 reads it; see ``allie_amd.checkpoint``."""
        from .checkpoint import load_checkpoint

        cfg, sd = load_checkpoint(path, n_head=n_head)
        return cls.from_state_dict(cfg, sd, mode=mode, device=device)

    def eval(self) -> "AllieModel":
        return self

    def to(self, *args, **kwargs) -> "AllieModel":
        return self

    def __call__(self, input_ids, attention_mask: Optional[torch.Tensor] = None, value_labels=None,
                 time_labels=None, output_hidden_states: bool = True, **kwargs) -> dict:
        return self.forward(input_ids, attention_mask)

    @torch.no_grad()
    def forward(self, input_ids, attention_mask=None) -> dict:
        dev = self.engine.device
        ids = torch.as_tensor(input_ids)
        if ids.dim() == 1:
            ids = ids[None]
        B = ids.shape[0]
        if attention_mask is None:
            mask = torch.ones_like(ids, dtype=torch.bool)
        else:
            mask = torch.as_tensor(attention_mask) != 0
        lens = mask.sum(dim=1).to(torch.int32).cpu().numpy()
        if (lens <= 0).any():
            raise ValueError("every row needs at least one real token")
        # real tokens, row by row (the ids of an unpacked word: id & 0x3FFF)
        words = ids.to(dev)[mask.to(dev)].to(torch.int32).contiguous()
        out = self.engine.prefill(words, np.ascontiguousarray(lens, dtype=np.int32))
        return {
            "logits": out.logits[:, None, :],
            "value_logits": out.value[:, None],
            "time_logits": out.time[:, None],
            # extras of the batched path: first argmax over the move logits and
            # their logsumexp at each row's last token
            "top1": out.top1,
            "lse": out.lse,
        }

    def close(self) -> None:
        self.engine.close()
