"""Reference checkpoint loader: ``best.pt`` -> (ModelConfig, state dict).

The reference saves ``{"iter_num", "best_val_loss", "model", "optimizer"}``
with ``torch.save`` (src/modeling/trainer.py:397-408), where ``model`` is the
state dict of ``CausalLMWithRegressionHead`` (unwrapped from DDP, :399), and
loads it with ``model.load_state_dict(ckpt["model"])``
(src/evaluation/evaluate.py:240-243).  Key names follow the module nesting
(model.py:20-24, 70-80): the GPT-2 LM at ``model.model.``, the control
embedding at ``model.control_embeds``, the heads at ``value_head.0`` and
``time_head.0``; ``allie_amd.weights`` lists them.

The file is read with ``torch.load(..., weights_only=True)``, which rebuilds
tensors and plain containers and executes nothing else from the file.  The
optimizer state is dropped.  Non-parameter buffers that some ``transformers``
versions store (``attn.bias``, ``attn.masked_bias``: the causal mask) are
ignored.  ``lm_head.weight`` must equal ``wte.weight``: GPT-2 ties them
(``tie_word_embeddings``), and the engine's heads matrix is built from
``wte``.

The state dict does not record ``n_head``.  Every reference config uses
64-wide heads (medium 1024/16, small 768/12), so ``n_head = d_model // 64``
unless given.
"""
from __future__ import annotations

import dataclasses
import os
import re
from typing import Optional

import numpy as np

from . import weights as W
from .config import ModelConfig

_PREFIXES = ("module.", "_orig_mod.")  # DDP / torch.compile wrappers, if a state dict kept them
_IGNORED = re.compile(r"(^|\.)attn\.(bias|masked_bias)$")


class CheckpointError(ValueError):
    pass


def _strip(key: str) -> str:
    changed = True
    while changed:
        changed = False
        for p in _PREFIXES:
            if key.startswith(p):
                key, changed = key[len(p):], True
    return key


def _to_numpy(v) -> np.ndarray:
    import torch

    if isinstance(v, torch.Tensor):
        return v.detach().to("cpu", torch.float32).numpy()
    return np.asarray(v, dtype=np.float32)


def config_from_state_dict(sd: dict, n_head: Optional[int] = None, base: Optional[ModelConfig] = None) -> ModelConfig:
    """Shape of the model a state dict holds (layers, width, positions)."""
    G = W.GLOBAL_KEYS
    for k in (G["wte"], G["wpe"]):
        if k not in sd:
            raise CheckpointError(f"state dict has no {k}")
    V, d = np.shape(sd[G["wte"]])
    n_pos = np.shape(sd[G["wpe"]])[0]
    layers = {int(m.group(1)) for k in sd for m in [re.match(re.escape(W.P) + r"h\.(\d+)\.", k)] if m}
    n_layer = len(layers)
    if n_layer == 0 or layers != set(range(n_layer)):
        raise CheckpointError(f"block indices are not 0..n-1: {sorted(layers)[:8]}")
    if n_head is None:
        if d % 64:
            raise CheckpointError(f"d_model {d} is not a multiple of 64; pass n_head")
        n_head = d // 64
    cfg = dataclasses.replace(base, n_layer=n_layer, d_model=d, n_head=n_head, n_positions=n_pos) if base \
        else ModelConfig(n_layer=n_layer, d_model=d, n_head=n_head, n_positions=n_pos)
    if V != cfg.vocab_size:
        raise CheckpointError(f"wte has {V} rows; this build's vocabulary has {cfg.vocab_size}")
    return cfg


def canonical_state_dict(raw: dict, cfg: ModelConfig) -> dict[str, np.ndarray]:
    """fp32 arrays under the reference's key names, every key the engine
    needs present with its shape; unknown keys are an error."""
    sd = {}
    for k, v in raw.items():
        k = _strip(k)
        if _IGNORED.search(k):
            continue
        sd[k] = _to_numpy(v)
    d, V = cfg.d_model, cfg.vocab_size
    want = {
        W.GLOBAL_KEYS["wte"]: (V, d), W.GLOBAL_KEYS["wpe"]: (cfg.n_positions, d),
        W.GLOBAL_KEYS["lnf_g"]: (d,), W.GLOBAL_KEYS["lnf_b"]: (d,), W.GLOBAL_KEYS["ctrl"]: (2, d),
        W.GLOBAL_KEYS["w_value"]: (1, d), W.GLOBAL_KEYS["b_value"]: (1,),
        W.GLOBAL_KEYS["w_time"]: (1, d), W.GLOBAL_KEYS["b_time"]: (1,),
    }
    shapes = {"ln1_g": (d,), "ln1_b": (d,), "w_qkv": (d, 3 * d), "b_qkv": (3 * d,), "w_o": (d, d), "b_o": (d,),
              "ln2_g": (d,), "ln2_b": (d,), "w_fc": (d, 4 * d), "b_fc": (4 * d,), "w_pr": (4 * d, d), "b_pr": (d,)}
    for i in range(cfg.n_layer):
        for name, key in W.layer_keys(i).items():
            want[key] = shapes[name]
    for k, shp in want.items():
        if k not in sd:
            raise CheckpointError(f"state dict has no {k}")
        if tuple(sd[k].shape) != shp:
            raise CheckpointError(f"{k}: shape {tuple(sd[k].shape)}, expected {shp}")
    lm = W.GLOBAL_KEYS["lm_head"]
    if lm in sd:
        if sd[lm].shape != sd[W.GLOBAL_KEYS["wte"]].shape or not np.array_equal(sd[lm], sd[W.GLOBAL_KEYS["wte"]]):
            raise CheckpointError("lm_head.weight differs from wte.weight; the engine needs them tied")
    else:
        sd[lm] = sd[W.GLOBAL_KEYS["wte"]]
    extra = sorted(set(sd) - set(want) - {lm})
    if extra:
        raise CheckpointError(f"unexpected keys: {extra[:6]}")
    return sd


def load_checkpoint(path: str, n_head: Optional[int] = None,
                    base: Optional[ModelConfig] = None) -> tuple[ModelConfig, dict[str, np.ndarray]]:
    """Read a reference ``best.pt`` (or a bare state dict saved with
    ``torch.save``) and return its config and fp32 state dict."""
    import torch

    if not os.path.isfile(path):
        raise FileNotFoundError(path)
    obj = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(obj, dict):
        raise CheckpointError(f"{path}: expected a dict, got {type(obj).__name__}")
    raw = obj["model"] if "model" in obj and isinstance(obj["model"], dict) else obj
    stripped = {_strip(k): v for k, v in raw.items()}
    cfg = config_from_state_dict(stripped, n_head=n_head, base=base)
    return cfg, canonical_state_dict(raw, cfg)
