"""Seeded weights in the reference's state-dict layout.

Key names are those of the reference checkpoint ``best.pt["model"]``
(written at src/modeling/trainer.py:400-408, loaded at
src/evaluation/evaluate.py:241-243): the GPT-2 LM sits at ``model.model``
inside ``CausalLMWithControlToken`` (model.py:20) inside
``CausalLMWithRegressionHead`` (model.py:70, 192-196).

Initialisation (there are no checkpoints or network here) follows GPT-2's
scheme [lib transformers GPT2PreTrainedModel._init_weights]: N(0, 0.02) for
Conv1D weights and embeddings, N(0, 0.02/sqrt(2 L)) for both ``c_proj``
weights, zero biases, unit LayerNorm.  ``control_embeds`` is N(0, 0.02)
(model.py:23-24); the value and time heads use ``nn.Linear``'s default
U(+-1/sqrt(d)).  Draws come from ``numpy.random.default_rng(seed)`` (PCG64,
platform stable), so a GPU box regenerates the same weights.

``perturb=True`` gives the correctness variant: non-zero biases, LayerNorm
gains 1 + N(0, 0.1), non-zero LayerNorm biases and query/key weights scaled
by 8 so attention is sharp.  With GPT-2's default init attention is nearly
uniform and biases are zero, which would hide masking and bias bugs.
"""
from __future__ import annotations

import numpy as np

from .config import ModelConfig

P = "model.model.transformer."


def layer_keys(i: int) -> dict[str, str]:
    b = f"{P}h.{i}."
    return {
        "ln1_g": b + "ln_1.weight",
        "ln1_b": b + "ln_1.bias",
        "w_qkv": b + "attn.c_attn.weight",
        "b_qkv": b + "attn.c_attn.bias",
        "w_o": b + "attn.c_proj.weight",
        "b_o": b + "attn.c_proj.bias",
        "ln2_g": b + "ln_2.weight",
        "ln2_b": b + "ln_2.bias",
        "w_fc": b + "mlp.c_fc.weight",
        "b_fc": b + "mlp.c_fc.bias",
        "w_pr": b + "mlp.c_proj.weight",
        "b_pr": b + "mlp.c_proj.bias",
    }


GLOBAL_KEYS = {
    "wte": P + "wte.weight",
    "wpe": P + "wpe.weight",
    "lnf_g": P + "ln_f.weight",
    "lnf_b": P + "ln_f.bias",
    "lm_head": "model.model.lm_head.weight",  # tied to wte
    "ctrl": "model.control_embeds.weight",
    "w_value": "value_head.0.weight",
    "b_value": "value_head.0.bias",
    "w_time": "time_head.0.weight",
    "b_time": "time_head.0.bias",
}


def init_weights(cfg: ModelConfig, seed: int = 0, perturb: bool = False) -> dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    d, L, V = cfg.d_model, cfg.n_layer, cfg.vocab_size
    f32 = np.float32

    def normal(shape, std):
        return (rng.standard_normal(shape, dtype=f32) * f32(std)).astype(f32)

    def uniform(shape, bound):
        return rng.uniform(-bound, bound, size=shape).astype(f32)

    sd: dict[str, np.ndarray] = {}
    sd[GLOBAL_KEYS["wte"]] = normal((V, d), 0.02)
    sd[GLOBAL_KEYS["wpe"]] = normal((cfg.n_positions, d), 0.02)
    proj_std = 0.02 / np.sqrt(2 * L)
    for i in range(L):
        k = layer_keys(i)
        sd[k["ln1_g"]] = np.ones(d, f32)
        sd[k["ln1_b"]] = np.zeros(d, f32)
        sd[k["w_qkv"]] = normal((d, 3 * d), 0.02)
        sd[k["b_qkv"]] = np.zeros(3 * d, f32)
        sd[k["w_o"]] = normal((d, d), proj_std)
        sd[k["b_o"]] = np.zeros(d, f32)
        sd[k["ln2_g"]] = np.ones(d, f32)
        sd[k["ln2_b"]] = np.zeros(d, f32)
        sd[k["w_fc"]] = normal((d, 4 * d), 0.02)
        sd[k["b_fc"]] = np.zeros(4 * d, f32)
        sd[k["w_pr"]] = normal((4 * d, d), proj_std)
        sd[k["b_pr"]] = np.zeros(d, f32)
    sd[GLOBAL_KEYS["lnf_g"]] = np.ones(d, f32)
    sd[GLOBAL_KEYS["lnf_b"]] = np.zeros(d, f32)
    sd[GLOBAL_KEYS["ctrl"]] = normal((2, d), 0.02)
    bound = 1.0 / np.sqrt(d)
    sd[GLOBAL_KEYS["w_value"]] = uniform((1, d), bound)
    sd[GLOBAL_KEYS["b_value"]] = uniform((1,), bound)
    sd[GLOBAL_KEYS["w_time"]] = uniform((1, d), bound)
    sd[GLOBAL_KEYS["b_time"]] = uniform((1,), bound)

    if perturb:
        for i in range(L):
            k = layer_keys(i)
            for g in ("ln1_g", "ln2_g"):
                sd[k[g]] = (1.0 + normal((d,), 0.1)).astype(f32)
            for b in ("ln1_b", "ln2_b"):
                sd[k[b]] = normal((d,), 0.05)
            for b, n in (("b_qkv", 3 * d), ("b_o", d), ("b_fc", 4 * d), ("b_pr", d)):
                sd[k[b]] = normal((n,), 0.05)
            w = sd[k["w_qkv"]].copy()
            w[:, : 2 * d] *= 8.0  # sharpen attention: scale Wq and Wk
            sd[k["w_qkv"]] = w
        sd[GLOBAL_KEYS["lnf_g"]] = (1.0 + normal((d,), 0.1)).astype(f32)
        sd[GLOBAL_KEYS["lnf_b"]] = normal((d,), 0.05)
    sd[GLOBAL_KEYS["lm_head"]] = sd[GLOBAL_KEYS["wte"]]
    return sd


def quantize_fp8_per_channel(w_in_out: np.ndarray):
    """fp8 e4m3fn (OCP, max 448) weights with one fp32 scale per output
    channel: ``s_j = max_k |W[k, j]| / 448`` and ``q = rne_e4m3(W / s_j)``.

    Input is a Conv1D weight ``[in, out]``; returns ``(q [out, in] uint8 bits,
    s [out] float32)`` in the engine's ``[N, K]`` layout.  Rounding uses
    torch's float8_e4m3fn conversion (round to nearest even).
    """
    import torch

    w = torch.from_numpy(np.ascontiguousarray(w_in_out.T))  # [out, in]
    amax = w.abs().amax(dim=1).clamp_min(1e-12)
    s = (amax / 448.0).to(torch.float32)
    q = (w / s[:, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).numpy(), s.numpy()


def dequantize_fp8(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """Inverse of :func:`quantize_fp8_per_channel`: returns ``[in, out]`` fp32."""
    import torch

    w = torch.from_numpy(q).view(torch.float8_e4m3fn).to(torch.float32) * torch.from_numpy(s)[:, None]
    return np.ascontiguousarray(w.numpy().T)
