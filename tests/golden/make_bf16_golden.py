"""Writes tests/golden/model_tiny_bf16.npz: known answers for the bf16 mode.

The reference's bf16 mode is ``torch.autocast(device_type, torch.bfloat16)``
around the model (src/evaluation/decode.py:74-78); its GPT-2 blocks are the
third-party ``transformers`` code (requirements.txt:11, built at
src/modeling/model.py:165-190; BetterTransformer routes attention to
``torch.nn.functional.scaled_dot_product_attention``).  This script runs the
``transformers`` and ``torch`` installed in this image -- ``GPT2LMHeadModel``
from a local ``GPT2Config``, ``attn_implementation="sdpa"``, no network --
under ``torch.autocast("cpu", dtype=torch.bfloat16)`` with the weights of
``allie_amd.weights.init_weights(TINY, seed=7, perturb=True)``.

CPU and CUDA autocast differ on one op of this model: CUDA's list casts
``pow`` to fp32, so the tanh GELU (``gelu_new``) runs in fp32 on a GPU, while
CPU autocast leaves it in bf16.  The fixture therefore holds two runs:

* ``cuda`` -- each block's GELU module replaced by the same formula computed
  in fp32 (what CUDA autocast does to it); the known answer for the
  oracle's bf16 mode;
* ``cpu``  -- stock CPU autocast, which tells the two op lists apart.

Per run it stores, for games given at batch 1 (the reference's call shape,
decode.py:199-203,356-360): the output of block 0 (``hidden_states[1]``,
fp32) on every third row, and at the last token the post-``ln_f`` hidden
state, the bf16 logits and the value / time heads (the heads written out
here as ``nn.Linear`` modules under the same autocast, model.py:72-80).

Run here (CPU):  python tests/golden/make_bf16_golden.py
"""
import math
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from allie_amd import config, weights  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "model_tiny_bf16.npz")
SEED = 7
LENS = [1, 5, 17, 40, 77, 130, 200, 300]
ROW_STRIDE = 3


class GeluFp32(torch.nn.Module):
    """gelu_new with autocast's CUDA treatment of pow: computed in fp32."""

    def forward(self, x):
        with torch.autocast("cpu", enabled=False):
            x = x.float()
            return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * torch.pow(x, 3.0))))


def games():
    rng = np.random.default_rng(SEED + 100)
    return [rng.integers(0, 1968, n).astype(np.int64) for n in LENS]


def build(sd, cfg, fp32_gelu):
    from transformers import GPT2Config, GPT2LMHeadModel

    hf_cfg = GPT2Config(vocab_size=cfg.vocab_size, n_positions=cfg.n_positions, n_embd=cfg.d_model,
                        n_layer=cfg.n_layer, n_head=cfg.n_head, activation_function="gelu_new",
                        layer_norm_epsilon=cfg.eps, resid_pdrop=0.0, embd_pdrop=0.0, attn_pdrop=0.0,
                        bos_token_id=1993, eos_token_id=1994, pad_token_id=1996, attn_implementation="sdpa")
    model = GPT2LMHeadModel(hf_cfg).eval()
    hf_sd = {k[len("model.model."):]: torch.from_numpy(np.asarray(v)).float()
             for k, v in sd.items() if k.startswith("model.model.")}
    missing, unexpected = model.load_state_dict(hf_sd, strict=False)
    assert not unexpected, unexpected
    if fp32_gelu:
        for blk in model.transformer.h:
            blk.mlp.act = GeluFp32()
    return model


def heads(sd, d):
    g = weights.GLOBAL_KEYS
    vh, th = torch.nn.Linear(d, 1), torch.nn.Linear(d, 1)
    vh.weight.data = torch.from_numpy(np.asarray(sd[g["w_value"]])).float().reshape(1, d)
    vh.bias.data = torch.from_numpy(np.asarray(sd[g["b_value"]])).float().reshape(1)
    th.weight.data = torch.from_numpy(np.asarray(sd[g["w_time"]])).float().reshape(1, d)
    th.bias.data = torch.from_numpy(np.asarray(sd[g["b_time"]])).float().reshape(1)
    return vh, th


def run(model, vh, th, seqs):
    block0, hL, logits, value, time = [], [], [], [], []
    with torch.no_grad(), torch.autocast("cpu", dtype=torch.bfloat16):
        for s in seqs:
            o = model(input_ids=torch.from_numpy(s)[None], output_hidden_states=True)
            block0.append(o.hidden_states[1][0, ::ROW_STRIDE].float().numpy())
            last = o.hidden_states[-1][:, -1]  # post ln_f, fp32
            hL.append(last[0].float().numpy())
            logits.append(o.logits[0, -1].float().numpy())
            value.append(float(torch.tanh(vh(last))[0, 0].float()))
            time.append(float(th(last)[0, 0].float()))
    return dict(block0=np.concatenate(block0), hL=np.stack(hL), logits=np.stack(logits),
                value=np.array(value, np.float32), time=np.array(time, np.float32))


def main() -> None:
    import transformers

    cfg = config.TINY
    sd = weights.init_weights(cfg, seed=SEED, perturb=True)
    seqs = games()
    vh, th = heads(sd, cfg.d_model)
    out = {"ids": np.concatenate(seqs), "lens": np.array(LENS), "row_stride": ROW_STRIDE, "seed": SEED,
           "transformers_version": np.array(transformers.__version__),
           "torch_version": np.array(torch.__version__)}
    for tag, fp32_gelu in (("cuda", True), ("cpu", False)):
        r = run(build(sd, cfg, fp32_gelu), vh, th, seqs)
        for k, v in r.items():
            out[f"{tag}_{k}"] = v
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
