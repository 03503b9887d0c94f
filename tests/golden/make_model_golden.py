"""Writes tests/golden/model_tiny.npz: known answers for the model forward.

The GPT-2 block arithmetic of the reference lives in the third-party
``transformers`` package (pinned ``transformers==4.39.3`` at
requirements.txt:11; built at src/modeling/model.py:165-174).  This script
runs the ``transformers`` installed in this image (``GPT2LMHeadModel`` from a
local ``GPT2Config``, eager attention, no network) as the known-answer source
for the blocks, with:

* weights from ``allie_amd.weights.init_weights(TINY, seed=7, perturb=True)``
  (seeded PCG64, regenerated identically by the tests);
* the embedding of ``CausalLMWithControlToken.forward``
  (src/modeling/model.py:35-48) and the value/time heads of
  ``CausalLMWithRegressionHead`` (model.py:72-80,105-110) written out here in
  float64 numpy, independently of the oracle's torch code;
* a right-padded batch with ``attention_mask`` and ``position_ids`` exactly
  as ``UCITokenizer.pad_and_collate`` builds them (data.py:310-327).

The fixture stores the inputs and the outputs at each game's last real token
(logits, value, time), plus value/time at every real position.

Run here (CPU):  python tests/golden/make_model_golden.py
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from allie_amd import config, weights  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "model_tiny.npz")
SEED = 7
PAD = 1996


def games(rng):
    lens = [1, 2, 9, 40, 77, 130]
    seqs = []
    for n in lens:
        s = rng.integers(0, 1968, n).astype(np.int64)
        if n >= 9:  # Elo words, time-control token and UNK as the tokenizer writes them
            s[0] = 1997 + int(rng.integers(300, 3300))
            s[1] = 1997 + int(rng.integers(300, 3300))
            s[2] = 1968 + int(rng.integers(0, 24))
            s[3] = 1995
        seqs.append(s)
    return seqs


def main() -> None:
    from transformers import GPT2Config, GPT2LMHeadModel

    cfg = config.TINY
    sd = weights.init_weights(cfg, seed=SEED, perturb=True)
    V, d = cfg.vocab_size, cfg.d_model
    hf_cfg = GPT2Config(vocab_size=V, n_positions=cfg.n_positions, n_embd=d, n_layer=cfg.n_layer,
                        n_head=cfg.n_head, activation_function="gelu_new", layer_norm_epsilon=cfg.eps,
                        resid_pdrop=0.0, embd_pdrop=0.0, attn_pdrop=0.0, bos_token_id=1993,
                        eos_token_id=1994, pad_token_id=PAD, attn_implementation="eager")
    model = GPT2LMHeadModel(hf_cfg).eval().double()
    hf_sd = {k[len("model.model."):]: torch.from_numpy(np.asarray(v)).double()
             for k, v in sd.items() if k.startswith("model.model.")}
    missing, unexpected = model.load_state_dict(hf_sd, strict=False)
    assert not unexpected, unexpected
    assert all(m.endswith("attn.bias") or m.endswith("masked_bias") for m in missing), missing

    rng = np.random.default_rng(SEED)
    seqs = games(rng)
    B, T = len(seqs), max(len(s) for s in seqs)
    ids = np.full((B, T), PAD, np.int64)
    for i, s in enumerate(seqs):
        ids[i, : len(s)] = s
    mask = ids != PAD
    pos = np.maximum(np.cumsum(mask, axis=1) - 1, 0)

    # model.py:35-48 in float64
    ctrl = np.asarray(sd[weights.GLOBAL_KEYS["ctrl"]], np.float64)
    wte = np.asarray(sd[weights.GLOBAL_KEYS["wte"]], np.float64)
    e = (np.clip(ids - V, 500, 3000) - 500) / 2500.0
    ce = e[..., None] * ctrl[0] + (1.0 - e)[..., None] * ctrl[1]
    te = wte[np.clip(ids, 0, V - 1)]
    emb = np.where((ids >= V)[..., None], ce, te)

    with torch.no_grad():
        out = model(inputs_embeds=torch.from_numpy(emb), attention_mask=torch.from_numpy(mask.astype(np.float64)),
                    position_ids=torch.from_numpy(pos), output_hidden_states=True)
    hL = out.hidden_states[-1].numpy()  # post ln_f
    logits = out.logits.numpy()
    wv = np.asarray(sd[weights.GLOBAL_KEYS["w_value"]], np.float64)[0]
    bv = float(sd[weights.GLOBAL_KEYS["b_value"]][0])
    wt = np.asarray(sd[weights.GLOBAL_KEYS["w_time"]], np.float64)[0]
    bt = float(sd[weights.GLOBAL_KEYS["b_time"]][0])
    value = np.tanh(hL @ wv + bv)
    time = hL @ wt + bt
    last = mask.sum(1) - 1
    ar = np.arange(B)
    np.savez_compressed(
        OUT,
        ids=ids, attention_mask=mask, position_ids=pos, lens=mask.sum(1),
        last_logits=logits[ar, last].astype(np.float32),
        last_value=value[ar, last], last_time=time[ar, last],
        value_all=np.where(mask, value, 0.0), time_all=np.where(mask, time, 0.0),
        seed=SEED, transformers_version=np.array(__import__("transformers").__version__),
    )
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
