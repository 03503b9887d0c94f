"""Reference checkpoint loader (allie_amd/checkpoint.py).

The checkpoint is made the way the reference makes it: the module nesting of
``CausalLMWithRegressionHead(CausalLMWithControlToken(GPT2LMHeadModel))``
(src/modeling/model.py:13-24, 60-80) built around the installed
``transformers`` GPT-2, and ``torch.save({"iter_num", "best_val_loss",
"model": state_dict(), "optimizer": ...})`` (trainer.py:397-408).  The key
names therefore come from the library, not from this build's key table.
"""
import os

import numpy as np
import pytest
import torch
from torch import nn

from allie_amd import config, weights
from allie_amd.checkpoint import CheckpointError, canonical_state_dict, config_from_state_dict, load_checkpoint


class _ControlToken(nn.Module):  # attribute names of model.py:13-24
    def __init__(self, lm):
        super().__init__()
        self.model = lm
        self.control_embeds = nn.Embedding(2, lm.config.n_embd)


class _RegressionHead(nn.Module):  # attribute names of model.py:60-80
    def __init__(self, m):
        super().__init__()
        self.model = m
        d = m.model.config.n_embd
        self.value_head = nn.Sequential(nn.Linear(d, 1), nn.Flatten(start_dim=1), nn.Tanh())
        self.time_head = nn.Sequential(nn.Linear(d, 1), nn.Flatten(start_dim=1))


def _reference_module(cfg, seed=0):
    from transformers import GPT2Config, GPT2LMHeadModel

    torch.manual_seed(seed)
    hf = GPT2Config(vocab_size=cfg.vocab_size, n_positions=cfg.n_positions, n_embd=cfg.d_model,
                    n_layer=cfg.n_layer, n_head=cfg.n_head, activation_function="gelu_new")
    return _RegressionHead(_ControlToken(GPT2LMHeadModel(hf))).eval()


def _save(tmp_path, module, **extra):
    path = os.path.join(tmp_path, "best.pt")
    opt = torch.optim.AdamW(module.parameters(), lr=1e-4)
    torch.save({"iter_num": 7, "best_val_loss": 1.5, "model": module.state_dict(),
                "optimizer": opt.state_dict(), **extra}, path)
    return path


def test_load_reference_layout(tmp_path):
    cfg = config.TINY
    mod = _reference_module(cfg)
    path = _save(tmp_path, mod)
    got_cfg, sd = load_checkpoint(path)
    assert (got_cfg.n_layer, got_cfg.d_model, got_cfg.n_head, got_cfg.n_positions) == \
        (cfg.n_layer, cfg.d_model, cfg.n_head, cfg.n_positions)
    ref = {k: v.float().numpy() for k, v in mod.state_dict().items()}
    # every tensor the engine reads, under the build's key table, equals the module's
    G = weights.GLOBAL_KEYS
    for k in list(G.values()) + [k for i in range(cfg.n_layer) for k in weights.layer_keys(i).values()]:
        assert k in ref, k
        np.testing.assert_array_equal(sd[k], ref[k])
    # Conv1D weights are [in, out], as the engine expects
    assert sd[weights.layer_keys(0)["w_qkv"]].shape == (cfg.d_model, 3 * cfg.d_model)
    assert sd[weights.layer_keys(0)["w_pr"]].shape == (4 * cfg.d_model, cfg.d_model)


def test_bare_state_dict_and_wrapper_prefixes(tmp_path):
    cfg = config.TINY
    mod = _reference_module(cfg, seed=1)
    path = os.path.join(tmp_path, "sd.pt")
    torch.save({"module." + k: v for k, v in mod.state_dict().items()}, path)
    got_cfg, sd = load_checkpoint(path, n_head=8)
    assert got_cfg.n_head == 8 and got_cfg.n_layer == cfg.n_layer
    np.testing.assert_array_equal(sd[weights.GLOBAL_KEYS["wte"]], mod.model.model.transformer.wte.weight.detach().numpy())


def test_rejects_untied_missing_and_unknown(tmp_path):
    cfg = config.TINY
    base = {k: torch.from_numpy(np.asarray(v)) for k, v in weights.init_weights(cfg, seed=2).items()}
    canonical_state_dict(base, cfg)  # the build's own seeded dict is complete
    untied = dict(base)
    untied[weights.GLOBAL_KEYS["lm_head"]] = base[weights.GLOBAL_KEYS["wte"]] + 1
    with pytest.raises(CheckpointError, match="tied"):
        canonical_state_dict(untied, cfg)
    missing = dict(base)
    del missing[weights.layer_keys(1)["b_fc"]]
    with pytest.raises(CheckpointError, match="no .*mlp.c_fc.bias"):
        canonical_state_dict(missing, cfg)
    unknown = dict(base, **{"model.model.transformer.h.0.mlp.extra": torch.zeros(3)})
    with pytest.raises(CheckpointError, match="unexpected"):
        canonical_state_dict(unknown, cfg)
    wrong = dict(base)
    wrong[weights.layer_keys(0)["w_o"]] = torch.zeros(cfg.d_model + 1, cfg.d_model)
    with pytest.raises(CheckpointError, match="shape"):
        canonical_state_dict(wrong, cfg)
    small_vocab = dict(base)
    small_vocab[weights.GLOBAL_KEYS["wte"]] = torch.zeros(100, cfg.d_model)
    with pytest.raises(CheckpointError, match="vocabulary"):
        config_from_state_dict(small_vocab)


def test_refuses_pickled_objects(tmp_path):
    path = os.path.join(tmp_path, "obj.pt")
    torch.save({"model": {"x": torch.zeros(1)}, "note": _ControlToken.__name__, "obj": object()}, path)
    with pytest.raises(Exception):
        load_checkpoint(path)


@pytest.mark.gpu
def test_gpu_model_from_checkpoint_matches_oracle(tmp_path, cuda):
    """A checkpoint in the reference layout through the loader and the GPU
    engine (fp32 check mode) against the oracle on the loaded weights."""
    from allie_amd.model import AllieModel
    from oracle.model_ref import RefModel

    cfg = config.TINY
    mod = _reference_module(cfg, seed=3)
    g = torch.Generator().manual_seed(3)
    with torch.no_grad():  # non-zero biases and LayerNorm parameters, so bias and LN bugs show
        for name, p in mod.named_parameters():
            if name.endswith("bias") or ".ln_" in name:
                p.add_(0.05 * torch.randn(p.shape, generator=g))
    path = _save(tmp_path, mod)
    gpu = AllieModel.from_checkpoint(path, mode="float32")
    try:
        _, sd = load_checkpoint(path)
        ref = RefModel(cfg, sd, mode="float32")
        rng = np.random.default_rng(3)
        lens = [1, 5, 40, 120]
        T = max(lens)
        ids = torch.full((len(lens), T), 1996, dtype=torch.int64)
        mask = torch.zeros(len(lens), T)
        for i, n in enumerate(lens):
            ids[i, :n] = torch.from_numpy(rng.integers(0, 1968, n))
            mask[i, :n] = 1
        ids[2, 0], ids[2, 1] = 1997 + 1800, 1997 + 2400  # Elo words
        got = gpu(input_ids=ids, attention_mask=mask)
        want = ref.forward_padded(ids, mask, last_only=True)
        np.testing.assert_allclose(got["logits"][:, -1].cpu().numpy(), want["logits"].numpy(), atol=1e-4, rtol=0)
        np.testing.assert_allclose(got["value_logits"][:, -1].cpu().numpy(), want["value_logits"].numpy(), atol=1e-4)
        np.testing.assert_allclose(got["time_logits"][:, -1].cpu().numpy(), want["time_logits"].numpy(), atol=1e-4)
    finally:
        gpu.close()
