"""Pins the CPU oracle of the model forward (oracle/model_ref.py).

* against ``transformers``' own GPT2LMHeadModel (the library the reference
  runs its blocks in, src/modeling/model.py:165-190), through the committed
  known answers of tests/golden/model_tiny.npz;
* against a float64 brute force written with explicit per-token loops at a
  tiny shape (no padding, no batching, no matrix reshapes), which catches a
  wrong causal mask, a wrong head split or a dropped bias;
* the Elo control embedding against its closed form at the clamp edges
  (model.py:35-48);
* the bf16 emulation and fp8 quantisation against their definitions.
"""
import math
import os

import numpy as np
import pytest
import torch

from allie_amd import config, weights
from oracle.model_ref import RefModel, gelu_new, policy_summary

GOLD = os.path.join(os.path.dirname(__file__), "golden", "model_tiny.npz")


def test_oracle_matches_transformers_fixture():
    g = np.load(GOLD)
    cfg = config.TINY
    sd = weights.init_weights(cfg, seed=int(g["seed"]), perturb=True)
    ref = RefModel(cfg, sd, mode="float32")
    out = ref.forward_padded(torch.from_numpy(g["ids"]), torch.from_numpy(g["attention_mask"]).float(),
                             torch.from_numpy(g["position_ids"]))
    B = g["ids"].shape[0]
    last = g["lens"] - 1
    ar = np.arange(B)
    np.testing.assert_allclose(out["logits"].numpy()[ar, last], g["last_logits"], atol=2e-5, rtol=0)
    np.testing.assert_allclose(out["value_logits"].numpy()[ar, last], g["last_value"], atol=2e-6)
    np.testing.assert_allclose(out["time_logits"].numpy()[ar, last], g["last_time"], atol=2e-5)
    m = g["attention_mask"]
    np.testing.assert_allclose(np.where(m, out["value_logits"].numpy(), 0), g["value_all"], atol=2e-6)
    # forward_last (the sub-batched path the GPU tests use) agrees too
    seqs = [g["ids"][i, : g["lens"][i]] for i in range(B)]
    fl = ref.forward_last(seqs, batch=4)
    np.testing.assert_allclose(fl["logits"], g["last_logits"], atol=2e-5, rtol=0)


def _brute(cfg, sd, ids):
    """float64, one game, explicit loops over tokens/heads/keys."""
    d, H = cfg.d_model, cfg.n_head
    hd = d // H
    V = cfg.vocab_size
    f = lambda k: np.asarray(sd[k], np.float64)
    G = weights.GLOBAL_KEYS
    n = len(ids)

    def ln(x, g_, b_):
        mu = sum(x) / d
        var = sum((xi - mu) ** 2 for xi in x) / d
        return np.array([(x[i] - mu) / math.sqrt(var + cfg.eps) * g_[i] + b_[i] for i in range(d)])

    h = []
    for t, i in enumerate(ids):
        if i >= V:
            e = (min(max(i - V, 500), 3000) - 500) / 2500.0
            x = e * f(G["ctrl"])[0] + (1 - e) * f(G["ctrl"])[1]
        else:
            x = f(G["wte"])[i].copy()
        h.append(x + f(G["wpe"])[t])
    for l in range(cfg.n_layer):
        k = weights.layer_keys(l)
        a = [ln(x, f(k["ln1_g"]), f(k["ln1_b"])) for x in h]
        qkv = [x @ f(k["w_qkv"]) + f(k["b_qkv"]) for x in a]
        o = []
        for t in range(n):
            row = np.zeros(d)
            for hh in range(H):
                q = qkv[t][hh * hd:(hh + 1) * hd]
                sc = []
                for j in range(t + 1):  # causal: keys 0..t
                    kk = qkv[j][d + hh * hd: d + (hh + 1) * hd]
                    sc.append(float(q @ kk) / math.sqrt(hd))
                mx = max(sc)
                p = [math.exp(s - mx) for s in sc]
                z = sum(p)
                for j in range(t + 1):
                    row[hh * hd:(hh + 1) * hd] += p[j] / z * qkv[j][2 * d + hh * hd: 2 * d + (hh + 1) * hd]
            o.append(row)
        h = [h[t] + o[t] @ f(k["w_o"]) + f(k["b_o"]) for t in range(n)]
        a = [ln(x, f(k["ln2_g"]), f(k["ln2_b"])) for x in h]
        ff = []
        for x in a:
            u = x @ f(k["w_fc"]) + f(k["b_fc"])
            gl = np.array([0.5 * v * (1 + math.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3))) for v in u])
            ff.append(gl @ f(k["w_pr"]) + f(k["b_pr"]))
        h = [h[t] + ff[t] for t in range(n)]
    hl = ln(h[-1], f(G["lnf_g"]), f(G["lnf_b"]))
    logits = f(G["wte"]) @ hl
    value = math.tanh(float(hl @ f(G["w_value"])[0]) + float(f(G["b_value"])[0]))
    time = float(hl @ f(G["w_time"])[0]) + float(f(G["b_time"])[0])
    return logits, value, time


def test_oracle_matches_float64_brute_force():
    cfg = config.ModelConfig(n_layer=2, d_model=32, n_head=2)
    sd = weights.init_weights(cfg, seed=3, perturb=True)
    rng = np.random.default_rng(4)
    games = [rng.integers(0, 1968, n).astype(np.int64) for n in (1, 5, 12)]
    games[2][0] = 1997 + 2600  # an Elo word inside the clamp range
    games[2][1] = 1997 + 100   # below the clamp
    ref = RefModel(cfg, sd, mode="float32").forward_last(games, batch=3)  # padded together
    for b, s in enumerate(games):
        lg, v, t = _brute(cfg, sd, list(s))
        np.testing.assert_allclose(ref["logits"][b], lg, atol=1e-5, rtol=0)
        assert abs(ref["value_logits"][b] - v) < 1e-6
        assert abs(ref["time_logits"][b] - t) < 1e-5


def test_elo_embedding_closed_form():
    cfg = config.ModelConfig(n_layer=1, d_model=8, n_head=1)
    sd = weights.init_weights(cfg, seed=1)
    r = RefModel(cfg, sd)
    V = cfg.vocab_size
    ids = torch.tensor([[V + 0, V + 500, V + 1750, V + 3000, V + 9000, 5]])
    pos = torch.zeros_like(ids)
    x = r.embed(ids, pos) - r.wpe[0]
    c = r.ctrl
    for j, e in enumerate([0.0, 0.0, 0.5, 1.0, 1.0]):
        torch.testing.assert_close(x[0, j], e * c[0] + (1 - e) * c[1])
    torch.testing.assert_close(x[0, 5], r.wte[5])


def test_gelu_new_is_tanh_gelu():
    x = torch.linspace(-8, 8, 1001, dtype=torch.float64)
    torch.testing.assert_close(gelu_new(x), torch.nn.functional.gelu(x, approximate="tanh"))


def test_bf16_emulation_close_to_fp32():
    cfg = config.TINY
    sd = weights.init_weights(cfg, seed=2)
    rng = np.random.default_rng(0)
    games = [rng.integers(0, 1968, n).astype(np.int64) for n in (3, 50)]
    a = RefModel(cfg, sd, "float32").forward_last(games)
    b = RefModel(cfg, sd, "bfloat16").forward_last(games)
    d = np.abs(a["logits"] - b["logits"]).max()
    assert 0 < d < 5e-2
    # every bf16-mode output is a bf16 value
    for k in ("logits", "value_logits", "time_logits"):
        v = torch.from_numpy(b[k])
        assert torch.equal(v, v.to(torch.bfloat16).float())


def test_fp8_quantisation():
    rng = np.random.default_rng(0)
    w = rng.standard_normal((64, 48)).astype(np.float32) * 0.05
    w[3, 7] = 0.0
    q, s = weights.quantize_fp8_per_channel(w)
    assert q.shape == (48, 64) and s.shape == (48,)
    np.testing.assert_allclose(s, np.abs(w).max(0) / 448.0, rtol=1e-7)
    deq = weights.dequantize_fp8(q, s)
    # e4m3 keeps 3 mantissa bits: relative error <= 2^-4 for normal values
    big = np.abs(w) > s[None, :] * 2 ** -6 * 8
    assert (np.abs(deq - w)[big] <= np.abs(w)[big] * 2 ** -4 + 1e-12).all()
    # the channel maximum maps to exactly +-448
    qf = torch.from_numpy(q).view(torch.float8_e4m3fn).float().numpy()
    assert np.allclose(np.abs(qf).max(1), 448.0)


def test_policy_summary_first_argmax():
    l = np.zeros((2, 1997), np.float32)
    l[0, [5, 9]] = 3.0  # tie: the first index wins (torch.argmax)
    l[1, 1990] = 50.0   # outside the move range: ignored
    l[1, 7] = 1.0
    ps = policy_summary(l)
    assert list(ps["top1"]) == [5, 7]
    m = np.float64(3.0)
    want = m + np.log(np.exp(l[0, :1968].astype(np.float64) - m).sum())
    assert abs(ps["lse"][0] - want) < 1e-12
    assert ps["margin"][0] == 0.0
