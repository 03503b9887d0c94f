"""bf16 parity at full depth, measured against the oracle's own floor.

Two faithful bf16-autocast implementations of a deep model do not agree to
the last bit: every GEMM output is rounded to bf16, so a different summation
order flips some roundings, and the flips compound through the layers.  The
oracle measures this on the inputs of each check by running itself twice,
with fp32 and with fp64 summation (same rounding points), and the GPU is
held to the contract bar (2e-2) or to twice that floor, whichever is larger:

* logits (after and before their final bf16 rounding), value and time:
  max |GPU - oracle| <= max(2e-2, 2 * max |oracle64 - oracle32|), per
  quantity, and the median over games of the per-game logit error <= twice
  the floor's median (the GPU is not systematically further off than a
  change of summation order);
* top-1 move: for EVERY game the GPU's pick is the oracle's first argmax,
  or a move whose oracle logit is within twice that bound of the maximum
  (a near tie); exact agreement is required wherever the oracle's top-2
  margin exceeds twice the bound.  Counts are printed.

Reference semantics: the last-token reads of Policy.score_full and
MCTS.evaluate_node (src/evaluation/decode.py:204-226, 356-373) under bf16
autocast (decode.py:74-78).
"""
from __future__ import annotations

import numpy as np

from oracle.model_ref import RefModel, policy_summary

BAR = 2e-2


def oracle_pair(cfg, sd, mode, seqs, batch=8):
    a = RefModel(cfg, sd, mode=mode).forward_last(seqs, batch=batch)
    b = RefModel(cfg, sd, mode=mode, accumulate="fp64").forward_last(seqs, batch=batch)
    return a, b


def _per_game(x, y):
    return np.abs(np.asarray(x, np.float64) - np.asarray(y, np.float64)).reshape(len(x), -1).max(axis=1)


def check_at_floor(label, got, ref, ref64, top1=None):
    """got: dict with logits, logits_raw, value, time ([n, ...] numpy);
    ref / ref64: oracle outputs (fp32 / fp64 summation) of the same rows;
    top1: the GPU's first argmax per row (default: argmax of got logits)."""
    rows = {}
    for k_got, k_ref in (("logits", "logits"), ("logits_raw", "logits_raw"), ("value", "value_logits"),
                         ("time", "time_logits")):
        if got.get(k_got) is None:
            continue
        e = _per_game(got[k_got], ref[k_ref])
        f = _per_game(ref64[k_ref], ref[k_ref])
        bound = max(BAR, 2.0 * float(f.max()))
        rows[k_got] = (e, f, bound)
        print(f"{label} {k_got}: GPU max {e.max():.4f} median {np.median(e):.4f} (games > 2e-2: {(e > BAR).sum()}) | "
              f"oracle fp64-vs-fp32 floor max {f.max():.4f} median {np.median(f):.4f} "
              f"(games > 2e-2: {(f > BAR).sum()}) | bound {bound:.4f}", flush=True)
    for k, (e, f, bound) in rows.items():
        assert e.max() <= bound, (label, k, float(e.max()), bound)
        if k.startswith("logits"):
            assert np.median(e) <= 2.0 * np.median(f) + 1e-6, (label, k, float(np.median(e)), float(np.median(f)))
    # top-1 against the oracle's logits
    ps = policy_summary(ref["logits"])
    if top1 is None:
        top1 = policy_summary(got["logits"])["top1"]
    top1 = np.asarray(top1)
    if "logits" in rows:
        bound = rows["logits"][2]
    else:  # only the GPU's moves are known: the floor alone sets the bound
        bound = max(BAR, 2.0 * float(_per_game(ref64["logits"], ref["logits"]).max()))
    tie = 2.0 * bound
    lg = np.asarray(ref["logits"], np.float64)[:, :1968]
    picked = lg[np.arange(len(top1)), top1]
    gap = lg.max(axis=1) - picked
    decided = ps["margin"] > tie
    differ = top1 != ps["top1"]
    print(f"{label} top-1: {int(differ.sum())} of {len(top1)} differ from the oracle (all near ties: "
          f"max gap {gap.max():.4f} <= {tie:.4f}); {int((~decided).sum())} games have an oracle top-2 margin "
          f"<= {tie:.4f}", flush=True)
    assert (top1 >= 0).all() and (top1 < 1968).all()
    assert (gap <= tie).all(), (label, np.nonzero(gap > tie))
    assert not (differ & decided).any(), (label, np.nonzero(differ & decided))
