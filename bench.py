"""Benchmark of the batched policy/value inference path on one MI355X.

``python bench.py`` (the driver's line) measures the headline configuration:
medium shape (24 layers, d_model 1024, 16 heads), bf16, one ragged packed
batch of 256 game prefixes with lengths ``default_rng(2).integers(8, 401,
256)`` and uniform move-token ids; one step = one prefill forward emitting
policy logits, value and time at every game's last token.  ``value`` is leaf
(prefix) evaluations per second with the inputs already resident in HBM.

On the same JSON line:
* ``roofline`` for the dominant kernel (the MLP c_fc GEMM + gelu): its
  algorithmic FLOPs per launch (2 * T * 4096 * 1024) over its average launch
  duration, measured with HIP events around each of its launches inside the
  timed forwards (on the stream they run on), against the dense bf16 MFMA
  peak; ``traffic`` is the copy-calibrated HBM bytes per launch from the
  committed rocprofv3 counter summary;
* ``cpu_baseline``: the CPU oracle (fp32, the reference's execution shape:
  one B=1 forward per game as Policy.score_full / MCTS.evaluate_node do,
  src/evaluation/decode.py:199-203,356-360) timed on a bounded sample of the
  same games on the host cores.

``--config c3|c4|c5`` measures the other synthetic workloads, one JSON line
each: MCTS tree expansion (leaf evals/s), continuous-batching self-play
decode (tokens/s and step latency), and the fp8-weight 2x model (leaf
evals/s, top-1 agreement with bf16).  ``--config search`` times one MCTS
decision (50 simulations) with the reference's per-leaf recompute, with the
KV-cached search, and with KV plus leaf batching; ``--config serve``
times 256 concurrent policy requests through the batching front end.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MFMA_BF16_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBS = 8000.0
METRIC = "leaf evals/sec @ medium, ragged batch 256; % of MFMA / HBM roofline"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_gemm_fc_c2.txt")
ATTN_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_attn_c3_c4.txt")


def c2_batch():
    rng = np.random.default_rng(2)
    lens = rng.integers(8, 401, 256).astype(np.int32)
    seqs = [rng.integers(0, 1968, n).astype(np.uint32) for n in lens]
    return seqs, lens


def alg_flops(cfg, lens):
    """Algorithmic FLOPs of one forward over ragged games: linear layers,
    causal attention (QK^T and PV over n(n+1)/2 pairs per head), heads."""
    T = int(np.sum(lens))
    P = cfg.linear_params
    attn = 2 * cfg.n_layer * cfg.d_model * int(np.sum(lens.astype(np.int64) * (lens + 1)))
    heads = 2 * len(lens) * cfg.d_model * (cfg.vocab_size + 2)
    return 2 * P * T + attn + heads


def executed_flops(cfg, lens):
    """FLOPs the prefill executes: the algorithmic count less what the last
    block skips -- its attention c_proj and MLP run on each game's last row
    only, and its attention on the 32-query tile holding that row (when
    2 B <= T, as in C2)."""
    lens = np.minimum(np.asarray(lens, np.int64), cfg.max_length)
    T, B, d = int(lens.sum()), len(lens), cfg.d_model
    full = alg_flops(cfg, lens)
    if 2 * B > T:
        return full
    gemm_skip = 2 * (T - B) * (d * d + 2 * d * cfg.d_ff)
    last_tile = lambda n: sum(range(32 * ((n - 1) // 32) + 1, n + 1))  # key counts of the tile's queries
    attn_skip = 4 * d * int(sum(n * (n + 1) // 2 - last_tile(int(n)) for n in lens))
    return full - gemm_skip - attn_skip


def read_traffic(key: str = "", one_piece: bool = False):
    """HBM bytes per launch of a dominant kernel, measured with rocprofv3
    --pmc FETCH_SIZE / WRITE_SIZE and scaled by the copy calibration: the
    line ``hbm_bytes_per_launch: N`` of the fc GEMM's committed summary, or
    ``hbm_bytes_per_launch[key]: N`` of the attention kernels' one, or (with
    one_piece) the fc GEMM's launch over the whole batch in one piece; None
    when the summary is absent."""
    path = TRAFFIC_FILE if not key else ATTN_TRAFFIC_FILE
    tag = "hbm_bytes_per_launch:" if not key else f"hbm_bytes_per_launch[{key}]:"
    if one_piece:
        tag = "hbm_bytes_per_launch_one_piece:"
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith(tag):
                return float(line.split(":", 1)[1])
    return None


def traffic_commit(key: str = "") -> str | None:
    """The kernel source and commit the traffic summary was measured on (its
    ``kernel_commit:`` line), printed next to ``traffic``."""
    path = TRAFFIC_FILE if not key else ATTN_TRAFFIC_FILE
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("kernel_commit:"):
                return line.split(":", 1)[1].strip()
    return None


def calibrate_copy(mib: int = 512, reps: int = 3):
    """A plain device-to-device copy of known size, for scaling the HBM byte
    counters (FETCH_SIZE / WRITE_SIZE) of the profiled kernels."""
    import torch

    x = torch.empty(mib * 1024 * 1024, dtype=torch.uint8, device="cuda:0").fill_(1)
    y = torch.empty_like(x)
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"calibration_copy_bytes": x.numel(), "reps": reps}), flush=True)


def _cpu_info():
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model


def cpu_baseline(cfg, sd, leaves, unit, budget_s: float = 20.0, per_leaf: float = 1.0, extrapolate=None):
    """The reference's CPU execution shape, timed on this host's cores: the
    oracle in fp32 with all-position logits and no KV cache (the reference
    model, src/modeling/model.py:85-147), over a fixed sample of ``leaves``
    (token id sequences, each one evaluation the reference makes) in two
    modes, each the median of 3 timed runs after one warm-up:

    (i)  ``b1``: one B=1 forward per leaf, as Policy.score_full and
         MCTS.evaluate_node call the model (src/evaluation/decode.py:199-203,
         356-360) -- the reported ``value``;
    (ii) ``padded``: the same leaves as ONE right-padded batch with an
         attention mask, as pad_and_collate builds it (data.py:281-337).

    The sample is the first leaves that fit the budget (about budget_s / 10
    seconds per B=1 run; a padded run takes longer).  ``per_leaf`` converts leaves to the metric's unit
    (e.g. tokens appended per leaf); ``extrapolate`` = (units, label) adds the
    linear extrapolation of the B=1 rate to a whole workload.  Threads: the
    cores this process may run on (its CPU affinity), which on a shared host
    is the process's share rather than every core of the machine."""
    import statistics

    import torch

    from oracle.model_ref import RefModel

    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(avail)
    ref = RefModel(cfg, sd, mode="float32")
    fwd = lambda s: ref.forward_padded(torch.as_tensor(np.asarray(s, np.int64))[None])
    fwd(leaves[0])  # warm-up
    t0 = time.perf_counter()
    fwd(leaves[0])
    one = time.perf_counter() - t0
    run_s = budget_s / 10.0
    n = 1
    est = one
    while n < len(leaves) and est + one * len(leaves[n]) / max(len(leaves[0]), 1) < run_s:
        est += one * len(leaves[n]) / max(len(leaves[0]), 1)
        n += 1
    sample = leaves[:n]

    def b1():
        t = time.perf_counter()
        for s in sample:
            fwd(s)
        return time.perf_counter() - t

    T = max(len(s) for s in sample)
    ids = torch.full((n, T), 1996, dtype=torch.int64)
    mask = torch.zeros(n, T)
    for i, s in enumerate(sample):
        ids[i, : len(s)] = torch.as_tensor(np.asarray(s, np.int64))
        mask[i, : len(s)] = 1

    def padded():
        t = time.perf_counter()
        ref.forward_padded(ids, mask)
        return time.perf_counter() - t

    modes = {}
    b1()  # warm-up (the padded batch runs the same kernels)
    for name, fn in (("b1", b1), ("padded", padded)):
        runs = [fn() for _ in range(3)]
        med = statistics.median(runs)
        modes[name] = {"value": n * per_leaf / med, "runs_s": [round(r, 3) for r in runs]}
    res = {
        "value": modes["b1"]["value"],
        "unit": unit,
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{n} leaves of {min(len(s) for s in sample)}-{T} tokens; mode b1 (one fp32 B=1 forward "
                   f"per leaf, all-position logits, no KV cache; the value) and mode padded (one right-padded "
                   f"batch of them), each the median of 3 runs; os.cpu_count()={os.cpu_count()}, "
                   f"affinity={avail}, torch threads={torch.get_num_threads()}; cpu {_cpu_info()!r}; "
                   f"torch {torch.__version__}"),
        "modes": modes,
    }
    if extrapolate is not None:
        units, label = extrapolate
        res["extrapolated"] = {"workload": label, "seconds_at_b1_rate": units / modes["b1"]["value"],
                               "note": "linear extrapolation of the timed sample"}
    return res


class Probe:
    """HIP events around every launch of one kernel kind inside the engine's
    calls (recorded on the stream the kernels run on)."""

    def __init__(self, kind, max_launches):
        from allie_amd import capi

        self.capi = capi
        capi.check(capi.lib().allie_probe_begin(kind, max_launches), "probe")

    def span(self):
        """Time during which at least one probed launch ran (ms)."""
        sp = C.c_float()
        self.capi.check(self.capi.lib().allie_probe_span(C.byref(sp)), "probe span")
        return sp.value

    def end(self):
        tot, n = C.c_float(), C.c_int()
        self.capi.check(self.capi.lib().allie_probe_end(C.byref(tot), C.byref(n)), "probe end")
        return tot.value, n.value


def base_result(args, value, unit, ms, dtype, workload, **config):
    return {
        "metric": METRIC, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dtype,
        "data": "synthetic (seeded inputs, random-init GPT-2 weights)",
        "config": {"workload": workload, **config, "parallelism": "single GPU"},
    }


# ------------------------------------------------------------------- C2 / C5
def run_prefill(args, cfg, mode, workload):
    import torch

    from allie_amd import capi, weights
    from allie_amd.engine import Engine

    sd = weights.init_weights(cfg, seed=0)
    seqs, lens = c2_batch()
    T = int(lens.sum())
    eng = Engine(cfg, sd, mode=mode, device="cuda:0")
    words = torch.from_numpy(np.concatenate(seqs).view(np.int32)).cuda()
    out = eng.prefill(words, lens)
    for _ in range(args.warmup):
        eng.prefill(words, lens, out=out)
    torch.cuda.synchronize()
    # a large batch runs as two halves (two launches per layer); room for up to four
    probe = Probe(capi.PROBE_FC, 4 * args.steps * cfg.n_layer)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        eng.prefill(words, lens, out=out)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    fc_span = probe.span()
    fc_tot, fc_n = probe.end()
    ms = el * 1000.0 / args.steps
    flops = alg_flops(cfg, lens)
    # the c_fc FLOPs of one forward: every row in the first L - 1 blocks, the
    # games' last rows in the last block when it runs on those only (2 B <= T)
    B = len(lens)
    fc_rows = (cfg.n_layer - 1) * T + (B if 2 * B <= T else T)
    fc_flops = 2.0 * fc_rows * cfg.d_ff * cfg.d_model
    fc_ms = fc_tot / max(fc_n, 1)
    # a split batch's two halves run their c_fc launches on two streams, and
    # those may overlap in time: the rate is the FLOPs over the time during
    # which a c_fc launch was running (equal to the summed durations when no
    # two overlap)
    fc_tflops = args.steps * fc_flops / (fc_span * 1e-3) / 1e12
    res = base_result(args, len(lens) / (ms / 1000.0), "leaf evals/s", ms,
                      "bf16" if mode == "bfloat16" else "fp8 e4m3 weights, bf16 activations", workload,
                      n_seq=len(lens), n_tokens=T, tokens_per_s=T / (ms / 1000.0),
                      alg_tflop_per_step=flops / 1e12,
                      whole_forward_mfma_frac=flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                      executed_tflop_per_step=executed_flops(cfg, lens) / 1e12,
                      whole_forward_mfma_frac_executed=executed_flops(cfg, lens) / (ms * 1e-3) / 1e12
                      / MFMA_BF16_PEAK_TFLOPS)
    # the same kernel with the batch in one piece (no second stream beside it)
    one_status = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    eng.prefill(words, lens, out=out, status=one_status)
    torch.cuda.synchronize()
    iso_steps = 3
    probe = Probe(capi.PROBE_FC, iso_steps * cfg.n_layer)
    for _ in range(iso_steps):
        eng.prefill(words, lens, out=out, status=one_status)
    torch.cuda.synchronize()
    iso_span = probe.span()
    iso_tot, iso_n = probe.end()
    iso_tflops = iso_steps * fc_flops / (iso_span * 1e-3) / 1e12
    res["roofline"] = {
        "kernel": ("gemm_big_kernel<EPI_GELU> (MLP c_fc, persistent 256x256 tiles)" if mode == "bfloat16"
                   else "widen_fp8_kernel + gemm_big_kernel<EPI_GELU,SCALED> (MLP c_fc, fp8 weights "
                        "widened to bf16 per call, per-channel scale in the epilogue)"),
        "bound": "mfma", "achieved": fc_tflops, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
        "frac": fc_tflops / MFMA_BF16_PEAK_TFLOPS,
        "traffic": read_traffic() if (mode == "bfloat16" and cfg.d_model == 1024) else None,
        "traffic_measured_on": traffic_commit() if (mode == "bfloat16" and cfg.d_model == 1024) else None,
        "avg_launch_ms": fc_ms, "launches": fc_n,
        "alg_flop_per_launch": args.steps * fc_flops / max(fc_n, 1),
        "achieved_is": "c_fc FLOPs of the timed forwards / the time during which one of their c_fc launches ran",
        "launch_span_ms": fc_span / args.steps, "launch_sum_ms": fc_tot / args.steps,
        "one_piece": {"note": "the same forward with the batch in one piece on one stream",
                      "avg_launch_ms": iso_tot / max(iso_n, 1), "launches": iso_n, "achieved": iso_tflops,
                      "frac": iso_tflops / MFMA_BF16_PEAK_TFLOPS,
                      "traffic": read_traffic(one_piece=True) if (mode == "bfloat16" and cfg.d_model == 1024) else None},
    }
    return res, eng, sd, seqs, lens, words, out


def bench_c2(args):
    from allie_amd import config

    res, eng, sd, seqs, lens, _, _ = run_prefill(
        args, config.MEDIUM, "bfloat16",
        "C2 ragged prefill: medium shape 24x1024x16, 256 prefixes, lens U[8,400] seed 2")
    eng.close()
    res["cpu_baseline"] = None if args.no_cpu_baseline else cpu_baseline(
        config.MEDIUM, sd, seqs, "leaf evals/s", args.cpu_budget, extrapolate=(len(seqs), "the 256-game C2 batch"))
    return res


def fp8_quality(fp8_logits, fp8_top1, bf_logits, bf_top1) -> dict:
    """The ablation's quality bar (pretrain_config/ablations/large.yaml:20):
    raw top-1 agreement of the fp8-weight model with the same weights in
    bf16, required >= 0.99; beside it the agreement over the games whose bf16
    top-2 margin exceeds twice their own fp8 logit error, and the margin and
    error distributions that explain the difference."""
    lf = fp8_logits.float().cpu().numpy()
    lb = bf_logits.float().cpu().numpy()
    agree = fp8_top1.cpu().numpy() == bf_top1.cpu().numpy()
    err = np.abs(lf - lb).max(axis=1)
    srt = np.sort(lb[:, :1968], axis=1)
    margin = srt[:, -1] - srt[:, -2]
    clear = margin > 2 * err
    return {"top1_agreement": float(agree.mean()), "bar": 0.99, "meets_bar": bool(agree.mean() >= 0.99),
            "top1_agreement_where_margin_exceeds_2x_err": float(agree[clear].mean()) if clear.any() else None,
            "games_with_clear_margin": int(clear.sum()), "games": int(len(agree)),
            "bf16_top2_margin_median": float(np.median(margin)), "fp8_logit_err_median": float(np.median(err)),
            "fp8_logit_err_max": float(err.max()), "bf16_logit_rms": float(np.sqrt((lb[:, :1968] ** 2).mean()))}


def c5_quality_sweep(cfg, words, lens, scales=(1.0, 2.0, 4.0, 8.0)) -> list:
    """fp8 quality on weights whose logit margins come closer to a trained
    policy's: the perturbed variant (non-zero biases, LN gains 1 + N(0, 0.1),
    Wq/Wk x 8) with wte -- the input embedding and the tied lm_head -- scaled
    by s, which widens the top-2 margins relative to the fp8 error."""
    import torch

    from allie_amd import weights
    from allie_amd.engine import Engine

    out = []
    for sc in scales:
        sd = weights.init_weights(cfg, seed=0, perturb=True)
        w = sd[weights.GLOBAL_KEYS["wte"]] * np.float32(sc)
        sd[weights.GLOBAL_KEYS["wte"]] = w
        sd[weights.GLOBAL_KEYS["lm_head"]] = w
        r = {}
        for mode in ("fp8w", "bfloat16"):
            e = Engine(cfg, sd, mode=mode, device="cuda:0")
            o = e.prefill(words, lens)
            torch.cuda.synchronize()
            r[mode] = (o.logits.clone(), o.top1.clone())
            e.close()
            del e, o
            torch.cuda.empty_cache()
        q = fp8_quality(r["fp8w"][0], r["fp8w"][1], r["bfloat16"][0], r["bfloat16"][1])
        out.append({"wte_scale": sc, **q})
        print(json.dumps({"c5_quality_sweep": out[-1]}), file=sys.stderr, flush=True)
    return out


def bench_c5(args):
    """2x shape with fp8 e4m3 per-output-channel weights on the C2 batch;
    quality against the bf16 engine on the same weights."""
    import torch

    from allie_amd import config
    from allie_amd.engine import Engine

    cfg = config.LARGE2X
    res, eng, sd, seqs, lens, words, out = run_prefill(
        args, cfg, "fp8w", "C5 fp8-weight ablation: 32x1280x20, C2 batch (256 prefixes, lens U[8,400] seed 2)")
    ref_logits = out.logits.clone()
    ref_top1 = out.top1.clone()
    eng.close()
    del eng
    torch.cuda.empty_cache()
    bf = Engine(cfg, sd, mode="bfloat16", device="cuda:0")
    ob = bf.prefill(words, lens)
    torch.cuda.synchronize()
    q = fp8_quality(ref_logits, ref_top1, ob.logits, ob.top1)
    bf.close()
    del bf, ob
    torch.cuda.empty_cache()
    res["config"].update(top1_agreement_vs_bf16=q["top1_agreement"], max_abs_logit_err_vs_bf16=q["fp8_logit_err_max"],
                         quality=q)
    if args.quality_sweep:
        res["config"]["quality_sweep_perturbed_scaled_wte"] = c5_quality_sweep(cfg, words, lens)
    res["cpu_baseline"] = None if args.no_cpu_baseline else cpu_baseline(
        cfg, sd, seqs, "leaf evals/s", args.cpu_budget, extrapolate=(len(seqs), "the 256-game C2 batch, 2x shape"))
    return res


# ------------------------------------------------------------------------ C3
def bench_c3(args):
    import torch

    from allie_amd import capi, config, weights
    from allie_amd.engine import Engine
    from allie_amd.tree import TreeExpansion, TreeLayout

    cfg = config.MEDIUM
    lay = TreeLayout(n_roots=64, prefix_len=200, branching=8, depth=4)
    tx_sd = weights.init_weights(cfg, seed=0)
    eng = Engine(cfg, tx_sd, mode="bfloat16", device="cuda:0")
    tx = TreeExpansion(eng, lay, seed=3)
    outs = [None] * lay.depth

    def run_tree(probe_levels=()):
        tx.prefill_roots()
        times, attn = [], {}
        for k in range(1, lay.depth + 1):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            # a large level runs as two halves: two launches per layer
            p = Probe(capi.PROBE_ATTN, 2 * cfg.n_layer) if k in probe_levels else None
            e0.record()
            outs[k - 1] = tx.expand_level(k, out=outs[k - 1])
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1))
            if p:
                span = p.span()
                attn[k] = p.end() + (span,)
        return times, attn

    for _ in range(max(args.warmup, 1)):
        run_tree()
    assert int(tx.status.item()) == 0, "extend status"
    level_ms = np.zeros(lay.depth)
    attn = {}
    for _ in range(args.steps):
        t, attn = run_tree(probe_levels=(1, 2, 4))
        level_ms += np.array(t)
    level_ms /= args.steps
    # the same tree with every level in one piece (no two-stream split), for
    # level 4's attention on its own: in two halves its launches share the
    # GPU with the other half's GEMMs
    eng.set_split_tokens(0, 0)
    t1, attn1 = run_tree(probe_levels=(4,))
    eng.set_split_tokens(24576, 512)
    d, L, P = cfg.d_model, cfg.n_layer, lay.prefix_len
    kv_tok = 2 * d * 2  # bytes of one token's keys + values, one layer
    roof = {}
    for k in (1, 2, 4):
        n = lay.level_size(k)
        bytes_ = lay.n_roots * P * kv_tok + n * k * kv_tok + n * 2 * d * 2
        tot, cnt, span = attn[k]
        # per layer: the time during which the layer's attention launches ran (the
        # union of their intervals; two overlapping launches when the level runs as
        # two halves on two streams, one otherwise)
        ms = span / L
        roof[k] = {"ms_per_layer": ms, "avg_launch_ms": tot / max(cnt, 1), "launches_per_layer": cnt / L,
                   "alg_bytes_per_layer": bytes_, "achieved_GBs": bytes_ / (ms * 1e-3) / 1e9}
    # level 4: every pool row once (ancestors shared by siblings), and its MFMA work
    n4 = lay.level_size(4)
    uniq = lay.n_roots * P * kv_tok + sum(lay.level_size(j) for j in range(1, 5)) * kv_tok + n4 * 2 * d * 2
    fl4 = 4 * d * n4 * (P + 4)  # QK^T and PV over each node's P + 4 keys
    roof[4].update(unique_bytes_per_layer=uniq, achieved_unique_GBs=uniq / (roof[4]["ms_per_layer"] * 1e-3) / 1e9,
                   alg_flop_per_layer=fl4, achieved_TFLOPs=fl4 / (roof[4]["ms_per_layer"] * 1e-3) / 1e12)
    roof[4]["note"] = ("the level runs as two halves on two streams: each half's attention launch runs beside the "
                       "other half's GEMMs, at a different time from the other's, so ms_per_layer is the union of "
                       "two launches that share the GPU; one_piece times the attention alone")
    tot1, cnt1, span1 = attn1[4]
    roof[4]["one_piece"] = {"note": "the same level in one piece on one stream (split threshold 0)",
                            "level_ms": t1[3], "ms_per_layer": span1 / L, "avg_launch_ms": tot1 / max(cnt1, 1),
                            "achieved_TFLOPs": fl4 / (span1 / L * 1e-3) / 1e12,
                            "achieved_unique_GBs": uniq / (span1 / L * 1e-3) / 1e9}
    total_ms = float(level_ms.sum())
    leaves = lay.level_size(lay.depth)
    flops = sum(2 * cfg.linear_params * lay.level_size(k) + 4 * d * L * lay.level_size(k) * (P + k)
                for k in range(1, lay.depth + 1))
    res = base_result(args, leaves / (total_ms / 1000.0), "leaf evals/s", total_ms, "bf16",
                      "C3 MCTS tree expansion: medium bf16, 64 roots x 200-token prefix (paged, block 16), "
                      "depth 4, branching 8 (262,144 leaves)",
                      level_ms=[float(x) for x in level_ms],
                      node_evals_per_s=lay.n_nodes / (total_ms / 1000.0),
                      whole_tree_mfma_frac=flops / (total_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                      roots_prefill_untimed=True)
    a1 = roof[1]
    res["roofline"] = {"kernel": "attn_extend_fan_kernel (level 1: 512 nodes in groups of 8 over 64 shared "
                                 "prefixes; level2: attn_extend_tree_kernel)",
                       "bound": "hbm", "achieved": a1["achieved_GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": a1["achieved_GBs"] / HBM_PEAK_GBS, "traffic": read_traffic("c3_level1"),
                       "traffic_measured_on": traffic_commit("c3_level1"),
                       "level2": dict(roof[2], traffic=read_traffic("c3_level2")),
                       "level4": dict(roof[4], traffic=read_traffic("c3_level4"))}
    res["roofline"]["level4"]["one_piece"]["traffic"] = read_traffic("c3_level4_one_piece")
    eng.close()
    res["cpu_baseline"] = None
    if not args.no_cpu_baseline:
        # the reference evaluates every leaf by a full recompute of its game
        # (root prefix + ancestors + leaf), decode.py:356-360
        from allie_amd.tree import node_path

        paths = [node_path(lay, tx.prefixes, tx.levels, lay.depth, j) for j in range(0, leaves, 4097)]
        res["cpu_baseline"] = cpu_baseline(cfg, tx_sd, paths, "leaf evals/s", args.cpu_budget,
                                           extrapolate=(lay.level_size(lay.depth), "262,144 depth-4 leaves"))
    return res


# ------------------------------------------------------------------------ C4
def bench_c4(args):
    import torch

    from allie_amd import capi, config, weights
    from allie_amd.batcher import ContinuousBatcher
    from allie_amd.engine import Engine

    cfg = config.MEDIUM
    c4_sd = weights.init_weights(cfg, seed=0)
    eng = Engine(cfg, c4_sd, mode="bfloat16", device="cuda:0")
    cb = ContinuousBatcher(eng, n_slots=args.slots)
    for _ in range(args.warmup):
        cb.step()
    torch.cuda.synchronize()
    assert int(cb.status.item()) == 0, "extend status"
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    probed = args.steps  # every decode attention launch of the timed steps is timed
    # a step of many games runs as two halves on two streams: two launches per layer
    probe = Probe(capi.PROBE_DECODE, 2 * probed * cfg.n_layer)
    tok0, keys0 = cb.tokens, cb.keys_read
    keys_probed = dec_probed = 0
    t0 = time.perf_counter()
    evs[0].record()
    for i in range(args.steps):
        k_before, d_before = cb.decode_keys, cb.decoded
        cb.step()
        if i < probed:
            keys_probed += cb.decode_keys - k_before
            dec_probed += cb.decoded - d_before
        evs[i + 1].record()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    att_span = probe.span()
    att_tot, att_n = probe.end()
    lat = np.array([evs[i].elapsed_time(evs[i + 1]) for i in range(args.steps)])
    ms = el * 1000.0 / args.steps
    appended = cb.tokens - tok0
    tok_s = appended / el
    mean_keys = (cb.keys_read - keys0) / args.steps
    games_started = cb.games_started
    # the same self-play continued with every step in one piece (decode split
    # off), for the attention kernel on its own
    n1 = max(args.steps // 10, 20)
    eng.set_split_tokens(24576, 0)
    probe1 = Probe(capi.PROBE_DECODE, 2 * n1 * cfg.n_layer)
    k1, dd1 = cb.decode_keys, cb.decoded
    for _ in range(n1):
        cb.step()
    torch.cuda.synchronize()
    span1 = probe1.span()
    tot1, cnt1 = probe1.end()
    k1, dd1 = cb.decode_keys - k1, cb.decoded - dd1
    eng.set_split_tokens(24576, 512)
    d = cfg.d_model
    att_ms = att_tot / max(att_n, 1)
    # per layer of a step: the running games' keys and values read (all
    # heads), their queries read and outputs written; over the time during
    # which a decode-attention launch of that layer ran (the union of the
    # launches' intervals: one launch, or one per half)
    att_bytes = (keys_probed / probed) * 2 * d * 2 + (dec_probed / probed) * 2 * d * 2
    layer_ms = att_span / (probed * cfg.n_layer)
    achieved = att_bytes / (layer_ms * 1e-3) / 1e9
    bytes1 = (k1 / n1) * 2 * d * 2 + (dd1 / n1) * 2 * d * 2
    layer1_ms = span1 / (n1 * cfg.n_layer)
    achieved1 = bytes1 / (layer1_ms * 1e-3) / 1e9
    res = base_result(args, tok_s, "tokens/s", ms, "bf16",
                      f"C4 continuous-batching self-play decode: medium bf16, {cb.S} slots, prefixes U[1,50], "
                      "game length Geometric(mean 80) capped 512, greedy argmax, refill on finish",
                      step_ms_p50=float(np.percentile(lat, 50)), step_ms_p90=float(np.percentile(lat, 90)),
                      step_ms_p99=float(np.percentile(lat, 99)),
                      mean_keys_per_step=mean_keys,
                      moves_appended=appended, games_started=games_started)
    res["roofline"] = {"kernel": "attn_extend_wave_kernel (decode: one token per running game over its paged KV)",
                       "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": achieved / HBM_PEAK_GBS, "traffic": read_traffic("c4_decode"),
                       "traffic_measured_on": traffic_commit("c4_decode"),
                       "achieved_is": "decode-attention bytes of a layer / the time during which that layer's "
                                      "attention launches ran (two per layer when the step runs as two halves, "
                                      "each beside the other half's projections)",
                       "alg_bytes_per_layer": att_bytes, "ms_per_layer": layer_ms, "avg_launch_ms": att_ms,
                       "launches_per_layer": att_n / (probed * cfg.n_layer),
                       "one_piece": {"note": f"{n1} more steps of the same self-play, each in one piece on one "
                                             "stream (decode split threshold 0)",
                                     "ms_per_layer": layer1_ms, "alg_bytes_per_layer": bytes1,
                                     "achieved": achieved1, "frac": achieved1 / HBM_PEAK_GBS,
                                     "traffic": read_traffic("c4_decode_one_piece"),
                                     "launches_per_layer": cnt1 / (n1 * cfg.n_layer)}}
    eng.close()
    res["cpu_baseline"] = None
    if not args.no_cpu_baseline:
        # the reference appends a move with a full forward of the game so far
        # (Policy.score_full, decode.py:199-203): leaves are the games of the
        # same seeded queue at each length they pass through
        from allie_amd.batcher import GameQueue

        prefixes, P, total = GameQueue().draw(16)
        rng = np.random.default_rng(0)
        leaves = []
        for p, tot in zip(prefixes, total):
            g = list(p) + rng.integers(0, 1968, int(tot) - len(p)).tolist()
            leaves += [g[:L] for L in range(len(p), int(tot), 16)]
        order = np.random.default_rng(1).permutation(len(leaves))
        leaves = [leaves[i] for i in order]
        res["cpu_baseline"] = cpu_baseline(cfg, c4_sd, leaves, "tokens/s", args.cpu_budget,
                                           extrapolate=(appended, f"the {args.steps} timed steps ({appended} moves)"))
    return res


# ------------------------------------------------------------------ search
def search_games(n_games: int, plies: int, seed: int = 11):
    """Seeded random legal games of ``plies`` moves (the search roots)."""
    from allie_amd.tokenizer import Game

    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n_games:
        g = Game("300+0", 1500, 1600, None, False, [], [], None)
        while len(g.moves) < plies and g.board.outcome() is None:
            legal = g.legal_moves
            g = g.make_move(legal[int(rng.integers(len(legal)))])
        if len(g.moves) == plies and g.board.outcome() is None:
            out.append(Game("300+0", 1500, 1600, None, False, g.moves, [3] * plies, None))
    return out


def bench_search(args):
    """One MCTS decision (``score_full``, n_sims simulations) on the medium
    bf16 model: the reference's full recompute per leaf, the KV-cached
    search (same sequential semantics; each leaf replayed from a captured
    HIP graph, and launched eagerly), and KV with leaf batching."""
    import torch

    from allie_amd import config, weights
    from allie_amd.decode import DECODE_STRATEGIES
    from allie_amd.model import AllieModel
    from allie_amd.tokenizer import UCITokenizer

    cfg = config.MEDIUM
    n_sims = 50
    model = AllieModel.from_state_dict(cfg, weights.init_weights(cfg, seed=0), mode="bfloat16")
    tok = UCITokenizer(max_length=512)
    games = search_games(args.warmup + args.steps, plies=60)
    modes = {"recompute": {}, "kv": {"kv_cache": True}, "kv_eager": {"kv_cache": True, "kv_graph": False},
             "kv_batch16": {"kv_cache": True, "leaf_batch": 16}}
    ms = {}
    leaf_us = None
    for name, kw in modes.items():
        strat = DECODE_STRATEGIES["mcts"](model, tok, device="cuda", precision="bfloat16", n_sims=n_sims, **kw)
        for g in games[: args.warmup]:
            strat.score_full(g, g.legal_moves)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for g in games[args.warmup:]:
            strat.score_full(g, g.legal_moves)
        torch.cuda.synchronize()
        ms[name] = (time.perf_counter() - t0) * 1000.0 / args.steps
        if name == "kv":
            # GPU time of one leaf: the captured graph replayed with the last
            # leaf's inputs (it rewrites that leaf's keys and values with the
            # same numbers), timed by events on the replay stream
            lg = strat._kv.leaf_graph
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(100):
                lg.graph.replay()
            e1.record()
            torch.cuda.synchronize()
            leaf_us = e0.elapsed_time(e1) * 10.0
    model.close()
    res = base_result(args, n_sims / (ms["kv"] / 1000.0), "simulations/s", ms["kv"], "bf16",
                      "MCTS decision: medium 24x1024x16, 50 simulations, roots = random legal games of 60 plies "
                      "(63 tokens)",
                      ms_per_decision={k: round(v, 2) for k, v in ms.items()},
                      sims_per_s={k: round(n_sims / (v / 1000.0), 1) for k, v in ms.items()},
                      speedup_kv_vs_recompute=ms["recompute"] / ms["kv"],
                      kv_leaf_gpu_us=round(leaf_us, 1),
                      note="kv replays each leaf from a captured HIP graph, kv_eager launches it kernel by "
                           "kernel; kv_batch16 is a different (virtual-loss batched) search; recompute, kv and "
                           "kv_eager make the same decisions")
    res["metric"] = "MCTS simulations/s per decision (not the headline metric)"
    res["roofline"] = None
    res["cpu_baseline"] = None
    return res


def bench_serve(args):
    """256 concurrent ``policy`` requests (random legal games of 20-120
    plies) on the medium bf16 model: the reference server's one-at-a-time
    ``decode_full`` against the batching front end (allie_amd.serve)."""
    import threading

    import torch

    from allie_amd import config, weights
    from allie_amd.decode import DECODE_STRATEGIES
    from allie_amd.model import AllieModel
    from allie_amd.serve import PolicyBatcher
    from allie_amd.tokenizer import UCITokenizer

    cfg = config.MEDIUM
    model = AllieModel.from_state_dict(cfg, weights.init_weights(cfg, seed=0), mode="bfloat16")
    tok = UCITokenizer(max_length=512)
    rng = np.random.default_rng(5)
    n_req = 256
    games = []
    for p in rng.integers(20, 121, n_req):
        games += search_games(1, int(p), seed=int(rng.integers(1 << 30)))
    for g in games:
        g.legal_moves  # host rules outside the timed region, as a server holds the position
    seq = DECODE_STRATEGIES["policy"](model, tok, device="cuda", precision="bfloat16")
    for g in games[:4]:
        seq.decode_full(g)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for g in games[: 64]:
        seq.decode_full(g)
    torch.cuda.synchronize()
    seq_rps = 64 / (time.perf_counter() - t0)
    b = PolicyBatcher(DECODE_STRATEGIES["policy"](model, tok, device="cuda", precision="bfloat16"), max_batch=256,
                      max_wait_ms=2.0)
    futs = [None] * n_req
    for rep in range(args.warmup + args.steps):
        if rep == args.warmup:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
        ths = [threading.Thread(target=lambda i=i: futs.__setitem__(i, b.submit(games[i]))) for i in range(n_req)]
        for t in ths:
            t.start()
        for t in ths:
            t.join()
        for f in futs:
            f.result(timeout=300)
    el = time.perf_counter() - t0
    batches, reqs = b.batches, b.requests
    b.close()
    model.close()
    rps = n_req * args.steps / el
    res = base_result(args, rps, "requests/s", el * 1000 / args.steps, "bf16",
                      "policy serving: medium 24x1024x16 bf16, 256 concurrent decode_full requests, random legal "
                      "games of 20-120 plies",
                      sequential_requests_per_s=seq_rps, speedup_vs_sequential=rps / seq_rps,
                      mean_batch=reqs / max(batches, 1))
    res["metric"] = "policy requests/s (not the headline metric)"
    res["roofline"] = None
    res["cpu_baseline"] = None
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--config", choices=["c2", "c3", "c4", "c5", "search", "serve"], default="c2")
    ap.add_argument("--slots", type=int, default=1024, help="c4: concurrent games")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--quality-sweep", action="store_true",
                    help="c5: fp8 top-1 agreement on perturbed weights with wte scaled 1, 2, 4, 8")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 512 MiB device copy (counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(games never exchange data, so the batch would shard by game, one "
                                   "shard per GPU)"}))
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy()
        return
    defaults = {"c2": (10, 3), "c3": (3, 1), "c4": (2000, 200), "c5": (10, 3), "search": (5, 1), "serve": (5, 1)}[args.config]
    args.steps = defaults[0] if args.steps is None else args.steps
    args.warmup = defaults[1] if args.warmup is None else args.warmup
    res = {"c2": bench_c2, "c3": bench_c3, "c4": bench_c4, "c5": bench_c5, "search": bench_search, "serve": bench_serve}[args.config](args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
