"""Benchmark of the batched policy/value inference path on one MI355X.

Default workload (the headline metric's configuration): medium shape
(24 layers, d_model 1024, 16 heads), bf16, one ragged packed batch of 256
game prefixes with lengths ``default_rng(2).integers(8, 401, 256)`` and
uniform move-token ids; one step = one prefill forward emitting policy
logits, value and time at every game's last token.  ``value`` is leaf
(prefix) evaluations per second with the inputs already resident in HBM.

Also reported, on the same JSON line:
* ``roofline`` for the dominant kernel (the MLP c_fc GEMM + gelu): its
  algorithmic FLOPs per launch (2 * T * 4096 * 1024) over its average launch
  duration, measured with HIP events around each of its launches inside the
  timed forwards, against the dense bf16 MFMA peak;
* ``cpu_baseline``: the CPU oracle (fp32, the reference's execution shape:
  one B=1 forward per game as Policy.score_full / MCTS.evaluate_node do,
  src/evaluation/decode.py:199-203,356-360) timed on a bounded sample of the
  same games on the host cores.
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


def cpu_baseline(cfg, sd, seqs, budget_s: float = 20.0):
    import torch

    from oracle.model_ref import RefModel

    cores = min(16, os.cpu_count() or 1)
    torch.set_num_threads(cores)
    ref = RefModel(cfg, sd, mode="float32")
    # one warm-up game, then B=1 forwards (as Policy.score_full calls the model)
    ids0 = torch.as_tensor(seqs[0].astype(np.int64))[None]
    ref.forward_padded(ids0)
    done, t0 = 0, time.perf_counter()
    for s in seqs:
        ref.forward_padded(torch.as_tensor(s.astype(np.int64))[None])
        done += 1
        if time.perf_counter() - t0 > budget_s:
            break
    el = time.perf_counter() - t0
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": done / el,
        "unit": "leaf evals/s",
        "cores": cores,
        "kind": "port",
        "sample": f"first {done} games of the same batch, one fp32 B=1 forward each "
                  f"(all-position logits, no KV cache), {el:.1f} s; cpu {cpu_model!r}; "
                  f"torch {torch.__version__}",
    }


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_gemm_fc_c2.txt")


def read_traffic():
    """HBM bytes per launch of the fc GEMM, measured with rocprofv3 --pmc
    FETCH_SIZE / WRITE_SIZE and scaled by the copy calibration (the line
    ``hbm_bytes_per_launch: N`` of the committed summary), or None."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        for line in f:
            if line.startswith("hbm_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 512 MiB device copy (counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(the path shards by game with no exchange; see DESIGN.md)"}))
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy()
        return

    import torch

    from allie_amd import capi, config, weights
    from allie_amd.engine import Engine

    cfg = config.MEDIUM
    sd = weights.init_weights(cfg, seed=0)
    seqs, lens = c2_batch()
    T = int(lens.sum())
    eng = Engine(cfg, sd, mode="bfloat16", device="cuda:0")
    words = torch.from_numpy(np.concatenate(seqs).view(np.int32)).cuda()
    out = eng.prefill(words, lens)
    for _ in range(args.warmup):
        eng.prefill(words, lens, out=out)
    torch.cuda.synchronize()

    L = capi.lib()
    capi.check(L.allie_probe_begin(capi.PROBE_FC, args.steps * cfg.n_layer), "probe")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        eng.prefill(words, lens, out=out)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    tot_ms, n_l = C.c_float(), C.c_int()
    capi.check(L.allie_probe_end(C.byref(tot_ms), C.byref(n_l)), "probe end")

    ms = el * 1000.0 / args.steps
    flops = alg_flops(cfg, lens)
    fc_flops = 2.0 * T * cfg.d_ff * cfg.d_model
    fc_ms = tot_ms.value / max(n_l.value, 1)
    fc_tflops = fc_flops / (fc_ms * 1e-3) / 1e12
    traffic = read_traffic()
    res = {
        "metric": "leaf evals/sec @ medium, ragged batch 256; % of MFMA / HBM roofline",
        "value": 256.0 / (ms / 1000.0),
        "unit": "leaf evals/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded ragged prefixes, random-init GPT-2 weights)",
        "config": {
            "workload": "C2 ragged prefill: medium shape 24x1024x16, 256 prefixes, lens U[8,400] seed 2",
            "n_seq": 256,
            "n_tokens": T,
            "tokens_per_s": T / (ms / 1000.0),
            "alg_tflop_per_step": flops / 1e12,
            "whole_forward_mfma_frac": flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "parallelism": "single GPU",
        },
        "roofline": {
            "kernel": "gemm_mfma_kernel<EPI_GELU,W_BF16> (MLP c_fc)",
            "bound": "mfma",
            "achieved": fc_tflops,
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": fc_tflops / MFMA_BF16_PEAK_TFLOPS,
            "traffic": traffic,
            "avg_launch_ms": fc_ms,
            "launches": n_l.value,
        },
        "cpu_baseline": None,
    }
    eng.close()
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(cfg, sd, seqs, args.cpu_budget)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
