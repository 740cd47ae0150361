"""Benchmark: fused linear-CE forward+backward on one MI355X.

Default workload is BASELINE config C2 (Qwen2.5-0.5B-shaped head: N=16384,
d=896, V=151936, bf16, 5% ignore_index, mean).  A step is one
cut_cross_entropy forward plus backward producing dHidden and dW.  Prints one
JSON line (the driver's contract).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

PEAK_BF16_TFLOPS = 2516.6   # 256 CU x 4096 FLOP/clk x 2.4 GHz (dense bf16 MFMA)
PEAK_HBM_GBS = 8000.0


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(cfg, rows: int, seed: int = 0) -> dict:
    """Oracle (numpy restatement of the reference CPU path) fwd+bwd on a row slice; tokens/s."""
    import numpy as np
    import torch

    from oracle import cce_oracle
    from tests.cce_common import make_inputs

    h, w, lab = make_inputs(cfg, seed=seed, N=rows)
    hn = h.float().numpy()
    wn = w.float().numpy()
    ln = lab.numpy()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    cce_oracle.loss_and_grads(hn[: max(8, rows // 8)], wn, ln[: max(8, rows // 8)], chunk_size=8192)  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        cce_oracle.loss_and_grads(hn, wn, ln, chunk_size=8192)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    del torch
    return {"value": rows / t, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{cfg.name} rows[:{rows}] of N={cfg.N} (full d={cfg.d}, V={cfg.V}), fp32 numpy, "
                      f"median of 3 after a warm-up, {t:.2f} s per run; extrapolated linearly in N",
            "cpu": cpu_model()}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="C2")
    ap.add_argument("--chunk", type=int, default=8192)
    ap.add_argument("--cpu-rows", type=int, default=512)
    ap.add_argument("--skip-cpu", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build runs the fused linear-CE path on a single MI355X "
              "(use --gpus 1)", file=sys.stderr)
        return 2

    import torch

    from chronicals_amd.kernels.cut_cross_entropy import cut_cross_entropy
    from tests.cce_common import CONFIGS, make_inputs

    cfg = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    h, w, lab = make_inputs(cfg, seed=0, device=dev, gen_device="cuda")
    h = h.to(torch.bfloat16).requires_grad_(True)
    w = w.to(torch.bfloat16).requires_grad_(True)
    N, d, V = cfg.N, cfg.d, cfg.V

    def step():
        h.grad = None
        w.grad = None
        loss = cut_cross_entropy(h, w, lab, None, args.chunk, -100, 0.0, 0.0, reduction=cfg.reduction)
        loss.backward()
        return loss

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    base_mem = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        loss = step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    peak_extra = torch.cuda.max_memory_allocated() - base_mem

    flops = 6.0 * N * V * d
    achieved = flops / (ms * 1e-3) / 1e12
    tokens_per_s = N / (ms * 1e-3)
    out = {
        "metric": "fused linear-CE fwd+bwd tokens/s and % bf16 MFMA peak, N=16k V=152k",
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) hidden, N(0,0.02) W, uniform labels)",
        "config": {"workload": f"{cfg.name}: fused linear-CE fwd+bwd N={N} d={d} V={V} bf16, "
                               f"{int(cfg.ignore_frac * 100)}% ignore_index, {cfg.reduction}",
                   "N": N, "d": d, "V": V, "chunk_size": args.chunk},
        "pct_bf16_peak": 100.0 * achieved / PEAK_BF16_TFLOPS,
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS, "traffic": None,
                     "kernel": "whole fwd+bwd step (6*N*V*d algorithmic FLOPs)"},
        "peak_extra_mem_bytes": int(peak_extra),
        "loss": float(loss.item()),
    }
    if not args.skip_cpu:
        out["cpu_baseline"] = cpu_baseline(cfg, args.cpu_rows)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
