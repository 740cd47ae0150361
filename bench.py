"""Benchmark: fused linear-CE forward+backward on one MI355X.

Default workload is BASELINE config C2 (Qwen2.5-0.5B-shaped head: N=16384,
d=896, V=151936, bf16, 5% ignore_index, mean).  A step is one
cut_cross_entropy forward plus backward producing dHidden and dW, with the
inputs already resident in HBM.  Prints one JSON line (the driver's contract).

Roofline: the dominant credited kernel kind (the largest share of step time
among launches that carry algorithmic work: the forward GEMM, and the per-band
launch holding the dHidden / dWeight GEMMs — with the next band's logits
recompute, which is executed but not credited, as the algorithmic work of a
fwd+bwd step is 6*N*V*d FLOPs) is timed with HIP events on its own launch
stream by the library (cce_kernel_timing_enable) over K further steps after the
K timed steps; the library reports each launch's credited and executed FLOPs.
The timed steps carry no per-launch events (one event between steps only):
events between a step's kernels add about 0.5% to a C2 step.

``--workload logits`` measures the logits-in cross-entropy instead
(chunked_cross_entropy_loss over [N, V] bf16 logits of the same C2 shape,
forward + backward producing dlogits); its kernels are HBM-bound and the
roofline is algorithmic bytes (N*V*2 read forward; N*V*2 read + N*V*2
written backward) over the HIP-event launch time.
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
# The rate a 256 x 256-tile bf16 MFMA loop reaches on this chip with random
# operands (LDS pre-filled, no global memory; the chip is power-limited and
# clocks down with the operands' bit activity): measured 1616-1660 TFLOP/s.
# A design that recomputes the logits executes 8*N*V*d for 6*N*V*d credited,
# so its step cannot exceed 6/8 of this.
CEILING_BF16_TFLOPS = 1640.0
PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic.json")
TRAFFIC_LOGITS_FILE = os.path.join(REPO, "profiles", "traffic_logits.json")


def timed_steps(step, steps: int):
    """Mean ms per step over `steps` steps, the sorted per-step times and the
    last step's result.  One event on the current stream between consecutive
    steps; nothing is recorded between the kernels of a step."""
    import torch

    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    out = None
    torch.cuda.synchronize()
    evs[0].record()
    for i in range(steps):
        out = step()
        evs[i + 1].record()
    torch.cuda.synchronize()
    return (evs[0].elapsed_time(evs[-1]) / steps, sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(steps)),
            out)


def kernel_timed_steps(step, steps: int) -> None:
    """`steps` further steps with the library's per-launch HIP events on each
    launch's stream (read back with kernel_timing_read).  The events sit
    between kernels and add about 0.5% to a C2 step, so the headline step
    time is measured without them."""
    import torch
    from chronicals_amd import _lib

    torch.cuda.synchronize()
    for k in range(_lib.CCE_KERNEL_KINDS):
        _lib.kernel_timing_read(k)  # drop anything recorded so far
    _lib.kernel_timing_enable(True)
    try:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    finally:
        _lib.kernel_timing_enable(False)


def cpu_model() -> str:
    """CPU model string (with the x86 family / model / stepping numbers, which name
    the core generation where the model name is generic) plus the host's logical
    CPU count and the CPUs this process may run on."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block is enough
                key, _, val = line.partition(":")
                fields.setdefault(key.strip(), val.strip())
    except OSError:
        pass
    name = fields.get("model name") or platform.processor() or "unknown"
    ids = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if fields.get(k)]
    if ids:
        name = f"{name}, " + ", ".join(ids)
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = None
    return f"{name} ({os.cpu_count()} logical CPUs on the host, {allowed} usable by this process)"


def blas_threads() -> int:
    """Threads the BLAS under numpy uses (threadpoolctl), else OMP_NUM_THREADS / the CPU count."""
    try:
        from threadpoolctl import threadpool_info
        blas = [p for p in threadpool_info() if p.get("user_api") == "blas"]
        mine = [p for p in blas if "numpy" in p.get("filepath", "")] or blas
        if mine:
            return int(mine[0]["num_threads"])
    except Exception:  # noqa: BLE001 - threadpoolctl is optional
        pass
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def cpu_baseline(cfg, h, w, lab, rows: int) -> dict:
    """Oracle (numpy restatement of the reference CPU path) fwd+bwd on the first
    `rows` rows of the timed inputs (h, w, lab: the CPU tensors the GPU run was
    given), upcast exactly to fp32; tokens/s."""
    from oracle import cce_oracle

    rows = min(rows, h.shape[0])
    hn = h[:rows].float().numpy()
    wn = w.float().numpy()
    ln = lab[:rows].numpy()
    threads = blas_threads()
    warm = max(8, rows // 8)
    cce_oracle.loss_and_grads(hn[:warm], wn, ln[:warm], chunk_size=8192)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        cce_oracle.loss_and_grads(hn, wn, ln, chunk_size=8192)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": rows / t, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{cfg.name}: the first {rows} of the timed N={h.shape[0]} rows and labels with the full "
                      f"weight (d={cfg.d}, V={cfg.V}), the same values the GPU step ran on, upcast to fp32; fp32 "
                      f"numpy/BLAS restatement of the reference CPU path (V-chunk 8192); median of 3 runs after a "
                      f"warm-up, {t:.2f} s per run; tokens/s = rows / time (linear in N)",
            "cpu": cpu_model()}


def cpu_baseline_logits(cfg, rows: int, seed: int = 0) -> dict:
    """Oracle (numpy restatement of chunked_cross_entropy_loss + its gradient) on a row slice; tokens/s."""
    import numpy as np
    import torch

    from oracle import cce_oracle

    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(rows, cfg.V, generator=g) * 3.0).to(torch.bfloat16).float().numpy()
    lab = torch.randint(0, cfg.V, (rows,), generator=g).numpy()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))

    def run(xs, ls):
        loss, lse, valid = cce_oracle.logits_forward(xs, ls, 8192)
        return cce_oracle.logits_backward(xs, ls, lse, valid, np.ones(1))

    run(x[: max(8, rows // 8)], lab[: max(8, rows // 8)])
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run(x, lab)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": rows / t, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{rows} rows of [N={cfg.N}, V={cfg.V}] logits (bf16 values in fp32); numpy restatement of "
                      f"chunked_cross_entropy_loss forward (V-chunk 8192) + its gradient, single-threaded "
                      f"elementwise numpy; median of 3 runs after a warm-up, {t:.2f} s per run; tokens/s = rows / "
                      f"time (linear in N)",
            "cpu": cpu_model()}


def copy_calibration(nbytes: int) -> None:
    """A plain device copy of known size, for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "launches": 3}), flush=True)


def blas_reference(cfg, chunk: int) -> None:
    """Library speed-of-light reference: torch.matmul (hipBLASLt) bf16 GEMMs of the path's shapes at cfg, each
    timed with events over 10 calls after 3 warm-ups; one JSON line per GEMM."""
    import torch

    N, d, V = cfg.N, cfg.d, cfg.V

    def run(name, M, Nn, K, a_t=False, b_t=True):
        a = (torch.randn(K, M, device="cuda").to(torch.bfloat16).t() if a_t
             else torch.randn(M, K, device="cuda").to(torch.bfloat16))
        b = torch.randn(Nn, K, device="cuda").to(torch.bfloat16).t() if b_t else torch.randn(K, Nn, device="cuda").to(
            torch.bfloat16)
        for _ in range(3):
            a @ b
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            a @ b
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 10
        print(json.dumps({"blas_reference": name, "M": M, "N": Nn, "K": K, "us": ms * 1e3,
                          "tflops": 2.0 * M * Nn * K / (ms * 1e-3) / 1e12}), flush=True)
        del a, b

    run("8192^3 A.B^T", 8192, 8192, 8192)
    run(f"{cfg.name} forward logits H.W^T", N, V, d)
    run(f"{cfg.name} band recompute H.W_b^T", N, chunk, d)
    run(f"{cfg.name} band dH G_b.W_b", N, d, chunk, b_t=False)
    run(f"{cfg.name} band dW G_b^T.H", chunk, d, N, a_t=True, b_t=False)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C2")
    ap.add_argument("--chunk", type=int, default=8192)
    ap.add_argument("--rows", type=int, default=None,
                    help="run the configuration with this many rows (N) instead of its own (smaller batches at "
                         "the configuration's d and V)")
    ap.add_argument("--cpu-rows", type=int, default=None,
                    help="rows of the CPU baseline sample (default 4096 fused, 8192 logits)")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain device copy of BYTES (PMC calibration) and exit")
    ap.add_argument("--frozen-weight", action="store_true",
                    help="lm_head weight frozen (LoRA): the step computes dHidden only, 4*N*V*d credited FLOPs")
    ap.add_argument("--trainer", action="store_true",
                    help="the reference trainer's call (chronicals_trainer.py:577-594, :1747-1771): fp32 hidden "
                         "states and fp32 master lm_head weight under bf16 autocast (cast to bf16 per call, fp32 "
                         "gradients), chunk from get_optimal_chunk_size, z_loss_weight 1e-4, through "
                         "CutCrossEntropyLoss")
    ap.add_argument("--blas-reference", action="store_true",
                    help="only time torch.matmul (hipBLASLt) on the path's GEMM shapes and exit")
    ap.add_argument("--workload", choices=("fused", "logits", "logits-fused"), default="fused",
                    help="fused: linear-CE from hidden + lm_head (default); logits: CE over existing logits, "
                         "forward + autograd backward; logits-fused: loss and gradient in one kernel "
                         "(liger_cross_entropy_forward with compute_grads)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build runs the fused linear-CE path on a single MI355X "
              "(use --gpus 1)", file=sys.stderr)
        return 2
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return 0

    if args.workload in ("logits", "logits-fused"):
        return bench_logits(args)
    if args.blas_reference:
        from tests.cce_common import CONFIGS
        blas_reference(CONFIGS[args.config], args.chunk)
        return 0

    import torch

    from chronicals_amd import _lib
    from chronicals_amd.kernels.cut_cross_entropy import (CutCrossEntropyLoss, cut_cross_entropy,
                                                          get_optimal_chunk_size)
    from tests.cce_common import CONFIGS, make_inputs

    cfg = CONFIGS[args.config]
    if args.rows:
        import dataclasses
        cfg = dataclasses.replace(cfg, N=int(args.rows))
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    # inputs by the configuration's CPU recipe (one seeded generator: hidden,
    # W, labels, ignore mask), then moved to the device; the CPU baseline runs
    # on a row slice of these same values
    h_cpu, w_cpu, lab_cpu = make_inputs(cfg, seed=0)
    h, w, lab = h_cpu.to(dev), w_cpu.to(dev), lab_cpu.to(dev)
    # the configuration's input dtype goes through the boundary as it is: C1's
    # fp32 operands are rounded to bf16 inside the op (bf16 MFMA arithmetic with
    # fp32 accumulation) and get fp32 gradients back; the trainer mode keeps
    # fp32 hidden states and an fp32 master weight
    io_dtype = torch.float32 if args.trainer else cfg.dtype
    h = h.to(io_dtype).requires_grad_(True)
    w = w.to(io_dtype).requires_grad_(not args.frozen_weight)
    N, d, V = cfg.N, cfg.d, cfg.V
    credited_step = (4.0 if args.frozen_weight else 6.0) * N * V * d
    # forward and backward skip the row tiles past the labelled rows (the
    # autograd path needs no lse of an ignored row): the figure over labelled
    # rows only is reported beside
    n_valid = int((lab != -100).sum())
    credited_valid = (4.0 if args.frozen_weight else 6.0) * n_valid * V * d
    chunk = get_optimal_chunk_size(V, d) if args.trainer else args.chunk
    z_loss = 1e-4 if args.trainer else 0.0
    loss_fn = CutCrossEntropyLoss(chunk_size=None, ignore_index=-100, z_loss_weight=z_loss,
                                  reduction=cfg.reduction) if args.trainer else None

    def step():
        h.grad = None
        w.grad = None
        if args.trainer:
            # chronicals_trainer.py:1747-1771: the loss runs under bf16 autocast on
            # the model's fp32 hidden states and lm_head.weight
            with torch.autocast("cuda", dtype=torch.bfloat16):
                loss = loss_fn(h, w, lab, None)
        else:
            loss = cut_cross_entropy(h, w, lab, None, chunk, -100, 0.0, z_loss, reduction=cfg.reduction)
        loss.backward()
        return loss

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    base_mem = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    # the mean over the K timed steps is the headline, the per-step spread is
    # reported beside it
    ms, step_ms, loss = timed_steps(step, args.steps)

    def pct(q):
        return step_ms[min(len(step_ms) - 1, int(round(q * (len(step_ms) - 1))))]
    peak_extra = torch.cuda.max_memory_allocated() - base_mem

    # per-kernel breakdown over K further steps, with the library's own FLOP
    # accounting per launch: credited = algorithmic (forward logits, dHidden,
    # dWeight), executed adds the backward's logits recompute
    kernel_timed_steps(step, args.steps)
    kernels = {}
    for k, name in _lib.KERNEL_KIND_NAMES.items():
        tot_ms, n, cr, ex = _lib.kernel_timing_read(k)
        if n == 0:
            continue
        kernels[name] = {
            "launches_per_step": n / args.steps,
            "avg_launch_us": tot_ms / n * 1e3,
            "ms_per_step": tot_ms / args.steps,
            "credited_gflop_per_launch": cr / n / 1e9,
            "tflops_credited": cr / (tot_ms * 1e-3) / 1e12,
            "tflops_executed": ex / (tot_ms * 1e-3) / 1e12,
        }
    credited = [k for k in kernels if kernels[k]["tflops_credited"] > 0]
    dom = max(credited, key=lambda k: kernels[k]["ms_per_step"])
    kd = kernels[dom]
    achieved = kd["tflops_credited"]
    traffic = None
    clock = None
    traffic_from = None
    try:
        with open(TRAFFIC_FILE) as f:
            tr = json.load(f)
        if (tr.get("config") == cfg.name and tr.get("kernel") == dom and not args.frozen_weight
                and not args.trainer and not args.rows and chunk == tr.get("chunk_size", 8192)):
            traffic = tr.get("hbm_bytes_per_launch")
            clock = tr.get("mfma_busy_and_clock", {}).get(dom, {}).get("clock_ghz")
            # traffic and clock come from separate rocprofv3 runs of the same
            # command (counters are collected in runs of their own), on the box
            # the profile names, not from this run
            traffic_from = (f"{tr.get('source')}: rocprofv3 --pmc runs on {tr.get('box', 'another box')}"
                            + (f", where {dom} averaged {tr['avg_launch_us']:.1f} us per launch by HIP events"
                               if tr.get("avg_launch_us") else "")
                            + "; achieved/frac here are this run's own HIP-event times")
    except (OSError, ValueError):
        pass

    step_tflops = credited_step / (ms * 1e-3) / 1e12
    # the same kernel over the labelled rows only (the GEMMs skip the 256-row
    # tiles past them; the last live tile is counted whole)
    valid_frac = min(1.0, (-(-n_valid // 256) * 256) / N)
    # ceiling of this kernel kind: the random-operand MFMA loop rate scaled by
    # its credited share of the executed FLOPs
    ceiling = CEILING_BF16_TFLOPS * kd["tflops_credited"] / kd["tflops_executed"]
    step_ceiling = CEILING_BF16_TFLOPS * (4.0 if args.frozen_weight else 6.0) / (6.0 if args.frozen_weight else 8.0)
    if args.trainer:
        workload = (f"{cfg.name} in the reference trainer's call: CutCrossEntropyLoss(chunk_size=None -> {chunk}, "
                    f"z_loss_weight=1e-4) on fp32 hidden [{N}, {d}] and an fp32 master lm_head weight [{V}, {d}] "
                    f"under bf16 autocast (both cast to bf16 per call, bf16 MFMA with fp32 accumulation, fp32 "
                    f"dHidden and dW), {int(cfg.ignore_frac * 100)}% ignore_index, {cfg.reduction}")
    else:
        workload = (f"{cfg.name}: fused linear-CE fwd+bwd N={N} d={d} V={V} "
                    + ("fp32 inputs (rounded to bf16 at the boundary: bf16 MFMA with fp32 accumulation; fp32 "
                       "gradients)" if io_dtype == torch.float32 else "bf16")
                    + f", {int(cfg.ignore_frac * 100)}% ignore_index, {cfg.reduction}; grads "
                    + ("dHidden only (frozen lm_head weight)" if args.frozen_weight else "dHidden, dW"))
    # BASELINE.json's metric names the C2 workload; other runs name their own
    headline = cfg.name == "C2" and not (args.rows or args.frozen_weight or args.trainer or chunk != 8192)
    metric = ("fused linear-CE fwd+bwd tokens/s and % bf16 MFMA peak, N=16k V=152k" if headline else
              f"fused linear-CE fwd+bwd tokens/s and % bf16 MFMA peak, {cfg.name} N={N} d={d} V={V}"
              + (", frozen lm_head (dHidden only)" if args.frozen_weight else "")
              + (", reference trainer call" if args.trainer else ""))
    ignore_txt = ("first token of each packed sequence" if cfg.labels == "packed"
                  else f"{cfg.ignore_frac:.0%} of rows") + " set to ignore_index"
    out = {
        "metric": metric,
        "value": N / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "step_ms": {"median": pct(0.5), "p10": pct(0.1), "p90": pct(0.9)},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # the arithmetic: bf16 MFMA operands with fp32 accumulation, whatever
        # the operands' dtype at the boundary (config.input_dtype)
        "dtype": "bf16",
        "data": (f"synthetic: one CPU torch.Generator seeded 0 draws hidden ~ N(0,1) [{N},{d}], W ~ N(0,0.02) "
                 f"[{V},{d}] (fp32, cast to {str(cfg.dtype).replace('torch.', '')}), labels "
                 f"{'Zipf(1.1)' if cfg.labels == 'zipf' else 'uniform'} over [0,V), then the ignore mask "
                 f"({ignore_txt}); then moved to the GPU"),
        "host": platform.node(),
        "config": {"workload": workload, "N": N, "d": d, "V": V, "chunk_size": chunk,
                   "frozen_weight": bool(args.frozen_weight), "trainer_call": bool(args.trainer),
                   "input_dtype": str(io_dtype).replace("torch.", ""), "z_loss_weight": z_loss},
        "pct_bf16_peak": 100.0 * step_tflops / PEAK_BF16_TFLOPS,
        "step_tflops_algorithmic": step_tflops,
        "valid_rows": n_valid,
        "pct_bf16_peak_valid_rows": 100.0 * credited_valid / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        # the step against the random-operand MFMA ceiling times the credited
        # share of a recomputing design's executed work (6/8; frozen W 4/6)
        "step_ceiling_tflops": step_ceiling,
        "pct_of_step_ceiling": 100.0 * step_tflops / step_ceiling,
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS, "traffic": traffic,
                     "ceiling": ceiling, "frac_of_ceiling": achieved / ceiling,
                     "achieved_valid_rows": achieved * valid_frac,
                     "frac_valid_rows": achieved * valid_frac / PEAK_BF16_TFLOPS,
                     # the chip runs below its 2.4 GHz peak clock under this load (power-limited); the
                     # clock the profile measured for this kernel, and the fraction of the peak at it
                     "clock_ghz_profiled": clock,
                     "traffic_and_clock_from": traffic_from,
                     "frac_at_profiled_clock": (achieved / (PEAK_BF16_TFLOPS * clock / 2.4)) if clock else None,
                     "kernel": f"{dom}: credited (algorithmic) FLOPs per launch "
                               f"({kd['credited_gflop_per_launch']:.1f} GFLOP) over its HIP-event average launch "
                               f"time ({kd['avg_launch_us']:.1f} us, {kd['launches_per_step']:g} launches/step); "
                               f"executed incl. recompute {kd['tflops_executed']:.0f} TFLOP/s; both count all N "
                               f"rows; the GEMMs run only the row tiles holding the {n_valid} labelled rows"},
        "kernels": kernels,
        "peak_extra_mem_bytes": int(peak_extra),
        "loss": float(loss.item()),
    }
    if not args.skip_cpu:
        out["cpu_baseline"] = cpu_baseline(cfg, h_cpu, w_cpu, lab_cpu, args.cpu_rows or 4096)
    print(json.dumps(out), flush=True)
    return 0


def bench_logits(args) -> int:
    """chunked_cross_entropy_loss fwd+bwd over [N, V] bf16 logits of config C2's shape."""
    import torch

    from chronicals_amd import _lib
    from chronicals_amd.kernels.logits_cross_entropy import chunked_cross_entropy_loss, liger_cross_entropy_forward
    from tests.cce_common import CONFIGS

    fused = args.workload == "logits-fused"

    cfg = CONFIGS[args.config]
    N, V = cfg.N, cfg.V
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    x = (torch.randn(N, V, generator=g, device=dev) * 3.0).to(torch.bfloat16).requires_grad_(True)
    lab = torch.randint(0, V, (N,), generator=g, device=dev)
    lab[torch.rand(N, generator=g, device=dev) < cfg.ignore_frac] = -100

    def step():
        if fused:
            # the gradient overwrites the logits, as the reference's kernel does; later steps run on those values
            return liger_cross_entropy_forward(xf, lab, compute_grads=True)[0]
        x.grad = None
        loss = chunked_cross_entropy_loss(x, lab)
        loss.backward()
        return loss

    xf = x.detach() if fused else None

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ms, step_ms, loss = timed_steps(step, args.steps)

    def pct(q):
        return step_ms[min(len(step_ms) - 1, int(round(q * (len(step_ms) - 1))))]

    kernel_timed_steps(step, args.steps)
    kernels = {}
    for k in (_lib.CCE_KERNEL_LOGITS_FWD, _lib.CCE_KERNEL_LOGITS_BWD, _lib.CCE_KERNEL_LOGITS_FUSED):
        tot_ms, n, by, _ = _lib.kernel_timing_read(k)
        if n == 0:
            continue
        kernels[_lib.KERNEL_KIND_NAMES[k]] = {
            "launches_per_step": n / args.steps,
            "avg_launch_us": tot_ms / n * 1e3,
            "ms_per_step": tot_ms / args.steps,
            "algorithmic_gb_per_launch": by / n / 1e9,
            "gbs": by / (tot_ms * 1e-3) / 1e9,
        }
    dom = max(kernels, key=lambda k: kernels[k]["ms_per_step"])
    kd = kernels[dom]
    step_bytes = (2.0 if fused else 3.0) * N * V * 2
    traffic = None
    try:
        with open(TRAFFIC_LOGITS_FILE) as f:
            tr = json.load(f)
        if tr.get("config") == cfg.name and tr.get("kernel") == dom:
            traffic = tr.get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        pass
    out = {
        "metric": ("logits-in CE loss+gradient (one kernel) tokens/s and % HBM peak, N=16k V=152k bf16 logits"
                   if fused else "logits-in CE fwd+bwd tokens/s and % HBM peak, N=16k V=152k bf16 logits"),
        "value": N / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "step_ms": {"median": pct(0.5), "p10": pct(0.1), "p90": pct(0.9)},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,9) bf16 logits, uniform labels, 5% ignore_index)",
        "config": {"workload": (f"logits-in CE loss + gradient in one kernel (liger_cross_entropy_forward, "
                                f"compute_grads) over [{N}, {V}] bf16 logits, mean; gradient bf16 over the logits"
                                if fused else
                                f"logits-in CE (chunked_cross_entropy_loss) fwd+bwd over [{N}, {V}] bf16 logits, "
                                f"mean; grad dlogits bf16"), "N": N, "V": V},
        "step_gbs_algorithmic": step_bytes / (ms * 1e-3) / 1e9,
        "roofline": {"bound": "hbm", "achieved": kd["gbs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": kd["gbs"] / PEAK_HBM_GBS, "traffic": traffic,
                     "kernel": f"{dom}: algorithmic bytes per launch ({kd['algorithmic_gb_per_launch']:.2f} GB) "
                               f"over its HIP-event average launch time ({kd['avg_launch_us']:.1f} us)"},
        "kernels": kernels,
        "loss": float(loss.item()),
    }
    if not args.skip_cpu:
        out["cpu_baseline"] = cpu_baseline_logits(cfg, args.cpu_rows or 8192)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
