"""Benchmark of the NCA rollout on one MI355X: cell-updates/s and roofline fraction.

Workload (one bench "step" = one pass of the hot path over one batch): 256 random valid Sudoku
boards (17-30 clues, seed 0), K=128 trials each (32,768 rows), 9x9 grid, C=64, 4 perception
kernels (identity / Sobel-x / Sobel-y / Laplacian), MLP 256 -> 256 -> 64, p_fire=0.5, D=256
steps in one launch of the LDS-resident kernel, then the conf@K selection over the 128 trials.
Weights N(0, 0.02) (synthetic), states zero-initialised and clamped; inputs resident in HBM
before the timed region.

value = rows * 81 * D * steps / wall seconds (cell-updates/s). The roofline block prices the
rollout kernel's algorithmic FLOPs (2 * (36 C + F * hidden + hidden * C) = 168,448 per
cell-update) against the MI355X dense MFMA peak of the compute type, with the kernel's average
duration taken from HIP events recorded around every launch on its stream. The cpu_baseline
times the CPU oracle (PyTorch-CPU restatement of the reference step, fp32, all host threads) on
a bounded row sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_TFLOPS = {"bf16": 2500.0, "fp32": 157.3}
N_BOARDS, K_TRIALS, DEPTH, GRID = 256, 128, 256, 9
C, F, HID = 64, 256, 256
FLOP_PER_CELL_UPDATE = 2 * (36 * C + F * HID + HID * C)  # 168,448


def make_workload(device, seed=0):
    from ncas_amd.model import build_model, init_weights
    from ncas_amd.tasks import sudoku_boards

    model = init_weights(build_model("sudoku_c64"), seed=seed, std=0.02, zero_last=False)
    model = model.to(device)
    boards = sudoku_boards(N_BOARDS, seed)
    inputs = torch.from_numpy(np.repeat(boards.inputs, K_TRIALS, 0)).to(device)
    given = torch.from_numpy(np.repeat(boards.given, K_TRIALS, 0)).to(device)
    x = torch.zeros((inputs.shape[0], C, GRID, GRID), device=device)
    given4 = given[:, None]
    clamp = model.clamp_values(inputs)
    x = model.apply_clamp(x, given4, clamp).contiguous()
    return model, x, given4, clamp


def traffic_from_profiles(precision):
    path = os.path.join(ROOT, "profiles", f"rollout_c3_{precision}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def cpu_baseline(budget_s: float = 15.0):
    """The CPU oracle (fp32) on a row sample of the workload; cell-updates/s."""
    from ncas_amd.model import build_model, init_weights
    from ncas_amd.tasks import sudoku_boards
    from oracle import nca_oracle as O

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from cells import oracle_cell

    torch.set_num_threads(os.cpu_count() or 1)
    model = init_weights(build_model("sudoku_c64"), seed=0, std=0.02, zero_last=False)
    cell = oracle_cell(model)
    rows = 256
    boards = sudoku_boards(rows // 8, 0)
    inputs = torch.from_numpy(np.repeat(boards.inputs, 8, 0))
    given4 = torch.from_numpy(np.repeat(boards.given, 8, 0))[:, None]
    clamp = model.clamp_values(inputs)
    x = model.apply_clamp(torch.zeros(rows, C, GRID, GRID), given4, clamp)
    with torch.no_grad():
        O.rollout(cell, x, given4, clamp, 1, "fp32", seed=0, p_fire=0.5)  # warm-up
        t0 = time.perf_counter()
        O.rollout(cell, x, given4, clamp, 2, "fp32", seed=0, p_fire=0.5)
        per_step = (time.perf_counter() - t0) / 2
        steps = max(2, min(DEPTH, int(budget_s / max(per_step, 1e-6))))
        t0 = time.perf_counter()
        O.rollout(cell, x, given4, clamp, steps, "fp32", seed=0, p_fire=0.5)
        dt = time.perf_counter() - t0
    return {
        "value": rows * GRID * GRID * steps / dt,
        "unit": "cell-updates/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{rows} rows of the 9x9 C=64 workload x {steps} steps, fp32, {dt:.1f} s",
    }


def calibration_copy(mib: int) -> None:
    """One device-to-device copy of `mib` MiB: reads and writes exactly that many bytes."""
    n = mib * (1 << 20) // 4
    a = torch.ones(n, device="cuda:0")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    del a, b


def run_gpu(precision, steps, warmup):
    from ncas_amd.inference import rollout_steps
    from ncas_amd.readout import conf_select

    dev = torch.device("cuda:0")
    model, x, given4, clamp = make_workload(dev)
    model.packed(precision, dev)
    rows = x.shape[0]
    out = torch.empty_like(x)
    stream = torch.cuda.current_stream(dev)

    def one(seed, ev=None):
        if ev:
            ev[0].record(stream)
        _, conf, _ = rollout_steps(model, x, given4, clamp, DEPTH, seed=seed, p_fire=0.5,
                                   precision=precision, out=out, want_conf=True)
        if ev:
            ev[1].record(stream)
        best = conf_select(conf.view(N_BOARDS, K_TRIALS), None, K_TRIALS)
        return best

    with torch.no_grad():
        for i in range(warmup):
            one(1000 + i)
        torch.cuda.synchronize()
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(steps)]
        t0 = time.perf_counter()
        for i in range(steps):
            best = one(i, events[i])
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    kernel_ms = [a.elapsed_time(b) for a, b in events]
    cell_updates = rows * GRID * GRID * DEPTH
    avg_kernel_s = float(np.mean(kernel_ms)) / 1e3
    achieved = cell_updates * FLOP_PER_CELL_UPDATE / avg_kernel_s / 1e12
    return {
        "value": cell_updates * steps / wall,
        "ms_per_step": wall / steps * 1e3,
        "kernel_ms": kernel_ms,
        "achieved_tflops": achieved,
        "frac": achieved / PEAK_TFLOPS[precision],
        "best_first": best[:4].tolist(),
        "rows": rows,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--precision", choices=["bf16", "fp32"], default="bf16")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-fp32", action="store_true", help="skip the secondary fp32 run")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first copy this many MiB device-to-device (a kernel of known traffic "
                         "for scaling HBM counters), outside the timed region")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus must be 1"}))
        sys.exit(2)

    if args.calib_copy_mib:
        calibration_copy(args.calib_copy_mib)
    res = run_gpu(args.precision, args.steps, args.warmup)
    print(f"# gpu {args.precision}: {res['value']:.4g} cell-updates/s, kernel ms {res['kernel_ms']}",
          file=sys.stderr, flush=True)
    other = None
    if not args.no_fp32 and args.precision == "bf16":
        o = run_gpu("fp32", max(1, min(args.steps, 2)), 0)
        other = {"dtype": "fp32", "value": o["value"], "ms_per_step": o["ms_per_step"],
                 "roofline_frac": o["frac"], "achieved_tflops": o["achieved_tflops"]}
        print(f"# gpu fp32: {o['value']:.4g} cell-updates/s", file=sys.stderr, flush=True)
    cpu = None if args.no_cpu else cpu_baseline()
    line = {
        "metric": "cell-updates/sec on 1 MI355X (9x9 K=128 D=256) + % of roofline",
        "value": res["value"],
        "unit": "cell-updates/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.precision,
        "data": "synthetic",
        "config": {
            "workload": "sudoku 9x9: 256 boards x K=128 trials = 32768 rows, D=256 steps, "
                        "C=64, 4 kernels, MLP 256-256-64, p_fire=0.5, conf@K selection",
            "rows": res["rows"],
            "grid": [GRID, GRID],
            "depth": DEPTH,
            "k_trials": K_TRIALS,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": res["achieved_tflops"],
            "peak": PEAK_TFLOPS[args.precision],
            "unit": "TFLOP/s",
            "frac": res["frac"],
            "traffic": traffic_from_profiles(args.precision),
        },
        "cpu_baseline": cpu,
        "kernel_ms": res["kernel_ms"],
        "secondary": other,
    }
    if cpu:
        line["speedup_vs_cpu"] = res["value"] / cpu["value"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
