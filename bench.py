"""Benchmark of the NCA rollout on one MI355X: cell-updates/s and roofline fraction.

Default workload (one bench "step" = one pass of the hot path over one batch): 256 random valid
Sudoku boards (17-30 clues, seed 0), K=128 trials each (32,768 rows), 9x9 grid, C=64, 4
perception kernels (identity / Sobel-x / Sobel-y / Laplacian), MLP 256 -> 256 -> 64,
p_fire=0.5, D=256 steps in one launch of the LDS-resident kernel, then the conf@K selection over
the 128 trials. Weights N(0, 0.02) (synthetic), states zero-initialised and clamped; inputs
resident in HBM before the timed region.

`--workload maze13` (8 DFS mazes 13x13, K=1, D=300, fp32: the smoke maze configuration) times the
resident kernel. `--workload maze201` (16 DFS mazes 201x201, C=16, MLP 64 -> 128 -> 16,
D=13,000, p_fire=0.5) times the per-step path (one launch of the wave-per-tile kernel per step)
the same way, and beside it the temporally blocked regime (2 steps per launch on LDS-resident
windows, `--window-steps`), and
`--workload hardmaze30` (1,000 hard mazes
30x30 with 10 % extra openings, K=64 -> 64,000 rows, C=32, MLP 128 -> 256 -> 32, D=200, p_fire=0.8
gated to 0.2 above confidence 0.9) the streamed C=32 kernel (one board per workgroup, the whole
rollout in one launch). `--workload bptt30` times one training iteration: 64
states sampled from a replay pool of 1,024 (30x30 DFS mazes, C=32 cell, bf16 forward with fp32
master weights), a 32-step BPTT chunk with the per-cell cross-entropy on the 2-class path
targets, the fused clip + AdamW + EMA update, write-back; it reports cell-steps/s and the peak
activation memory. Its roofline
prices 4x the forward FLOPs per cell-step against the dense MFMA peak of the chunk's compute
type (bf16: the forward and every product of the backward run on bf16 MFMA, the backward with
the reference's bf16 gradient rounding points), with the same rate against the fp32 peak beside
it (frac_of_fp32_peak).

The default run (the Sudoku workload) adds a `configs` block with every other configuration
measured the same way, each with its roofline and CPU baseline: maze13 (C1), maze201 (C2, both
regimes), hardmaze30 (C4) and bptt30 (C5, with the peak activation memory); `--no-configs`
skips it.

value = rows * H * W * D * steps / wall seconds (cell-updates/s). The roofline block prices the
rollout kernel's algorithmic FLOPs (2 * (36 C + F * hidden + hidden * C) per cell-update, the
reference's count_step_flops convention) against the MI355X dense MFMA peak of the compute type,
or, for the per-step path (maze201) when it is lower, its algorithmic HBM bytes (the fp32 state read and
written once per step plus the given mask: 8 C + 1 bytes per cell-update) against 8 TB/s. The
kernel time comes from HIP events recorded on the launch stream around every rollout call. The
cpu_baseline times the CPU oracle (PyTorch-CPU restatement of the reference step, fp32, all host
threads) on a bounded row sample of the same workload.
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
PEAK_HBM_GBS = 8000.0

WORKLOADS = {
    "maze13": dict(
        preset="maze_c16", task="maze", boards=8, k=1, depth=300, grid=13, p_fire=0.5,
        precision="fp32",
        desc="smoke maze 13x13: 8 DFS mazes, K=1, D=300 steps, C=16, 4 kernels, MLP 64-128-16, "
             "p_fire=0.5, fp32, one launch of the resident kernel"),
    "sudoku9": dict(
        preset="sudoku_c64", task="sudoku", boards=256, k=128, depth=256, grid=9, p_fire=0.5,
        desc="sudoku 9x9: 256 boards x K=128 trials = 32768 rows, D=256 steps, C=64, 4 kernels, "
             "MLP 256-256-64, p_fire=0.5, conf@K selection"),
    "maze201": dict(
        preset="maze_c16", task="maze", boards=16, k=1, depth=13000, grid=201, p_fire=0.5,
        desc="maze 201x201: 16 DFS mazes, D=13000 steps, C=16, 4 kernels, MLP 64-128-16, "
             "p_fire=0.5, one launch per step (wave-per-tile kernel)"),
    "bptt30": dict(
        preset="maze_hard_c32", task="maze", boards=1024, k=1, depth=32, grid=30, p_fire=0.8,
        batch=64, extra=0.10,
        desc="BPTT 30x30: batch 64 from a replay pool of 1024 maze states, 32-step chunk, C=32, "
             "MLP 128-256-32 bf16 with fp32 master weights, per-cell CE on path targets, AdamW"),
    "hardmaze30": dict(
        preset="maze_hard_c32", task="maze", boards=1000, k=64, depth=200, grid=30, p_fire=0.8,
        p_low=0.2, tau=0.9, extra=0.10,
        desc="hard maze 30x30 (+10% openings): 1000 boards x K=64 = 64000 rows, D=200 steps, "
             "C=32, MLP 128-256-32, p_fire=0.8 gated to 0.2 above confidence 0.9, conf@K, "
             "one streamed launch per rollout (one board per workgroup)"),
}


def _cell_dims(preset):
    from ncas_amd.model import build_model

    cfg = build_model(preset).cfg
    C, hid = cfg.channels, cfg.hidden
    return C, 4 * C, hid


def flop_per_cell_update(preset):
    C, F, hid = _cell_dims(preset)
    return 2 * (36 * C + F * hid + hid * C)


def hbm_bytes_per_cell_update(preset):
    C, _, _ = _cell_dims(preset)
    return 8 * C + 1


def make_boards(wl, seed=0):
    from ncas_amd.tasks import maze_boards, sudoku_boards

    if wl["task"] == "sudoku":
        return sudoku_boards(wl["boards"], seed)
    return maze_boards(wl["boards"], wl["grid"], seed, extra_openings=wl.get("extra", 0.0))


def make_workload(wl, device, seed=0):
    from ncas_amd.model import build_model, init_weights

    model = init_weights(build_model(wl["preset"]), seed=seed, std=0.02, zero_last=False)
    model = model.to(device)
    boards = make_boards(wl, seed)
    inputs = torch.from_numpy(np.repeat(boards.inputs, wl["k"], 0)).to(device)
    given = torch.from_numpy(np.repeat(boards.given, wl["k"], 0)).to(device)
    C = model.cfg.channels
    x = torch.zeros((inputs.shape[0], C, *inputs.shape[1:]), device=device)
    given4 = given[:, None]
    clamp = model.clamp_values(inputs)
    x = model.apply_clamp(x, given4, clamp).contiguous()
    return model, x, given4, clamp


def traffic_from_profiles(name, precision):
    path = os.path.join(ROOT, "profiles", f"rollout_{name}_{precision}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def cpu_baseline(wl, budget_s: float = 15.0):
    """The CPU oracle (fp32) on a row sample of the workload; cell-updates/s."""
    from ncas_amd.model import build_model, init_weights
    from oracle import nca_oracle as O

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from cells import oracle_cell

    torch.set_num_threads(os.cpu_count() or 1)
    model = init_weights(build_model(wl["preset"]), seed=0, std=0.02, zero_last=False)
    cell = oracle_cell(model)
    sub = dict(wl, boards=max(1, min(wl["boards"], 4096 // (wl["grid"] ** 2) + 1)))
    boards = make_boards(sub, 0)
    k = max(1, min(wl["k"], 1024 // len(boards.inputs)))
    inputs = torch.from_numpy(np.repeat(boards.inputs, k, 0))
    given4 = torch.from_numpy(np.repeat(boards.given, k, 0))[:, None]
    clamp = model.clamp_values(inputs)
    rows, H, W = inputs.shape
    x = model.apply_clamp(torch.zeros(rows, model.cfg.channels, H, W), given4, clamp)
    kw = dict(seed=0, p_fire=wl["p_fire"], p_low=wl.get("p_low"), tau=wl.get("tau"))
    with torch.no_grad():
        O.rollout(cell, x, given4, clamp, 1, "fp32", **kw)  # warm-up
        t0 = time.perf_counter()
        O.rollout(cell, x, given4, clamp, 2, "fp32", **kw)
        per_step = (time.perf_counter() - t0) / 2
        steps = max(2, min(wl["depth"], int(budget_s / max(per_step, 1e-6))))
        t0 = time.perf_counter()
        O.rollout(cell, x, given4, clamp, steps, "fp32", **kw)
        dt = time.perf_counter() - t0
    return {
        "value": rows * H * W * steps / dt,
        "unit": "cell-updates/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "cpu_model": cpu_model(),
        "sample": f"{rows} rows of the {H}x{W} C={model.cfg.channels} workload x {steps} steps, "
                  f"fp32, {dt:.1f} s",
    }


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo, what lscpu prints as "Model name")."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_bptt(wl, budget_s: float = 8.0):
    """The CPU oracle's BPTT chunk (fp32 autograd of the restated chunk loss, the reference's
    unfused path) on a board sample of the workload; cell-steps/s."""
    from ncas_amd.model import build_model, init_weights
    from oracle import nca_oracle as O

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from cells import oracle_cell

    torch.set_num_threads(os.cpu_count() or 1)
    model = init_weights(build_model(wl["preset"]), seed=0, std=0.02, zero_last=False)
    base = oracle_cell(model)
    names = ("kernels", "w1", "b1", "w2", "b2", "head_w", "head_b")
    boards = make_boards(dict(wl, boards=2), 0)
    inputs = torch.from_numpy(boards.inputs)
    given4 = torch.from_numpy(boards.given)[:, None]
    clamp = model.clamp_values(inputs)
    B, H, W = inputs.shape
    x0 = model.apply_clamp(torch.zeros(B, model.cfg.channels, H, W), given4, clamp)
    targets = model.output_index(torch.from_numpy(boards.targets))
    n = wl["depth"]
    masks = torch.stack([O.fire_masks_np(0, 0, B, s, H, W, wl["p_fire"]) for s in range(n)])
    weights = [1.0] * n

    def once():
        params = {k: getattr(base, k).detach().float().clone().requires_grad_(True)
                  for k in names}
        cell = O.OracleCell(**{**base.__dict__, **params})
        loss = O.chunk_loss(cell, x0, given4, clamp, masks, targets, weights, "fp32",
                            dtype=torch.float32)
        loss.backward()

    once()  # warm-up
    reps, t0 = 0, time.perf_counter()
    while reps < 1 or (time.perf_counter() - t0 < budget_s and reps < 20):
        once()
        reps += 1
    dt = time.perf_counter() - t0
    return {"value": B * H * W * n * reps / dt, "unit": "cell-steps/s",
            "cores": torch.get_num_threads(), "kind": "port", "cpu_model": cpu_model(),
            "sample": f"{B} boards of the {H}x{W} C={model.cfg.channels} chunk x {n} steps x "
                      f"{reps} forward + backward, fp32 autograd, {dt:.1f} s"}


def calibration_copy(mib: int) -> None:
    """One device-to-device copy of `mib` MiB: reads and writes exactly that many bytes."""
    n = mib * (1 << 20) // 4
    a = torch.ones(n, device="cuda:0")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    del a, b


def run_gpu(wl, precision, steps, warmup, window_steps=0):
    from ncas_amd import _lib
    from ncas_amd.inference import rollout_steps
    from ncas_amd.readout import conf_select

    if _lib.load().nca_set_window_steps(window_steps) != 0:
        raise ValueError(f"window steps {window_steps}")
    dev = torch.device("cuda:0")
    model, x, given4, clamp = make_workload(wl, dev)
    model.packed(precision, dev)
    rows, _, H, W = x.shape
    out = torch.empty_like(x)
    stream = torch.cuda.current_stream(dev)
    n_boards, k = wl["boards"], wl["k"]

    def one(seed, ev=None):
        if ev:
            ev[0].record(stream)
        _, conf, _ = rollout_steps(model, x, given4, clamp, wl["depth"], seed=seed,
                                   p_fire=wl["p_fire"], p_low=wl.get("p_low"), tau=wl.get("tau"),
                                   precision=precision, out=out, want_conf=True)
        if ev:
            ev[1].record(stream)
        return conf_select(conf.view(n_boards, k), None, k)

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
    cell_updates = rows * H * W * wl["depth"]
    avg_kernel_s = float(np.mean(kernel_ms)) / 1e3
    rate = cell_updates / avg_kernel_s
    tflops = rate * flop_per_cell_update(wl["preset"]) / 1e12
    return {
        "value": cell_updates * steps / wall,
        "ms_per_step": wall / steps * 1e3,
        "kernel_ms": kernel_ms,
        "kernel_rate": rate,
        "achieved_tflops": tflops,
        "frac": tflops / PEAK_TFLOPS[precision],
        "best_first": best[:4].tolist(),
        "rows": rows,
        "cell_updates": cell_updates,
    }


def run_bptt(wl, precision, steps, warmup):
    """Training iterations: pool sample -> 32-step BPTT chunk -> fused clip + AdamW + EMA ->
    write-back."""
    from ncas_amd.model import build_model, init_weights
    from ncas_amd.optim import FusedUpdate
    from ncas_amd.train import Engine, ReplayPool

    dev = torch.device("cuda:0")
    model = init_weights(build_model(wl["preset"]), seed=0, std=0.02, zero_last=False).to(dev)
    ema = init_weights(build_model(wl["preset"]), seed=0, std=0.02, zero_last=False).to(dev)
    boards = make_boards(wl, 0)
    pool = ReplayPool(model, boards, wl["boards"], np.random.default_rng(0),
                      torch.Generator(device=dev).manual_seed(0))
    eng = Engine(model, None, {"rollout": wl["depth"], "chunk": wl["depth"], "amp": precision == "bf16"}, dev)
    # The reference's hard-maze training settings (configs/maze_hard.yaml: lr 5e-4, weight decay
    # 1e-4, clip 1.0, linear warm-up over the first quarter of 10,000 steps), EMA 0.999.
    upd = FusedUpdate(model, ema, 5e-4, weight_decay=1e-4)
    rng = np.random.default_rng(1)
    weights = [1.0] * wl["depth"]
    it = [0]

    def one():
        idx, batch = pool.sample(wl["batch"], 0.25)
        seeds = rng.integers(0, 2**62, size=wl["depth"])
        lr = 5e-4 * min(1.0, (it[0] + 1) / 2500)
        d = min(0.999, (1 + it[0]) / (10 + it[0]))
        x, loss, _ = eng.train_iteration(batch, seeds, 0, weights, None,
                                         lambda _g: upd.step(lr, d, 1.0))
        it[0] += 1
        batch["x"] = x
        pool.write_back(idx, batch)
        return loss

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    t0 = time.perf_counter()
    losses = [one() for _ in range(steps)]
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    peak = torch.cuda.max_memory_allocated(dev) - base
    cell_steps = wl["batch"] * wl["grid"] ** 2 * wl["depth"]
    rate = cell_steps * steps / wall
    flops = 4 * flop_per_cell_update(wl["preset"])  # forward + recompute + dX + dW
    tflops = rate * flops / 1e12
    res = eng.last_chunk
    return {
        "value": rate, "ms_per_step": wall / steps * 1e3, "kernel_ms": None,
        "kernel_rate": rate, "achieved_tflops": tflops,
        "rows": wl["batch"], "loss": [float(v) for v in losses],
        "peak_activation_bytes": int(peak),
        "states_bytes": res.states_bytes, "workspace_bytes": res.workspace_bytes,
        "skipped": int(upd.skipped),
    }


# LDS ceiling of the streamed C=64 kernel (9x9 bf16): per 16-cell tile its waves read 70 KB
# from LDS (the stencil's taps, Z four times, H twice, the state) and write 22 KB (Z, H, the state
# and its bf16 copy); gfx950's LDS serves 256 B/cycle of conflict-free ds_read_b128 and 80 B/cycle
# of ds_write_b128 / b64 per CU (measured), at the 2.4 GHz peak clock of the MFMA figure.
LDS_CYCLES_PER_CELL_STREAM64 = (70 * 1024 / 256 + 22 * 1024 / 80) / 16
CLOCK_HZ = 2.4e9
N_CU = 256


def roofline(name, wl, precision, res):
    """Binding ceiling of the workload's dominant kernel: the lowest of its MFMA (FLOPs), LDS
    (the streamed C=64 kernel's own LDS traffic) and HBM (algorithmic bytes) ceilings, each in
    cell-updates/s; MFMA for the resident kernels (sudoku9, hardmaze30, maze13), the lower of
    MFMA and HBM for the per-step path (maze201)."""
    flops = flop_per_cell_update(wl["preset"])
    mfma_ceiling = PEAK_TFLOPS[precision] * 1e12 / flops
    block = {"bound": "mfma", "achieved": res["achieved_tflops"], "peak": PEAK_TFLOPS[precision],
             "unit": "TFLOP/s", "frac": res["frac"], "traffic": traffic_from_profiles(name, precision)}
    ceilings = {"unit": "cell-updates/s", "mfma": mfma_ceiling, "lds": None, "hbm": None}
    if name == "sudoku9" and precision == "bf16":
        ceilings["lds"] = N_CU * CLOCK_HZ / LDS_CYCLES_PER_CELL_STREAM64
    if name == "maze201":
        nbytes = hbm_bytes_per_cell_update(wl["preset"])
        hbm_ceiling = PEAK_HBM_GBS * 1e9 / nbytes
        ceilings["hbm"] = hbm_ceiling
        if hbm_ceiling < mfma_ceiling:
            gbs = res["kernel_rate"] * nbytes / 1e9
            block.update(bound="hbm", achieved=gbs, peak=PEAK_HBM_GBS, unit="GB/s",
                         frac=gbs / PEAK_HBM_GBS)
    elif block["traffic"]:
        # the resident kernels touch HBM once per launch: the measured bytes per cell-update
        ceilings["hbm"] = PEAK_HBM_GBS * 1e9 / (block["traffic"] / res["cell_updates"])
    if name == "maze13":
        # one board per workgroup of the resident kernel (ceil(rows / 256) boards each): with
        # fewer boards than CUs the rest of the chip idles, so the fraction of the occupied CUs'
        # peak is given beside the chip's
        rows = wl["boards"] * wl["k"]
        per_wg = max(1, -(-rows // N_CU))
        wgs = -(-rows // per_wg)
        if wgs < N_CU:
            block["workgroups"] = wgs
            block["frac_of_occupied_cus"] = block["frac"] * N_CU / wgs
    block["ceilings"] = ceilings
    return block


def bptt_entry(wl, precision, steps, warmup, cpu_budget=None):
    """The BPTT workload's measurement: cell-steps/s of whole training iterations, the roofline
    of 4x the forward FLOPs per cell-step against the dense MFMA peak of the chunk's compute type
    (fp32 peak beside it), the peak activation memory and the CPU oracle's chunk."""
    res = run_bptt(wl, precision, steps, warmup)
    return {
        "metric": "BPTT cell-steps/sec on 1 MI355X (30x30 C=32, batch 64, 32-step chunk)",
        "value": res["value"], "unit": "cell-steps/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": res["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": precision, "data": "synthetic",
        "config": {"workload": wl["desc"], "rows": res["rows"], "grid": [wl["grid"]] * 2,
                   "depth": wl["depth"]},
        "roofline": {"bound": "mfma", "achieved": res["achieved_tflops"],
                     "peak": PEAK_TFLOPS[precision], "unit": "TFLOP/s",
                     "frac": res["achieved_tflops"] / PEAK_TFLOPS[precision], "traffic": None,
                     "frac_of_fp32_peak": res["achieved_tflops"] / PEAK_TFLOPS["fp32"]},
        "peak_activation_bytes": res["peak_activation_bytes"],
        "states_bytes": res["states_bytes"], "workspace_bytes": res["workspace_bytes"],
        "skipped_updates": res["skipped"], "loss": res["loss"],
        "cpu_baseline": None if cpu_budget is None else cpu_baseline_bptt(wl, cpu_budget),
    }


def rollout_entry(name, wl, precision, steps, warmup, window_steps=0, cpu_budget=None,
                  fp32=False, regimes=False):
    """A rollout workload's measurement: cell-updates/s over the wall clock, the dominant
    kernel's roofline (HIP events on its stream), optionally the fp32 run beside a bf16 one, the
    other C2 regime, and the CPU oracle on a row sample."""
    res = run_gpu(wl, precision, steps, warmup, window_steps)
    print(f"# gpu {name} {precision}: {res['value']:.4g} cell-updates/s, kernel ms "
          f"{[round(v, 3) for v in res['kernel_ms']]}", file=sys.stderr, flush=True)
    H = W = wl["grid"]
    entry = {
        "metric": f"cell-updates/sec on 1 MI355X ({H}x{W} {name})",
        "value": res["value"], "unit": "cell-updates/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": res["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": precision, "data": "synthetic",
        "config": {"workload": wl["desc"], "rows": res["rows"], "grid": [H, W],
                   "depth": wl["depth"], "k_trials": wl["k"]},
        "roofline": roofline(name, wl, precision, res),
        "kernel_ms": res["kernel_ms"],
    }
    if fp32 and precision == "bf16":
        o = run_gpu(wl, "fp32", max(1, min(steps, 2)), 0)
        entry["secondary"] = {"dtype": "fp32", "value": o["value"],
                              "ms_per_step": o["ms_per_step"], "roofline_frac": o["frac"],
                              "achieved_tflops": o["achieved_tflops"]}
        print(f"# gpu fp32: {o['value']:.4g} cell-updates/s", file=sys.stderr, flush=True)
    if regimes:
        # the other C2 regime: per-step launches vs the temporally blocked kernel
        alt = 2 if window_steps == 0 else 0
        r2 = run_gpu(wl, precision, 1, 0, alt)
        label = lambda t: "per_step" if t == 0 else f"temporal_T{t}"  # noqa: E731
        entry["regimes"] = {
            label(t): {"kernel_ms_per_step": float(np.mean(r["kernel_ms"])) / wl["depth"],
                       "cell_updates_per_s": r["kernel_rate"],
                       "roofline": roofline(name, wl, precision, r)}
            for t, r in ((window_steps, res), (alt, r2))}
        print(f"# regimes {entry['regimes']}", file=sys.stderr, flush=True)
    cpu = None if cpu_budget is None else cpu_baseline(wl, cpu_budget)
    entry["cpu_baseline"] = cpu
    if cpu:
        # the CPU baseline is the fp32 oracle: the like-for-like ratio is the fp32 GPU run's
        entry["speedup_vs_cpu"] = res["value"] / cpu["value"]
        fp32_value = res["value"] if precision == "fp32" else entry.get("secondary", {}).get("value")
        if fp32_value:
            entry["speedup_vs_cpu_fp32"] = fp32_value / cpu["value"]
    return entry


# every configuration beside the headline: (workload, precision, steps, warmup, CPU seconds)
CONFIG_RUNS = (("maze13", "fp32", 10, 2, 4.0), ("maze201", "bf16", 2, 1, 4.0),
               ("hardmaze30", "bf16", 2, 1, 4.0), ("bptt30", "bf16", 20, 3, 6.0))


def configs_block() -> dict:
    """C1, C2 (both regimes), C4 and C5 measured the same way as the headline."""
    out = {}
    for name, precision, steps, warmup, budget in CONFIG_RUNS:
        wl = dict(WORKLOADS[name])
        if name == "bptt30":
            e = bptt_entry(wl, precision, steps, warmup, budget)
        else:
            e = rollout_entry(name, wl, precision, steps, warmup, cpu_budget=budget,
                              regimes=name == "maze201")
        e.pop("kernel_ms", None)
        e.pop("loss", None)
        out[name] = e
        print(f"# config {name}: {e['value']:.4g} {e['unit']}", file=sys.stderr, flush=True)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--workload", choices=list(WORKLOADS), default="sudoku9")
    ap.add_argument("--precision", choices=["bf16", "fp32"], default=None,
                    help="compute type (default: the workload's, bf16 unless it names fp32)")
    ap.add_argument("--window-steps", type=int, default=0,
                    help="steps per launch of the temporally blocked kernel (maze201; 0: one "
                         "step per launch)")
    ap.add_argument("--no-regimes", action="store_true",
                    help="maze201: skip the secondary timing of the other regime")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-fp32", action="store_true", help="skip the secondary fp32 run")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other configurations of the default run")
    ap.add_argument("--depth", type=int, default=0,
                    help="steps per rollout instead of the workload's own (profiling runs only)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first copy this many MiB device-to-device (a kernel of known traffic "
                         "for scaling HBM counters), outside the timed region")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus must be 1"}))
        sys.exit(2)

    wl = dict(WORKLOADS[args.workload])
    if args.precision is None:
        args.precision = wl.get("precision", "bf16")
    if args.depth:  # a shorter rollout of the same workload, for counter runs
        wl["depth"] = args.depth
    if args.calib_copy_mib:
        calibration_copy(args.calib_copy_mib)
    budget = None if args.no_cpu else 15.0
    if args.workload == "bptt30":
        line = bptt_entry(wl, args.precision, args.steps, args.warmup,
                          None if args.no_cpu else 8.0)
        print(json.dumps(line), flush=True)
        return
    line = rollout_entry(args.workload, wl, args.precision, args.steps, args.warmup,
                         args.window_steps, budget, fp32=not args.no_fp32,
                         regimes=args.workload == "maze201" and not args.no_regimes)
    if args.workload == "sudoku9":
        line["metric"] = "cell-updates/sec on 1 MI355X (9x9 K=128 D=256) + % of roofline"
        if not args.no_configs and not args.depth:
            line["configs"] = configs_block()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
