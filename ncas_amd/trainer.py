"""The training recipe around the HIP engine: a counterpart of the reference's `train_fast`
(reference src/nca/engine/train.py:87-386) for the cells and tasks of this engine.

Every iteration: draw a batch from the replay pool (fresh boards at `seed_ratio`), perturb it
(target swap, damage discs, then the clamp; optionally the public code's batch noise), draw a
chunk start and the per-step seeds from the run's numpy generator, run
`Engine.train_iteration` (step noise inside the rollout when `train.noise` is active), and in its
update callback step AdamW when the gradient norm is finite, advance the learning-rate schedule
(linear warm-up, then constant or cosine) and the exponential moving average of the weights;
then write the rollout's final states back to the pool. Checkpoints hold the model, the EMA, the
optimiser, the schedule, the pool, both random generators and the step, so a run interrupted at a
checkpoint resumes exactly (bit for bit: every kernel of the path sums in a fixed order).

Files of a run directory, like the reference's: `run.json` (config, seed, parameter count, model
config, engine), `log.jsonl` (loss, grad norm, lr, batch accuracy, pool age, iteration seconds,
peak memory; evaluations), `checkpoint.pt`, `final.pt` (the EMA weights and the model config)
and `summary.json`. Checkpoints are read back with `weights_only=True`.

Config sections: `task` ({name, args, train: {n, size, seed}, val: {n, size, seed}}), `model`
({preset, overrides}), `train` (the keys of `DEFAULTS`), `engine` (`train.EngineConfig`).
"""

from __future__ import annotations

import copy
import json
import math
import time
from pathlib import Path

import numpy as np
import torch

from . import _lib
from .model import NCA, NCAConfig, build_model
from .rng import step_seeds
from .rollout import RolloutConfig, rollout
from .tasks import get_task
from .train import Engine, EngineConfig, ReplayPool, loss_weights

# the reference's training defaults (reference src/nca/train.py:44-87), for the keys this
# trainer implements
DEFAULTS = dict(
    steps=5000, batch_size=64, pool_mult=4, seed_ratio=0.25, rollout=100, chunk=100,
    loss_window="all", loss="mse", lr=4e-4, schedule="constant", warmup_ratio=0.0,
    init_lr_ratio=None, weight_decay=0.0, betas=(0.9, 0.999), grad_clip=1.0, ema=0.999,
    ema_warmup=True, noise=dict(p_t=0.1, p_s=0.2, sigma=0.15),
    damage=dict(p=0.1, n=1, r_min=0.1, r_max=0.4, fill=0.0, geometry="ours"),
    swap=dict(p=0.1), swap_source="fresh", batch_noise=None, augment=True, asynchronous=True,
    replay=True, perturb=True, log_every=50, eval_every=500, checkpoint_every=500, amp=False,
    eval=dict(n=256, depth=None, k=1),
)
BATCH_NOISE = dict(p=0.1, ps=0.2, sigma=0.15)


def resolve_train_cfg(cfg: dict) -> dict:
    """The `train` section merged into `DEFAULTS`, sub-dicts key by key (reference
    src/nca/train.py:111-134)."""
    given = cfg.get("train") or {}
    unknown = set(given) - set(DEFAULTS)
    if unknown:
        raise ValueError(f"train options not implemented by this trainer: {sorted(unknown)}")
    tr = {**DEFAULTS, **given}
    for k in ("noise", "damage", "swap", "eval"):
        tr[k] = {**DEFAULTS[k], **(given.get(k) or {})}
    if tr["batch_noise"] is not None:
        tr["batch_noise"] = {**BATCH_NOISE, **tr["batch_noise"]}
    if tr["swap_source"] not in ("fresh", "pool"):
        raise ValueError("train.swap_source must be fresh or pool")
    if tr["damage"]["geometry"] not in ("ours", "official"):
        raise ValueError("train.damage.geometry must be ours or official")
    if tr["schedule"] not in ("constant", "cosine"):
        raise ValueError("train.schedule must be constant or cosine")
    return tr


def lr_at(step: int, total: int, tr: dict) -> float:
    """Learning-rate multiplier of iteration `step` of `total` (reference src/nca/train.py:
    151-170): a linear warm-up over warmup_ratio * total iterations, from 1 / warm (or from
    init_lr_ratio), then constant or a cosine decay to cosine_floor."""
    warm = int(tr["warmup_ratio"] * total)
    if step < warm:
        r0 = tr.get("init_lr_ratio")
        return (step + 1) / warm if r0 is None else r0 + (1 - r0) * step / warm
    if tr["schedule"] == "constant":
        return 1.0
    frac = (step - warm) / max(1, total - warm)
    floor = tr.get("cosine_floor", 0.0)
    return floor + (1 - floor) * 0.5 * (1 + math.cos(math.pi * frac))


def ema_decay(tr: dict, step: int) -> float:
    """EMA decay of iteration `step` (reference src/nca/train.py:210-216): with `ema_warmup`,
    min(ema, (1 + t) / (10 + t))."""
    return min(tr["ema"], (1 + step) / (10 + step)) if tr["ema_warmup"] else tr["ema"]


# ------------------------------------------------------------------------------ perturbations
def damage_masks(B: int, H: int, W: int, n: int, r_min: float, r_max: float,
                 rng: np.random.Generator, hit: np.ndarray, geometry: str = "ours") -> np.ndarray:
    """(B, H, W) bool union of `n` random discs on each board with `hit` (reference
    src/nca/perturb.py:43-83). "ours": centres anywhere on the grid, radius r ~ U(r_min, r_max)
    times min(H, W), closed discs; "official": coordinates in [-1, 1], centres in
    [-0.5, 0.5]^2, radius in those units, open discs."""
    out = np.zeros((B, H, W), dtype=bool)
    if geometry == "official":
        ys = np.linspace(-1.0, 1.0, H)[:, None]
        xs = np.linspace(-1.0, 1.0, W)[None, :]
    else:
        ys = np.arange(H)[:, None].astype(np.float64)
        xs = np.arange(W)[None, :].astype(np.float64)
    for b in np.nonzero(hit)[0]:
        for _ in range(n):
            if geometry == "official":
                cy, cx = rng.uniform(-0.5, 0.5, size=2)
                r = rng.uniform(r_min, r_max)
                out[b] |= (ys - cy) ** 2 + (xs - cx) ** 2 < r * r
            else:
                cy, cx = rng.uniform(0, H), rng.uniform(0, W)
                r = rng.uniform(r_min, r_max) * min(H, W)
                out[b] |= (ys - cy) ** 2 + (xs - cx) ** 2 <= r * r
    return out


def perturb_batch(model, pool: ReplayPool, batch: dict, tr: dict, rng: np.random.Generator,
                  gen_dev: torch.Generator) -> None:
    """The pre-rollout perturbations, in place (reference src/nca/train.py:219-252): target
    swap (fresh boards or other pool entries), damage (the state set to `fill` inside random
    discs of a fraction `p` of the boards), the clamp, and the optional batch noise."""
    B = batch["x"].shape[0]
    which = np.nonzero(rng.random(B) < tr["swap"]["p"])[0]
    if tr["swap_source"] == "pool":
        pool.swap_from_pool(batch, which)
    else:
        pool.replace_boards(batch, which)
    d = tr["damage"]
    hit = rng.random(B) < d["p"]
    if hit.any():
        _, _, H, W = batch["x"].shape
        m = damage_masks(B, H, W, d["n"], d["r_min"], d["r_max"], rng, hit, d["geometry"])
        batch["x"] = batch["x"].masked_fill(_lib.upload(m, pool.device)[:, None], d["fill"])
    batch["x"] = model.apply_clamp(batch["x"], batch["given4"], batch["clamp"])
    bn = tr["batch_noise"]
    if bn is not None:
        x = batch["x"]
        Bn, C, H, W = x.shape
        dev = x.device
        boards = torch.rand((Bn, 1, 1, 1), generator=gen_dev, device=dev) < bn["p"]
        cells = torch.rand((Bn, 1, H, W), generator=gen_dev, device=dev) < bn["ps"]
        noise = torch.randn(x.shape, generator=gen_dev, device=dev) * bn["sigma"]
        keep = boards & cells
        in_ch = torch.zeros((1, C, 1, 1), dtype=torch.bool, device=dev)
        in_ch[:, model.cfg.in_slice] = True
        keep = keep & ~(batch["given4"] & in_ch)
        batch["x"] = model.apply_clamp(x + noise * keep.to(x.dtype), batch["given4"],
                                       batch["clamp"])


# ------------------------------------------------------------------------------ run pieces
def build_task_and_data(tcfg: dict):
    """(task, train boards, validation boards or None) from the task section; boards come from
    the task's seeded generator (`task.load` caches them when a data root is given)."""
    task = get_task(tcfg["name"], **tcfg.get("args", {}))
    tr = {"seed": 0, **tcfg["train"]}
    train = task.generate(tr["n"], tr["size"], tr["seed"])
    val = None
    if tcfg.get("val"):
        va = {"seed": 1, **tcfg["val"]}
        val = task.generate(va["n"], va["size"], va["seed"])
    return task, train, val


def build_run_model(cfg: dict) -> NCA:
    mcfg = cfg.get("model", {})
    model = build_model(mcfg.get("preset"), **mcfg.get("overrides", {}))
    if not resolve_train_cfg(cfg)["asynchronous"]:
        model.cfg.fire_rate = 1.0
    return model


def load_model(path) -> tuple[NCA, dict]:
    """(model, checkpoint) of a `final.pt`, read with weights_only=True."""
    ck = torch.load(path, map_location="cpu", weights_only=True)
    model = NCA(NCAConfig.from_dict(ck["model_config"]))
    model.load_state_dict(ck["model"])
    return model, ck


@torch.no_grad()
def evaluate(model, task, boards, ev: dict, rollout_steps: int, seed: int) -> dict:
    """Quick validation: one rollout of ev["n"] boards for ev["depth"] (default: the training
    rollout) steps with ev["k"] trials, first trial's exact rate and cell accuracy."""
    n = min(ev["n"], len(boards))
    sub = boards.subset(np.arange(n))
    rc = RolloutConfig(depth=ev["depth"] or rollout_steps, k=ev["k"])
    res = rollout(model, task, sub, rc, seed=seed)
    m = task.metrics(res.pred[:, 0], sub)
    return {"val_exact": float(m["exact"].mean()), "val_cell_acc": float(m["cell_acc"].mean())}


def _rng_state(rng: np.random.Generator) -> dict:
    st = rng.bit_generator.state
    return {"bit_generator": st["bit_generator"], "state": str(st["state"]["state"]),
            "inc": str(st["state"]["inc"]), "has_uint32": st["has_uint32"],
            "uinteger": st["uinteger"]}


def _set_rng_state(rng: np.random.Generator, d: dict) -> None:
    rng.bit_generator.state = {"bit_generator": d["bit_generator"],
                               "state": {"state": int(d["state"]), "inc": int(d["inc"])},
                               "has_uint32": d["has_uint32"], "uinteger": d["uinteger"]}


def _json_line(rec: dict) -> str:
    return json.dumps(rec) + "\n"


def train_fast(cfg: dict, out_dir, seed: int = 0, device=None, resume: bool = True,
               quiet: bool = False, stop_at_step: int | None = None) -> dict:
    """Train one model on the HIP engine; resumable from `out_dir/checkpoint.pt`. With
    `stop_at_step` the run stops there (the learning-rate horizon stays `train.steps`) and marks
    its summary `training_complete: false`. Returns the last evaluation."""
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    tr = resolve_train_cfg(cfg)
    end_step = tr["steps"] if stop_at_step is None else int(stop_at_step)
    if not 0 < end_step <= tr["steps"]:
        raise ValueError("stop_at_step must be in 1..train.steps")
    dev = torch.device(device or "cuda")
    if dev.type != "cuda":
        raise ValueError("the HIP engine trains on the GPU")
    torch.cuda.reset_peak_memory_stats(dev)
    torch.manual_seed(seed)
    rng = np.random.default_rng(seed)
    gen_dev = torch.Generator(device=dev)
    gen_dev.manual_seed(seed)

    task, train_boards, val_boards = build_task_and_data(cfg["task"])
    model = build_run_model(cfg).to(dev)
    ema = copy.deepcopy(model).eval()
    for p in ema.parameters():
        p.requires_grad_(False)
    opt = torch.optim.AdamW(model.parameters(), lr=tr["lr"], weight_decay=tr["weight_decay"],
                            betas=tuple(tr["betas"]))
    sched = torch.optim.lr_scheduler.LambdaLR(opt, lambda s: lr_at(s, tr["steps"], tr))
    pool_size = (tr["pool_mult"] if tr["replay"] else 1) * tr["batch_size"]
    seed_ratio = tr["seed_ratio"] if tr["replay"] else 1.0
    pool = ReplayPool(model, train_boards, pool_size, rng, gen_dev, task=task,
                      augment=tr["augment"])
    ecfg = EngineConfig.from_dict(cfg.get("engine"))
    engine = Engine(model, ecfg, tr, dev)
    N, Nc = engine.N, engine.Nc
    weights = loss_weights(tr["loss_window"], Nc, dev)

    step0 = 0
    ckpt_path, log_path = out / "checkpoint.pt", out / "log.jsonl"
    if resume and ckpt_path.exists():
        ck = torch.load(ckpt_path, map_location=dev, weights_only=True)
        model.load_state_dict(ck["model"])
        ema.load_state_dict(ck["ema"])
        opt.load_state_dict(ck["opt"])
        sched.load_state_dict(ck["sched"])
        pool.load_state_dict(ck["pool"])
        _set_rng_state(rng, ck["rng"])
        gen_dev.set_state(ck["gen_dev"].cpu())
        step0 = int(ck["step"])
        if step0 >= end_step:
            raise ValueError("stop_at_step must be after the resumed checkpoint")
        if not quiet:
            print(f"resumed from step {step0}")
    n_params = sum(p.numel() for p in model.parameters())
    (out / "run.json").write_text(json.dumps({
        "config": cfg, "seed": seed, "params": n_params, "model_config": model.cfg.to_dict(),
        "engine": engine.to_dict(), "device": f"{dev} ({torch.cuda.get_device_name(dev)})",
        "torch": torch.__version__,
    }, indent=1, default=str))

    n_skipped = 0
    last_eval: dict = {}
    t_start = window_t0 = time.time()
    window_n = 0
    model.train()
    for step in range(step0, end_step):
        idx, batch = pool.sample(tr["batch_size"], seed_ratio)
        if tr["perturb"]:
            perturb_batch(model, pool, batch, tr, rng, gen_dev)
        c0 = int(rng.integers(0, N - Nc + 1))
        seeds = step_seeds(rng, N)

        def apply_update(gn, step=step):
            nonlocal n_skipped
            if bool(torch.isfinite(gn)):  # one host wait per iteration, like the reference
                opt.step()
            else:
                n_skipped += 1
            opt.zero_grad(set_to_none=True)
            sched.step()
            d = ema_decay(tr, step)
            with torch.no_grad():
                for pe, pm in zip(ema.parameters(), model.parameters()):
                    pe.mul_(d).add_(pm.detach(), alpha=1 - d)

        x, loss, gn = engine.train_iteration(batch, seeds, c0, weights, tr["grad_clip"],
                                             apply_update)
        batch["x"] = x.detach()
        pool.write_back(idx, batch)
        window_n += 1
        if (step + 1) % tr["log_every"] == 0 or step == step0:
            with torch.no_grad():
                from .rollout import decode_tokens

                dec, _ = decode_tokens(model, x, batch["given4"][:, 0], batch["inputs"],
                                       task.fill_given)
                lm = batch.get("loss_mask")
                scored = ~batch["given4"][:, 0] if lm is None else lm > 0
                right = ((dec == batch["targets"]) & scored).sum(dim=(1, 2)).float()
                n_sc = scored.sum(dim=(1, 2)).clamp_min(1)
                stats = torch.stack([(right / n_sc).mean(), (right == n_sc).float().mean(),
                                     batch["age"].float().mean(), loss, gn]).tolist()
            now = time.time()
            rec = dict(step=step + 1, loss=stats[3], grad_norm=stats[4],
                       lr=sched.get_last_lr()[0], batch_cell_acc=stats[0], batch_exact=stats[1],
                       mean_age=stats[2], skipped_steps=n_skipped, elapsed=now - t_start,
                       iter_seconds=(now - window_t0) / max(1, window_n),
                       peak_mem_gb=torch.cuda.max_memory_allocated(dev) / 2**30)
            window_t0, window_n = now, 0
            with open(log_path, "a") as f:
                f.write(_json_line(rec))
            if not quiet:
                print(f"step {step + 1}/{tr['steps']} loss {rec['loss']:.4f} "
                      f"cell {rec['batch_cell_acc']:.3f} exact {rec['batch_exact']:.3f} "
                      f"{rec['iter_seconds']:.3f} s/it")
        if val_boards is not None and ((step + 1) % tr["eval_every"] == 0 or step + 1 == end_step):
            last_eval = evaluate(ema, task, val_boards, tr["eval"], N, seed)
            last_eval["step"] = step + 1
            with open(log_path, "a") as f:
                f.write(_json_line({"eval": last_eval}))
            model.train()
            window_t0 = time.time()
        if (step + 1) % tr["checkpoint_every"] == 0 or step + 1 == end_step:
            torch.save(dict(model=model.state_dict(), ema=ema.state_dict(),
                            opt=opt.state_dict(), sched=sched.state_dict(),
                            pool={k: v for k, v in pool.state_dict().items() if v is not None},
                            rng=_rng_state(rng), gen_dev=gen_dev.get_state(), step=step + 1),
                       ckpt_path)

    final = dict(model=ema.state_dict(), model_config=model.cfg.to_dict(), seed=seed,
                 step=end_step)
    if end_step < tr["steps"]:
        final.update(target_steps=tr["steps"], training_complete=False)
    torch.save(final, out / "final.pt")
    summary = {"final_eval": last_eval, "train_seconds": time.time() - t_start,
               "steps": end_step, "start_step": step0, "params": n_params,
               "skipped_steps": n_skipped, "engine": engine.to_dict(),
               "training_complete": end_step == tr["steps"],
               "peak_mem_gb": torch.cuda.max_memory_allocated(dev) / 2**30}
    if end_step < tr["steps"]:
        summary["target_steps"] = tr["steps"]
    (out / "summary.json").write_text(json.dumps(summary, indent=1))
    return last_eval
