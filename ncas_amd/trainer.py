"""The training recipe around the HIP engine: a counterpart of the reference's `train_fast`
(reference src/nca/engine/train.py:87-386) for the cells and tasks of this engine.

The run is an object (`_Run`) with one method per phase: restore, iterate, log, checkpoint,
finish. An iteration samples a batch from the replay pool (fresh boards at `seed_ratio`),
perturbs it (target swaps; the damage discs and the clamp in one GPU pass; optionally the
public code's batch noise), draws a chunk start and the per-step seeds from the run's numpy
generator, and runs `Engine.train_iteration` (step noise inside the rollout when `train.noise`
is active) whose update callback is one launch of the fused update (`optim.FusedUpdate`,
`nca_adamw_ema`): gradient norm, clipping, the finiteness test, AdamW with this iteration's
learning rate (linear warm-up, then constant or cosine), the EMA and the zeroing of the
gradient, with the skip decision and the step counts kept on the device, so nothing waits for
the host. The final states go back to the pool. Checkpoints hold the model, the EMA, the
update's moments and counters, the schedule's position, the pool, both random generators and
the step; a run interrupted at a checkpoint resumes bit for bit (every kernel of the path,
the update's norm included, sums in a fixed order).

Files of a run directory, like the reference's: `run.json` (config, seed, parameter count, model
config, engine), `log.jsonl` (loss, grad norm, lr, batch accuracy, pool age, iteration seconds,
peak memory; evaluations), `checkpoint.pt`, `final.pt` (the EMA weights, the model config and
the run config) and `summary.json`. Checkpoints are read back with `weights_only=True`.

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

from . import perturb
from .model import NCA, NCAConfig, build_model
from .optim import FusedUpdate
from .rng import step_seeds
from .rollout import RolloutConfig, decode_tokens, rollout
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
def perturb_batch(model, pool: ReplayPool, batch: dict, tr: dict, rng: np.random.Generator,
                  gen_dev: torch.Generator) -> None:
    """The pre-rollout perturbations, in place (reference src/nca/train.py:219-252): target
    swaps (fresh boards or other pool entries), then the damage discs and the clamp in one pass
    on the GPU (`perturb.damage_clamp`), then the optional batch noise. The host draws only the
    swap rows and the discs' geometry from the run's generator."""
    B, _, H, W = batch["x"].shape
    rows = perturb.swap_rows(rng, B, tr["swap"]["p"])
    (pool.swap_from_pool if tr["swap_source"] == "pool" else pool.replace_boards)(batch, rows)
    d = tr["damage"]
    hit = rng.random(B) < d["p"]
    discs = perturb.draw_discs(rng, hit, H, W, d["n"], d["r_min"], d["r_max"], d["geometry"])
    batch["x"] = perturb.damage_clamp(model, batch["x"].float().contiguous(), batch["given4"],
                                      batch["clamp"], discs, d["fill"], d["geometry"])
    if tr["batch_noise"] is not None:
        perturb.batch_noise(model, batch, tr["batch_noise"], gen_dev)


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


def load_model(path, device=None) -> tuple[NCA, dict]:
    """(model with the EMA weights, run config) of a `final.pt` (reference src/nca/train.py:
    694-701), read with weights_only=True."""
    ck = torch.load(path, map_location="cpu", weights_only=True)
    model = NCA(NCAConfig.from_dict(ck["model_config"]))
    model.load_state_dict(ck["model"])
    if device is not None:
        model = model.to(device)
    return model.eval(), ck.get("config")


@torch.no_grad()
def evaluate(model, task, boards, ev: dict, rollout_steps: int, seed: int) -> dict:
    """Quick validation (reference src/nca/train.py:674-691): one rollout of ev["n"] boards for
    ev["depth"] (default: the training rollout) steps with ev["k"] trials; the mean of every task
    metric over the trials, trial 0's cell accuracy and the mean board confidence."""
    n = min(ev["n"] or len(boards), len(boards))
    sub = boards.subset(np.arange(n))
    res = rollout(model, task, sub, RolloutConfig(depth=ev["depth"] or rollout_steps, k=ev["k"]),
                  seed=seed)
    out = {f"val_{k}": float(np.mean(v)) for k, v in res.metrics.items()}
    out["val_cell_acc"] = float(np.mean(res.metrics["cell_acc"][:, 0]))
    out["val_conf"] = float(res.conf.mean())
    return out


def _rng_state(rng: np.random.Generator) -> dict:
    st = rng.bit_generator.state
    return {"bit_generator": st["bit_generator"], "state": str(st["state"]["state"]),
            "inc": str(st["state"]["inc"]), "has_uint32": st["has_uint32"],
            "uinteger": st["uinteger"]}


def _set_rng_state(rng: np.random.Generator, d: dict) -> None:
    rng.bit_generator.state = {"bit_generator": d["bit_generator"],
                               "state": {"state": int(d["state"]), "inc": int(d["inc"])},
                               "has_uint32": d["has_uint32"], "uinteger": d["uinteger"]}


def _append_json(path: Path, rec: dict) -> None:
    with open(path, "a") as f:
        f.write(json.dumps(rec) + "\n")


class _Run:
    """One training run's state and its phases. Everything that a checkpoint must restore for an
    exact resume lives here: the model and its EMA (views of the fused update's flat buffers),
    the update's moments and counters, the replay pool, the numpy generator (swaps, damage,
    chunk starts, step seeds) and the device generator (fresh states, batch noise)."""

    def __init__(self, cfg: dict, out: Path, seed: int, dev: torch.device, quiet: bool):
        self.cfg, self.out, self.seed, self.dev, self.quiet = cfg, out, seed, dev, quiet
        self.tr = tr = resolve_train_cfg(cfg)
        torch.manual_seed(seed)
        self.rng = np.random.default_rng(seed)
        self.gen_dev = torch.Generator(device=dev)
        self.gen_dev.manual_seed(seed)
        self.task, self.train_boards, self.val_boards = build_task_and_data(cfg["task"])
        self.model = build_run_model(cfg).to(dev)
        self.ema = copy.deepcopy(self.model).eval()
        for p in self.ema.parameters():
            p.requires_grad_(False)
        self.update = FusedUpdate(self.model, self.ema, tr["lr"], tr["betas"],
                                  weight_decay=tr["weight_decay"])
        mult = tr["pool_mult"] if tr["replay"] else 1
        self.seed_ratio = tr["seed_ratio"] if tr["replay"] else 1.0
        self.pool = ReplayPool(self.model, self.train_boards, mult * tr["batch_size"], self.rng,
                               self.gen_dev, task=self.task, augment=tr["augment"])
        self.engine = Engine(self.model, EngineConfig.from_dict(cfg.get("engine")), tr, dev)
        self.weights = loss_weights(tr["loss_window"], self.engine.Nc, dev)
        self.n_params = sum(p.numel() for p in self.model.parameters())
        self.step0 = 0
        self.last_eval: dict = {}

    @property
    def ckpt_path(self) -> Path:
        return self.out / "checkpoint.pt"

    # ------------------------------------------------------------------ checkpoints
    def save_checkpoint(self, step: int) -> None:
        torch.save(dict(model=self.model.state_dict(), ema=self.ema.state_dict(),
                        opt=self.update.state_dict(), sched={"last_epoch": step},
                        pool={k: v for k, v in self.pool.state_dict().items() if v is not None},
                        rng=_rng_state(self.rng), gen_dev=self.gen_dev.get_state(), step=step),
                   self.ckpt_path)

    def restore(self) -> int:
        """Load the checkpoint into every piece of state; returns its step."""
        ck = torch.load(self.ckpt_path, map_location=self.dev, weights_only=True)
        self.model.load_state_dict(ck["model"])
        self.ema.load_state_dict(ck["ema"])
        self.update.load_state_dict(ck["opt"])
        self.pool.load_state_dict(ck["pool"])
        _set_rng_state(self.rng, ck["rng"])
        self.gen_dev.set_state(ck["gen_dev"].cpu())
        self.step0 = int(ck["step"])
        return self.step0

    # ------------------------------------------------------------------ one iteration
    def iterate(self, step: int):
        """Sample and perturb a batch, run the engine's iteration with the fused update, write
        the final states back. Returns (batch, final state, loss)."""
        tr, eng = self.tr, self.engine
        idx, batch = self.pool.sample(tr["batch_size"], self.seed_ratio)
        if tr["perturb"]:
            perturb_batch(self.model, self.pool, batch, tr, self.rng, self.gen_dev)
        c0 = int(self.rng.integers(0, eng.N - eng.Nc + 1))
        seeds = step_seeds(self.rng, eng.N)
        lr = tr["lr"] * lr_at(step, tr["steps"], tr)
        update = lambda _gn: self.update.step(lr, ema_decay(tr, step), tr["grad_clip"])  # noqa: E731
        x, loss, _ = eng.train_iteration(batch, seeds, c0, self.weights, None, update)
        batch["x"] = x.detach()
        self.pool.write_back(idx, batch)
        return batch, x, loss

    def log_record(self, step: int, batch: dict, x, loss, t0: float, t_window: float,
                   n_window: int) -> dict:
        """The log line of iteration `step` (one host copy of the device statistics)."""
        with torch.no_grad():
            dec, _ = decode_tokens(self.model, x, batch["given4"][:, 0], batch["inputs"],
                                   self.task.fill_given)
            lm = batch.get("loss_mask")
            scored = ~batch["given4"][:, 0] if lm is None else lm > 0
            right = ((dec == batch["targets"]) & scored).sum(dim=(1, 2)).float()
            n_sc = scored.sum(dim=(1, 2)).clamp_min(1)
            cell, exact, age, lo, gn, skipped = torch.stack([
                (right / n_sc).mean(), (right == n_sc).float().mean(),
                batch["age"].float().mean(), loss.float(), self.update.grad_norm,
                self.update.skipped.float()]).tolist()
        now = time.time()
        tr = self.tr
        return dict(step=step + 1, loss=lo, grad_norm=gn,
                    lr=tr["lr"] * lr_at(step + 1, tr["steps"], tr), batch_cell_acc=cell,
                    batch_exact=exact, mean_age=age, skipped_steps=int(skipped),
                    elapsed=now - t0, iter_seconds=(now - t_window) / max(1, n_window),
                    peak_mem_gb=torch.cuda.max_memory_allocated(self.dev) / 2**30)

    # ------------------------------------------------------------------ files
    def write_run_json(self) -> None:
        (self.out / "run.json").write_text(json.dumps({
            "config": self.cfg, "seed": self.seed, "params": self.n_params,
            "model_config": self.model.cfg.to_dict(), "engine": self.engine.to_dict(),
            "device": f"{self.dev} ({torch.cuda.get_device_name(self.dev)})",
            "torch": torch.__version__, "update": "nca_adamw_ema",
        }, indent=1, default=str))

    def finish(self, end_step: int, seconds: float) -> dict:
        tr = self.tr
        final = dict(model=self.ema.state_dict(), model_config=self.model.cfg.to_dict(),
                     config=self.cfg, seed=self.seed, step=end_step)
        summary = {"final_eval": self.last_eval, "train_seconds": seconds, "steps": end_step,
                   "start_step": self.step0, "params": self.n_params,
                   "skipped_steps": int(self.update.skipped), "engine": self.engine.to_dict(),
                   "training_complete": end_step == tr["steps"],
                   "peak_mem_gb": torch.cuda.max_memory_allocated(self.dev) / 2**30}
        if end_step < tr["steps"]:
            final.update(target_steps=tr["steps"], training_complete=False)
            summary["target_steps"] = tr["steps"]
        torch.save(final, self.out / "final.pt")
        (self.out / "summary.json").write_text(json.dumps(summary, indent=1))
        return self.last_eval


def train_fast(cfg: dict, out_dir, seed: int = 0, device=None, resume: bool = True,
               quiet: bool = False, stop_at_step: int | None = None) -> dict:
    """Train one model on the HIP engine, resumable from `out_dir/checkpoint.pt` (the reference's
    `train_fast`, src/nca/engine/train.py:87-386, and its run files). With `stop_at_step` the run
    stops there (the learning-rate horizon stays `train.steps`) and marks its summary
    `training_complete: false`. A finished run is not trained again: its summary's last
    evaluation is returned. Returns the last evaluation."""
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
    run = _Run(cfg, out, seed, dev, quiet)
    if resume and run.ckpt_path.exists():
        step0 = run.restore()
        summary = out / "summary.json"
        if step0 >= tr["steps"] and summary.exists():
            return json.loads(summary.read_text()).get("final_eval", {})
        if step0 >= end_step:
            raise ValueError("stop_at_step must be after the resumed checkpoint")
        if not quiet:
            print(f"resumed from step {step0}")
    run.write_run_json()
    log_path = out / "log.jsonl"
    t0 = t_window = time.time()
    n_window = 0
    run.model.train()
    for step in range(run.step0, end_step):
        batch, x, loss = run.iterate(step)
        n_window += 1
        last = step + 1 == end_step
        if (step + 1) % tr["log_every"] == 0 or step == run.step0:
            rec = run.log_record(step, batch, x, loss, t0, t_window, n_window)
            t_window, n_window = time.time(), 0
            _append_json(log_path, rec)
            if not quiet:
                print(f"step {step + 1}/{tr['steps']} loss {rec['loss']:.4f} "
                      f"cell {rec['batch_cell_acc']:.3f} exact {rec['batch_exact']:.3f} "
                      f"{rec['iter_seconds']:.3f} s/it")
        if run.val_boards is not None and ((step + 1) % tr["eval_every"] == 0 or last):
            run.last_eval = {**evaluate(run.ema, run.task, run.val_boards, tr["eval"],
                                        run.engine.N, seed), "step": step + 1}
            _append_json(log_path, {"eval": run.last_eval})
            run.model.train()
            t_window = time.time()
        if (step + 1) % tr["checkpoint_every"] == 0 or last:
            run.save_checkpoint(step + 1)
    return run.finish(end_step, time.time() - t0)
