"""The fused training update and the fused damage + clamp pass on the GPU, through the C ABI.

* `nca_adamw_ema` (optim.FusedUpdate) against torch's clip_grad_norm_ + AdamW + EMA loop +
  zero_grad (the reference's update, src/nca/engine/train.py:262-273) over several iterations,
  with and without clipping and weight decay; a non-finite gradient skips AdamW (its step count
  too) but not the EMA; its state_dict loads into torch.optim.AdamW, which then continues the
  same way.
* `nca_damage_clamp` (perturb.damage_clamp) equals the oracle's rasterised discs and clamp bit for
  bit, in both geometries, including discs whose edge falls on a grid coordinate.
* train_fast's final.pt carries the reference's keys (config included) and load_model returns
  (model, config); running a finished run again returns its last evaluation without training.
"""

from __future__ import annotations

import copy
import json

import numpy as np
import pytest
import torch

from ncas_amd import perturb
from ncas_amd.model import build_model
from ncas_amd.optim import FusedUpdate
from ncas_amd.trainer import load_model, train_fast
from oracle import perturb as OP

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _models(seed=0):
    torch.manual_seed(seed)
    m = build_model("maze_hard_c32")
    with torch.no_grad():
        for p in m.parameters():
            p.normal_(0, 0.05)
    m = m.to(DEV)
    return m, copy.deepcopy(m), copy.deepcopy(m), copy.deepcopy(m)


def _grads(params, gen, scale):
    return [torch.randn(p.shape, generator=gen, device=DEV) * scale for p in params]


@pytest.mark.parametrize("clip,wd,scale", [(None, 0.0, 1e-3), (1.0, 1e-4, 1e-1), (0.5, 1e-2, 1.0)])
def test_fused_update_matches_torch(clip, wd, scale):
    m, ema, mt, ema_t = _models()
    lr, betas = 5e-4, (0.9, 0.999)
    fu = FusedUpdate(m, ema, lr, betas, weight_decay=wd)
    opt = torch.optim.AdamW(mt.parameters(), lr=lr, betas=betas, weight_decay=wd)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(1)
    for it in range(12):
        gs = _grads(list(m.parameters()), gen, scale)
        lr_it = lr * (it + 1) / 12
        d = min(0.999, (1 + it) / (10 + it))
        for p, g in zip(m.parameters(), gs):
            p.grad.add_(g)
        gn = fu.step(lr_it, d, clip).clone()
        for p, g in zip(mt.parameters(), gs):
            p.grad = g.clone()
        gn_t = (torch.nn.utils.clip_grad_norm_(mt.parameters(), clip) if clip is not None else
                torch.linalg.vector_norm(torch.stack([g.norm() for g in gs])))
        for grp in opt.param_groups:
            grp["lr"] = lr_it
        opt.step()
        opt.zero_grad(set_to_none=True)
        with torch.no_grad():
            for pe, pm in zip(ema_t.parameters(), mt.parameters()):
                pe.mul_(d).add_(pm, alpha=1 - d)
        assert abs(gn.item() - gn_t.item()) <= 1e-5 * gn_t.item()
        for a, b in zip(list(m.parameters()) + list(ema.parameters()),
                        list(mt.parameters()) + list(ema_t.parameters())):
            assert torch.allclose(a, b, rtol=2e-6, atol=1e-8), (it, (a - b).abs().max().item())
        assert all(not p.grad.any() for p in m.parameters())
    assert fu.counters.tolist() == [12, 0]


def test_nonfinite_gradient_skips_adamw_not_the_ema():
    m, ema, _, _ = _models(1)
    fu = FusedUpdate(m, ema, 1e-3)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(2)
    for p, g in zip(m.parameters(), _grads(list(m.parameters()), gen, 1e-2)):
        p.grad.add_(g)
    fu.step(1e-3, 0.5, 1.0)
    before = [p.detach().clone() for p in m.parameters()]
    moments = (fu.exp_avg.clone(), fu.exp_avg_sq.clone())
    ema_before = [p.detach().clone() for p in ema.parameters()]
    grads = _grads(list(m.parameters()), gen, 1e-2)
    grads[1][0, 0] = float("inf")
    for p, g in zip(m.parameters(), grads):
        p.grad.add_(g)
    gn = fu.step(1e-3, 0.5, 1.0)
    assert not torch.isfinite(gn).item()
    assert fu.counters.tolist() == [1, 1]
    for a, b in zip(m.parameters(), before):
        assert torch.equal(a, b)
    assert torch.equal(fu.exp_avg, moments[0]) and torch.equal(fu.exp_avg_sq, moments[1])
    for e, e0, p in zip(ema.parameters(), ema_before, m.parameters()):
        assert torch.allclose(e, 0.5 * e0 + 0.5 * p, rtol=1e-6, atol=0)
    assert all(not p.grad.any() for p in m.parameters())
    # the packed-weight cache sees the parameters' new values
    assert m.update.fc1.weight._version > 0


def test_state_dict_continues_in_torch_adamw():
    m, ema, mt, _ = _models(2)
    fu = FusedUpdate(m, ema, 1e-3, weight_decay=1e-4)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(3)
    for _ in range(3):
        for p, g in zip(m.parameters(), _grads(list(m.parameters()), gen, 1e-2)):
            p.grad.add_(g)
        fu.step(1e-3, 0.9, None)
    sd = fu.state_dict()
    with torch.no_grad():
        for a, b in zip(mt.parameters(), m.parameters()):
            a.copy_(b)
    opt = torch.optim.AdamW(mt.parameters(), lr=1e-3, weight_decay=1e-4)
    opt.load_state_dict({k: v for k, v in sd.items() if k != "skipped"})
    gs = _grads(list(m.parameters()), gen, 1e-2)
    for p, g in zip(m.parameters(), gs):
        p.grad.add_(g)
    fu.step(1e-3, 0.9, None)
    for p, g in zip(mt.parameters(), gs):
        p.grad = g.clone()
    opt.step()
    for a, b in zip(m.parameters(), mt.parameters()):
        assert torch.allclose(a, b, rtol=2e-6, atol=1e-8)
    # and back: a fresh fused update restored from the state continues identically
    m2, ema2, _, _ = _models(2)
    with torch.no_grad():
        for a, b in zip(list(m2.parameters()) + list(ema2.parameters()),
                        list(m.parameters()) + list(ema.parameters())):
            a.copy_(b)
    fu2 = FusedUpdate(m2, ema2, 1e-3, weight_decay=1e-4)
    fu2.load_state_dict(fu.state_dict())
    gs = _grads(list(m.parameters()), gen, 1e-2)
    for fx, mm in ((fu, m), (fu2, m2)):
        for p, g in zip(mm.parameters(), gs):
            p.grad.add_(g)
        fx.step(1e-3, 0.9, 1.0)
    for a, b in zip(list(m.parameters()) + list(ema.parameters()),
                    list(m2.parameters()) + list(ema2.parameters())):
        assert torch.equal(a, b)


@pytest.mark.parametrize("geometry", ["ours", "official"])
def test_damage_clamp_matches_oracle(geometry):
    model = build_model("maze_hard_c32").to(DEV)
    rng = np.random.default_rng(4)
    B, C, H, W = 12, 32, 11, 17
    hit = rng.random(B) < 0.6
    discs = perturb.draw_discs(rng, hit, H, W, 2, 0.1, 0.4, geometry)
    if geometry == "official":  # an edge on grid coordinates: linspace rounding decides
        discs = np.concatenate([discs, [[B - 1, 0.0, 0.0, 0.2 ** 2]]])
    else:
        discs = np.concatenate([discs, [[B - 1, 5.0, 8.0, 9.0]]])
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    given = rng.random((B, H, W)) < 0.3
    sl = model.cfg.in_slice
    clamp = rng.standard_normal((B, sl.stop - sl.start, H, W)).astype(np.float32)
    xd = torch.from_numpy(x).to(DEV)
    perturb.damage_clamp(model, xd, torch.from_numpy(given).to(DEV)[:, None],
                         torch.from_numpy(clamp).to(DEV), discs, 0.25, geometry)
    masks = OP.disc_masks(discs, B, H, W, geometry)
    want = OP.damage_clamp(x, masks, 0.25, given, clamp, sl)
    assert masks.any() and np.array_equal(xd.cpu().numpy(), want)


def _cfg(steps):
    return {
        "task": {"name": "maze", "train": {"n": 32, "size": 9, "seed": 0},
                 "val": {"n": 4, "size": 9, "seed": 1}},
        "model": {"preset": "maze_hard_c32"},
        "train": dict(steps=steps, batch_size=4, pool_mult=2, rollout=4, chunk=3, loss="ce",
                      lr=5e-4, log_every=1, eval_every=steps, checkpoint_every=steps,
                      noise={"sigma": 0.0}, eval={"n": 4, "depth": 4, "k": 2}),
    }


def test_final_checkpoint_keys_and_rerun(tmp_path):
    cfg = _cfg(3)
    res = train_fast(cfg, tmp_path, seed=0, quiet=True)
    ck = torch.load(tmp_path / "final.pt", weights_only=True)
    assert set(ck) == {"model", "model_config", "config", "seed", "step"}
    model, conf = load_model(tmp_path / "final.pt")
    assert conf == cfg and not model.training
    assert {"val_exact", "val_valid", "val_optimal", "val_cell_acc", "val_conf"} <= set(res)
    log = (tmp_path / "log.jsonl").read_text()
    again = train_fast(cfg, tmp_path, seed=0, quiet=True)
    assert again == json.loads(json.dumps(res))
    assert (tmp_path / "log.jsonl").read_text() == log  # nothing trained again
