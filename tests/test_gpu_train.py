"""Training on the GPU through the C ABI: the differentiable step (`nca_step_backward`) and the
engine's train_iteration, against the fp64 autograd oracle.

* The step's vector-Jacobian product (state, clamp values, noise, every step parameter) within a
  relative norm error of 1e-4 (fp32) / 1e-3 (bf16: straight-through rounding points, with the
  gradients of dx, h and z rounded to bf16 like the reference's bf16 backward) of the oracle,
  for every cell (mlp and l2 heads), fire masks {Philox, 0, 1, 0.5} and noise; `make_step`
  under autograd gives the same gradients (reference tests/test_engine_ops.py:251-294).
* `Engine(model, cfg, train_cfg, device).train_iteration` equals its composition (prefix, chunk,
  suffix with global step keys); with `amp` the prefix and suffix run in fp32 (reference
  engine.py:285-292) and the chunk in bf16, each checked against the oracle; the step-by-step
  chunk equals the fused chunk; the MSE loss of an l2-head cell and step noise run through the
  step-by-step chunk and match the oracle.
"""

from __future__ import annotations

import copy
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, __file__.rsplit("/", 1)[0])
from cells import CELLS, boards_for, initial_state, make_model, oracle_cell  # noqa: E402

from ncas_amd.inference import rollout_steps  # noqa: E402
from ncas_amd.step import make_step, step_vjp  # noqa: E402
from ncas_amd.train import Engine, EngineConfig, bptt_chunk  # noqa: E402
from oracle import nca_oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
STEP_NAMES = ("kernels", "w1", "b1", "w2", "b2")
NAMES = STEP_NAMES + ("head_w", "head_b")
VJP_TOL = {"fp32": 1e-4, "bf16": 1e-3}


def _say(*a):
    print(*a, flush=True)


def _rel(a, b):
    a = a.detach().double().cpu().reshape(-1)
    b = b.detach().double().cpu().reshape(-1)
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _case(name, n_boards=2, k=3, sigma=0.15, seed=0):
    preset, size = CELLS[name]
    m = make_model(name, seed)
    b = boards_for(preset, n_boards, size, seed)
    x, g4, cl = initial_state(m, b, k=k, sigma=sigma, seed=seed)
    return m, copy.deepcopy(m).to(DEV), x, g4, cl, b


def oracle_step_vjp(m, x, g4, cl, fire, noise, cot, precision):
    """fp64 autograd of sum(step(x) * cot) through the oracle's step: grads of x, clamp, noise
    and the step parameters."""
    cell = oracle_cell(m)
    dt = torch.float64
    params = {k: getattr(cell, k).detach().to(dt).clone().requires_grad_(True) for k in STEP_NAMES}
    c = O.OracleCell(**{**cell.__dict__, **params})
    xx = x.detach().to(dt).clone().requires_grad_(True)
    cc = cl.detach().to(dt).clone().requires_grad_(True)
    nz = None if noise is None else noise.detach().to(dt).clone().requires_grad_(True)
    y = O.step(c, xx, g4, cc, fire.to(dt), precision, nz, dtype=dt, ste=True,
               grad_round=precision == "bf16")
    wrt = [xx, cc] + ([nz] if nz is not None else []) + [params[k] for k in STEP_NAMES]
    g = torch.autograd.grad((y * cot.to(dt)).sum(), wrt, allow_unused=True)
    g = [torch.zeros_like(w) if v is None else v for v, w in zip(g, wrt)]
    out = {"x": g[0], "clamp": g[1]}
    if nz is not None:
        out["noise"] = g[2]
    out.update(zip(STEP_NAMES, g[-len(STEP_NAMES):]))
    return out


def _grads(md) -> dict:
    """The model's accumulated .grad by C ABI name."""
    u = md.update
    g = {"kernels": md.perceive.weight.grad, "w1": u.fc1.weight.grad, "b1": u.fc1.bias.grad,
         "w2": u.fc2.weight.grad, "b2": u.fc2.bias.grad}
    if md.cfg.head == "mlp":
        g.update(head_w=md.head.weight.grad, head_b=md.head.bias.grad)
    return g


def _fires(B, H, W):
    return {
        "philox": O.fire_masks_np(3, 0, B, 0, H, W, 0.5),
        "zeros": torch.zeros(B, 1, H, W),
        "ones": torch.ones(B, 1, H, W),
        "half": torch.full((B, 1, H, W), 0.5),
    }


# ------------------------------------------------------------------------------ step VJP
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
@pytest.mark.parametrize("name", list(CELLS))
def test_step_vjp_matches_oracle(name, precision):
    _say("step vjp", name, precision)
    m, md, x, g4, cl, _ = _case(name)
    B, C, H, W = x.shape
    cot = torch.randn(x.shape, generator=torch.Generator().manual_seed(7))
    for fname, fire in _fires(B, H, W).items():
        gx, gp = step_vjp(md, x.to(DEV), g4.to(DEV), fire.to(DEV), cot.to(DEV), precision)
        ref = oracle_step_vjp(m, x, g4, cl, fire, None, cot, precision)
        errs = {"x": _rel(gx, ref["x"])}
        errs.update({k: _rel(g, ref[k]) for k, g in zip(STEP_NAMES, gp)})
        assert max(errs.values()) <= VJP_TOL[precision], (fname, errs)
        if fname == "zeros":  # nothing fires: the MLP and the kernels get no gradient
            assert all(float(g.abs().max()) == 0.0 for g in gp)


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
@pytest.mark.parametrize("name", ["maze_c16", "sudoku_c64", "ref_maze_hard"])
def test_make_step_under_autograd_matches_oracle(name, precision):
    """The reference's check of the step (tests/test_engine_ops.py:251-294): outputs and the
    gradients of the state and every parameter (the head gets none), with and without noise;
    the clamp values and the noise get their gradients too."""
    _say("make_step autograd", name, precision)
    m, md, x, g4, cl, _ = _case(name)
    B, C, H, W = x.shape
    fire = O.fire_masks_np(9, 0, B, 0, H, W, 0.6)
    noise = torch.randn(x.shape, generator=torch.Generator().manual_seed(1)) * 0.2
    step = make_step(md, precision=precision)
    params = list(md.parameters())
    for nz in (None, noise):
        xa = x.to(DEV).requires_grad_(True)
        ca = cl.to(DEV).requires_grad_(True)
        na = None if nz is None else nz.to(DEV).requires_grad_(True)
        y = step(xa, g4.to(DEV), ca, fire.to(DEV), na)
        cot = 0.2 * y.detach()  # d/dy of 0.1 * sum(y^2)
        wrt = [xa, ca] + ([na] if na is not None else []) + params
        grads = torch.autograd.grad((0.1 * y.pow(2)).sum(), wrt, allow_unused=True)
        with torch.no_grad():
            y_ref = O.step(oracle_cell(m), x, g4, cl, fire, precision, nz)
        tol = 1e-4 if precision == "fp32" else 2e-2
        assert (y.detach().cpu() - y_ref).abs().max().item() <= tol
        ref = oracle_step_vjp(m, x, g4, cl, fire, nz, cot.cpu(), precision)
        got = dict(zip(["x", "clamp"] + (["noise"] if na is not None else []), grads))
        named = dict(md.named_parameters())
        pmap = {"kernels": "perceive.weight", "w1": "update.fc1.weight", "b1": "update.fc1.bias",
                "w2": "update.fc2.weight", "b2": "update.fc2.bias"}
        pgrads = dict(zip([n for n, _ in md.named_parameters()], grads[len(wrt) - len(params):]))
        for k, pn in pmap.items():
            got[k] = pgrads[pn]
        for pn in named:
            if pn.startswith("head."):
                assert pgrads[pn] is None  # the step does not use the readout head
        for k, g in got.items():
            assert _rel(g, ref[k]) <= VJP_TOL[precision], (k, nz is None, _rel(g, ref[k]))


def test_step_refuses_gradient_wrt_fire():
    m, md, x, g4, cl, _ = _case("maze_c16")
    fire = torch.ones(x.shape[0], 1, *x.shape[2:], device=DEV, requires_grad=True)
    with pytest.raises(ValueError):
        make_step(md)(x.to(DEV), g4.to(DEV), cl.to(DEV), fire)


# ------------------------------------------------------------------------------ the engine
def _train_cfg(rollout, chunk, amp=False, loss="ce", noise=None):
    return {"rollout": rollout, "chunk": chunk, "amp": amp, "loss": loss,
            "noise": noise or {"p_t": 0.0, "p_s": 0.0, "sigma": 0.0}, "perturb": noise is not None}


def _masks(seeds, step0, B, H, W, p):
    return torch.stack([O.fire_masks_np(int(s), 0, B, step0 + i, H, W, p)
                        for i, s in enumerate(seeds)])


def _engine_case(name="maze_hard_c32", n_boards=2, k=2):
    m, md, x, g4, cl, b = _case(name, n_boards=n_boards, k=k)
    tokens = torch.from_numpy(np.repeat(b.targets, k, 0))
    batch = {"x": x.to(DEV), "given4": g4.to(DEV), "clamp": cl.to(DEV), "targets": tokens.to(DEV)}
    return m, md, batch


def test_engine_has_the_reference_constructor_and_composes():
    """Engine(model, EngineConfig, train_cfg, device): prefix / chunk / suffix with global step
    keys equal the separate operators, the update runs once after the rollout."""
    m, md, batch = _engine_case()
    seeds = np.arange(100, 110, dtype=np.int64)
    eng = Engine(md, EngineConfig.from_dict({"backend": "fused", "compile": False}),
                 _train_cfg(10, 4), DEV)
    assert eng.fused_chunk
    calls = []
    for p in md.parameters():
        p.grad = None
    w = torch.tensor([1.0, 0.0, 1.0, 1.0], device=DEV)
    xf, loss, gn = eng.train_iteration(batch, seeds, 3, w, grad_clip=1e9, apply_update=calls.append)
    assert len(calls) == 1 and torch.equal(calls[0], gn)
    p = m.cfg.fire_rate
    tgt = md.output_index(batch["targets"])
    with torch.no_grad():
        x3, _, _ = rollout_steps(md, batch["x"], batch["given4"], batch["clamp"], 3,
                                 step_seeds=seeds[:3], p_fire=p)
        ref = bptt_chunk(md, x3, batch["given4"], batch["clamp"], tgt, [1, 0, 1, 1],
                         step_seeds=seeds[3:7], step0=3, p_fire=p)
        xe, _, _ = rollout_steps(md, ref.x, batch["given4"], batch["clamp"], 3,
                                 step_seeds=seeds[7:], step0=7, p_fire=p)
    assert torch.equal(xf, xe) and torch.equal(loss, ref.loss)
    assert torch.equal(md.update.fc1.weight.grad, ref.grads["w1"].reshape(md.update.fc1.weight.shape))
    total = torch.sqrt(sum((ref.grads[k].double() ** 2).sum() for k in NAMES))
    assert abs(float(gn) - float(total)) <= 1e-5 * float(total)


def test_engine_update_right_after_the_backward():
    m, md, batch = _engine_case()
    seeds = np.arange(10, dtype=np.int64)
    order = []
    eng = Engine(md, EngineConfig(update_after_rollout=False), _train_cfg(10, 4), DEV)
    orig = eng.forward_steps

    def spy(*a, **kw):
        order.append("steps")
        return orig(*a, **kw)

    eng.forward_steps = spy
    eng.train_iteration(batch, seeds, 2, [1, 1, 1, 1], None, lambda g: order.append("update"))
    assert order == ["steps", "update", "steps"]


def test_engine_amp_runs_prefix_and_suffix_in_fp32():
    """train_cfg amp: the chunk is bf16 (gradients within the bf16 chunk bar of the oracle from
    the same state), the steps before and after it fp32 (within 1e-4 of the fp32 oracle, and not
    the bf16 trajectory)."""
    m, md, batch = _engine_case()
    B, C, H, W = batch["x"].shape
    seeds = np.arange(500, 512, dtype=np.int64)
    c0, Nc, N = 4, 3, 12
    eng = Engine(md, EngineConfig(), _train_cfg(N, Nc, amp=True), DEV)
    for p in md.parameters():
        p.grad = None
    w = [1.0, 0.0, 1.0]
    xf, loss, _ = eng.train_iteration(batch, seeds, c0, w, None, None)
    cell = oracle_cell(m)
    p = m.cfg.fire_rate
    x0 = batch["x"].cpu()
    g4, cl = batch["given4"].cpu(), batch["clamp"].cpu()
    # the prefix: fp32
    xp_ref, _ = O.rollout(cell, x0, g4, cl, c0, "fp32", masks=_masks(seeds[:c0], 0, B, H, W, p))
    with torch.no_grad():
        xp = eng.forward_steps(batch["x"], batch["given4"], batch["clamp"], seeds[:c0], 0)
    assert (xp.cpu() - xp_ref).abs().max().item() <= 1e-4
    # the chunk: bf16, from the GPU's prefix state
    tgt = md.output_index(batch["targets"]).cpu()
    cmasks = _masks(seeds[c0:c0 + Nc], c0, B, H, W, p)
    ref_loss, ref = O.bptt_chunk(cell, xp.cpu(), g4, cl, cmasks.double(), tgt, w, "bf16",
                                 grad_round=True)
    assert abs(float(loss) - ref_loss) <= 1e-2 * abs(ref_loss)
    got = _grads(md)
    for k in NAMES:
        assert _rel(got[k], ref[k]) <= 1e-2, (k, _rel(got[k], ref[k]))
    # the suffix: fp32 from the chunk's final state
    xc = eng.last_chunk.x
    xs_ref, _ = O.rollout(cell, xc.cpu(), g4, cl, N - c0 - Nc, "fp32",
                          masks=_masks(seeds[c0 + Nc:], c0 + Nc, B, H, W, p))
    err32 = (xf.cpu() - xs_ref).abs().max().item()
    with torch.no_grad():
        x16, _, _ = rollout_steps(md, xc, batch["given4"], batch["clamp"], N - c0 - Nc,
                                  step_seeds=seeds[c0 + Nc:], step0=c0 + Nc, p_fire=p,
                                  precision="bf16")
    _say("suffix error fp32", err32, "bf16 path differs by", (x16 - xf).abs().max().item())
    assert err32 <= 1e-4
    assert (x16 - xf).abs().max().item() > 1e-4  # the bf16 trajectory is a different one


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_step_by_step_chunk_equals_the_fused_chunk(precision):
    m, md, batch = _engine_case()
    seeds = np.arange(40, 46, dtype=np.int64)
    eng = Engine(md, EngineConfig(), _train_cfg(6, 6, amp=precision == "bf16"), DEV)
    w = np.array([0.5, 1.0, 0.0, 1.0, 0.0, 1.0], np.float32)
    tgt = md.output_index(batch["targets"])
    res = bptt_chunk(md, batch["x"], batch["given4"], batch["clamp"], tgt, w, step_seeds=seeds,
                     step0=0, p_fire=m.cfg.fire_rate, precision=precision)
    for p in md.parameters():
        p.grad = None
    with torch.enable_grad():
        x, loss = eng._chunk_steps(batch["x"], batch, seeds, 0, w, precision)
        loss.backward()
    tol = 1e-4 if precision == "fp32" else 1e-2
    assert abs(float(loss.detach()) - float(res.loss)) <= tol * abs(float(res.loss))
    assert (x.detach() - res.x).abs().max().item() <= (1e-4 if precision == "fp32" else 2e-2)
    got = _grads(md)
    for k in NAMES:
        assert _rel(got[k], res.grads[k]) <= tol, (k, _rel(got[k], res.grads[k]))


def _oracle_mse_chunk(m, x0, g4, cl, masks, targets_tokens, weights, noises=None):
    """fp64 autograd of the MSE chunk loss (reference train.py:183-207, "mse") through the
    oracle's step: (loss, grads of the step parameters)."""
    cell = oracle_cell(m)
    dt = torch.float64
    params = {k: getattr(cell, k).detach().to(dt).clone().requires_grad_(True) for k in STEP_NAMES}
    c = O.OracleCell(**{**cell.__dict__, **params})
    x = x0.to(dt)
    emb = m.target_embedding(targets_tokens).to(dt)
    total = x.new_zeros(())
    sl = m.cfg.out_slice
    for t in range(masks.shape[0]):
        nz = None if noises is None or noises[t] is None else noises[t].to(dt)
        x = O.step(c, x, g4, cl, masks[t].to(dt), "fp32", nz, dtype=dt)
        if weights[t] != 0:
            total = total + weights[t] * ((x[:, sl] - emb) ** 2).sum(dim=1).mean()
    total = total / max(sum(weights), 1.0)
    grads = torch.autograd.grad(total, [params[k] for k in STEP_NAMES])
    return float(total.detach()), dict(zip(STEP_NAMES, grads))


def test_engine_mse_loss_with_an_l2_head():
    """The reference's trained maze cell (l2 head) with the MSE loss: the chunk runs step by step
    through the differentiable HIP step; loss and gradients match the fp64 oracle."""
    m, md, batch = _engine_case("ref_maze_hard")
    B, C, H, W = batch["x"].shape
    seeds = np.arange(7, 12, dtype=np.int64)
    eng = Engine(md, EngineConfig(), _train_cfg(5, 4, loss="mse"), DEV)
    assert not eng.fused_chunk
    for p in md.parameters():
        p.grad = None
    w = [1.0, 0.0, 1.0, 1.0]
    xf, loss, _ = eng.train_iteration(batch, seeds, 1, w, None, None)
    with torch.no_grad():
        x1 = eng.forward_steps(batch["x"], batch["given4"], batch["clamp"], seeds[:1], 0)
    masks = _masks(seeds[1:5], 1, B, H, W, m.cfg.fire_rate)
    ref_loss, ref = _oracle_mse_chunk(m, x1.cpu(), batch["given4"].cpu(), batch["clamp"].cpu(),
                                      masks, batch["targets"].cpu(), w)
    assert abs(float(loss) - ref_loss) <= 1e-5 * abs(ref_loss)
    got = _grads(md)
    for k in STEP_NAMES:
        assert _rel(got[k], ref[k]) <= 1e-4, (k, _rel(got[k], ref[k]))


@pytest.mark.parametrize("name", ["maze_c16", "sudoku_c64", "maze_hard_c32", "ref_maze_ood"])
@pytest.mark.parametrize("uniform", [False, True])
def test_init_state_matches_the_reference_expressions(name, uniform):
    """nca_init_state (model.init_state on the GPU) against the reference's torch expressions
    (src/nca/model.py:384-412: noise scaled, embed[inputs] as clamp, the clamp on the given
    cells' input channels) evaluated on the same draw: bit for bit."""
    preset, size = CELLS[name]
    m = make_model(name, 0)
    m.cfg.init_uniform = uniform
    m.cfg.sigma_init = 0.37
    md = copy.deepcopy(m).to(DEV)
    b = boards_for(preset, 5, size, 3)
    inputs = torch.as_tensor(np.asarray(b.inputs)).to(DEV, torch.int64)
    given = torch.as_tensor(np.asarray(b.given)).to(DEV, torch.bool)
    _say("init_state", name, uniform, tuple(inputs.shape))
    x, g4, cl = md.init_state(inputs, given, None, torch.Generator(device=DEV).manual_seed(11))
    gen = torch.Generator(device=DEV).manual_seed(11)
    shape = (inputs.shape[0], md.cfg.channels) + tuple(inputs.shape[1:])
    if uniform:
        rx = (torch.rand(shape, generator=gen, device=DEV) * 2 - 1) * md.cfg.sigma_init
    else:
        rx = torch.randn(shape, generator=gen, device=DEV) * md.cfg.sigma_init
    rcl = md.embed.detach()[inputs].permute(0, 3, 1, 2).contiguous()
    sl = md.cfg.in_slice
    rx[:, sl] = torch.where(given[:, None], rcl, rx[:, sl])
    assert given.any() and (~given).any()
    assert torch.equal(g4, given[:, None])
    assert torch.equal(cl, rcl)
    assert torch.equal(x, rx)


def test_engine_step_noise():
    """Step noise (p_t, p_s, sigma): every step's noise is drawn from its seed; the rollout
    outside the chunk and the chunk's gradients match the oracle fed the same noise."""
    m, md, batch = _engine_case("maze_hard_c32")
    B, C, H, W = batch["x"].shape
    seeds = np.arange(900, 906, dtype=np.int64)
    noise = {"p_t": 0.9, "p_s": 0.4, "sigma": 0.1}
    eng = Engine(md, EngineConfig(), _train_cfg(6, 3, loss="ce", noise=noise), DEV)
    assert eng.noise_cfg is not None and not eng.fused_chunk
    d0 = eng.draw(seeds[0], 0, batch["x"].shape)
    d0b = eng.draw(seeds[0], 0, batch["x"].shape)
    assert torch.equal(d0.noise, d0b.noise) and float(d0.noise.abs().sum()) > 0
    for p in md.parameters():
        p.grad = None
    w = [1.0, 1.0, 1.0]
    xf, loss, _ = eng.train_iteration(batch, seeds, 2, w, None, None)
    cell = oracle_cell(m)
    draws = [eng.draw(s, i, batch["x"].shape) for i, s in enumerate(seeds)]
    x = batch["x"].cpu().double()
    g4, cl = batch["given4"].cpu(), batch["clamp"].cpu()
    with torch.no_grad():
        for i in range(2):
            x = O.step(cell, x, g4, cl, draws[i].fire.cpu(), "fp64", draws[i].noise.cpu())
    tgt = md.output_index(batch["targets"]).cpu()
    # the chunk with its noise: oracle by fp64 autograd
    dt = torch.float64
    params = {k: getattr(cell, k).detach().to(dt).clone().requires_grad_(True) for k in NAMES}
    c = O.OracleCell(**{**cell.__dict__, **params})
    xc = x.clone()
    total = xc.new_zeros(())
    for i in range(2, 5):
        xc = O.step(c, xc, g4, cl, draws[i].fire.cpu(), "fp64", draws[i].noise.cpu(), dtype=dt)
        logits = torch.einsum("vc,bchw->bvhw", c.head_w, xc[:, m.cfg.out_slice]) \
            + c.head_b[None, :, None, None]
        total = total + torch.nn.functional.cross_entropy(logits, tgt).to(dt)
    total = total / 3.0
    grads = dict(zip(NAMES, torch.autograd.grad(total, [params[k] for k in NAMES])))
    assert abs(float(loss) - float(total)) <= 1e-4 * abs(float(total))
    got = _grads(md)
    for k in NAMES:
        assert _rel(got[k], grads[k]) <= 1e-4, (k, _rel(got[k], grads[k]))
    with torch.no_grad():
        x = xc.detach()
        x = O.step(cell, x, g4, cl, draws[5].fire.cpu(), "fp64", draws[5].noise.cpu())
    assert (xf.cpu().double() - x).abs().max().item() <= 1e-4
