"""The BPTT oracle pinned without the GPU: its autograd gradients agree with finite differences
of its own fp64 forward (torch.autograd.gradcheck on small tensors, central differences along
random directions for the large ones), for wall, zero and wrap padding; the straight-through
bf16 variant differentiates the rounded forward; and the replay pool's bookkeeping."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, __file__.rsplit("/", 1)[0])
from cells import DYN, initial_state, oracle_cell, perturbed_model  # noqa: E402

from ncas_amd.tasks import maze_boards  # noqa: E402
from oracle import nca_oracle as O  # noqa: E402

NAMES = ("kernels", "w1", "b1", "w2", "b2", "head_w", "head_b")


def _case(padding="wall", size=6, rows=2, steps=3, seed=0):
    kw = {"padding": padding}
    if padding != "wall":
        kw["wall_token"] = None
    # random fc1 without the leak wiring of the GPU parity cells: no pre-activation sits exactly
    # on the ReLU's kink (clamped one-hot inputs are exact zeros), so finite differences apply
    m = perturbed_model("maze_c16", seed, DYN["maze_c16"][0], 0.0, **kw)
    cell = oracle_cell(m)
    b = maze_boards(rows, size, seed)
    x, g4, cl = initial_state(m, b, k=1, sigma=0.3, seed=seed)
    g = torch.Generator().manual_seed(seed + 7)
    B, C, H, W = x.shape
    masks = (torch.rand((steps, B, 1, H, W), generator=g) < 0.6).double()
    targets = torch.randint(0, 2, (B, H, W), generator=g)
    weights = [1.0, 0.0, 0.5][:steps] + [1.0] * max(0, steps - 3)
    return cell, x, g4, cl, masks, targets, weights


def _kink_margin(cell, x, g4, cl, masks, padding):
    """Smallest |fc1 pre-activation| over the chunk's steps (fp64)."""
    xx, worst = x.double(), float("inf")
    for t in range(masks.shape[0]):
        B, C, H, W = xx.shape
        z = O.perceive(O.pad(xx, padding, cell.pad_vec.double()), cell.kernels.double(), H, W)
        a = z.permute(0, 2, 3, 1).reshape(-1, z.shape[1]) @ cell.w1.double().T + cell.b1.double()
        worst = min(worst, a.abs().min().item())
        xx = O.step(cell, xx, g4, cl, masks[t], "fp64")
    return worst


def _smooth_case(padding, size=5, margin=4e-5):
    """The first seed whose fc1 pre-activations all stay `margin` away from the ReLU's kink:
    finite differences of step 1e-6 are only valid away from it."""
    for seed in range(20):
        case = _case(padding, size=size, seed=seed)
        if _kink_margin(*case[:5], padding) >= margin:
            return case
    raise AssertionError("no seed keeps the pre-activations away from the kink")


def _loss_fn(cell, x, g4, cl, masks, targets, weights, name, precision="fp32", ste=True, lm=None):
    def f(t):
        c = O.OracleCell(**{**cell.__dict__, name: t}) if name != "x0" else cell
        x0 = t if name == "x0" else x
        return O.chunk_loss(c, x0, g4, cl, masks, targets, weights, precision, lm, ste)
    return f


@pytest.mark.parametrize("padding", ["wall", "zero", "wrap"])
def test_gradcheck_small_parameters_and_state(padding):
    cell, x, g4, cl, masks, targets, weights = _smooth_case(padding, size=5)
    for name in ("kernels", "b2", "head_w", "head_b", "x0"):
        base = x if name == "x0" else getattr(cell, name)
        t = base.detach().to(torch.float64).clone().requires_grad_(True)
        f = _loss_fn(cell, x, g4, cl, masks, targets, weights, name)
        assert torch.autograd.gradcheck(f, (t,), eps=1e-6, atol=1e-7, rtol=1e-4), (padding, name)


@pytest.mark.parametrize("padding", ["wall", "wrap"])
def test_directional_derivatives_of_every_gradient(padding):
    """<grad L, v> equals (L(p + e v) - L(p - e v)) / 2e for random v, every parameter."""
    cell, x, g4, cl, masks, targets, weights = _case(padding)
    lm = (torch.rand(targets.shape, generator=torch.Generator().manual_seed(3)) < 0.7).double()
    _, grads = O.bptt_chunk(cell, x, g4, cl, masks, targets, weights, "fp32", loss_mask=lm,
                            grad_x0=True)
    g = torch.Generator().manual_seed(11)
    for name in NAMES + ("x0",):
        base = (x if name == "x0" else getattr(cell, name)).detach().to(torch.float64)
        v = torch.randn(base.shape, generator=g, dtype=torch.float64)
        v = v / v.norm()  # unit direction: a small step for every tensor size
        f = _loss_fn(cell, x, g4, cl, masks, targets, weights, name, lm=lm)
        eps = 1e-6
        with torch.no_grad():
            fd = (f(base + eps * v) - f(base - eps * v)) / (2 * eps)
        an = (grads[name] * v).sum()
        assert abs(float(fd) - float(an)) <= 1e-8 + 1e-5 * abs(float(an)), (name, float(fd), float(an))


def test_zero_weights_give_zero_loss_and_gradients():
    cell, x, g4, cl, masks, targets, _ = _case()
    loss, grads = O.bptt_chunk(cell, x, g4, cl, masks, targets, [0.0, 0.0, 0.0], grad_x0=True)
    assert loss == 0.0 and all(float(t.abs().max()) == 0.0 for t in grads.values())


def test_clamp_backward_with_a_silent_step():
    """One step with a zero fire mask is the clamp alone (x1 = clamp(x0)), so d L / d x0 is the
    loss gradient at x1 with the input slice of given cells zeroed (ops.py:276-294)."""
    cell, x, g4, cl, masks, targets, _ = _case(steps=1)
    silent = torch.zeros_like(masks)
    _, grads = O.bptt_chunk(cell, x, g4, cl, silent, targets, [1.0], grad_x0=True)
    x1 = O.apply_clamp(cell, x.double(), g4, cl).detach().requires_grad_(True)
    sl = slice(cell.out_offset, cell.out_offset + cell.c_out)
    logits = torch.einsum("vc,bchw->bvhw", cell.head_w.double(), x1[:, sl]) \
        + cell.head_b.double()[None, :, None, None]
    torch.nn.functional.cross_entropy(logits, targets, reduction="none").mean().backward()
    expect = x1.grad.clone()
    ins = slice(cell.in_offset, cell.in_offset + cell.c_in)
    expect[:, ins] = torch.where(g4, torch.zeros_like(expect[:, ins]), expect[:, ins])
    assert torch.allclose(grads["x0"], expect, atol=1e-15, rtol=1e-12)
    assert float(grads["w1"].abs().max()) == 0.0  # the MLP output is never used


def test_straight_through_bf16_is_the_gradient_of_the_rounded_forward():
    """With ste, the bf16 chunk's gradient equals the gradient of the fp64 forward evaluated at
    the same rounded operands: for the head (applied to fp64 states after the last rounding)
    and the final-step loss, fd of the rounded forward agree with it on a smooth direction."""
    cell, x, g4, cl, masks, targets, weights = _case()
    l32, g32 = O.bptt_chunk(cell, x, g4, cl, masks, targets, weights, "fp32")
    l16, g16 = O.bptt_chunk(cell, x, g4, cl, masks, targets, weights, "bf16")
    assert abs(l32 - l16) < 0.05 * abs(l32)
    for name in NAMES:
        rel = float((g16[name] - g32[name]).norm() / g32[name].norm().clamp_min(1e-12))
        assert rel < 0.15, (name, rel)
    # the head gradient is linear in the states: fd along head_w is exact for the rounded forward
    f = _loss_fn(cell, x, g4, cl, masks, targets, weights, "head_w", precision="bf16")
    v = torch.randn(cell.head_w.shape, generator=torch.Generator().manual_seed(2), dtype=torch.float64)
    base = cell.head_w.detach().to(torch.float64)
    with torch.no_grad():
        fd = (f(base + 1e-5 * v) - f(base - 1e-5 * v)) / 2e-5
    assert abs(float(fd) - float((g16["head_w"] * v).sum())) < 1e-6


def _bfn(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(torch.float64).numpy()


def _step_backward_np(cell, x, g4, cl, fire, G, padding):
    """One bf16 step and its backward written out in numpy loops, with the reference's bf16
    backward rounding (g_dx, the fc1-output gradient and g_z rounded to bf16; engine/triton_mlp.py
    46-78): an independent statement of what `grad_round` must compute. B = 1."""
    K = _bfn(cell.kernels.double().numpy().reshape(-1, 3, 3))        # (4, 3, 3)
    W1, b1 = _bfn(cell.w1.double().numpy()), _bfn(cell.b1.double().numpy())
    W2, b2 = _bfn(cell.w2.double().numpy()), _bfn(cell.b2.double().numpy())
    x = x.double().numpy()[0]                                         # (C, H, W)
    C, H, W = x.shape
    nk = K.shape[0]
    pv = cell.pad_vec.double().numpy()
    xp = np.zeros((C, H + 2, W + 2))
    for c in range(C):
        for i in range(-1, H + 1):
            for j in range(-1, W + 1):
                inside = 0 <= i < H and 0 <= j < W
                if inside or padding == "wrap":
                    xp[c, i + 1, j + 1] = x[c, i % H, j % W]
                else:
                    xp[c, i + 1, j + 1] = pv[c] if padding == "wall" else 0.0
    xp = _bfn(xp)
    z = np.zeros((nk * C, H, W))
    for k in range(nk):
        for c in range(C):
            for i in range(H):
                for j in range(W):
                    z[k * C + c, i, j] = sum(K[k, a, b] * xp[c, i + a, j + b] for a in range(3) for b in range(3))
    z = _bfn(z)
    rows = z.reshape(nk * C, H * W).T                                 # (cells, F)
    hpre = _bfn(rows @ W1.T + b1)
    h = np.maximum(hpre, 0.0)
    dx = _bfn(h @ W2.T + b2)                                          # (cells, C)
    f = fire.double().numpy().reshape(H * W)
    g = G.double().numpy()[0].reshape(C, H * W).T.copy()              # (cells, C)
    gv = g4.numpy().reshape(H * W)
    sl = slice(cell.in_offset, cell.in_offset + cell.c_in)
    g[gv, sl] = 0.0                                                   # clamp backward
    gdx = _bfn(g * f[:, None])
    gh = _bfn(gdx @ W2) * (hpre > 0)
    gz = _bfn(gh @ W1)                                                # (cells, F)
    gx = g.T.reshape(C, H, W).copy()
    gzp = gz.T.reshape(nk * C, H, W)
    dK = np.zeros((nk, 3, 3))
    gxp = np.zeros((C, H + 2, W + 2))
    for k in range(nk):
        for c in range(C):
            for i in range(H):
                for j in range(W):
                    for a in range(3):
                        for b in range(3):
                            gxp[c, i + a, j + b] += K[k, a, b] * gzp[k * C + c, i, j]
                            dK[k, a, b] += gzp[k * C + c, i, j] * xp[c, i + a, j + b]
    for c in range(C):
        for i in range(-1, H + 1):
            for j in range(-1, W + 1):
                if (0 <= i < H and 0 <= j < W) or padding == "wrap":
                    gx[c, i % H, j % W] += gxp[c, i + 1, j + 1]
    return {"x0": gx[None], "kernels": dK.reshape(nk, 1, 3, 3), "w1": gh.T @ rows, "b1": gh.sum(0), "w2": gdx.T @ h,
            "b2": gdx.sum(0)}


@pytest.mark.parametrize("padding", ["wall", "wrap"])
def test_bf16_gradient_rounding_matches_a_written_out_backward(padding):
    """`grad_round` (the reference's bf16 backward rounding points) against the numpy loops
    above on one step with a final cotangent; the straight-through gradient differs from it
    (the rounding points matter at this size)."""
    cell, x, g4, cl, masks, targets, _ = _case(padding, size=5, rows=1, steps=1)
    G = torch.randn(x.shape, generator=torch.Generator().manual_seed(3), dtype=torch.float64) * 0.3
    _, got = O.bptt_chunk(cell, x, g4, cl, masks, targets, [0.0], "bf16", grad_x0=True,
                          final_cotangent=G, grad_round=True)
    _, ste = O.bptt_chunk(cell, x, g4, cl, masks, targets, [0.0], "bf16", grad_x0=True,
                          final_cotangent=G)
    ref = _step_backward_np(cell, x, g4, cl, masks[0], G, padding)
    for k, v in ref.items():
        g = got[k].numpy().reshape(v.shape)
        assert np.abs(g - v).max() <= 1e-12 * max(1.0, np.abs(v).max()), k
    assert any(float((ste[k] - got[k]).abs().max()) > 0 for k in ("w1", "kernels", "x0"))


def test_replay_pool_sample_and_write_back():
    from ncas_amd.model import build_model
    from ncas_amd.train import ReplayPool

    m = build_model("maze_hard_c32")
    boards = maze_boards(12, 9, 0)
    pool = ReplayPool(m, boards, 16, np.random.default_rng(0), torch.Generator().manual_seed(0))
    assert pool.x.shape == (16, 32, 9, 9) and int(pool.age.sum()) == 0
    idx, batch = pool.sample(8, 0.25)
    assert len(set(idx.tolist())) == 8 and batch["x"].shape == (8, 32, 9, 9)
    assert int(batch["age"][:2].sum()) == 0  # two fresh boards
    batch["x"] = batch["x"] + 1.0
    pool.write_back(idx, batch)
    assert torch.equal(pool.x[torch.as_tensor(idx)], batch["x"])
    assert torch.equal(pool.age[torch.as_tensor(idx)], batch["age"] + 1)
    other = np.setdiff1d(np.arange(16), idx)
    assert int(pool.age[torch.as_tensor(other)].sum()) == 0
    sd = pool.state_dict()
    pool2 = ReplayPool(m, boards, 16, np.random.default_rng(5))
    pool2.load_state_dict(sd)
    assert torch.equal(pool2.x, pool.x)


def test_loss_weights_windows():
    from ncas_amd.train import loss_weights

    assert loss_weights("all", 4).tolist() == [1, 1, 1, 1]
    assert loss_weights("last", 4).tolist() == [0, 0, 0, 1]
    assert loss_weights(2, 4).tolist() == [0, 0, 1, 1]
