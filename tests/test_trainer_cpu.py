"""Host logic of the training recipe: config resolution, learning-rate schedule, EMA decay and
damage discs (the draws, and the oracle's rasterisation pinned by lattice-point counts), checked
against their closed forms (reference src/nca/train.py:111-216, src/nca/perturb.py:43-106)."""

from __future__ import annotations

import math

import numpy as np
import pytest

from ncas_amd.perturb import draw_discs
from ncas_amd.trainer import DEFAULTS, ema_decay, lr_at, resolve_train_cfg
from oracle.perturb import disc_masks


def test_resolve_merges_sub_dicts_and_refuses_unknown_keys():
    tr = resolve_train_cfg({"train": {"noise": {"sigma": 0.3}, "steps": 7}})
    assert tr["steps"] == 7 and tr["noise"] == {**DEFAULTS["noise"], "sigma": 0.3}
    assert tr["damage"] == DEFAULTS["damage"]
    with pytest.raises(ValueError):
        resolve_train_cfg({"train": {"not_an_option": 1}})
    with pytest.raises(ValueError):
        resolve_train_cfg({"train": {"schedule": "linear"}})


def test_lr_schedule_closed_forms():
    tr = resolve_train_cfg({"train": {"schedule": "cosine", "warmup_ratio": 0.25}})
    total = 100
    assert [lr_at(s, total, tr) for s in (0, 1, 24)] == [1 / 25, 2 / 25, 1.0]
    assert lr_at(25, total, tr) == 1.0  # cosine starts at its top
    assert abs(lr_at(25 + 75 // 2, total, tr) - 0.5 * (1 + math.cos(math.pi * 37 / 75))) < 1e-15
    assert lr_at(100, total, tr) == pytest.approx(0.0, abs=1e-15)
    const = resolve_train_cfg({"train": {}})
    assert all(lr_at(s, 10, const) == 1.0 for s in range(10))
    tr2 = resolve_train_cfg({"train": {"warmup_ratio": 0.5, "init_lr_ratio": 0.1}})
    assert lr_at(0, 10, tr2) == 0.1 and abs(lr_at(4, 10, tr2) - (0.1 + 0.9 * 4 / 5)) < 1e-15


def test_ema_decay_warm_up():
    tr = resolve_train_cfg({"train": {"ema": 0.999}})
    assert ema_decay(tr, 0) == 0.1 and ema_decay(tr, 10) == 11 / 20
    assert ema_decay(tr, 10**6) == 0.999
    assert ema_decay({**tr, "ema_warmup": False}, 0) == 0.999


def test_damage_discs():
    rng = np.random.default_rng(0)
    hit = np.array([True, False, True, True])
    discs = draw_discs(rng, hit, 20, 30, 2, 0.2, 0.2)
    assert discs.shape == (6, 4) and list(discs[:, 0]) == [0, 0, 2, 2, 3, 3]
    assert np.allclose(discs[:, 3], (0.2 * 20) ** 2)
    assert (0 <= discs[:, 1]).all() and (discs[:, 1] < 20).all() and (discs[:, 2] < 30).all()
    m = disc_masks(discs, 4, 20, 30)
    assert not m[1].any() and m[0].any() and m[2].any()
    # a disc of radius 4 holds at most the 49 lattice points of x^2 + y^2 <= 16; two at most 98
    for b in (0, 2, 3):
        assert 30 <= m[b].sum() <= 98
    # lattice-point counts of discs centred on a cell: 5 (r^2 = 1), 9 (2), 13 (4), 49 (16)
    for r2, want in ((1, 5), (2, 9), (4, 13), (16, 49)):
        assert disc_masks(np.array([[0, 10, 10, r2]]), 1, 21, 21).sum() == want
    # official discs on linspace(-1, 1) coordinates (grid step 0.2 on 11 points): a radius
    # below one step around the centre keeps only the centre cell, a radius above it adds the
    # four neighbours, and below sqrt(2) steps not the diagonals
    assert disc_masks(np.array([[0, 0.0, 0.0, 0.19 ** 2]]), 1, 11, 11, "official").sum() == 1
    assert disc_masks(np.array([[0, 0.0, 0.0, 0.21 ** 2]]), 1, 11, 11, "official").sum() == 5
    assert disc_masks(np.array([[0, 0.0, 0.0, 0.28 ** 2]]), 1, 11, 11, "official").sum() == 5
    rng = np.random.default_rng(1)
    do = draw_discs(rng, np.array([True, True]), 11, 11, 1, 0.3, 0.3, "official")
    assert (np.abs(do[:, 1:3]) <= 0.5).all() and np.allclose(do[:, 3], 0.09)
    mo = disc_masks(do, 2, 11, 11, "official")
    # centres in [-0.5, 0.5]^2, radius 0.3: the corners are never inside
    assert mo.any(axis=(1, 2)).all() and not mo[:, 0, 0].any() and not mo[:, -1, -1].any()
    with pytest.raises(ValueError):
        draw_discs(rng, hit, 5, 5, 1, 0.1, 0.2, "square")
