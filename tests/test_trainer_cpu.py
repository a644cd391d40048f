"""Host logic of the training recipe: config resolution, learning-rate schedule, EMA decay and
damage discs, checked against their closed forms (reference src/nca/train.py:111-216,
src/nca/perturb.py:43-106)."""

from __future__ import annotations

import math

import numpy as np
import pytest

from ncas_amd.trainer import DEFAULTS, damage_masks, ema_decay, lr_at, resolve_train_cfg


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
    m = damage_masks(4, 20, 30, 2, 0.2, 0.2, rng, hit)
    assert not m[1].any() and m[0].any() and m[2].any()
    # a disc of radius 0.2 * 20 = 4 cells holds about pi * 16 cells; two discs at most twice
    for b in (0, 2, 3):
        assert 30 <= m[b].sum() <= 2 * math.pi * 16 + 20
    rng = np.random.default_rng(1)
    mo = damage_masks(2, 11, 11, 1, 0.3, 0.3, rng, np.array([True, True]), "official")
    # official discs: centres in [-0.5, 0.5]^2 on a [-1, 1] grid, radius 0.3: the centre cell
    # row / column of the grid (coordinate 0) is within 0.5 + 0.3 of the centre, and the
    # corners never are
    assert mo.any(axis=(1, 2)).all() and not mo[:, 0, 0].any() and not mo[:, -1, -1].any()
