"""The oracle's Philox4x32-10 and fire-mask rule (CPU)."""

import numpy as np
import pytest

from oracle import philox

# Random123 known-answer vectors (kat_vectors, philox4x32 10 rounds): ctr, key -> output
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,expected", KAT)
def test_numpy_philox_known_answers(ctr, key, expected):
    assert tuple(int(v) for v in philox.philox4x32_10(ctr, key)) == expected


@pytest.mark.parametrize("ctr,key,expected", KAT)
def test_c_philox_known_answers(oracle_lib, ctr, key, expected):
    assert tuple(int(v) for v in oracle_lib.philox(ctr, key)) == expected


def test_c_and_numpy_philox_agree(oracle_lib):
    rng = np.random.default_rng(0)
    for _ in range(200):
        ctr = rng.integers(0, 2**32, 4, dtype=np.uint64)
        key = rng.integers(0, 2**32, 2, dtype=np.uint64)
        a = oracle_lib.philox(ctr.astype(np.uint32), key.astype(np.uint32))
        b = philox.philox4x32_10(tuple(ctr), tuple(key))
        assert np.array_equal(a, b)


@pytest.mark.parametrize("hw", [1, 3, 81, 169, 900])
def test_fire_masks_agree_and_are_keyed(oracle_lib, hw):
    seed = 0x1234_5678_9ABC_DEF
    a = oracle_lib.fire_mask(seed, 5, 7, 11, hw, 0.5)
    b = philox.fire_mask(seed, 5, 7, 11, hw, 0.5)
    assert np.array_equal(a, b)
    # a row's mask depends only on (seed, row, step): shifting row0 shifts rows
    c = philox.fire_mask(seed, 6, 6, 11, hw, 0.5)
    assert np.array_equal(a[1:], c)
    # another step or seed gives another mask
    if hw >= 81:
        assert not np.array_equal(a, philox.fire_mask(seed, 5, 7, 12, hw, 0.5))
        assert not np.array_equal(a, philox.fire_mask(seed + 1, 5, 7, 11, hw, 0.5))


def test_uniforms_are_24_bit_and_rate_matches():
    u = philox.cell_uniforms(3, 0, 2000, 0, 81)
    assert u.min() >= 0.0 and u.max() < 1.0
    assert np.all(u * 2**24 == np.floor(u * 2**24))
    for p in (0.25, 0.5, 0.8):
        m = philox.fire_mask(3, 0, 2000, 0, 81, p)
        assert abs(m.mean() - p) < 0.01  # 162k draws: 4 sigma < 0.005
    assert philox.fire_mask(3, 0, 10, 0, 81, 0.0).sum() == 0
    assert philox.fire_mask(3, 0, 10, 0, 81, 1.0).all()


def test_adaptive_rule(oracle_lib):
    rng = np.random.default_rng(1)
    rows, hw = 400, 81
    conf = rng.random((rows, hw)).astype(np.float32)
    given = rng.random((rows, hw)) < 0.3
    a = oracle_lib.fire_mask(9, 0, rows, 4, hw, 0.8, 0.2, 0.9, conf, given)
    b = philox.fire_mask(9, 0, rows, 4, hw, 0.8, 0.2, 0.9, conf, given)
    assert np.array_equal(a, b)
    confident = (conf > 0.9) | given
    assert abs(a[confident].mean() - 0.2) < 0.02
    assert abs(a[~confident].mean() - 0.8) < 0.02
    # strict threshold: a cell exactly at tau is not confident
    c = np.full((1, 8), 0.5, np.float32)
    m1 = philox.fire_mask(9, 0, 1, 0, 8, 1.0, 0.0, 0.5, c, None)
    assert m1.all()
