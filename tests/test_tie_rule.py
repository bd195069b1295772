"""The near-tie rule the GPU parity tests use for greedy tokens
(conftest.assert_argmax_parity), checked on the CPU with planted
differences: a swap between near-tied logits is excused, any other swap
fails, and so do too many excused rows."""
import numpy as np
import pytest

from conftest import NEAR_TIE, assert_argmax_parity


def logits(rows=50, vocab=300, seed=0):
    return np.random.default_rng(seed).standard_normal((rows, vocab)).astype(np.float32) * 3.0


def test_identical_tokens_pass():
    lg = logits()
    assert assert_argmax_parity(lg.argmax(axis=1), lg) == 0


def test_first_index_wins_exact_ties():
    lg = np.zeros((1, 8), np.float32)
    lg[0, [2, 5]] = 1.0  # sampler::argmax keeps the first maximum (src/sampler.rs:42-51)
    assert assert_argmax_parity(np.array([2]), lg) == 0
    assert assert_argmax_parity(np.array([5]), lg) == 1  # an exact tie is a near-tie


def test_near_tie_is_excused_and_a_real_difference_fails():
    lg = logits()
    dev = lg.argmax(axis=1).copy()
    r = 7
    top = int(dev[r])
    second = int(np.argsort(lg[r])[-2])
    scale = float(np.abs(lg[r]).max())
    lg[r, second] = lg[r, top] - 0.5 * NEAR_TIE * scale  # within the bar
    dev[r] = second
    assert assert_argmax_parity(dev, lg) == 1
    lg[r, second] = lg[r, top] - 4 * NEAR_TIE * scale  # outside it
    with pytest.raises(AssertionError, match="near-tie bar"):
        assert_argmax_parity(dev, lg)


def test_too_many_near_ties_fail():
    lg = logits(rows=20)
    dev = lg.argmax(axis=1).copy()
    for r in range(3):
        second = int(np.argsort(lg[r])[-2])
        lg[r, second] = np.nextafter(lg[r, dev[r]], np.float32(-np.inf))  # just below the top
        dev[r] = second
    with pytest.raises(AssertionError, match="near-tie rows"):
        assert_argmax_parity(dev, lg)  # 3 of 20 rows > 1% + 1
    assert assert_argmax_parity(dev, lg, max_ties=3) == 3
