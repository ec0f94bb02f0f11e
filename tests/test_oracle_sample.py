"""Pins the oracle's greedy selection with the repetition penalty
(oracle/sample_ref.py, restating alpacca/sample.py:31-45) by hand-built
cases whose answer follows from the definition, and the vectorized form
against the list form on random inputs."""
import numpy as np
import pytest

from oracle.sample_ref import (RepeatWindow, penalized_argmax, penalized_argmax_pure,
                               penalized_margin)

BOTH = [penalized_argmax, penalized_argmax_pure]


@pytest.mark.parametrize("f", BOTH)
def test_no_penalty_is_first_argmax(f):
    v = np.array([1.0, 3.0, -2.0, 3.0, 0.5], np.float32)
    for p in (1.0, 0.0):  # sample.py:40: 0 and 1 leave the logits alone
        assert f(v, [1, 3], p) == 1
    assert f(v, [], 1.1) == 1  # an empty window changes nothing


@pytest.mark.parametrize("f", BOTH)
def test_positive_winner_divided(f):
    v = np.array([0.0, 3.0, 2.9, 1.0], np.float32)
    assert f(v, [1], 1.1) == 2          # 3.0 / 1.1 = 2.727 < 2.9
    assert f(v, [1], 1.01) == 1         # 3.0 / 1.01 = 2.97 > 2.9
    assert f(v, [2], 1.1) == 1


@pytest.mark.parametrize("f", BOTH)
def test_negative_values_multiplied(f):
    v = np.array([-1.0, -1.05, -3.0], np.float32)
    assert f(v, [0], 1.1) == 1          # -1.0 * 1.1 = -1.1 < -1.05
    assert f(v, [0], 0.9) == 0          # a penalty below 1 raises negatives: -0.9
    z = np.array([0.0, -1e-30], np.float32)
    assert f(z, [0], 1.1) == 0          # 0 is not > 0: 0 * 1.1 = 0 stays the max


@pytest.mark.parametrize("f", BOTH)
def test_duplicates_penalized_once(f):
    # set(recent): a token twice in the window is penalized once
    v = np.array([2.6, 0.0, 3.0], np.float32)
    assert f(v, [2, 2], 1.1) == 2       # once: 2.727 > 2.6; twice would be 2.479


@pytest.mark.parametrize("f", BOTH)
def test_ties_take_the_lower_index(f):
    # penalty 2 is exact in binary: 4 / 2 == 2 ties with the plain 2.0
    v = np.array([0.0, 2.0, 0.0, 4.0, 2.0], np.float32)
    assert f(v, [3], 2.0) == 1          # 1 (plain 2.0) before 3 (penalized 2.0)
    w = np.array([0.0, 4.0, 0.0, 2.0], np.float32)
    assert f(w, [1], 2.0) == 1          # penalized 2.0 at 1 before plain 2.0 at 3


def test_penalty_in_double_not_float():
    # the penalized value is a double: rounding it to float32 would tie
    a = np.float32(1.0)
    b = np.float32(np.float64(a) * 1.1)  # float32 nearest to 1.1
    v = np.array([a, b], np.float32)
    exact = float(b) / 1.1               # 1.0000000217 in double, 1.0 in float32
    assert exact > 1.0 and np.float32(exact) == a
    assert penalized_argmax(v, [1], 1.1) == 1 == penalized_argmax_pure(v, [1], 1.1)


def test_window_keeps_last_n():
    w = RepeatWindow(2)
    for t in (5, 6, 7):
        w.accept(t)
    assert w.recent == [6, 7]
    w0 = RepeatWindow(0)  # max(repeat_last_n, 1)
    w0.accept(1), w0.accept(2)
    assert w0.recent == [2]


def test_vectorized_matches_list_form():
    rng = np.random.default_rng(3)
    for trial in range(300):
        n = int(rng.integers(1, 60))
        v = rng.standard_normal(n).astype(np.float32)
        if trial % 3 == 0:  # many ties
            v = np.round(v * 2).astype(np.float32) / 2
        recent = [int(t) for t in rng.integers(0, n, int(rng.integers(0, 10)))]
        p = float(rng.choice([1.1, 1.3, 0.8, 2.0, 1.0]))
        assert penalized_argmax(v, recent, p) == penalized_argmax_pure(v, recent, p)


def test_margin():
    v = np.array([1.0, 3.0, 2.5], np.float32)
    assert penalized_margin(v, [], 1.0) == pytest.approx(0.5)
    assert penalized_margin(v, [1], 2.0) == pytest.approx(1.0)  # 2.5 vs 1.5
