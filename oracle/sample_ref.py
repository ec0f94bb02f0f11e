"""Oracle: greedy selection with the repetition penalty (TEST INFRASTRUCTURE -
see oracle/__init__.py).

Restates the reference's sampler at temperature <= 0 (alpacca/sample.py):

* ``RepeatWindow`` - Sampler.accept (sample.py:31-34): the last
  max(repeat_last_n, 1) accepted tokens.
* ``penalized_argmax`` - Sampler.sample's penalty and greedy branch
  (sample.py:36-45): the float32 logits become Python floats
  (tensor.to_list, tensor.py:74-77); every distinct recent token t gets
  v / penalty when v > 0, else v * penalty, in double; the result is the
  first index of the maximum (max over range with a key keeps the first).
  Vectorized over NumPy float64, whose division and product are the same
  IEEE double operations as Python's.
* ``penalized_argmax_pure`` - the same in the reference's own list form, for
  small inputs (the vectorized form is checked against it).
"""
from __future__ import annotations

import numpy as np


class RepeatWindow:
    """The recent-token list of the sampler (sample.py:31-34)."""

    def __init__(self, last_n: int = 64):
        self.last_n = last_n
        self.recent: list[int] = []

    def accept(self, token: int) -> None:
        self.recent.append(int(token))
        if len(self.recent) > max(self.last_n, 1):
            self.recent.pop(0)


def penalized_argmax(logits, recent, penalty: float) -> int:
    vals = np.asarray(logits, dtype=np.float32).astype(np.float64)
    if penalty and penalty != 1.0 and len(recent):
        for t in set(int(r) for r in recent):
            v = vals[t]
            vals[t] = v / penalty if v > 0 else v * penalty
    return int(np.argmax(vals))


def penalized_argmax_pure(logits, recent, penalty: float) -> int:
    vals = np.asarray(logits, dtype=np.float32).tolist()
    if penalty and penalty != 1.0 and recent:
        for t in set(recent):
            v = vals[t]
            vals[t] = v / penalty if v > 0 else v * penalty
    return max(range(len(vals)), key=vals.__getitem__)


def penalized_margin(logits, recent, penalty: float) -> float:
    """Gap between the largest and second-largest penalized value."""
    vals = np.asarray(logits, dtype=np.float32).astype(np.float64)
    if penalty and penalty != 1.0 and len(recent):
        for t in set(int(r) for r in recent):
            v = vals[t]
            vals[t] = v / penalty if v > 0 else v * penalty
    top2 = np.partition(vals, -2)[-2:]
    return float(top2.max() - top2.min())
