"""Helpers of the sampler tests: whether a sampling decision lies far
enough from its thresholds that the reference's f32 running sums and exact
running sums must decide it the same way.

The margin is twice the drift the reference's own f32 running sum shows on
the case (measured against an f64 sum), plus `rel`, the largest relative
difference between the two sides' probabilities (the reference's f32
softmax sum over 10^5 terms is itself off by ~1e-5 relative, which scales
every probability), plus `slack`.
"""

from __future__ import annotations

import numpy as np


def _margin(p_sorted: np.ndarray, rel: float, slack: float) -> tuple[np.ndarray, float]:
    cum64 = np.cumsum(p_sorted.astype(np.float64))
    cum32 = np.add.accumulate(p_sorted.astype(np.float32), dtype=np.float32)
    return cum64, 2.0 * float(np.max(np.abs(cum32 - cum64), initial=0.0)) + rel + slack


def rel_diff(p_a: np.ndarray, p_b: np.ndarray) -> float:
    """Largest relative difference of two probability vectors (over the
    entries above 1e-30)."""
    a, b = np.asarray(p_a, np.float64), np.asarray(p_b, np.float64)
    big = b > 1e-30
    return float(np.max(np.abs(a[big] - b[big]) / b[big], initial=0.0))


def robust_topp(p: np.ndarray, topp: float, coin: float, rel: float = 0.0, slack: float = 1e-6) -> bool:
    n = p.size
    with np.errstate(divide="ignore", invalid="ignore"):  # n == 1: cutoff inf
        cutoff = np.float32((np.float32(1) - np.float32(topp)) / (np.float32(n) - np.float32(1)))
        cand = np.nonzero(p >= cutoff)[0]
    if cand.size == 0:
        return True
    order = cand[np.lexsort((cand, -p[cand]))]
    cum, delta = _margin(p[order], rel, slack)
    if np.min(np.abs(cum - np.float64(topp))) < delta:
        return False
    hit = np.nonzero(cum > topp)[0]
    last = int(hit[0]) if hit.size else order.size - 1
    r = np.float64(coin) * cum[last]
    return bool(np.min(np.abs(cum[: last + 1] - r)) >= delta)


def robust_mult(p: np.ndarray, coin: float, rel: float = 0.0, slack: float = 1e-6) -> bool:
    cdf, delta = _margin(np.asarray(p), rel, slack)
    return bool(np.min(np.abs(cdf - np.float64(coin))) >= delta)
