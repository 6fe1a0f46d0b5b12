"""Host-side schedule maths of the approximate top-k (trace-time logic of the
reference, computed in Python exactly as the reference does it in numpy).

Reference: tallax/top_k_convergence_theory.py:5-128 and top_dynamic_k's
schedule handling (tallax/_src/top_k.py:472-478).  Throwing k balls
uniformly into `num_bins` bins, the maximum occupancy is <= m with
probability k! / num_bins^k * [x^k] (sum_{i<=m} x^i / i!)^num_bins; the
polynomial power is taken by repeated squaring in log space (shifted by the
maximum before exponentiating) and truncated at degree k.
"""
from __future__ import annotations

import functools
import math

import numpy as np


def _lgamma(a: np.ndarray) -> np.ndarray:
    return np.array([math.lgamma(float(v)) for v in np.ravel(a)]).reshape(np.shape(a))


def _log_poly_mul(log_a: np.ndarray, log_b: np.ndarray, trunc: int) -> np.ndarray:
    sa, sb = np.max(log_a), np.max(log_b)
    if sa == -np.inf or sb == -np.inf:
        return np.full(min(len(log_a) + len(log_b) - 1, trunc), -np.inf)
    lin = np.convolve(np.exp(log_a - sa), np.exp(log_b - sb))[:trunc]
    with np.errstate(divide="ignore"):
        return np.log(lin) + sa + sb


def max_occupancy_pdf(k: int, num_bins: int) -> np.ndarray:
    """P(max bin occupancy == m) for m = 1..k (index m - 1)."""
    log_k_fact = math.lgamma(k + 1)
    log_denom = k * math.log(num_bins)
    pdf = np.zeros(k)
    prev = 0.0
    for m in range(1, k + 1):
        base = -_lgamma(np.arange(min(m + 1, k + 1)) + 1.0)   # log(1 / i!)
        acc = np.array([0.0])
        p = num_bins
        while p > 0:
            if p & 1:
                acc = _log_poly_mul(acc, base, k + 1)
            if p > 1:
                base = _log_poly_mul(base, base, k + 1)
            p >>= 1
        log_cdf = (acc[k] if len(acc) > k else -np.inf) + log_k_fact - log_denom
        cdf = min(1.0, math.exp(log_cdf) if log_cdf > -700 else 0.0)
        pdf[m - 1] = max(0.0, cdf - prev)
        prev = cdf
        if cdf >= 1.0 - 1e-14:
            break
    return pdf


def calculate_depth_thresholds(k: int, num_bins: int, block_size: int = 8,
                               target_yields=(0.66, 0.95, 0.9999)) -> tuple:
    """Smallest depths d (1-based) with P(max occupancy <= d)**block_size >=
    each target yield (top_k_convergence_theory.py:106-128)."""
    cdf = np.cumsum(max_occupancy_pdf(k, num_bins))
    block = cdf ** block_size
    out = set()
    for target in target_yields:
        hit = np.nonzero(block >= target)[0]
        if hit.size:
            out.add(int(hit[0]) + 1)
    return tuple(sorted(out))


@functools.lru_cache(maxsize=256)
def _auto_schedule(max_k: int, num_bins: int, block_token: int) -> tuple:
    # computed once per shape, as the reference computes it once per trace
    # (a few hundred microseconds of polynomial arithmetic on the host)
    return tuple(t + 1 for t in calculate_depth_thresholds(max_k, num_bins, block_token,
                                                           target_yields=(0.8, 0.98, 0.9999)))


def topm_schedule(max_k: int, num_bins: int, block_token: int, schedule=None) -> tuple:
    """The depths top_dynamic_k evaluates (top_k.py:472-478), without the
    leading 0: the automatic one is the depth thresholds at yields
    (0.8, 0.98, 0.9999) plus one; user schedules are deduplicated and sorted."""
    if schedule is None:
        schedule = _auto_schedule(int(max_k), int(num_bins), int(block_token))
    return tuple(sorted(set(int(m) for m in schedule)))
