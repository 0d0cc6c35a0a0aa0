"""Host metrics over logits rows (x0ne-core/runtime/src/metrics.rs): the greedy argmax, log-sum-exp
and KL, in f64."""
from __future__ import annotations

import numpy as np


def argmax(row):
    """metrics.rs:10-21: first index of the largest value; None for an empty row or any NaN."""
    row = np.asarray(row, np.float32)
    if row.size == 0 or np.isnan(row).any():
        return None
    return int(np.argmax(row))


def logsumexp(row) -> float:
    x = np.asarray(row, np.float64)
    m = x.max()
    if not np.isfinite(m):
        return float(m)
    return float(m + np.log(np.exp(x - m).sum()))


def kl(p, q) -> float:
    """KL(p || q) in nats of two logits rows."""
    a = np.asarray(p, np.float64) - logsumexp(p)
    b = np.asarray(q, np.float64) - logsumexp(q)
    return float((np.exp(a) * (a - b)).sum())
