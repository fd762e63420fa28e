"""mHC Sinkhorn oracle (test infrastructure only: imported by tests/ and
bench.py's cpu_baseline as the checker, never by the product path)."""
from __future__ import annotations

import numpy as np


def sinkhorn4(logits: np.ndarray, iterations: int) -> np.ndarray:
    """Log-domain Sinkhorn over the last two axes (4 x 4 matrices).

    Restates the PyTorch path of sample_standalone.py:2582-2586: per
    iteration subtract each row's logsumexp, then each column's; return exp
    of the result.  fp64.
    """
    m = np.asarray(logits, dtype=np.float64).copy()
    for _ in range(int(iterations)):
        for axis in (-1, -2):
            mx = m.max(axis=axis, keepdims=True)
            lse = mx + np.log(np.exp(m - mx).sum(axis=axis, keepdims=True))
            m = m - lse
    return np.exp(m)
