"""Sampling oracle: greedy argmax and temperature + top-p (test infrastructure only)."""
from __future__ import annotations

import numpy as np
import torch


def argmax(logits: torch.Tensor) -> np.ndarray:
    """First index of the row maximum (NaN counts as the maximum).

    Restates sample_standalone.py:5609-5610 (torch.argmax).  Implemented with
    numpy's argmax, which has the same first-occurrence and NaN rules, so the
    oracle does not share code with the call it restates.
    """
    return np.argmax(logits.detach().float().cpu().numpy(), axis=-1).astype(np.int64)


def top_p_sample(logits: torch.Tensor, temperature: float, top_p: float, u: torch.Tensor,
                 top_k: int = 0) -> np.ndarray:
    """Temperature + nucleus sampling with a caller-supplied uniform per row.

    Restates sample_standalone.py:5611-5636 and the C twin
    llmy_cuda/src/llmy.cpp:158-201:
      * logits / temperature; optional top-k (0 = off);
      * sort descending (ties -> lower token id first);
      * probs = softmax; keep the smallest prefix whose cumulative probability
        reaches top_p (first element always kept; llmy.cpp:179-185);
      * renormalise; return the first kept token i with u < cumsum_i
        (inverse CDF, llmy.cpp:195-200), the last kept one if none.
    Arithmetic in fp64.
    """
    x = logits.detach().double().cpu().numpy() / float(temperature)
    rows, V = x.shape
    uu = u.detach().double().cpu().numpy().reshape(-1)
    out = np.empty(rows, dtype=np.int64)
    ids = np.arange(V)
    for r in range(rows):
        order = np.lexsort((ids, -x[r]))
        if top_k > 0:
            order = order[:top_k]
        vals = x[r][order]
        p = np.exp(vals - vals[0])
        p /= p.sum()
        cut = len(order)
        if 0.0 < top_p < 1.0:
            c = np.cumsum(p)
            hit = np.nonzero(c >= top_p)[0]
            if hit.size:
                cut = int(hit[0]) + 1
        kept = p[:cut] / p[:cut].sum()
        cdf = np.cumsum(kept)
        pick = np.nonzero(uu[r] < cdf)[0]
        out[r] = order[int(pick[0])] if pick.size else order[cut - 1]
    return out
