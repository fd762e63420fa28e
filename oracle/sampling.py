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
                 top_k: int = 0, return_margin: bool = False):
    """Temperature + nucleus sampling with a caller-supplied uniform per row.

    Restates sample_standalone.py:5611-5636 and the C twin
    llmy_cuda/src/llmy.cpp:158-201:
      * logits / temperature; optional top-k (0 = off);
      * sort descending (ties -> lower token id first);
      * probs = softmax; keep the smallest prefix whose cumulative probability
        reaches top_p (first element always kept; llmy.cpp:179-185);
      * renormalise; return the first kept token i with u < cumsum_i
        (inverse CDF, llmy.cpp:195-200), the last kept one if none.
    Arithmetic in fp64.  With return_margin, also returns per row the distance
    of the two decisions from a flip: for the nucleus, how far the cumulative
    probabilities either side of the cut are from top_p; for the draw, how far
    u is from the two CDF steps that bound the picked token.  An implementation
    whose cumulative probabilities are off by less than that margin must pick
    the same id.
    """
    x = logits.detach().double().cpu().numpy() / float(temperature)
    rows, V = x.shape
    uu = u.detach().double().cpu().numpy().reshape(-1)
    out = np.empty(rows, dtype=np.int64)
    margin = np.full(rows, np.inf)
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
            margin[r] = abs(c[cut - 1] - top_p)
            if cut >= 2:
                margin[r] = min(margin[r], abs(top_p - c[cut - 2]))
        kept = p[:cut] / p[:cut].sum()
        cdf = np.cumsum(kept)
        pick = np.nonzero(uu[r] < cdf)[0]
        i = int(pick[0]) if pick.size else cut - 1
        out[r] = order[i]
        lo = cdf[i - 1] if i > 0 else -np.inf
        margin[r] = min(margin[r], abs(cdf[i] - uu[r]), abs(uu[r] - lo))
    return (out, margin) if return_margin else out


def top_p_error_bound(logits: torch.Tensor, temperature: float, top_k: int = 0) -> np.ndarray:
    """Per row, a bound on how far the cumulative probabilities of an fp32
    implementation of top_p_sample can lie from its fp64 ones.

    An fp32 implementation forms each exponent a_i = (x_i - max) / T with a
    few roundings (the reciprocal temperature, the difference and the
    product: relative error <= 4 * 2^-24 of |a_i|, in part common to every
    term) and exponentiates it with <= 1 ulp error (2^-23), so each
    unnormalised probability carries a
    relative error delta_i <= 2^-23 (1 + 2 |a_i|).  With the sums taken
    exactly (fixed point) or in fp64, a ratio of two partial sums of such
    terms (a cumulative probability of the kept set) then moves by at most
    2 sum_i p_i |delta_i| = 2^-22 (1 + 2 E_p|a|), p the fp64 softmax over
    the top-k set; one more 2^-22 covers the fp32 products that place the
    thresholds (top_p and u times a total).  This follows the fp32 arithmetic
    the reference itself does (logits / temperature and the softmax in fp32:
    sample_standalone.py:5611-5636).
    """
    x = logits.detach().double().cpu().numpy() / float(temperature)
    rows, V = x.shape
    out = np.empty(rows)
    for r in range(rows):
        v = np.sort(x[r])[::-1]
        if top_k > 0:
            v = v[:top_k]
        v = v[np.isfinite(v)]          # -inf (masked) ids carry no mass
        if v.size == 0:
            out[r] = 2.0 ** -21
            continue
        a = v - v[0]
        p = np.exp(a)
        p /= p.sum()
        out[r] = 2.0 ** -22 * (2.0 + 2.0 * float(np.sum(p * np.abs(a))))
    return out


def repetition_penalty(logits: torch.Tensor, recent, penalty: float) -> torch.Tensor:
    """sample_standalone.py:5601-5605: each distinct id of recent[r] (ids outside
    [0, V) ignored) has its logit divided by penalty if > 0, else multiplied.
    The arithmetic is one IEEE fp32 operation with the penalty rounded to fp32,
    as it is on fp32 logits."""
    x = logits.detach().float().cpu().numpy().copy()
    V = x.shape[1]
    pen = np.float32(penalty)
    rec = np.asarray(recent)
    for r in range(x.shape[0]):
        for t in sorted(set(int(i) for i in rec[r] if 0 <= int(i) < V)):
            v = x[r, t]
            x[r, t] = v / pen if v > 0 else v * pen
    return torch.from_numpy(x)
