"""mHC oracle (test infrastructure only: imported by tests/ and bench.py's
cpu_baseline as the checker, never by the product path): the Sinkhorn of the
llmy_mhc_sinkhorn4 hook, and the hyper-connection maps, stream read and write
of model/layers/mhc.py:156-231.  Pinned by tests/test_oracle_mhc.py against
the reference module's own outputs (tests/golden/mhc_golden.npz) and closed
forms."""
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


# ---------------------------------------------------------------------------
# Multi-stream hyper-connection maps and stream read / write (torch, fp32 as
# the reference computes them).  Streams X [..., S, D].

F32_EPS = float(np.finfo(np.float32).eps)   # nn.RMSNorm(eps=None) on fp32 input


def sinkhorn_t(logits, iterations: int):
    """The same log-domain Sinkhorn in torch fp32 (mhc.py:12-17)."""
    import torch
    m = logits.float()
    for _ in range(int(iterations)):
        m = m - torch.logsumexp(m, dim=-1, keepdim=True)
        m = m - torch.logsumexp(m, dim=-2, keepdim=True)
    return m.exp()


def mhc_maps(X, theta, map_norm_w, pre_bias, post_bias, res_bias, alpha, iterations,
             eps: float = F32_EPS, act_round=None):
    """compute_mappings (mhc.py:156-177): RMSNorm of the flattened streams
    (weight map_norm_w, eps = fp32 machine epsilon), theta [2S + S^2, S D]
    projection, pre = sigmoid(a0 pre_raw + pre_bias), post = 2 sigmoid(a1
    post_raw + post_bias), residual = Sinkhorn(a2 res_raw + res_bias).
    ``act_round`` (optional) rounds the normalised input of the projection.
    Returns (pre [..., S], post [..., S], residual [..., S, S])."""
    import torch
    S, D = X.shape[-2], X.shape[-1]
    flat = X.reshape(*X.shape[:-2], S * D).float()
    flat = flat * torch.rsqrt(flat.pow(2).mean(-1, keepdim=True) + eps) * map_norm_w.float()
    if act_round is not None:
        flat = act_round(flat)
    raw = flat @ theta.float().t()
    pre_raw, post_raw, res_raw = raw.split([S, S, S * S], dim=-1)
    a = alpha.float()
    pre = torch.sigmoid(a[0] * pre_raw + pre_bias.float())
    post = 2.0 * torch.sigmoid(a[1] * post_raw + post_bias.float())
    res = sinkhorn_t(a[2] * res_raw.reshape(*res_raw.shape[:-1], S, S) + res_bias.float(),
                     iterations)
    return pre, post, res


def mhc_read(X, pre, ln_w, ln_b, eps: float = 1e-5):
    """read (mhc.py:195-206): sum_s pre_s X_s, then LayerNorm (weight, bias)."""
    import torch
    import torch.nn.functional as F
    value = torch.einsum("...s,...sd->...d", pre.float(), X.float())
    return F.layer_norm(value, (value.shape[-1],), ln_w.float(), ln_b.float(), eps)


def mhc_write(X, U, post, residual, scale, gating_logit):
    """write (mhc.py:208-227): X_i + sigmoid(gating) scale_i (sum_j R_ij X_j + post_i U)."""
    import torch
    mixed = torch.einsum("...ij,...jd->...id", residual.float(), X.float())
    upd = (mixed + post.float()[..., None] * U.float()[..., None, :]) * scale.float()
    return X.float() + torch.sigmoid(gating_logit.float().reshape(())) * upd
