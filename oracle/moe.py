"""SwiGLU MoE oracle (test infrastructure only)."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def swiglu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor,
           w_down: torch.Tensor) -> torch.Tensor:
    """``W_down (silu(W_gate x) * W_up x)`` in fp32.

    Restates model/layers/expert.py:14-15 (nn.Linear layout [out, in]).
    """
    xf = x.float()
    return (F.silu(xf @ w_gate.float().t()) * (xf @ w_up.float().t())) @ w_down.float().t()


def moe_grouped(x: torch.Tensor, idx: np.ndarray, gates: torch.Tensor, w_gate: torch.Tensor,
                w_up: torch.Tensor, w_down: torch.Tensor, act_round=None) -> torch.Tensor:
    """Routed SwiGLU MoE, grouped by expert, fp32 accumulation.

    out[t] = sum_j gates[t,j] * expert_{idx[t,j]}(x[t]).
    Restates the dispatch of model/layers/moe.py:29-82 (group routes by expert,
    gate_up bmm, silu(g)*u, down bmm, gate-weighted combine) without capacity
    padding (no token dropping, moe.py:56-58).  Experts: w_gate, w_up [E,H,D],
    w_down [E,D,H].  ``act_round`` (e.g. a bf16 round trip) is applied to the
    SwiGLU activation before the down projection, where a bf16 kernel stores it.
    """
    T, D = x.shape
    k = idx.shape[1]
    E = w_gate.shape[0]
    xf = x.float()
    flat = np.asarray(idx).reshape(-1)
    out = torch.zeros(T, D, dtype=torch.float32)
    contrib = torch.zeros(T * k, D, dtype=torch.float32)
    gflat = gates.reshape(-1).float()
    for e in range(E):
        routes = np.nonzero(flat == e)[0]
        if routes.size == 0:
            continue
        r = torch.from_numpy(routes)
        xe = xf[r // k]
        act = F.silu(xe @ w_gate[e].float().t()) * (xe @ w_up[e].float().t())
        if act_round is not None:
            act = act_round(act)
        contrib[r] = (act @ w_down[e].float().t()) * gflat[r].unsqueeze(-1)
    for j in range(k):
        out += contrib.view(T, k, D)[:, j]
    return out


def moe_per_token(x: torch.Tensor, idx: np.ndarray, gates: torch.Tensor, w_gate: torch.Tensor,
                  w_up: torch.Tensor, w_down: torch.Tensor) -> torch.Tensor:
    """Brute-force routed MoE, one token and one route at a time (tiny sizes).

    Independent restatement of expert.py:15 + moe.py:78-81 used to pin
    ``moe_grouped``.
    """
    T, D = x.shape
    k = idx.shape[1]
    out = torch.zeros(T, D, dtype=torch.float64)
    for t in range(T):
        for j in range(k):
            e = int(idx[t, j])
            xv = x[t].double()
            g = w_gate[e].double() @ xv
            u = w_up[e].double() @ xv
            a = g / (1.0 + torch.exp(-g)) * u
            out[t] += float(gates[t, j]) * (w_down[e].double() @ a)
    return out.float()
