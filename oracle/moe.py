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


def shared_experts(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor,
                   w_down: torch.Tensor, act_round=None) -> torch.Tensor:
    """Shared experts: every token through each of the S dense SwiGLU experts,
    summed, then scaled by 1/sqrt(S); fp32.  Restates model/layers/moe.py:
    185-199 (``sum(expert(flat) for expert in self.shared) / sqrt(S)``) and
    llmy_cuda/src/model.cpp:1205-1225 (sum, then scale by 1/sqrt(S)).
    w_gate, w_up [S,H,D], w_down [S,D,H]; ``act_round`` as in moe_grouped."""
    S = w_gate.shape[0]
    xf = x.float()
    out = torch.zeros(x.shape[0], w_down.shape[1], dtype=torch.float32)
    for s in range(S):
        act = F.silu(xf @ w_gate[s].float().t()) * (xf @ w_up[s].float().t())
        if act_round is not None:
            act = act_round(act)
        out += act @ w_down[s].float().t()
    return out / np.float32(np.sqrt(S))


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


def moe_selected_fp32(x: np.ndarray, idx: np.ndarray, prob: np.ndarray, gate_up: np.ndarray,
                      down: np.ndarray):
    """One-token selected-expert MoE with the packed gate_up [E, 2H, D] layout.

    Restates the PyTorch path of sample_standalone.py:3065-3075 (index_select
    the k experts, gate_up GEMV, silu(g) * u, down GEMV, prob-weighted sum)
    and the scratch contents of llmy_cuda/src/kernels/moe.cu:174-267
    (activation [k, H], route_output [k, D] = prob * expert output).  Routes
    with an id outside [0, E) contribute zeros.  fp64; returns
    (activation, route_output, out).
    """
    x = np.asarray(x, dtype=np.float64).reshape(-1)
    E, H2, D = gate_up.shape
    H = H2 // 2
    k = idx.size
    act = np.zeros((k, H))
    ro = np.zeros((k, D))
    for j in range(k):
        e = int(idx.reshape(-1)[j])
        if not 0 <= e < E:
            continue
        gu = gate_up[e].astype(np.float64) @ x
        g, u = gu[:H], gu[H:]
        act[j] = g / (1.0 + np.exp(-g)) * u
        ro[j] = float(prob.reshape(-1)[j]) * (down[e].astype(np.float64) @ act[j])
    return act, ro, ro.sum(0)
