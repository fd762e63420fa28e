"""Gated delta-rule (GDN) recurrence oracle (test infrastructure only).

The reference transition (model/layers/gated_deltanet.py:140-149) is

    pred_t = k_t^T S_{t-1}                      (undecayed state)
    S_t    = g_t S_{t-1} + beta_t k_t (v_t - pred_t)^T
    o_t    = (q_t^T S_t) * gate_t

with S [dk, dv] fp32 per (batch, head).  The reference's decay is the
per-head constant sigmoid(decay_logit[h]) (gated_deltanet.py:132); here g is
per (b, t, h), of which the reference is the special case.
"""
from __future__ import annotations

import torch


def gdn_sequential(q, k, v, beta, g, state, gate=None, dtype=torch.float32, reset=None):
    """Sequential recurrence over T, restating gated_deltanet.py:140-149.

    q, k [B,T,H,dk]; v [B,T,H,dv]; beta, g [B,T,H]; state [B,H,dk,dv];
    gate [B,T,H,dv] or None.  Arithmetic in ``dtype`` (fp32 as the reference;
    fp64 for pinning).  ``reset`` [B,T] bool or None: where set, the state is
    zeroed before token t's update (the carry reset of gated_deltanet.py:138-142).
    Returns (o [B,T,H,dv], final state [B,H,dk,dv]).
    """
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    S = state.to(dtype).clone()
    qd, kd, vd = q.to(dtype), k.to(dtype), v.to(dtype)
    bd, gd = beta.to(dtype), g.to(dtype)
    out = torch.empty(B, T, H, dv, dtype=dtype)
    rs = None if reset is None else torch.as_tensor(reset).to(torch.bool).view(B, T)
    for t in range(T):
        if rs is not None:
            S = torch.where(rs[:, t, None, None, None], torch.zeros_like(S), S)
        kt = kd[:, t]
        pred = torch.einsum("bhk,bhkv->bhv", kt, S)
        delta = vd[:, t] - pred
        S = gd[:, t, :, None, None] * S + bd[:, t, :, None, None] * torch.einsum(
            "bhk,bhv->bhkv", kt, delta)
        out[:, t] = torch.einsum("bhk,bhkv->bhv", qd[:, t], S)
    if gate is not None:
        out = out * gate.to(dtype)
    return out, S


def gdn_step(q, k, v, beta, g, state, gate=None, dtype=torch.float32, reset=None):
    """One-token update (T = 1) of ``gdn_sequential``; q,k,v [B,H,d], beta,g [B,H];
    reset [B] or None."""
    o, S = gdn_sequential(q[:, None], k[:, None], v[:, None], beta[:, None], g[:, None],
                          state, None if gate is None else gate[:, None], dtype,
                          None if reset is None else torch.as_tensor(reset).view(-1, 1))
    return o[:, 0], S


def causal_conv_reset(h, hist, w, reset=None):
    """Causal depthwise conv over a sequence with a carried history, restating
    gated_deltanet.py:56-78 (taps do not cross a reset) token by token, the
    decode rule of :257-270 (window = [history, h_t]; a reset clears the
    history first).  h [B,T,D], hist [B,K-1,D], w [D,K]; reset [B,T] or None.
    Returns (pre-sigmoid conv [B,T,D], new history [B,K-1,D])."""
    B, T, D = h.shape
    hist = hist.clone()
    out = torch.empty(B, T, D, dtype=h.dtype)
    rs = None if reset is None else torch.as_tensor(reset).to(torch.bool).view(B, T)
    for t in range(T):
        if rs is not None:
            hist = torch.where(rs[:, t, None, None], torch.zeros_like(hist), hist)
        window = torch.cat([hist, h[:, t:t + 1]], dim=1)      # [B, K, D]
        out[:, t] = (window * w.t()[None]).sum(1)
        hist = window[:, 1:]
    return out, hist


def gdn_chunked(q, k, v, beta, g, state, chunk=64, dtype=torch.float64):
    """Chunk-parallel form of the same recurrence (the build's own algorithm).

    Within a chunk starting from S0, with Gamma_t = prod_{j<=t} g_j (log-space
    cumulative sums, so every ratio used is <= 1):
      U  = (I + L)^{-1} [beta * (V - Gamma_{t-1} K S0)],
           L[t,i] = beta_t (Gamma_{t-1}/Gamma_i) k_t.k_i  for i < t
      O  = Gamma Q S0 + [(Gamma_t/Gamma_i)_{i<=t} * (Q K^T)] U
      S' = Gamma_C S0 + K^T diag(Gamma_C/Gamma_i) U
    Substituting S_t = Gamma_t S0 + sum_{i<=t} (Gamma_t/Gamma_i) k_i u_i^T into
    the recurrence gives u_t = beta_t (v_t - S_{t-1}^T k_t), hence the lower
    triangular system.  Checked against ``gdn_sequential``.
    """
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    S = state.to(dtype).clone()
    out = torch.empty(B, H, T, dv, dtype=dtype)
    qd = q.to(dtype).permute(0, 2, 1, 3)  # [B,H,T,dk]
    kd = k.to(dtype).permute(0, 2, 1, 3)
    vd = v.to(dtype).permute(0, 2, 1, 3)
    bd = beta.to(dtype).permute(0, 2, 1)  # [B,H,T]
    lg = torch.log(g.to(dtype)).permute(0, 2, 1)
    for c0 in range(0, T, chunk):
        c1 = min(T, c0 + chunk)
        C = c1 - c0
        Q, K, V = qd[:, :, c0:c1], kd[:, :, c0:c1], vd[:, :, c0:c1]
        bt = bd[:, :, c0:c1]
        cum = torch.cumsum(lg[:, :, c0:c1], dim=-1)            # log Gamma_t, t=1..C
        prev = torch.cat([torch.zeros_like(cum[..., :1]), cum[..., :-1]], dim=-1)  # log Gamma_{t-1}
        tri_strict = torch.tril(torch.ones(C, C, dtype=torch.bool), -1)
        tri = torch.tril(torch.ones(C, C, dtype=torch.bool))
        ratio_prev = torch.exp((prev[..., :, None] - cum[..., None, :]).masked_fill(~tri_strict, -torch.inf))
        L = bt[..., :, None] * ratio_prev * (K @ K.transpose(-1, -2))
        A = torch.eye(C, dtype=dtype) + L
        rhs = bt[..., None] * (V - torch.exp(prev)[..., None] * (K @ S))
        U = torch.linalg.solve_triangular(A, rhs, upper=False, unitriangular=True)
        ratio = torch.exp((cum[..., :, None] - cum[..., None, :]).masked_fill(~tri, -torch.inf))
        O = torch.exp(cum)[..., None] * (Q @ S) + (ratio * (Q @ K.transpose(-1, -2))) @ U
        out[:, :, c0:c1] = O
        last = cum[..., -1:]
        S = torch.exp(last)[..., None] * S + K.transpose(-1, -2) @ (torch.exp(last - cum)[..., None] * U)
    return out.permute(0, 2, 1, 3).contiguous(), S
