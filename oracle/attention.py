"""Banded (sliding-window) causal attention oracle (test infrastructure only)."""
from __future__ import annotations

import math

import torch


def banded_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int,
                     scale: float | None = None, block: int = 256) -> torch.Tensor:
    """o_i = sum_{j: 0 <= i-j < W} softmax_j(scale * q_i.k_j) v_j, per (b, h).

    Layout [B, T, H, hd]; fp32 scores and accumulation.  Mask restates
    runpod/kernels/fused_attention.py:27 (row >= col and row - col < W);
    scale 1/sqrt(hd) as runpod/kernels/triton_banded_attention.py:97-98.
    Queries are processed in blocks so memory stays O(block * (block + W)).
    """
    B, T, H, hd = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(hd)
    qf, kf, vf = (t.float().permute(0, 2, 1, 3) for t in (q, k, v))  # [B,H,T,hd]
    out = torch.empty(B, H, T, hd, dtype=torch.float32)
    for i0 in range(0, T, block):
        i1 = min(T, i0 + block)
        j0 = max(0, i0 - window + 1)
        s = torch.matmul(qf[:, :, i0:i1], kf[:, :, j0:i1].transpose(-1, -2)) * scale
        rows = torch.arange(i0, i1).view(-1, 1)
        cols = torch.arange(j0, i1).view(1, -1)
        mask = (rows >= cols) & (rows - cols < window)
        s = s.masked_fill(~mask, float("-inf"))
        p = torch.softmax(s, dim=-1)
        out[:, :, i0:i1] = torch.matmul(p, vf[:, :, j0:i1])
    return out.permute(0, 2, 1, 3).contiguous()


def banded_attention_decode(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                            k_cache: torch.Tensor, v_cache: torch.Tensor, pos: torch.Tensor,
                            scale: float | None = None):
    """One decode step of banded attention against a ring-buffer KV cache.

    q, k_new, v_new [B, H, hd]; caches [B, H, W, hd]; pos [B] = absolute
    position of the new token.  The new K/V is written to slot pos % W first,
    then the query attends to the last min(pos + 1, W) tokens, current one
    included — the decode window of model/layers/hca.py:119-128.  Returns
    (o [B, H, hd] fp32, k_cache', v_cache') without modifying the inputs.
    """
    B, H, W, hd = k_cache.shape
    if scale is None:
        scale = 1.0 / math.sqrt(hd)
    kc = k_cache.clone()
    vc = v_cache.clone()
    o = torch.empty(B, H, hd, dtype=torch.float32)
    for b in range(B):
        p = int(pos[b])
        slot = p % W
        kc[b, :, slot] = k_new[b]
        vc[b, :, slot] = v_new[b]
        n_valid = min(p + 1, W)
        if n_valid == W:
            keys, vals = kc[b].float(), vc[b].float()
        else:
            keys, vals = kc[b, :, :n_valid].float(), vc[b, :, :n_valid].float()
        s = torch.einsum("hd,hsd->hs", q[b].float(), keys) * scale
        o[b] = torch.einsum("hs,hsd->hd", torch.softmax(s, dim=-1), vals)
    return o, kc, vc
