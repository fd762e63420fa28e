"""Router and token permutation oracle (test infrastructure only)."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def rmsnorm(x: torch.Tensor, weight: torch.Tensor | None, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm in fp32: ``x * rsqrt(mean(x^2) + eps) * w``.

    Restates model/layers/norms.py:13-16 (fp32 variance, eps 1e-6).
    """
    xf = x.float()
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    out = xf * torch.rsqrt(var + eps)
    if weight is not None:
        out = out * weight.float()
    return out


def router_logits(x: torch.Tensor, w_router: torch.Tensor, norm_w: torch.Tensor | None = None,
                  eps: float = 1e-6) -> torch.Tensor:
    """fp32 router logits ``RMSNorm(x) @ W_r^T``.

    Restates model/layers/context_router.py:62,71-72 with context_aware=False.
    ``norm_w=None`` skips the router's own RMSNorm (the bare logits op).
    """
    h = rmsnorm(x, norm_w, eps) if norm_w is not None else x.float()
    return h @ w_router.float().t()


def layernorm(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, eps: float = 1e-5
              ) -> torch.Tensor:
    """``(x - mean) / sqrt(var + eps) * w + b`` over the last dim, biased
    variance, in fp64 then fp32.  Restates torch.nn.LayerNorm with its default
    eps 1e-5, the latent norm of model/layers/mla_memory.py:21,23-24."""
    xd = x.double()
    mu = xd.mean(-1, keepdim=True)
    var = (xd - mu).pow(2).mean(-1, keepdim=True)
    return ((xd - mu) / torch.sqrt(var + eps) * w.double() + b.double()).float()


def context_latents(h: torch.Tensor, norm_w: torch.Tensor, w_down: torch.Tensor,
                    ln_w: torch.Tensor, ln_b: torch.Tensor, eps: float = 1e-6
                    ) -> tuple[torch.Tensor, torch.Tensor]:
    """(local, lat): local = RMSNorm(h) * norm_w (context_router.py:61), lat =
    LayerNorm(local . W_down^T) (MLALatentMemory.encode, mla_memory.py:23-24)."""
    local = rmsnorm(h, norm_w, eps)
    lat = layernorm((local.double() @ w_down.double().t()).float(), ln_w, ln_b)
    return local, lat


def context_window_mean(lat: torch.Tensor, window: int) -> torch.Tensor:
    """Causal box mean over the last ``window`` latents of a sequence starting at
    position 0: ctx[t] = mean(lat[max(0, t-W+1) .. t]) along dim -2 (fp64 sums).

    Restates MLALatentMemory.forward (mla_memory.py:29-48: a width-W box filter
    with the first positions divided by t+1 instead of W) and, token by token,
    ContextAwareRouter.forward_step (context_router.py:108-128: the mean of the
    rolling history plus the current latent, its last W entries)."""
    x = lat.double()
    T = x.shape[-2]
    c = torch.cumsum(x, dim=-2)
    out = torch.empty_like(x)
    for t in range(T):
        lo = t - window
        s = c[..., t, :] - (c[..., lo, :] if lo >= 0 else 0.0)
        out[..., t, :] = s / min(t + 1, window)
    return out.float()


def context_route_logits(local: torch.Tensor, ctx: torch.Tensor, w_local_out: torch.Tensor,
                         w_ctx_out: torch.Tensor, route_gate: torch.Tensor,
                         w_router: torch.Tensor, act_round=lambda t: t,
                         global_ctx: torch.Tensor | None = None) -> torch.Tensor:
    """route = local + sigmoid(g) * context_out(local_context_out(ctx) [+
    global_ctx]); logits = route . W_r^T (context_router.py:65-72; global_ctx is
    the HCA global branch of :66-68, ``hca_global_context``).  ``act_round``
    rounds the inputs of the two projections where the HIP path stores them in
    bf16."""
    cl = act_round(act_round(ctx) @ w_local_out.float().t()
                   + (0.0 if global_ctx is None else global_ctx))
    c = cl @ w_ctx_out.float().t()
    route = local + torch.sigmoid(route_gate.float()) * c
    return route @ w_router.float().t()


def topk_lower_index(logits: torch.Tensor, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Indices and values of the k largest entries per row.

    Order: descending value; equal values -> lower index first; NaN above
    everything (torch.topk's comparison).  The reference uses torch.topk
    (context_router.py:73), whose tie order is unspecified; this pins it.
    Implemented as a lexicographic sort so it is independent of torch.topk.
    """
    v = logits.detach().float().cpu().numpy()
    rows, n = v.shape
    idx = np.empty((rows, k), dtype=np.int64)
    vals = np.empty((rows, k), dtype=np.float32)
    cols = np.arange(n)
    for r in range(rows):
        row = v[r]
        nan = np.isnan(row)
        clean = np.where(nan, 0.0, row)
        clean = np.where(clean == 0.0, 0.0, clean)  # -0.0 == +0.0
        order = np.lexsort((cols, -clean, ~nan))
        idx[r] = order[:k]
        vals[r] = row[order[:k]]
    return idx, vals


def router_topk(logits: torch.Tensor, k: int) -> tuple[np.ndarray, torch.Tensor]:
    """(expert ids [T,k] int64, gates [T,k] fp32 = softmax of the k values).

    Restates context_router.py:73-74 with the tie rule of topk_lower_index.
    """
    idx, vals = topk_lower_index(logits, k)
    gates = torch.from_numpy(vals).softmax(dim=-1)
    return idx, gates


def moe_permute(expert_ids: np.ndarray, num_experts: int) -> dict[str, np.ndarray]:
    """Stable counting sort of flat route ids ``r = t*k + j`` by expert.

    Restates model/layers/moe.py:42-60 (flat routes, sort by expert, bincount,
    exclusive-cumsum offsets) with the sort made stable (moe.py:46 uses an
    unstable torch.sort; the combined output does not depend on the order).
    Returns counts [E], offsets [E+1], sorted_routes [n], route_pos [n].
    """
    ids = np.asarray(expert_ids, dtype=np.int64).reshape(-1)
    counts = np.bincount(ids, minlength=num_experts).astype(np.int64)
    offsets = np.zeros(num_experts + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    sorted_routes = np.argsort(ids, kind="stable").astype(np.int64)
    route_pos = np.empty_like(sorted_routes)
    route_pos[sorted_routes] = np.arange(ids.size)
    return {"counts": counts, "offsets": offsets, "sorted_routes": sorted_routes,
            "route_pos": route_pos}


def hca_global_context(local: torch.Tensor, values: list, w_down, ln_w, ln_b, w_q, w_k, w_v,
                       w_o, heads: int, head_dim: int, act_round=lambda t: t) -> torch.Tensor:
    """The router's global branch (context_router.py:66-68,126-127;
    mla_memory.py:52-90) over an HCA block's summaries, as the native engine
    computes it (router_hca_latent_attention, llmy_cuda/src/model.cpp:972-1062:
    the block's own emitted summaries, masked to those visible): latents =
    LayerNorm(down . value) (hca_latent, mla_memory.py:23-24, eps 1e-5), then
    o(MHA(q(local), k(latents), v(latents))) with scale 1/sqrt(head_dim).
    ``values[b]`` [n_b, D] holds row b's visible summary values (n_b may be 0:
    that row's branch is 0).  Returns [B, D] fp32 (the o projection's input
    rounded by ``act_round``)."""
    B = local.shape[0]
    HQ = heads * head_dim
    q = act_round(act_round(local) @ w_q.float().t()).double().view(B, heads, head_dim)
    att = torch.zeros(B, HQ, dtype=torch.float64)
    for b in range(B):
        v = values[b]
        if v.shape[0] == 0:
            continue
        raw = act_round(v).double() @ w_down.double().t()
        lat = act_round(F.layer_norm(raw, (raw.shape[-1],), ln_w.double(), ln_b.double(),
                                     1e-5).float())
        kk = act_round(lat @ w_k.float().t()).double().view(-1, heads, head_dim)
        vv = act_round(lat @ w_v.float().t()).double().view(-1, heads, head_dim)
        sc = torch.einsum("hd,nhd->hn", q[b], kk) / head_dim ** 0.5
        att[b] = torch.einsum("hn,nhd->hd", sc.softmax(-1), vv).reshape(HQ)
    return act_round(att.float()) @ w_o.float().t()
