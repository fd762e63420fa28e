"""Torch-facing wrappers over the libllmy C ABI.

Each op checks device, dtype, contiguity and shape on the host, allocates its
outputs with torch (device memory is plumbing; kernels never allocate), and
launches on torch's current HIP stream.  A failed launch raises; there is no
eager/CPU fallback.
"""
from __future__ import annotations

import torch

from . import _lib


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _check(t: torch.Tensor, dtype: torch.dtype, name: str, shape: tuple | None = None) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} shape {tuple(t.shape)} != expected {tuple(shape)}")


# --------------------------------------------------------------------------- router
def router_topk(x: torch.Tensor, w_router: torch.Tensor, k: int,
                norm_w: torch.Tensor | None = None, eps: float = 1e-6,
                return_logits: bool = False):
    """(idx [T,k] int32, gates [T,k] fp32[, logits [T,E] fp32]) for bf16 x [T,D]."""
    T, D = x.shape
    E = w_router.shape[0]
    _check(x, torch.bfloat16, "x")
    _check(w_router, torch.float32, "w_router", (E, D))
    if norm_w is not None:
        _check(norm_w, torch.float32, "norm_w", (D,))
    idx = torch.empty(T, k, dtype=torch.int32, device=x.device)
    gates = torch.empty(T, k, dtype=torch.float32, device=x.device)
    logits = torch.empty(T, E, dtype=torch.float32, device=x.device) if return_logits else None
    _lib.call("llmy_router_topk_bf16", _ptr(x), _ptr(norm_w), _ptr(w_router), _ptr(logits),
              _ptr(idx), _ptr(gates), T, D, E, k, eps, _stream())
    return (idx, gates, logits) if return_logits else (idx, gates)


def router_topk_from_logits(logits: torch.Tensor, k: int, idx=None, gates=None):
    T, E = logits.shape
    _check(logits, torch.float32, "logits")
    if idx is None:
        idx = torch.empty(T, k, dtype=torch.int32, device=logits.device)
    if gates is None:
        gates = torch.empty(T, k, dtype=torch.float32, device=logits.device)
    _check(idx, torch.int32, "idx", (T, k))
    _check(gates, torch.float32, "gates", (T, k))
    _lib.call("llmy_router_topk_logits_f32", _ptr(logits), _ptr(idx), _ptr(gates), T, E, k,
              _stream())
    return idx, gates


def moe_permute(expert_ids: torch.Tensor, num_experts: int):
    """Stable expert-major permutation of flat routes; returns a dict of int32
    tensors: counts [E], offsets [E+1], sorted_routes [n], route_pos [n]."""
    _check(expert_ids, torch.int32, "expert_ids")
    n = expert_ids.numel()
    dev = expert_ids.device
    out = {
        "counts": torch.empty(num_experts, dtype=torch.int32, device=dev),
        "offsets": torch.empty(num_experts + 1, dtype=torch.int32, device=dev),
        "sorted_routes": torch.empty(n, dtype=torch.int32, device=dev),
        "route_pos": torch.empty(n, dtype=torch.int32, device=dev),
    }
    _lib.call("llmy_moe_permute", _ptr(expert_ids), n, num_experts, _ptr(out["counts"]),
              _ptr(out["offsets"]), _ptr(out["sorted_routes"]), _ptr(out["route_pos"]),
              _stream())
    return out


# --------------------------------------------------------------------------- sampling
def argmax(logits: torch.Tensor) -> torch.Tensor:
    R, V = logits.shape
    _check(logits, torch.float32, "logits")
    out = torch.empty(R, dtype=torch.int32, device=logits.device)
    _lib.call("llmy_sample_argmax_f32", _ptr(logits), R, V, _ptr(out), _stream())
    return out


def sample_top_p(logits: torch.Tensor, temperature: float, top_p: float, u: torch.Tensor,
                 top_k: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """Temperature + top-k + nucleus draw per row with the supplied uniforms u [R]
    (sample_standalone.py:5611-5636; llmy.cpp:132-202).  temperature <= 0 is greedy."""
    R, V = logits.shape
    _check(logits, torch.float32, "logits")
    _check(u, torch.float32, "u", (R,))
    if out is None:
        out = torch.empty(R, dtype=torch.int32, device=logits.device)
    _lib.call("llmy_sample_top_p_f32", _ptr(logits), R, V, float(temperature), int(top_k),
              float(top_p), _ptr(u), _ptr(out), _stream())
    return out


def repetition_penalty_(logits: torch.Tensor, recent: torch.Tensor, penalty: float) -> torch.Tensor:
    """In place: penalise each distinct id of recent[r] (int32 [R, n], -1 = none) in logits[r]
    (sample_standalone.py:5601-5605)."""
    R, V = logits.shape
    _check(logits, torch.float32, "logits")
    _check(recent, torch.int32, "recent")
    if recent.dim() != 2 or recent.shape[0] != R:
        raise ValueError("recent must be [rows, n]")
    _lib.call("llmy_repetition_penalty_f32", _ptr(logits), R, V, _ptr(recent), recent.shape[1],
              float(penalty), _stream())
    return logits


# --------------------------------------------------------------------------- projections
EPI_STORE_BF16, EPI_STORE_F32, EPI_RESID_ADD, EPI_RESID_GATED = 0, 1, 2, 3
# per-256-wide-K-block partial products [K/256, M, N] fp32 (M <= 64), folded by
# moe_route_decode(parts=...)
EPI_PARTIAL_F32 = 4


LAYOUT_ROWMAJOR, LAYOUT_PACKED = 0, 1


def pack_weights(w: torch.Tensor) -> torch.Tensor:
    """Row-major [..., N, K] bf16 -> the packed operand order (same shape/size)."""
    _check(w, torch.bfloat16, "w")
    N, K = w.shape[-2:]
    batch = w.numel() // (N * K)
    out = torch.empty_like(w)
    _lib.call("llmy_pack_weights_bf16", _ptr(w), _ptr(out), batch, N, K, _stream())
    return out


def linear(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None,
           epilogue: int = EPI_STORE_BF16, aux: torch.Tensor | None = None,
           layout: int = LAYOUT_ROWMAJOR) -> torch.Tensor:
    """x [M,K] bf16 . w [N,K]^T with a fused epilogue (see llmy_linear_bf16).
    ``layout=LAYOUT_PACKED`` when w came from pack_weights.  EPI_PARTIAL_F32
    returns the per-K-block products [K/256, M, N]."""
    M, K = x.shape
    N = w.shape[0]
    _check(x, torch.bfloat16, "x")
    _check(w, torch.bfloat16, "w", (N, K))
    if epilogue == EPI_PARTIAL_F32:
        if out is None:
            out = torch.empty(K // 256, M, N, dtype=torch.float32, device=x.device)
        _check(out, torch.float32, "out", (K // 256, M, N))
    elif out is None:
        if epilogue not in (EPI_STORE_BF16, EPI_STORE_F32):
            raise ValueError("residual epilogues need an explicit out tensor")
        dt = torch.bfloat16 if epilogue == EPI_STORE_BF16 else torch.float32
        out = torch.empty(M, N, dtype=dt, device=x.device)
    else:
        _check(out, torch.bfloat16 if epilogue == EPI_STORE_BF16 else torch.float32, "out", (M, N))
    if aux is not None:
        _check(aux, torch.float32, "aux", (M, N))
    _lib.call("llmy_linear_bf16", _ptr(x), _ptr(w), _ptr(out), _ptr(aux), M, N, K, epilogue,
              layout, _stream())
    return out


# --------------------------------------------------------------------------- MoE
def moe_experts(x: torch.Tensor, perm: dict, gates: torch.Tensor, w_gate_up: torch.Tensor,
                w_down: torch.Tensor, act: torch.Tensor | None = None,
                y: torch.Tensor | None = None, layout: int = LAYOUT_ROWMAJOR):
    """Routed SwiGLU experts over the permuted routes; returns (act, y)."""
    T, D = x.shape
    E, H2, D2 = w_gate_up.shape
    H = H2 // 2
    k = gates.shape[-1]
    _check(x, torch.bfloat16, "x")
    _check(w_gate_up, torch.bfloat16, "w_gate_up", (E, 2 * H, D))
    _check(w_down, torch.bfloat16, "w_down", (E, D, H))
    _check(gates, torch.float32, "gates", (T, k))
    n = T * k
    if act is None:
        act = torch.empty(n, H, dtype=torch.bfloat16, device=x.device)
    if y is None:
        y = torch.empty(n, D, dtype=torch.float32, device=x.device)
    _check(act, torch.bfloat16, "act", (n, H))
    _check(y, torch.float32, "y", (n, D))
    _lib.call("llmy_moe_experts_bf16", _ptr(x), _ptr(perm["offsets"]), _ptr(perm["sorted_routes"]),
              _ptr(gates), _ptr(w_gate_up), _ptr(w_down), _ptr(act), _ptr(y), T, D, H, E, k,
              layout, _stream())
    return act, y


def moe_experts_routed(x: torch.Tensor, ids: torch.Tensor, gates: torch.Tensor,
                       w_gate_up: torch.Tensor, w_down: torch.Tensor,
                       act: torch.Tensor | None = None, y: torch.Tensor | None = None,
                       layout: int = LAYOUT_ROWMAJOR):
    """Route-indexed experts (no permutation): act/y rows are route ids t*k+j."""
    T, D = x.shape
    E, H2, _ = w_gate_up.shape
    H = H2 // 2
    k = gates.shape[-1]
    _check(x, torch.bfloat16, "x")
    _check(ids, torch.int32, "ids", (T, k))
    _check(gates, torch.float32, "gates", (T, k))
    _check(w_gate_up, torch.bfloat16, "w_gate_up", (E, 2 * H, D))
    _check(w_down, torch.bfloat16, "w_down", (E, D, H))
    if act is None:
        act = torch.empty(T * k, H, dtype=torch.bfloat16, device=x.device)
    if y is None:
        y = torch.empty(T * k, D, dtype=torch.float32, device=x.device)
    _lib.call("llmy_moe_experts_routed_bf16", _ptr(x), _ptr(ids), _ptr(gates), _ptr(w_gate_up),
              _ptr(w_down), _ptr(act), _ptr(y), T, D, H, E, k, layout, _stream())
    return act, y


MOE_OUT_BF16, MOE_OUT_F32, MOE_OUT_RESID = 0, 1, 2


def moe_combine(y: torch.Tensor, route_pos: torch.Tensor, T: int, k: int,
                out: torch.Tensor | None = None, mode: int = MOE_OUT_BF16) -> torch.Tensor:
    D = y.shape[1]
    _check(y, torch.float32, "y", (T * k, D))
    if out is None:
        out = torch.empty(T, D, dtype=torch.bfloat16 if mode == MOE_OUT_BF16 else torch.float32,
                          device=y.device)
    _lib.call("llmy_moe_combine", _ptr(y), _ptr(route_pos), _ptr(out), T, D, k, mode, _stream())
    return out


def moe_forward(x: torch.Tensor, w_router: torch.Tensor, w_gate_up: torch.Tensor,
                w_down: torch.Tensor, k: int, router_norm: torch.Tensor | None = None,
                eps: float = 1e-6, layout: int = LAYOUT_ROWMAJOR) -> dict:
    """Full routed MoE layer op: router -> permute -> experts ->
    combine.  Returns a dict with idx, gates, perm, out (bf16 [T,D])."""
    T, D = x.shape
    E = w_router.shape[0]
    idx, gates = router_topk(x, w_router, k, router_norm, eps)
    perm = moe_permute(idx.view(-1), E)
    act, y = moe_experts(x, perm, gates, w_gate_up, w_down, layout=layout)
    out = moe_combine(y, perm["route_pos"], T, k)
    return {"idx": idx, "gates": gates, "perm": perm, "out": out}


# --------------------------------------------------------------------------- attention
def banded_attn_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int,
                        scale: float | None = None, out: torch.Tensor | None = None
                        ) -> torch.Tensor:
    """q, k, v [B,T,H,hd] bf16 -> o [B,T,H,hd] bf16 (banded causal attention)."""
    B, T, H, hd = q.shape
    _check(q, torch.bfloat16, "q")
    _check(k, torch.bfloat16, "k", (B, T, H, hd))
    _check(v, torch.bfloat16, "v", (B, T, H, hd))
    if out is None:
        out = torch.empty_like(q)
    scale = hd ** -0.5 if scale is None else scale
    _lib.call("llmy_banded_attn_prefill_bf16", _ptr(q), _ptr(k), _ptr(v), _ptr(out), B, T, H, hd,
              window, scale, _stream())
    return out


def banded_attn_decode(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                       k_cache: torch.Tensor, v_cache: torch.Tensor, pos: torch.Tensor,
                       scale: float | None = None, out: torch.Tensor | None = None
                       ) -> torch.Tensor:
    """q/k_new/v_new [B,H,hd] (or row-strided views of a fused projection),
    caches [B,H,W,hd] bf16 updated in place, pos [B] int32 -> out [B,H,hd] bf16."""
    B, H, W, hd = k_cache.shape
    for t, nm in ((q, "q"), (k_new, "k_new"), (v_new, "v_new")):
        if t.dtype != torch.bfloat16 or not t.is_cuda or tuple(t.shape) != (B, H, hd):
            raise ValueError(f"{nm} must be bf16 [B,H,hd] on the GPU")
        if t.stride(2) != 1 or t.stride(1) != hd:
            raise ValueError(f"{nm} must have contiguous heads")
    if k_new.stride(0) != v_new.stride(0):
        raise ValueError("k_new and v_new must share a batch stride")
    _check(k_cache, torch.bfloat16, "k_cache")
    _check(v_cache, torch.bfloat16, "v_cache", (B, H, W, hd))
    _check(pos, torch.int32, "pos", (B,))
    if out is None:
        out = torch.empty(B, H, hd, dtype=torch.bfloat16, device=q.device)
    scale = hd ** -0.5 if scale is None else scale
    _lib.call("llmy_banded_attn_decode_bf16", _ptr(q), _ptr(k_new), _ptr(v_new), q.stride(0),
              k_new.stride(0), _ptr(k_cache), _ptr(v_cache), _ptr(pos), _ptr(out), B, H, hd, W,
              scale, _stream())
    return out


def banded_attn_decode_parts(parts: torch.Tensor, k_off: int, v_off: int, k_cache: torch.Tensor,
                             v_cache: torch.Tensor, pos: torch.Tensor, scale: float | None = None,
                             out: torch.Tensor | None = None) -> torch.Tensor:
    """banded_attn_decode with q / k_new / v_new given as the partial products
    [P, B, row] fp32 of their projection (linear(..., epilogue=EPI_PARTIAL_F32)):
    q at column 0, k at k_off, v at v_off; the slices are summed in order and
    rounded to bf16 inside the kernel."""
    B, H, W, hd = k_cache.shape
    _check(parts, torch.float32, "parts")
    if parts.dim() != 3 or parts.shape[1] != B or parts.stride(2) != 1:
        raise ValueError("parts must be [P, B, row] fp32 with contiguous rows")
    _check(k_cache, torch.bfloat16, "k_cache")
    _check(v_cache, torch.bfloat16, "v_cache", (B, H, W, hd))
    _check(pos, torch.int32, "pos", (B,))
    if out is None:
        out = torch.empty(B, H, hd, dtype=torch.bfloat16, device=parts.device)
    scale = hd ** -0.5 if scale is None else scale
    _lib.call("llmy_banded_attn_decode_parts_bf16", _ptr(parts), parts.shape[0], parts.stride(0),
              parts.stride(1), k_off, v_off, _ptr(k_cache), _ptr(v_cache), _ptr(pos), _ptr(out),
              B, H, hd, W, scale, _stream())
    return out


# --------------------------------------------------------------------------- GDN
def _reset_arg(reset, shape, dev):
    """A reset mask as the device int32 array the kernels read (nonzero = reset)."""
    if reset is None:
        return None
    r = torch.as_tensor(reset, device=dev).to(torch.int32).contiguous()
    if tuple(r.shape) != tuple(shape):
        raise ValueError(f"reset: expected shape {tuple(shape)}, got {tuple(r.shape)}")
    return r


def gdn_prefill(q, k, v, beta, g, state, out=None, workspace=None, reset=None) -> torch.Tensor:
    """Chunked delta-rule scan; q,k [B,T,H,dk], v [B,T,H,dv] bf16, beta/g [B,T,H]
    fp32, state [B,H,dk,dv] fp32 updated in place.  Returns out [B,T,H,dv] bf16.
    ``reset`` [B, T] (bool/int): the state entering token t is zero where set
    (gated_deltanet.py:138-142)."""
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    _check(q, torch.bfloat16, "q")
    _check(k, torch.bfloat16, "k", (B, T, H, dk))
    _check(v, torch.bfloat16, "v", (B, T, H, dv))
    _check(beta, torch.float32, "beta", (B, T, H))
    _check(g, torch.float32, "g", (B, T, H))
    _check(state, torch.float32, "state", (B, H, dk, dv))
    nbytes = int(_lib.load().llmy_gdn_prefill_workspace_bytes(B, T, H, dk, dv))
    if workspace is None or workspace.numel() * workspace.element_size() < nbytes:
        workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q.device)
    if out is None:
        out = torch.empty(B, T, H, dv, dtype=torch.bfloat16, device=q.device)
    rs = _reset_arg(reset, (B, T), q.device)
    if rs is None:
        _lib.call("llmy_gdn_prefill_bf16", _ptr(q), _ptr(k), _ptr(v), _ptr(beta), _ptr(g),
                  _ptr(state), _ptr(out), _ptr(workspace), nbytes, B, T, H, dk, dv, _stream())
    else:
        _lib.call("llmy_gdn_prefill_reset_bf16", _ptr(q), _ptr(k), _ptr(v), _ptr(beta), _ptr(g),
                  _ptr(rs), _ptr(state), _ptr(out), _ptr(workspace), nbytes, B, T, H, dk, dv,
                  _stream())
    return out


def gdn_step(q, k, v, beta, g, state, gate=None, out=None, reset=None) -> torch.Tensor:
    """In-place state update; q,k [B,H,dk], v/gate [B,H,dv] bf16, beta/g [B,H] fp32,
    state [B,H,dk,dv] fp32.  Returns out [B,H,dv] bf16.  ``reset`` [B]: those
    rows start from a zero state."""
    B, H, dk = q.shape
    dv = v.shape[-1]
    _check(q, torch.bfloat16, "q")
    _check(k, torch.bfloat16, "k", (B, H, dk))
    _check(v, torch.bfloat16, "v", (B, H, dv))
    _check(beta, torch.float32, "beta", (B, H))
    _check(g, torch.float32, "g", (B, H))
    _check(state, torch.float32, "state", (B, H, dk, dv))
    if gate is not None:
        _check(gate, torch.bfloat16, "gate", (B, H, dv))
    if out is None:
        out = torch.empty(B, H, dv, dtype=torch.bfloat16, device=q.device)
    rs = _reset_arg(reset, (B,), q.device)
    if rs is None:
        _lib.call("llmy_gdn_step_bf16", _ptr(q), _ptr(k), _ptr(v), _ptr(beta), _ptr(g),
                  _ptr(gate), _ptr(state), _ptr(out), B, H, dk, dv, _stream())
    else:
        _lib.call("llmy_gdn_step_reset_bf16", _ptr(q), _ptr(k), _ptr(v), _ptr(beta), _ptr(g),
                  _ptr(gate), _ptr(rs), _ptr(state), _ptr(out), B, H, dk, dv, _stream())
    return out


def gdn_step_fused(proj, beta_bias, decay_logit, state, out=None, conv=None,
                   reset=None) -> torch.Tensor:
    """GDN step from the fused fp32 projection [B, ld] (or its per-K-block
    partial products [P, B, ld], summed in order); ``conv=(h, hist, w, cg_out)``
    also computes the causal conv gate in the same launch.  ``reset``: a device
    int32 [B] array (nonzero: the row starts from a zero state and history)."""
    B, H, dk, dv = state.shape
    _check(proj, torch.float32, "proj")
    nparts = proj.shape[0] if proj.dim() == 3 else 1
    if proj.dim() == 3 and proj.shape[1] != B:
        raise ValueError(f"proj: {tuple(proj.shape)} has {proj.shape[1]} rows, state {B}")
    _check(state, torch.float32, "state")
    if out is None:
        out = torch.empty(B, H * dv, dtype=torch.bfloat16, device=proj.device)
    ch = hist = cw = cg = None
    D = 0
    if conv is not None:
        ch, hist, cw, cg = conv
        D = ch.shape[1]
        _check(ch, torch.bfloat16, "conv_h", (B, D))
        _check(hist, torch.bfloat16, "conv_hist", (B, 3, D))
        _check(cw, torch.float32, "conv_w", (D, 4))
        _check(cg, torch.float32, "conv_out", (B, D))
    if reset is None:
        _lib.call("llmy_gdn_step_fused_f32", _ptr(proj), proj.shape[-1], nparts,
                  _ptr(beta_bias), _ptr(decay_logit), _ptr(state), _ptr(out), _ptr(ch),
                  _ptr(hist), _ptr(cw), _ptr(cg), D, 4, B, H, dk, dv, _stream())
    else:
        _check(reset, torch.int32, "reset", (B,))
        _lib.call("llmy_gdn_step_fused_reset_f32", _ptr(proj), proj.shape[-1], nparts,
                  _ptr(beta_bias), _ptr(decay_logit), _ptr(reset), _ptr(state), _ptr(out),
                  _ptr(ch), _ptr(hist), _ptr(cw), _ptr(cg), D, 4, B, H, dk, dv, _stream())
    return out


def moe_route_decode(x, ffn_w, router_w, w_router, k, eps=1e-6, bufs=None,
                     permute: bool = True, parts: torch.Tensor | None = None,
                     gate: torch.Tensor | None = None) -> dict:
    """Fused pre-MoE norm + router (+ the permutation unless permute=False).
    ``parts`` [P, T, D]: partial products of the preceding projection
    (EPI_PARTIAL_F32), folded into x first (x += sum, or x += gate * sum)."""
    T, D = x.shape
    E = w_router.shape[0]
    _check(x, torch.float32, "x")
    _check(w_router, torch.float32, "w_router", (E, D))
    nparts = 0
    if parts is not None:
        nparts = parts.shape[0]
        _check(parts, torch.float32, "parts", (nparts, T, D))
        if gate is not None:
            _check(gate, torch.float32, "gate", (T, D))
    elif gate is not None:
        raise ValueError("gate needs parts")
    dev = x.device
    if bufs is None:
        bufs = {"h": torch.empty(T, D, dtype=torch.bfloat16, device=dev),
                "idx": torch.empty(T, k, dtype=torch.int32, device=dev),
                "gates": torch.empty(T, k, dtype=torch.float32, device=dev),
                "counts": torch.empty(E, dtype=torch.int32, device=dev),
                "offsets": torch.empty(E + 1, dtype=torch.int32, device=dev),
                "sorted_routes": torch.empty(T * k, dtype=torch.int32, device=dev),
                "route_pos": torch.empty(T * k, dtype=torch.int32, device=dev)}
    b = bufs
    P = (lambda n: _ptr(b[n])) if permute else (lambda n: None)
    _lib.call("llmy_moe_route_decode", _ptr(x), _ptr(parts), nparts, _ptr(gate), _ptr(ffn_w),
              _ptr(router_w), _ptr(w_router),
              _ptr(b["h"]), _ptr(b["idx"]), _ptr(b["gates"]), P("counts"), P("offsets"),
              P("sorted_routes"), P("route_pos"), T, D, E, k, eps, _stream())
    return b


def moe_append_shared(idx, gates, n_experts: int, n_shared: int, idx_out=None, gates_out=None):
    """[T, k] router output -> [T, k + S] with every token also routed to the
    shared experts E .. E+S-1 at gate 1/sqrt(S)."""
    T, k = idx.shape
    _check(idx, torch.int32, "idx")
    _check(gates, torch.float32, "gates", (T, k))
    kx = k + n_shared
    if idx_out is None:
        idx_out = torch.empty(T, kx, dtype=torch.int32, device=idx.device)
    if gates_out is None:
        gates_out = torch.empty(T, kx, dtype=torch.float32, device=idx.device)
    _check(idx_out, torch.int32, "idx_out", (T, kx))
    _check(gates_out, torch.float32, "gates_out", (T, kx))
    _lib.call("llmy_moe_append_shared", _ptr(idx), _ptr(gates), _ptr(idx_out), _ptr(gates_out),
              T, k, n_experts, n_shared, _stream())
    return idx_out, gates_out


# ------------------------------------------------------------- context router
def router_context_latent(h, norm_w, w_down, ln_w, ln_b, eps: float = 1e-6,
                          ln_eps: float = 1e-5, local=None, lat=None):
    """h [rows, D] bf16 -> (local = RMSNorm(h) * norm_w fp32 [rows, D],
    lat = LayerNorm(local . w_down^T) fp32 [rows, L])."""
    rows, D = h.shape
    L = w_down.shape[0]
    _check(h, torch.bfloat16, "h")
    _check(w_down, torch.float32, "w_down", (L, D))
    for n, t in (("norm_w", norm_w), ("ln_w", ln_w), ("ln_b", ln_b)):
        _check(t, torch.float32, n)
    if local is None:
        local = torch.empty(rows, D, dtype=torch.float32, device=h.device)
    if lat is None:
        lat = torch.empty(rows, L, dtype=torch.float32, device=h.device)
    _check(local, torch.float32, "local", (rows, D))
    _check(lat, torch.float32, "lat", (rows, L))
    _lib.call("llmy_router_context_latent_f32", _ptr(h), _ptr(norm_w), _ptr(w_down), _ptr(ln_w),
              _ptr(ln_b), _ptr(local), _ptr(lat), rows, D, L, eps, ln_eps, _stream())
    return local, lat


def router_context_window(lat, ring, pos=None, ctx=None):
    """lat [B*T, L] (B sequences of T tokens) -> ctx bf16 [B*T, L], the mean of
    each token's window of W latents; ring [B, W, L] updated."""
    B, W, L = ring.shape
    rows = lat.shape[0]
    if rows % max(B, 1):
        raise ValueError("lat rows must be B * T")
    T = rows // B if B else 0
    _check(lat, torch.float32, "lat", (rows, L))
    _check(ring, torch.float32, "ring", (B, W, L))
    if pos is not None:
        _check(pos, torch.int32, "pos", (B,))
    if ctx is None:
        ctx = torch.empty(rows, L, dtype=torch.bfloat16, device=lat.device)
    _check(ctx, torch.bfloat16, "ctx", (rows, L))
    _lib.call("llmy_router_context_window", _ptr(lat), _ptr(ring), _ptr(pos), _ptr(ctx), B, T, W,
              L, _stream())
    return ctx


def router_context_logits(local, c, route_gate, w_router, logits=None):
    """logits = (local + sigmoid(route_gate) * c) . w_router^T, fp32 [rows, E]."""
    rows, D = local.shape
    E = w_router.shape[0]
    _check(local, torch.float32, "local")
    _check(c, torch.float32, "c", (rows, D))
    _check(route_gate, torch.float32, "route_gate")
    _check(w_router, torch.float32, "w_router", (E, D))
    if logits is None:
        logits = torch.empty(rows, E, dtype=torch.float32, device=local.device)
    _check(logits, torch.float32, "logits", (rows, E))
    _lib.call("llmy_router_context_logits_f32", _ptr(local), _ptr(c), _ptr(route_gate),
              _ptr(w_router), _ptr(logits), rows, D, E, _stream())
    return logits


def layernorm(x, w, b, eps: float = 1e-5, out=None) -> torch.Tensor:
    """bf16(LayerNorm(x) * w + b) of x [rows, L] fp32 (nn.LayerNorm, biased variance)."""
    rows, L = x.shape
    _check(x, torch.float32, "x")
    if out is None:
        out = torch.empty(rows, L, dtype=torch.bfloat16, device=x.device)
    _check(out, torch.bfloat16, "out", (rows, L))
    _lib.call("llmy_layernorm_f32_bf16", _ptr(x), _ptr(w), _ptr(b), _ptr(out), rows, L, eps,
              _stream())
    return out


def latent_attn(q, keys, vals, tag, heads: int, head_dim: int, pos=None, out=None):
    """Multi-head attention of q [B*T rows, heads*head_dim] over each row's C
    slots (keys / vals [B, C, heads*head_dim] bf16, tag [B, C]): query b*T + t
    at position pos[b] (None: t) sees slots with 1 <= tag <= position + 1."""
    B, C, HQ = keys.shape
    rows = q.shape[0]
    if rows % max(B, 1) or HQ != heads * head_dim:
        raise ValueError("latent_attn: rows must be B * T and keys heads * head_dim wide")
    _check(keys, torch.bfloat16, "keys")
    _check(vals, torch.bfloat16, "vals", (B, C, HQ))
    _check(tag, torch.int32, "tag", (B, C))
    if out is None:
        out = torch.empty(rows, HQ, dtype=torch.bfloat16, device=q.device)
    _lib.call("llmy_latent_attn_bf16", _ptr(q), _rows(q, "q", HQ), _ptr(keys), _ptr(vals),
              _ptr(tag), _ptr(pos), _ptr(out), _rows(out, "out", HQ), B, rows // max(B, 1), C,
              heads, head_dim, head_dim ** -0.5, _stream())
    return out


def router_context(h, w: dict, ring, k: int, pos=None, eps: float = 1e-6,
                   layout: int = LAYOUT_ROWMAJOR, bufs: dict | None = None,
                   glob: dict | None = None):
    """The whole context-aware routing of rows h [B*T, D] (bf16): returns
    (idx [rows, k] int32, gates [rows, k] fp32, logits [rows, E] fp32).
    ``w`` holds router_norm, ctx_down, ctx_ln_w, ctx_ln_b, ctx_local_out (bf16
    [D, L]), ctx_out (bf16 [D, D]), ctx_gate and w_router (fp32); ``layout``
    is that of the two bf16 matrices.  ``glob`` (HCA layers): the global
    branch's q ([HQ, D]) and o ([D, HQ]) weights, the block's summary keys /
    values / tags (rk, rv, rtag) and heads / head_dim; its output is added to
    local_context_out(ctx) before context_out."""
    b = bufs if bufs is not None else {}
    local, lat = router_context_latent(h, w["router_norm"], w["ctx_down"], w["ctx_ln_w"],
                                       w["ctx_ln_b"], eps, local=b.get("local"), lat=b.get("lat"))
    ctx = router_context_window(lat, ring, pos, ctx=b.get("ctx"))
    # a latent width (or query width) below a multiple of 256 reaches its GEMM
    # zero-padded to the padded weight's input width
    ctx = pad_cols(ctx, w["ctx_local_out"].shape[1], out=b.get("ctx_p"))
    if glob is None:
        cl = linear(ctx, w["ctx_local_out"], out=b.get("ctx_d"), epilogue=EPI_STORE_BF16,
                    layout=layout)
    else:
        t = linear(ctx, w["ctx_local_out"], out=b.get("ctx_t"), epilogue=EPI_STORE_F32,
                   layout=layout)
        lq = f32_to_bf16(local, out=b.get("lq"))
        gq = linear(lq, glob["q"], out=b.get("gq"), layout=layout)
        ga = latent_attn(gq, glob["rk"], glob["rv"], glob["rtag"], glob["heads"],
                         glob["head_dim"], pos=pos, out=b.get("gattn"))
        ga = pad_cols(ga, glob["o"].shape[1], out=b.get("gattn_p"))
        linear(ga, glob["o"], out=t, epilogue=EPI_RESID_ADD, layout=layout)
        cl = f32_to_bf16(t, out=b.get("ctx_d"))
    c = linear(cl, w["ctx_out"], out=b.get("ctx_c"), epilogue=EPI_STORE_F32, layout=layout)
    logits = router_context_logits(local, c, w["ctx_gate"], w["w_router"],
                                   logits=b.get("logits"))
    idx, gates = router_topk_from_logits(logits, k, idx=b.get("idx"), gates=b.get("gates"))
    return idx, gates, logits


def embed_norm(tokens, table, w, x, h, eps=1e-6) -> None:
    V, D = table.shape
    _check(tokens, torch.int32, "tokens")
    _check(table, torch.bfloat16, "table")
    B = tokens.numel()
    _check(x, torch.float32, "x", (B, D))
    _check(h, torch.bfloat16, "h", (B, D))
    _lib.call("llmy_embed_norm_bf16", _ptr(tokens), _ptr(table), _ptr(w), _ptr(x), _ptr(h), B, D,
              V, eps, _stream())


def moe_combine_norm(y, route_pos, x, h=None, w=None, k=2, eps=1e-6) -> None:
    """x += sum_j y[route_pos[t*k+j]] (route_pos None: route-indexed y), then
    h = bf16(RMSNorm(x) * w) when w is given."""
    T, D = x.shape
    _check(y, torch.float32, "y", (T * k, D))
    _check(x, torch.float32, "x")
    _lib.call("llmy_moe_combine_norm", _ptr(y), _ptr(route_pos), _ptr(w), _ptr(x), _ptr(h), T, D,
              k, eps, _stream())


def gdn_conv_gate(h, hist, w, out=None) -> torch.Tensor:
    B, D = h.shape
    _check(h, torch.bfloat16, "h")
    _check(hist, torch.bfloat16, "hist", (B, w.shape[1] - 1, D))
    _check(w, torch.float32, "w", (D, w.shape[1]))
    if out is None:
        out = torch.empty(B, D, dtype=torch.float32, device=h.device)
    _lib.call("llmy_gdn_conv_gate", _ptr(h), _ptr(hist), _ptr(w), _ptr(out), B, D, w.shape[1],
              _stream())
    return out


# --------------------------------------------------------------------------- mHC
MHC_MAP_EPS = 1.1920928955078125e-07   # nn.RMSNorm(eps=None) on fp32 (model/layers/mhc.py:72)


def mhc_embed(tokens, table, seed, out=None) -> torch.Tensor:
    """Streams [M, S, D] fp32: E[token] + seed[s] (model.py:442-444)."""
    M = tokens.numel()
    S, D = seed.shape
    _check(tokens, torch.int32, "tokens")
    _check(seed, torch.float32, "seed", (S, D))
    if out is None:
        out = torch.empty(M, S, D, dtype=torch.float32, device=tokens.device)
    _lib.call("llmy_mhc_embed", _ptr(tokens), _ptr(table), _ptr(seed), _ptr(out), M, S, D,
              table.shape[0], _stream())
    return out


def mhc_read(X, raw, p: dict, norm_w, iterations: int, maps=None, h=None, norm_eps: float = 1e-6):
    """Maps and read of one sublayer: X [M, S, D] streams, raw [M, >= 2S+S^2] fp32
    projection, p the layer's mHC parameters (pre_bias, post_bias, res_bias,
    alpha, ln_w, ln_b).  Returns (maps [M, S+S^2], h [M, D] bf16)."""
    M, S, D = X.shape
    _check(X, torch.float32, "X")
    if maps is None:
        maps = torch.empty(M, S + S * S, dtype=torch.float32, device=X.device)
    if h is None:
        h = torch.empty(M, D, dtype=torch.bfloat16, device=X.device)
    _lib.call("llmy_mhc_read", _ptr(X), _ptr(raw), raw.stride(0), _ptr(p["pre_bias"]),
              _ptr(p["post_bias"]), _ptr(p["res_bias"]), _ptr(p["alpha"]), iterations,
              _ptr(p["ln_w"]), _ptr(p["ln_b"]), 1e-5, _ptr(norm_w), norm_eps, _ptr(maps), _ptr(h),
              M, S, D, _stream())
    return maps, h


def mhc_write(X, U, maps, scale, gating_logit) -> None:
    """In place: X_i += sigmoid(g) scale_i (sum_j R_ij X_j + post_i U)."""
    M, S, D = X.shape
    _check(X, torch.float32, "X")
    _check(U, torch.float32, "U")
    _lib.call("llmy_mhc_write", _ptr(X), _ptr(U), U.stride(0), _ptr(maps), _ptr(scale),
              _ptr(gating_logit), M, S, D, _stream())


def pad_cols(x, Kp: int, out=None) -> torch.Tensor:
    """x [rows, K] bf16 -> [rows, Kp] with zero columns K .. Kp-1 (x itself when
    K == Kp): the input of a GEMM whose weight was zero-padded to Kp inputs."""
    rows, K = x.shape
    if K == Kp:
        return x
    _check(x, torch.bfloat16, "x")
    if out is None:
        out = torch.empty(rows, Kp, dtype=torch.bfloat16, device=x.device)
    _check(out, torch.bfloat16, "out", (rows, Kp))
    _lib.call("llmy_pad_cols_bf16", _ptr(x), _ptr(out), rows, K, Kp, _stream())
    return out


def f32_to_bf16(x, out=None) -> torch.Tensor:
    _check(x, torch.float32, "x")
    if out is None:
        out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    _lib.call("llmy_f32_to_bf16", _ptr(x), _ptr(out), x.numel(), _stream())
    return out


def zero_rows(t: torch.Tensor, mask: torch.Tensor) -> None:
    """Zero t[b] wherever mask[b] != 0; t contiguous [rows, ...] on the device,
    mask device int32 [rows] (a kernel, so it may sit in a captured graph)."""
    if not t.is_contiguous() or t.dim() < 1:
        raise ValueError("zero_rows: contiguous tensor with a row dimension expected")
    _check(mask, torch.int32, "mask", (t.shape[0],))
    row_bytes = t[0].numel() * t.element_size() if t.shape[0] else 0
    _lib.call("llmy_zero_rows", _ptr(t), row_bytes, t.shape[0], _ptr(mask), _stream())


# --------------------------------------------------------------------------- prefill glue
def kv_cache_fill(k, v, k_cache, v_cache) -> None:
    """K/V rows [B, T, ld] bf16 (head h at columns h*hd..; rows may be strided
    views of a fused qkv row) into ring caches [B, H, W, hd]: the last
    min(T, W) positions, position t at slot t % W."""
    B, H, W, hd = k_cache.shape
    T = k.shape[1]
    _check(k_cache, torch.bfloat16, "k_cache")
    _check(v_cache, torch.bfloat16, "v_cache", (B, H, W, hd))
    for name, t in (("k", k), ("v", v)):
        if t.dtype != torch.bfloat16 or t.shape[:2] != (B, T) or t.shape[2] < H * hd \
                or t.stride(-1) != 1 or t.stride(0) != T * t.stride(1) or not t.is_cuda:
            raise ValueError(f"{name}: expected bf16 rows [B, T, >=H*hd] with a common row stride")
    if k.stride(1) != v.stride(1):
        raise ValueError("k and v must share a row stride")
    _lib.call("llmy_kv_cache_fill_bf16", _ptr(k), _ptr(v), k.stride(1), _ptr(k_cache),
              _ptr(v_cache), B, T, H, hd, W, _stream())


def gdn_prefill_prep(proj, beta_bias, decay_logit, H, dk, dv, out=None):
    """q, k (L2-normalised), v bf16 [R, H, d] and beta, g fp32 [R, H] from the
    fused fp32 projection rows proj [R, ld]."""
    R = proj.shape[0]
    _check(proj, torch.float32, "proj")
    dev = proj.device
    if out is None:
        out = {"q": torch.empty(R, H, dk, dtype=torch.bfloat16, device=dev),
               "k": torch.empty(R, H, dk, dtype=torch.bfloat16, device=dev),
               "v": torch.empty(R, H, dv, dtype=torch.bfloat16, device=dev),
               "beta": torch.empty(R, H, dtype=torch.float32, device=dev),
               "g": torch.empty(R, H, dtype=torch.float32, device=dev)}
    _lib.call("llmy_gdn_prefill_prep_f32", _ptr(proj), proj.shape[1], _ptr(beta_bias),
              _ptr(decay_logit), _ptr(out["q"]), _ptr(out["k"]), _ptr(out["v"]),
              _ptr(out["beta"]), _ptr(out["g"]), R, H, dk, dv, _stream())
    return out


def gdn_gate(o, proj, gate_off, out=None) -> torch.Tensor:
    """bf16(o * sigmoid(proj[:, gate_off : gate_off + HV])); o [R, HV] bf16."""
    R, HV = o.shape
    _check(o, torch.bfloat16, "o")
    _check(proj, torch.float32, "proj")
    if out is None:
        out = torch.empty_like(o)
    _lib.call("llmy_gdn_gate_bf16", _ptr(o), _ptr(proj), proj.shape[1], gate_off, _ptr(out), R,
              HV, _stream())
    return out


def gdn_conv_gate_prefill(h, hist, w, out=None, reset=None) -> torch.Tensor:
    """Conv gate over a sequence: h [B, T, D] bf16, hist [B, K-1, D] updated.
    ``reset`` [B, T]: taps do not cross a reset (gated_deltanet.py:56-78)."""
    B, T, D = h.shape
    _check(h, torch.bfloat16, "h")
    _check(hist, torch.bfloat16, "hist", (B, w.shape[1] - 1, D))
    _check(w, torch.float32, "w", (D, w.shape[1]))
    if out is None:
        out = torch.empty(B, T, D, dtype=torch.float32, device=h.device)
    rs = _reset_arg(reset, (B, T), h.device)
    if rs is None:
        _lib.call("llmy_gdn_conv_gate_prefill", _ptr(h), _ptr(hist), _ptr(w), _ptr(out), B, T, D,
                  w.shape[1], _stream())
    else:
        _lib.call("llmy_gdn_conv_gate_prefill_reset", _ptr(h), _ptr(hist), _ptr(w), _ptr(rs),
                  _ptr(out), B, T, D, w.shape[1], _stream())
    return out


# --------------------------------------------------------------------------- glue
def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6, out=None) -> torch.Tensor:
    M, D = x.shape
    _check(x, torch.float32, "x")
    _check(w, torch.float32, "w", (D,))
    if out is None:
        out = torch.empty(M, D, dtype=torch.bfloat16, device=x.device)
    _lib.call("llmy_rmsnorm_f32_bf16", _ptr(x), _ptr(w), _ptr(out), M, D, eps, _stream())
    return out


def embed(tokens: torch.Tensor, table: torch.Tensor, out=None) -> torch.Tensor:
    V, D = table.shape
    _check(tokens, torch.int32, "tokens")
    _check(table, torch.bfloat16, "table")
    B = tokens.numel()
    if out is None:
        out = torch.empty(B, D, dtype=torch.float32, device=table.device)
    _lib.call("llmy_embed_bf16", _ptr(tokens), _ptr(table), _ptr(out), B, D, V, _stream())
    return out


# --------------------------------------------------------------------------- compressed memories
# CSA / HCA mixers (model/layers/csa.py, hca.py, compressed_attention.py): H
# heads of width Dh (HCA: H = 1, Dh = d_model), values of width Dv shared by
# the heads.  q / k / v may be column slices of one projection output: they
# are [rows, width] bf16 views with unit column stride at any row stride.
def _rows(t: torch.Tensor, name: str, width: int | None = None) -> int:
    if not t.is_cuda or t.dtype != torch.bfloat16 or t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a [rows, width] bf16 GPU view with unit column stride")
    if width is not None and t.shape[1] != width:
        raise ValueError(f"{name} width {t.shape[1]} != {width}")
    return t.stride(0)


def cmp_workspace(queries: int, H: int, slots: int, top_k: int, device,
                  decode: bool = False) -> torch.Tensor:
    n = _lib.load().llmy_cmp_workspace_bytes(queries, H, slots, top_k, int(decode))
    if n < 0:
        raise ValueError("bad compressed-attention workspace sizes")
    return torch.empty(max(int(n), 16), dtype=torch.uint8, device=device)


def cmp_local_prefill(q, k, v, B: int, T: int, H: int, Dh: int, W: int, out=None,
                      workspace=None) -> torch.Tensor:
    """Local branch over B fresh sequences of T tokens (rows b*T + t)."""
    Kw, Dv = H * Dh, v.shape[1]
    q_ld, k_ld, v_ld = _rows(q, "q", Kw), _rows(k, "k", Kw), _rows(v, "v")
    if out is None:
        out = torch.empty(B * T, Dv, dtype=torch.bfloat16, device=q.device)
    if workspace is None:
        workspace = cmp_workspace(B * T, H, W, 0, q.device)
    _lib.call("llmy_cmp_local_prefill_bf16", _ptr(q), q_ld, _ptr(k), k_ld, _ptr(v), v_ld,
              _ptr(out), _rows(out, "out", Dv), B, T, H, Dh, Dv, W, Dh ** -0.5, _ptr(workspace),
              workspace.numel(), _stream())
    return out


def cmp_memory_prefill(q, mk, mv, B: int, T: int, ratio: int, H: int, Dh: int, top_k: int,
                       out=None, workspace=None, slots: int = 0) -> torch.Tensor:
    """Memory branch over B fresh sequences; mk / mv rows b*n + i, n = T // ratio.
    ``slots`` > 0: a query sees only the last ``slots`` summaries emitted up to
    it (the decode memory's ring); 0: all of them."""
    Kw, Dv, n = H * Dh, mv.shape[1], T // ratio
    if mk.shape[0] != B * n or mv.shape[0] != B * n:
        raise ValueError("mk / mv must hold B * (T // ratio) rows")
    q_ld, mk_ld, mv_ld = _rows(q, "q", Kw), _rows(mk, "mk", Kw), _rows(mv, "mv")
    if out is None:
        out = torch.empty(B * T, Dv, dtype=torch.bfloat16, device=q.device)
    if workspace is None:
        workspace = cmp_workspace(B * T, H, max(n, 1), top_k, q.device)
    _lib.call("llmy_cmp_memory_prefill_bf16", _ptr(q), q_ld, _ptr(mk), mk_ld, _ptr(mv), mv_ld,
              _ptr(out), _rows(out, "out", Dv), B, T, n, ratio, H, Dh, Dv, top_k, slots,
              Dh ** -0.5, _ptr(workspace), workspace.numel(), _stream())
    return out


def cmp_local_decode(q, k_new, v_new, ring_k, ring_v, pos, H: int, Dh: int, out=None,
                     workspace=None) -> torch.Tensor:
    """Local branch for one token per row; k_new / v_new (rows at one stride) go
    into ring slot pos % W first."""
    B, W, Kw = ring_k.shape
    Dv = ring_v.shape[2]
    kv_ld = _rows(k_new, "k_new", Kw)
    if _rows(v_new, "v_new", Dv) != kv_ld:
        raise ValueError("k_new and v_new must share their row stride")
    _check(ring_k, torch.bfloat16, "ring_k", (B, W, H * Dh))
    _check(ring_v, torch.bfloat16, "ring_v", (B, W, Dv))
    _check(pos, torch.int32, "pos", (B,))
    if out is None:
        out = torch.empty(B, Dv, dtype=torch.bfloat16, device=q.device)
    if workspace is None:
        workspace = cmp_workspace(B, H, W, 0, q.device, decode=True)
    _lib.call("llmy_cmp_local_decode_bf16", _ptr(q), _rows(q, "q", Kw), _ptr(k_new), _ptr(v_new),
              kv_ld, _ptr(ring_k), _ptr(ring_v), _ptr(pos), _ptr(out), _rows(out, "out", Dv), B,
              H, Dh, Dv, W, Dh ** -0.5, _ptr(workspace), workspace.numel(), _stream())
    return out


def cmp_memory_decode(q, mk, mv, mtag, pos, H: int, Dh: int, top_k: int, out=None,
                      workspace=None) -> torch.Tensor:
    """Memory branch for one token per row over the C slots of each row."""
    B, C, Kw = mk.shape
    Dv = mv.shape[2]
    _check(mk, torch.bfloat16, "mk", (B, C, H * Dh))
    _check(mv, torch.bfloat16, "mv", (B, C, Dv))
    _check(mtag, torch.int32, "mtag", (B, C))
    _check(pos, torch.int32, "pos", (B,))
    if out is None:
        out = torch.empty(B, Dv, dtype=torch.bfloat16, device=q.device)
    if workspace is None:
        workspace = cmp_workspace(B, H, C, top_k, q.device, decode=True)
    _lib.call("llmy_cmp_memory_decode_bf16", _ptr(q), _rows(q, "q", Kw), _ptr(mk), _ptr(mv),
              _ptr(mtag), _ptr(pos), _ptr(out), _rows(out, "out", Dv), B, C, H, Dh, Dv, top_k,
              Dh ** -0.5, _ptr(workspace), workspace.numel(), _stream())
    return out


def cmp_pool_prefill(h, B: int, T: int, ratio: int, psum, pcnt, means=None) -> torch.Tensor:
    """Block means [B * (T // ratio), D] bf16; the tail's sum / count into psum / pcnt."""
    D = h.shape[1]
    n = T // ratio
    _check(psum, torch.float32, "psum", (B, D))
    _check(pcnt, torch.int32, "pcnt", (B,))
    if means is None:
        means = torch.empty(max(B * n, 1), D, dtype=torch.bfloat16, device=h.device)
    _lib.call("llmy_cmp_pool_prefill_bf16", _ptr(h), _rows(h, "h", D), _ptr(means), _ptr(psum),
              _ptr(pcnt), B, T, D, ratio, _stream())
    return means[:B * n]


def cmp_pool_step(h, psum, pcnt, ratio: int, mean=None, emit=None):
    B, D = h.shape
    _check(psum, torch.float32, "psum", (B, D))
    _check(pcnt, torch.int32, "pcnt", (B,))
    if mean is None:
        mean = torch.empty(B, D, dtype=torch.bfloat16, device=h.device)
    if emit is None:
        emit = torch.empty(B, dtype=torch.int32, device=h.device)
    _lib.call("llmy_cmp_pool_step_bf16", _ptr(h), _rows(h, "h", D), _ptr(psum), _ptr(pcnt),
              _ptr(mean), _ptr(emit), B, D, ratio, _stream())
    return mean, emit


def cmp_commit(kv, emit, pos, mk, mv, mtag, mcount) -> None:
    B, C, Kw = mk.shape
    Dv = mv.shape[2]
    _lib.call("llmy_cmp_commit_bf16", _ptr(kv), _rows(kv, "kv", Kw + Dv), _ptr(emit), _ptr(pos),
              _ptr(mk), _ptr(mv), _ptr(mtag), _ptr(mcount), B, C, Kw, Dv, _stream())


def cmp_memory_fill(kv, B: int, n: int, ratio: int, mk, mv, mtag, mcount) -> None:
    _, C, Kw = mk.shape
    Dv = mv.shape[2]
    if n:
        _lib.call("llmy_cmp_memory_fill_bf16", _ptr(kv), _rows(kv, "kv", Kw + Dv), _ptr(mk),
                  _ptr(mv), _ptr(mtag), _ptr(mcount), B, n, ratio, C, Kw, Dv, _stream())


def cmp_ring_fill(src, B: int, T: int, ring) -> None:
    _, W, width = ring.shape
    _lib.call("llmy_cmp_ring_fill_bf16", _ptr(src), _rows(src, "src", width), _ptr(ring), B, T,
              W, width, _stream())
