"""Configuration and deterministic synthetic weights for the hybrid block stack.

The block stack is the reference's looped recurrent core with mHC disabled
(model/model.py:119-126: ``_read`` = identity for one stream, ``_write`` =
residual add), i.e. a pre-norm residual block

    x <- x + Mixer(RMSNorm(x));  x <- x + MoE(RMSNorm(x))

with mixers alternating banded attention and GDN, looped ``num_loops`` times
with weights shared across loops and one KV cache / GDN state per
(loop, layer) (model/model.py:618-687, state namespace ``loop{i}`` at :645).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch


@dataclass(frozen=True)
class HybridConfig:
    d_model: int
    layer_kinds: tuple[str, ...]
    attn_heads: int
    attn_head_dim: int
    window: int
    gdn_heads: int
    gdn_dk: int
    gdn_dv: int
    n_experts: int
    top_k: int
    expert_hidden: int
    vocab: int
    num_loops: int
    conv_kernel: int = 4
    # shared experts per MoE (model/layers/moe.py:110,185-199): dense SwiGLU
    # experts of size expert_hidden on every token, summed and scaled by
    # 1/sqrt(shared_experts), added to the routed output
    shared_experts: int = 0
    # context-aware router, local-context branch (model/layers/context_router.py:
    # 13-27,59-76; mla_memory.py:18-24): a latent channel of width latent_dim
    # averaged over the last router_context tokens, added to the router input
    # through context_out at weight sigmoid(route_gate)
    context_router: bool = False
    latent_dim: int = 256
    router_context: int = 128
    route_gate_init: float = -4.59512  # context_router.py:25
    # the router's global branch (context_router.py:66-68,126-127): latent
    # attention with router_heads heads of router_head_dim over the HCA block's
    # summary latents (hca_latent: mla_memory.py:9-27), on HCA layers
    router_heads: int = 4      # model/config.py:48
    router_head_dim: int = 64  # model/config.py:49
    # multi-stream hyper-connections (model/layers/mhc.py:156-231; model.py:84-86,
    # 119-126,389-421,442-444,699-700): mhc_streams residual streams per token,
    # read before and written after every mixer and MoE sublayer through
    # input-dependent maps (pre / post weights, a Sinkhorn-normalised stream
    # mixing matrix), seeded from the embedding plus a per-stream vector and
    # collapsed by a linear map before the final norm; 1 = the single residual
    # stream of the schematic block (no mHC)
    mhc_streams: int = 1
    mhc_sinkhorn_iters: int = 10   # model/config.py:12
    mhc_gating_init: float = 0.01  # model/config.py:13
    # compressed-memory mixers (layer kinds "csa" / "hca"; model/layers/csa.py,
    # hca.py, defaults of model/config.py:56-70): index heads x head width of the
    # CSA scores (HCA: one head of width d_model), local window, temporal
    # compression ratio, top-k of the summaries (HCA: dense unless hca_dense is
    # off), and the decode memory's slots per row (the reference native engine's
    # fixed capacity, llmy_cuda/src/model.cpp:351-354; the oldest summary is
    # overwritten once a row has emitted more)
    csa_heads: int = 16
    csa_head_dim: int = 128
    csa_window: int = 128
    csa_ratio: int = 4
    csa_top_k: int = 32
    hca_window: int = 128
    hca_ratio: int = 32
    hca_dense: bool = True
    hca_top_k: int = 32
    cmp_slots: int = 256
    # stem and tail blocks (model/model.py:391-394,411-414): GDN mixers of the
    # core's GDN shape, each followed by a dense SwiGLU FFN of width dense_hidden
    # (model/layers/dense_ffn.py:7-15) instead of a MoE; the stem runs once
    # before the looped core and the tail once after it, each block with its
    # own GDN state (state keys stem.<i> / tail.<i>, model.py:600-606,689-695)
    stem_blocks: int = 0
    tail_blocks: int = 0
    dense_hidden: int = 0
    eps: float = 1e-6
    init_std: float = 0.02
    decay_logit_init: float = 2.0  # model/layers/gated_deltanet.py:113

    @property
    def n_layers(self) -> int:
        return len(self.layer_kinds)

    @property
    def attn_scale(self) -> float:
        return 1.0 / math.sqrt(self.attn_head_dim)

    def attn_layers(self) -> list[int]:
        return [i for i, k in enumerate(self.layer_kinds) if k == "attn"]

    def gdn_layers(self) -> list[int]:
        return [i for i, k in enumerate(self.layer_kinds) if k == "gdn"]

    def side_blocks(self, where: str) -> list[str]:
        """Weight prefixes of the stem ("S<i>.") or tail ("T<i>.") blocks."""
        n = self.stem_blocks if where == "stem" else self.tail_blocks
        return [f"{where[0].upper()}{i}." for i in range(n)]

    @property
    def has_gdn(self) -> bool:
        """Whether any block (core, stem or tail) runs a GDN mixer."""
        return bool(self.gdn_layers()) or self.stem_blocks > 0 or self.tail_blocks > 0

    def cmp_shape(self, kind: str) -> dict:
        """Heads, head width, window, ratio and top-k (0 = dense) of a CSA / HCA
        layer (model/model.py:95-106)."""
        if kind == "csa":
            return {"H": self.csa_heads, "Dh": self.csa_head_dim, "W": self.csa_window,
                    "ratio": self.csa_ratio, "top_k": self.csa_top_k}
        if kind == "hca":
            return {"H": 1, "Dh": self.d_model, "W": self.hca_window, "ratio": self.hca_ratio,
                    "top_k": 0 if self.hca_dense else self.hca_top_k}
        raise ValueError(kind)


def alternating(n: int) -> tuple[str, ...]:
    return tuple("attn" if i % 2 == 0 else "gdn" for i in range(n))


# random-init small LLMY (CPU reference, fp32).
C1 = HybridConfig(d_model=256, layer_kinds=alternating(4), attn_heads=4, attn_head_dim=64,
                  window=128, gdn_heads=4, gdn_dk=64, gdn_dv=64, n_experts=8, top_k=2,
                  expert_hidden=512, vocab=32000, num_loops=2)

# the bs=64 hybrid-MoE decode step.
C5 = HybridConfig(d_model=1024, layer_kinds=alternating(12), attn_heads=16, attn_head_dim=64,
                  window=2048, gdn_heads=16, gdn_dk=64, gdn_dv=64, n_experts=24, top_k=2,
                  expert_hidden=2048, vocab=32000, num_loops=2)


def _mhc_shapes(cfg: HybridConfig, p: str) -> list[tuple[str, tuple[int, ...], str]]:
    """A block's hyper-connection parameters (model/layers/mhc.py:63-84)."""
    Sm, D = cfg.mhc_streams, cfg.d_model
    if Sm <= 1:
        return []
    return [(p + "mhc_map_norm", (Sm * D,), "ones"),
            (p + "mhc_theta", (2 * Sm + Sm * Sm, Sm * D), "normal"),
            (p + "mhc_pre_bias", (Sm,), "mhc_pre"), (p + "mhc_post_bias", (Sm,), "zeros"),
            (p + "mhc_res_bias", (Sm, Sm), "eye4"), (p + "mhc_alpha", (3,), "alpha"),
            (p + "mhc_gating", (1,), "mhc_gate"), (p + "mhc_scale", (Sm, D), "ones"),
            (p + "mhc_ln_w", (D,), "ones"), (p + "mhc_ln_b", (D,), "zeros")]


def _gdn_shapes(cfg: HybridConfig, p: str) -> list[tuple[str, tuple[int, ...], str]]:
    """A GDN mixer's parameters (model/layers/gated_deltanet.py:104-113)."""
    D, Hg, dk, dv = cfg.d_model, cfg.gdn_heads, cfg.gdn_dk, cfg.gdn_dv
    return [(p + "wq", (Hg * dk, D), "normal"), (p + "wk", (Hg * dk, D), "normal"),
            (p + "wv", (Hg * dv, D), "normal"), (p + "wg", (Hg * dv, D), "normal"),
            (p + "wb", (Hg, D), "normal"), (p + "bb", (Hg,), "zeros"),
            (p + "wout", (D, Hg * dv), "normal"),
            (p + "conv", (D, cfg.conv_kernel), "normal"),
            (p + "decay", (Hg,), "decay")]


def weight_shapes(cfg: HybridConfig) -> list[tuple[str, tuple[int, ...], str]]:
    """(name, shape, kind) in generation order; kind in {normal, ones, zeros, decay, gate}."""
    D, E, Hf = cfg.d_model, cfg.n_experts, cfg.expert_hidden
    out: list[tuple[str, tuple[int, ...], str]] = [("embed", (cfg.vocab, D), "normal")]
    Sm = cfg.mhc_streams
    if Sm > 1:
        out.append(("stream_seed", (Sm, D), "seed"))
    for l, kind in enumerate(cfg.layer_kinds):
        p = f"L{l}."
        out += _mhc_shapes(cfg, p)
        out.append((p + "mix_norm", (D,), "ones"))
        if kind == "attn":
            w = cfg.attn_heads * cfg.attn_head_dim
            out += [(p + "wq", (w, D), "normal"), (p + "wk", (w, D), "normal"),
                    (p + "wv", (w, D), "normal"), (p + "wo", (D, w), "normal")]
        elif kind in ("csa", "hca"):
            cs = cfg.cmp_shape(kind)
            Kw = cs["H"] * cs["Dh"]
            out += [(p + "cmp_wq", (Kw, D), "normal"), (p + "cmp_wk", (Kw, D), "normal"),
                    (p + "cmp_wv", (D, D), "normal"), (p + "cmp_wlo", (D, D), "normal"),
                    (p + "cmp_wro", (D, D), "normal"), (p + "cmp_wout", (D, D), "normal"),
                    (p + "cmp_wck", (Kw, D), "normal"), (p + "cmp_wcv", (D, D), "normal")]
        else:
            out += _gdn_shapes(cfg, p)
        out += [(p + "ffn_norm", (D,), "ones"), (p + "router_norm", (D,), "ones"),
                (p + "w_router", (E, D), "normal"),
                (p + "w_gate", (E, Hf, D), "normal"), (p + "w_up", (E, Hf, D), "normal"),
                (p + "w_down", (E, D, Hf), "normal")]
        if cfg.context_router:
            L = cfg.latent_dim
            out += [(p + "ctx_down", (L, D), "normal"), (p + "ctx_ln_w", (L,), "ones"),
                    (p + "ctx_ln_b", (L,), "zeros"), (p + "ctx_local_out", (D, L), "normal"),
                    (p + "ctx_out", (D, D), "normal"), (p + "ctx_gate", (), "gate")]
        if cfg.shared_experts > 0:
            S = cfg.shared_experts
            out += [(p + "w_shared_gate", (S, Hf, D), "normal"),
                    (p + "w_shared_up", (S, Hf, D), "normal"),
                    (p + "w_shared_down", (S, D, Hf), "normal")]
    if Sm > 1:
        out.append(("mhc_collapse", (D, Sm * D), "collapse"))
    out.append(("final_norm", (D,), "ones"))
    if cfg.context_router:
        # the router's latent attention (every router has one) and the HCA
        # blocks' summary latents, drawn after every other weight
        L, HQ = cfg.latent_dim, cfg.router_heads * cfg.router_head_dim
        for l, kind in enumerate(cfg.layer_kinds):
            p = f"L{l}."
            out += [(p + "ctx_q", (HQ, D), "normal"), (p + "ctx_k", (HQ, L), "normal"),
                    (p + "ctx_v", (HQ, L), "normal"), (p + "ctx_o", (D, HQ), "normal")]
            if kind == "hca":
                out += [(p + "hca_lat_down", (L, D), "normal"),
                        (p + "hca_lat_ln_w", (L,), "ones"), (p + "hca_lat_ln_b", (L,), "zeros")]
    # stem then tail blocks, drawn last (so the core's weights do not depend on them)
    Hd = cfg.dense_hidden
    for p in cfg.side_blocks("stem") + cfg.side_blocks("tail"):
        out += _mhc_shapes(cfg, p)
        out.append((p + "mix_norm", (D,), "ones"))
        out += _gdn_shapes(cfg, p)
        out += [(p + "ffn_norm", (D,), "ones"), (p + "ffn_gate", (Hd, D), "normal"),
                (p + "ffn_up", (Hd, D), "normal"), (p + "ffn_down", (D, Hd), "normal")]
    return out


# Parameters kept in fp32 on the device; every other matrix is stored bf16.
FP32_PARAMS = ("mix_norm", "ffn_norm", "router_norm", "final_norm", "w_router", "bb", "conv",
               "decay", "ctx_down", "ctx_ln_w", "ctx_ln_b", "ctx_gate", "stream_seed",
               "mhc_map_norm", "mhc_pre_bias", "mhc_post_bias", "mhc_res_bias", "mhc_alpha",
               "mhc_gating", "mhc_scale", "mhc_ln_w", "mhc_ln_b", "hca_lat_ln_w", "hca_lat_ln_b")


def is_fp32_param(name: str) -> bool:
    return name.split(".")[-1] in FP32_PARAMS


def init_weights(cfg: HybridConfig, seed: int = 0, device: str | torch.device = "cpu"
                 ) -> dict[str, torch.Tensor]:
    """Random-init weights: every matrix N(0, init_std) drawn in ``weight_shapes``
    order from one generator seeded ``seed`` on ``device``; RMSNorm weights 1,
    biases 0, GDN decay logits 2.0, the context router's gate route_gate_init.  Matrices are rounded to bf16 except the
    fp32 parameters listed in FP32_PARAMS (the router is fp32 end to end).
    CPU and GPU generators give different streams: parity tests generate on
    the CPU and copy to the GPU.
    """
    gen = torch.Generator(device=device).manual_seed(seed)
    weights: dict[str, torch.Tensor] = {}
    for name, shape, kind in weight_shapes(cfg):
        if kind == "normal":
            t = torch.empty(shape, dtype=torch.float32, device=device)
            t.normal_(0.0, cfg.init_std, generator=gen)
        elif kind == "ones":
            t = torch.ones(shape, dtype=torch.float32, device=device)
        elif kind == "zeros":
            t = torch.zeros(shape, dtype=torch.float32, device=device)
        elif kind == "gate":
            t = torch.full(shape, cfg.route_gate_init, dtype=torch.float32, device=device)
        elif kind == "seed":       # stream_seed ~ N(0, 1e-3) (model.py:389-390)
            t = torch.empty(shape, dtype=torch.float32, device=device)
            t.normal_(0.0, 1e-3, generator=gen)
        elif kind == "mhc_pre":    # logit(1 / S) (mhc.py:75-77)
            S_ = shape[0]
            t = torch.full(shape, math.log((1.0 / S_) / (1.0 - 1.0 / S_)), dtype=torch.float32,
                           device=device)
        elif kind == "eye4":       # 4 I (mhc.py:79)
            t = 4.0 * torch.eye(shape[0], dtype=torch.float32, device=device)
        elif kind == "alpha":      # 0.01 each (mhc.py:80-82)
            t = torch.full(shape, 0.01, dtype=torch.float32, device=device)
        elif kind == "mhc_gate":   # logit(init gating factor) (mhc.py:83-84)
            gi = min(max(cfg.mhc_gating_init, 1e-5), 1 - 1e-5)
            t = torch.full(shape, math.log(gi / (1 - gi)), dtype=torch.float32, device=device)
        elif kind == "collapse":   # [I/S ... I/S] (model.py:415-421)
            D_, SD = shape
            t = (torch.eye(D_, dtype=torch.float32, device=device) / (SD // D_)).repeat(1, SD // D_)
        else:
            t = torch.full(shape, cfg.decay_logit_init, dtype=torch.float32, device=device)
        weights[name] = t if is_fp32_param(name) else t.to(torch.bfloat16)
    return weights
