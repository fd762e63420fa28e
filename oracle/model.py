"""Looped hybrid-block stack oracle (test infrastructure only).

Composes the pinned ops into the block of model/model.py:162-264, looping the
core ``num_loops`` times with one state per (loop, layer) (model.py:618-687,
:645), tied LM head (model.py:705).  Stem and tail blocks (GDN mixer, then a
dense SwiGLU FFN: model.py:89-93,391-394,411-414, dense_ffn.py:14-15) run once
before and after the loops (model.py:600-606,689-695; decode :842-845,906-909).  With ``mhc_streams`` > 1 the residual is
S streams read and written around each sublayer through the layer's
hyper-connection maps (model.py:119-126,177-264), seeded from the embedding
(:442-444) and collapsed before the final norm (:699-700); with 1 it is the
single residual stream of mHC disabled (model.py:119-126).

Mixers:
  * attention: q/k/v projections, banded attention over a ring KV cache
    (decode window of model/layers/hca.py:119-128), output projection;
  * CSA / HCA: the compressed-memory mixers of oracle/compressed.py (local
    window plus block summaries, model/layers/csa.py, hca.py) through their
    decode path;
  * GDN: gated_deltanet.py:125-149,254-275 — q/k/v/gate/beta projections,
    per-head L2 norm of q and k (clamp 1e-12), beta = sigmoid(.+bias),
    gate = sigmoid(.), decay = sigmoid(decay_logit) per head, the delta-rule
    step, o = (q^T S) * gate, out_proj, times sigmoid(causal depthwise conv)
    over the last ``conv_kernel`` normalised inputs.
MoE: router (own RMSNorm + fp32 logits + top-k + softmax; with the context-aware
router, the logits of context_router.py:94-137 from a per-(loop, layer)
history of the last router_context latents and, on HCA layers, the global
branch over the block's emitted summaries, hca_global_context), routed SwiGLU
experts (model/layers/moe.py:172-199) plus the shared experts when the config has
them (moe.py:185-199: their sum scaled by 1/sqrt(S), added to the routed output).

``act_bf16=True`` rounds activations to bf16 exactly where the HIP path
stores them in bf16 (GEMM inputs, the KV cache, the MoE activation), so the
comparison isolates accumulation-order differences; ``False`` is the plain
fp32 reference of BASELINE config 1.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from hybrid_llm_amd.config import HybridConfig

from .attention import banded_attention_decode
from .compressed import CompressedMixer
from .gdn import gdn_step
from .mhc import mhc_maps, mhc_read, mhc_write
from .moe import moe_grouped, shared_experts
from .router import (context_latents, context_route_logits, hca_global_context, rmsnorm,
                     router_logits, router_topk)


def _bf16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).float()


class HybridOracle:
    def __init__(self, cfg: HybridConfig, weights: dict[str, torch.Tensor], act_bf16: bool = False):
        self.cfg = cfg
        self.w = {k: v.float() for k, v in weights.items()}
        self.rnd = _bf16 if act_bf16 else (lambda t: t)
        # Discrete-decision forcing: when set to a list of [B, k] expert-id
        # arrays (one per MoE application, in execution order), the oracle
        # routes with those ids instead of its own top-k, and records in
        # route_gaps the logit gap of every token whose choice differed.
        self.forced_routes: list | None = None
        self.routes: list[np.ndarray] = []
        self.route_gaps: list[float] = []
        self.route_total = 0
        self.cmp = {l: CompressedMixer(self.w, f"L{l}.", *self._cmp_args(k), act_round=self.rnd)
                    for l, k in enumerate(cfg.layer_kinds) if k in ("csa", "hca")}

    def _cmp_args(self, kind: str):
        cs = self.cfg.cmp_shape(kind)
        return cs["H"], cs["Dh"], cs["W"], cs["ratio"], cs["top_k"] or None

    # ---- state -----------------------------------------------------------
    def new_state(self, batch: int) -> dict:
        cfg = self.cfg
        st: dict = {"pos": torch.zeros(batch, dtype=torch.long)}
        for loop in range(cfg.num_loops):
            for l, kind in enumerate(cfg.layer_kinds):
                if kind == "attn":
                    shape = (batch, cfg.attn_heads, cfg.window, cfg.attn_head_dim)
                    st[(loop, l)] = {"k": torch.zeros(shape), "v": torch.zeros(shape)}
                elif kind in ("csa", "hca"):
                    st[(loop, l)] = {"cmp": self.cmp[l].new_state(batch, cfg.d_model)}
                else:
                    st[(loop, l)] = {
                        "S": torch.zeros(batch, cfg.gdn_heads, cfg.gdn_dk, cfg.gdn_dv),
                        "hist": torch.zeros(batch, cfg.conv_kernel - 1, cfg.d_model),
                    }
                # the router's latent history (context_router.py:108-121)
                st[(loop, l)]["lat"] = torch.zeros(batch, 0, cfg.latent_dim)
        # stem / tail blocks: one GDN state and conv history each, outside the
        # loops' namespaces (model.py:181-184 with state keys stem.<i> / tail.<i>)
        for where in ("stem", "tail"):
            for i in range(len(cfg.side_blocks(where))):
                st[(where, i)] = {
                    "S": torch.zeros(batch, cfg.gdn_heads, cfg.gdn_dk, cfg.gdn_dv),
                    "hist": torch.zeros(batch, cfg.conv_kernel - 1, cfg.d_model)}
        return st

    # ---- blocks ----------------------------------------------------------
    def _attn(self, l: int, h: torch.Tensor, st: dict, pos: torch.Tensor) -> torch.Tensor:
        cfg, w, rnd = self.cfg, self.w, self.rnd
        B = h.shape[0]
        H, hd = cfg.attn_heads, cfg.attn_head_dim
        p = f"L{l}."
        q = rnd(h @ w[p + "wq"].t()).view(B, H, hd)
        k = rnd(h @ w[p + "wk"].t()).view(B, H, hd)
        v = rnd(h @ w[p + "wv"].t()).view(B, H, hd)
        o, st["k"], st["v"] = banded_attention_decode(q, k, v, st["k"], st["v"], pos,
                                                      cfg.attn_scale)
        return rnd(o).reshape(B, H * hd) @ w[p + "wo"].t()

    def _gdn(self, p: str, h: torch.Tensor, st: dict) -> torch.Tensor:
        """The GDN mixer of the block with weight prefix p."""
        cfg, w, rnd = self.cfg, self.w, self.rnd
        B = h.shape[0]
        H, dk, dv = cfg.gdn_heads, cfg.gdn_dk, cfg.gdn_dv
        q = (h @ w[p + "wq"].t()).view(B, H, dk)
        k = (h @ w[p + "wk"].t()).view(B, H, dk)
        v = (h @ w[p + "wv"].t()).view(B, H, dv)
        gate = torch.sigmoid(h @ w[p + "wg"].t()).view(B, H, dv)
        beta = torch.sigmoid(h @ w[p + "wb"].t() + w[p + "bb"])
        q = q * torch.rsqrt((q * q).sum(-1, keepdim=True).clamp_min(1e-12))
        k = k * torch.rsqrt((k * k).sum(-1, keepdim=True).clamp_min(1e-12))
        g = torch.sigmoid(w[p + "decay"]).expand(B, H)
        o, st["S"] = gdn_step(q, k, v, beta, g, st["S"], gate=gate)
        o = rnd(o.reshape(B, H * dv))
        window = torch.cat([st["hist"], h[:, None]], dim=1)  # [B, K, D]
        conv = (window * w[p + "conv"].t()[None]).sum(1)      # tap j -> position t-(K-1)+j
        st["hist"] = window[:, 1:].clone()
        return (o @ w[p + "wout"].t()) * torch.sigmoid(conv)

    def _moe(self, l: int, h2: torch.Tensor, s: dict | None = None) -> torch.Tensor:
        cfg, w = self.cfg, self.w
        p = f"L{l}."
        if cfg.context_router:
            # forward_step: mean of the last W latents (history + current)
            local, lat = context_latents(h2, w[p + "router_norm"], w[p + "ctx_down"],
                                         w[p + "ctx_ln_w"], w[p + "ctx_ln_b"], cfg.eps)
            hist = torch.cat([s["lat"], lat[:, None]], dim=1)[:, -cfg.router_context:]
            s["lat"] = hist
            if "lat_n" in s:
                # rows reset earlier hold fewer valid latents (the last n of the window)
                n = (s["lat_n"] + 1).clamp(max=cfg.router_context)
                s["lat_n"] = n
                W = hist.shape[1]
                ctx = torch.stack([hist[b, W - int(n[b]):].double().mean(0)
                                   for b in range(hist.shape[0])]).float()
            else:
                ctx = hist.double().mean(1).float()
            glob = None
            if cfg.layer_kinds[l] == "hca":
                # the global branch over this block's emitted summaries
                cm = s["cmp"]
                vals = [cm["mv"][b][cm["mpos"][b] >= 0] for b in range(h2.shape[0])]
                glob = hca_global_context(local, vals, w[p + "hca_lat_down"],
                                          w[p + "hca_lat_ln_w"], w[p + "hca_lat_ln_b"],
                                          w[p + "ctx_q"], w[p + "ctx_k"], w[p + "ctx_v"],
                                          w[p + "ctx_o"], cfg.router_heads, cfg.router_head_dim,
                                          self.rnd)
            logits = context_route_logits(local, ctx, w[p + "ctx_local_out"], w[p + "ctx_out"],
                                          w[p + "ctx_gate"], w[p + "w_router"], self.rnd,
                                          global_ctx=glob)
        else:
            logits = router_logits(h2, w[p + "w_router"], w[p + "router_norm"], cfg.eps)
        idx, gates = router_topk(logits, cfg.top_k)
        if self.forced_routes is not None:
            forced = np.asarray(self.forced_routes.pop(0)).reshape(idx.shape).astype(np.int64)
            self._check_forced(logits, idx, forced)
            idx = forced
            gates = torch.gather(logits, 1, torch.from_numpy(idx)).softmax(-1)
        self.routes.append(idx.copy())
        out = moe_grouped(h2, idx, gates, w[p + "w_gate"], w[p + "w_up"], w[p + "w_down"],
                          act_round=self.rnd)
        if cfg.shared_experts > 0:
            out = out + shared_experts(h2, w[p + "w_shared_gate"], w[p + "w_shared_up"],
                                       w[p + "w_shared_down"], act_round=self.rnd)
        return out

    def _check_forced(self, logits: torch.Tensor, own: np.ndarray, forced: np.ndarray) -> None:
        """Record how far a forced routing is from the oracle's own choice: for
        every token whose forced expert set differs, the logit gap between the
        oracle's weakest own pick and the forced set's weakest pick (0 for a tie)."""
        for t in range(own.shape[0]):
            if sorted(own[t]) != sorted(forced[t]):
                lo_own = float(logits[t, own[t]].min())
                lo_forced = float(logits[t, forced[t]].min())
                self.route_gaps.append(lo_own - lo_forced)
            self.route_total += 1

    # ---- step ------------------------------------------------------------
    def embed(self, tokens) -> torch.Tensor:
        """The residual stream's start: embedding rows (model.py:386); with
        mHC the S streams embed + stream_seed[s] (model.py:442-444), [B, S, D]."""
        tokens = torch.as_tensor(np.asarray(tokens), dtype=torch.long).view(-1)
        x = self.w["embed"][tokens].clone()
        if self.cfg.mhc_streams > 1:
            x = x[:, None, :] + self.w["stream_seed"][None]
        return x

    def _dense(self, p: str, h2: torch.Tensor) -> torch.Tensor:
        """The dense SwiGLU FFN of a stem / tail block (dense_ffn.py:14-15):
        down(silu(gate h) * up h), the activation rounded as the engine's bf16
        operand."""
        w = self.w
        a = self.rnd(F.silu(h2 @ w[p + "ffn_gate"].t()) * (h2 @ w[p + "ffn_up"].t()))
        return a @ w[p + "ffn_down"].t()

    def _mhc_read(self, p: str, X: torch.Tensor):
        """The maps of the hyper-connection of the block with weight prefix p
        and the read of the streams (model.py:119-123; mhc.py:156-206); the
        theta projection's input is rounded as the engine's bf16 GEMM operand."""
        cfg, w = self.cfg, self.w
        maps = mhc_maps(X, w[p + "mhc_theta"], w[p + "mhc_map_norm"], w[p + "mhc_pre_bias"],
                        w[p + "mhc_post_bias"], w[p + "mhc_res_bias"], w[p + "mhc_alpha"],
                        cfg.mhc_sinkhorn_iters, act_round=self.rnd)
        return mhc_read(X, maps[0], w[p + "mhc_ln_w"], w[p + "mhc_ln_b"]), maps

    def _mhc_write(self, p: str, X, U, maps):
        return mhc_write(X, U, maps[1], maps[2], self.w[p + "mhc_scale"], self.w[p + "mhc_gating"])

    def _block(self, p: str, mixer, ffn, x: torch.Tensor) -> torch.Tensor:
        """A block with weight prefix p (mixer branch then FFN branch, each a
        pre-norm residual branch: model.py:119-126,162-264) applied to the
        residual x; ``mixer`` / ``ffn`` map the normalised input to the branch
        output.  With mHC, x is the [B, S, D] streams, each branch reads them
        through the block's maps and writes its output back (model.py:177-264)."""
        cfg, w, rnd = self.cfg, self.w, self.rnd
        mhc = cfg.mhc_streams > 1
        hidden, maps = self._mhc_read(p, x) if mhc else (x, None)
        u = mixer(rnd(rmsnorm(hidden, w[p + "mix_norm"], cfg.eps)))
        x = self._mhc_write(p, x, u, maps) if mhc else x + u
        hidden, maps = self._mhc_read(p, x) if mhc else (x, None)
        u = ffn(rnd(rmsnorm(hidden, w[p + "ffn_norm"], cfg.eps)))
        return self._mhc_write(p, x, u, maps) if mhc else x + u

    def apply(self, l: int, x: torch.Tensor, s: dict, pos: torch.Tensor) -> torch.Tensor:
        """One application of core layer l (its mixer, then its MoE) to the
        residual x, updating that (loop, layer)'s state s in place; returns the
        new x."""
        kind = self.cfg.layer_kinds[l]
        if kind == "attn":
            mixer = lambda h: self._attn(l, h, s, pos)  # noqa: E731
        elif kind in ("csa", "hca"):
            mixer = lambda h: self.cmp[l].step(h, s["cmp"], pos)  # noqa: E731
        else:
            mixer = lambda h: self._gdn(f"L{l}.", h, s)  # noqa: E731
        return self._block(f"L{l}.", mixer, lambda h2: self._moe(l, h2, s), x)

    def apply_side(self, p: str, x: torch.Tensor, s: dict) -> torch.Tensor:
        """One stem / tail block (weight prefix p): its GDN mixer, then its
        dense SwiGLU FFN (model.py:89-93,391-394,411-414)."""
        return self._block(p, lambda h: self._gdn(p, h, s), lambda h2: self._dense(p, h2), x)

    def head(self, x: torch.Tensor) -> torch.Tensor:
        """Final RMSNorm and the tied LM head (model.py:705): fp32 logits.  With
        mHC the streams are first collapsed by mhc_collapse (model.py:699-700),
        whose input is rounded as the engine's bf16 GEMM operand."""
        if self.cfg.mhc_streams > 1:
            x = self.rnd(x.reshape(x.shape[0], -1)) @ self.w["mhc_collapse"].t()
        hf = self.rnd(rmsnorm(x, self.w["final_norm"], self.cfg.eps))
        return hf @ self.w["embed"].t()

    def reset_rows(self, st: dict, mask) -> None:
        """Rows b with mask[b] start a new sequence: their GDN states, conv
        histories, KV caches and router latent histories are zeroed and their
        position is 0 (RecurrentState.reset_rows, model/recurrent_state.py:213-225,
        applied by decode_step before a token whose reset_mask is set,
        model/model.py:814-822)."""
        rows = torch.as_tensor(np.asarray(mask)).to(torch.bool).view(-1)
        st["pos"] = torch.where(rows, torch.zeros_like(st["pos"]), st["pos"])
        for key, s in st.items():
            if key == "pos":
                continue
            for name in ("S", "hist", "k", "v"):
                if name in s:
                    s[name] = s[name].clone()
                    s[name][rows] = 0
            if "cmp" in s:
                CompressedMixer.reset_rows(s["cmp"], rows)
            if self.cfg.context_router and "lat" in s:
                n = s.get("lat_n", torch.full((rows.numel(),), s["lat"].shape[1],
                                              dtype=torch.long))
                s["lat_n"] = torch.where(rows, torch.zeros_like(n), n)
                s["lat"] = s["lat"].clone()
                s["lat"][rows] = 0

    def step(self, tokens, st: dict, num_loops: int | None = None, reset=None) -> torch.Tensor:
        """Decode one token per sequence; returns fp32 logits [B, V].  ``reset``
        [B]: those rows start a new sequence first (``reset_rows``)."""
        cfg = self.cfg
        if reset is not None:
            self.reset_rows(st, reset)
        pos = st["pos"].clone()
        x = self.embed(tokens)
        for i, p in enumerate(cfg.side_blocks("stem")):
            x = self.apply_side(p, x, st[("stem", i)])
        loops = cfg.num_loops if not num_loops else num_loops
        for loop in range(loops):
            for l in range(cfg.n_layers):
                x = self.apply(l, x, st[(loop, l)], pos)
        for i, p in enumerate(cfg.side_blocks("tail")):
            x = self.apply_side(p, x, st[("tail", i)])
        st["pos"] = pos + 1
        return self.head(x)

    def prefill(self, tokens, st: dict) -> torch.Tensor:
        """Token-by-token prefill of a [B, T] prompt; returns logits [B, T, V]."""
        tokens = torch.as_tensor(np.asarray(tokens), dtype=torch.long)
        if tokens.dim() == 1:
            tokens = tokens[None]
        outs = [self.step(tokens[:, t], st) for t in range(tokens.shape[1])]
        return torch.stack(outs, dim=1)
