"""Batched decode engine for the looped hybrid block stack on one MI355X.

Host orchestration in Python over the libllmy kernels (the reference's native
per-token step is llmy_cuda/src/model.cpp:1774-1935, batch 1 only; this one
decodes B sequences per step).  All device buffers — packed weights, per
(loop, layer) KV caches and GDN states, and every activation/scratch buffer —
are allocated once at construction, so ``step()`` enqueues kernels only and
the whole step can be captured into one HIP graph (``capture()``/``replay()``).

Packed weight layouts (built from the per-matrix weights of
``hybrid_llm_amd.config.init_weights``):
  * attention: wqkv [3*H*hd, D] = cat(wq, wk, wv); wo [D, H*hd];
  * GDN: wproj [N16, D] = cat(wq, wk, wv, wg, wb) padded with zero rows to a
    multiple of 16; the step kernel reads the fp32 projection row in place;
  * MoE: w_gate_up [E, 2H, D] = cat(w_gate, w_up, dim=1) (the reference's
    packing, llmy_cuda/include/llmy.h:80-82); w_down [E, D, H].
State layouts: KV caches [B, H, W, hd] bf16 (ring buffer, head-major);
GDN states [B, H, dk, dv] fp32; conv histories [B, K-1, D] bf16.
"""
from __future__ import annotations

import torch

from . import ops
from .config import HybridConfig


def _lib_load():
    from . import _lib
    return _lib.load()


def _pad_rows(w: torch.Tensor, mult: int) -> torch.Tensor:
    n = w.shape[0]
    pad = (-n) % mult
    if pad == 0:
        return w
    return torch.cat([w, torch.zeros(pad, *w.shape[1:], dtype=w.dtype, device=w.device)], 0)


CMP_PREFILL_MAX_SUMMARIES = 4000  # llmy_cmp_memory_prefill_bf16's limit per row


def check_prompt_length(cfg: HybridConfig, T: int) -> None:
    """Refuse, before any kernel runs, a prompt the compressed-memory prefill
    cannot take: more than 4000 summaries per row on a CSA / HCA block, or, on an
    HCA block with the context router, more summaries than the decode memory
    keeps (its latent attention reads the router's summary ring, which then no
    longer holds an early token's summaries; memory.decode_slots raises it)."""
    for kind in sorted({k for k in cfg.layer_kinds if k in ("csa", "hca")}):
        ratio = cfg.cmp_shape(kind)["ratio"]
        n = T // ratio
        if n > CMP_PREFILL_MAX_SUMMARIES:
            raise ValueError(f"prompt of {T} tokens: a {kind.upper()} block's prefill takes at most "
                             f"{CMP_PREFILL_MAX_SUMMARIES} summaries per row "
                             f"(T < {(CMP_PREFILL_MAX_SUMMARIES + 1) * ratio})")
        if kind == "hca" and cfg.context_router and n > cfg.cmp_slots:
            raise ValueError(f"prompt of {T} tokens emits {n} HCA summaries per row, more than the "
                             f"{cfg.cmp_slots} the router's summary memory keeps "
                             f"(memory.decode_slots); prefill at most "
                             f"{(cfg.cmp_slots + 1) * ratio - 1} tokens")


def round256(n: int) -> int:
    return (n + 255) // 256 * 256


def pad_hidden(gate_up: torch.Tensor, down: torch.Tensor):
    """Zero-pad the hidden width H of an expert stack (gate_up [E, 2H, D],
    down [E, D, H]) to the GEMM kernels' multiple of 256: zero gate and up rows
    give activations silu(0) * 0 = 0 and the zero down columns add nothing, so
    the result is the unpadded one (expert_hidden 320 / 640 of the reference's
    configs, model/config.py:33)."""
    E, H2, D = gate_up.shape
    H = H2 // 2
    Hp = round256(H)
    if Hp == H:
        return gate_up, down
    gu = gate_up.new_zeros(E, 2 * Hp, D)
    gu[:, :H] = gate_up[:, :H]
    gu[:, Hp:Hp + H] = gate_up[:, H:]
    dn = down.new_zeros(E, D, Hp)
    dn[:, :, :H] = down
    return gu, dn


def pad_cols(w: torch.Tensor) -> torch.Tensor:
    """Zero-pad the input width K of a [N, K] weight to a multiple of 256; its
    GEMM then reads an activation zero-padded the same way (``ops.pad_cols``)."""
    K = w.shape[-1]
    return w if K % 256 == 0 else torch.nn.functional.pad(w, (0, round256(K) - K))


class HybridDecoder:
    def __init__(self, cfg: HybridConfig, weights: dict[str, torch.Tensor], batch: int,
                 device: str | torch.device = "cuda",
                 sampling: tuple[float, float, int] | None = None):
        """``sampling`` = (temperature, top_p, top_k): each step then also draws
        ``buf["sampled"]`` with llmy_sample_top_p_f32 from the per-row uniforms
        in ``buf["u"]`` (set with ``set_uniforms``), beside the greedy
        ``buf["next"]``."""
        self.cfg = cfg
        self.sampling = sampling
        self.B = batch
        self.dev = torch.device(device)
        dev = self.dev
        D, B = cfg.d_model, batch

        def up(name, dtype=None):
            t = weights[name]
            return t.to(device=dev, dtype=dtype or t.dtype).contiguous()

        self.w: dict[str, torch.Tensor] = {"embed": up("embed"), "final_norm": up("final_norm")}

        def up_gdn(p):
            wproj = torch.cat([up(p + n) for n in ("wq", "wk", "wv", "wg", "wb")], 0)
            self.w[p + "wproj"] = _pad_rows(wproj, 16).contiguous()
            for n in ("wout", "bb", "conv", "decay"):
                self.w[p + n] = up(p + n)

        # stem / tail blocks: GDN mixer and the dense SwiGLU FFN as a one-expert
        # stack (gate | up [1, 2Hd, D], down [1, D, Hd]) run by the MoE kernels
        # with every token routed to it at gate 1
        self.side = {where: cfg.side_blocks(where) for where in ("stem", "tail")}
        for p in self.side["stem"] + self.side["tail"]:
            self.w[p + "mix_norm"] = up(p + "mix_norm")
            self.w[p + "ffn_norm"] = up(p + "ffn_norm")
            up_gdn(p)
            gu, dn = pad_hidden(torch.cat([up(p + "ffn_gate"), up(p + "ffn_up")], 0)[None],
                                up(p + "ffn_down")[None])
            self.w[p + "ffn_gate_up"], self.w[p + "ffn_down"] = gu.contiguous(), dn.contiguous()
        for l, kind in enumerate(cfg.layer_kinds):
            p = f"L{l}."
            self.w[p + "mix_norm"] = up(p + "mix_norm")
            if kind == "attn":
                self.w[p + "wqkv"] = torch.cat([up(p + "wq"), up(p + "wk"), up(p + "wv")], 0)
                self.w[p + "wo"] = up(p + "wo")
            elif kind in ("csa", "hca"):
                # q | k | v in one projection, the compressor's key | value in
                # another, [local_out | remote_out] over the branches' concat
                self.w[p + "cmp_wqkv"] = torch.cat([up(p + "cmp_wq"), up(p + "cmp_wk"),
                                                    up(p + "cmp_wv")], 0)
                self.w[p + "cmp_wc"] = torch.cat([up(p + "cmp_wck"), up(p + "cmp_wcv")], 0)
                self.w[p + "cmp_wlr"] = torch.cat([up(p + "cmp_wlo"), up(p + "cmp_wro")], 1)
                self.w[p + "cmp_wout"] = up(p + "cmp_wout")
            else:
                up_gdn(p)
            self.w[p + "ffn_norm"] = up(p + "ffn_norm")
            self.w[p + "router_norm"] = up(p + "router_norm")
            self.w[p + "w_router"] = up(p + "w_router")
            if cfg.context_router:
                # latent encoder and gate fp32; the two wide projections bf16,
                # packed below like the other GEMM weights
                # (the GEMMs over a latent_dim or heads x head_dim input not a
                # multiple of 256 read their input zero-padded: pad_cols)
                for n in ("ctx_down", "ctx_ln_w", "ctx_ln_b", "ctx_gate", "ctx_out"):
                    self.w[p + n] = up(p + n)
                self.w[p + "ctx_local_out"] = pad_cols(up(p + "ctx_local_out"))
                if kind == "hca":
                    # the global branch: the block's summary latents (hca_latent)
                    # and the router's latent attention; k | v in one projection
                    for n in ("hca_lat_down", "hca_lat_ln_w", "hca_lat_ln_b", "ctx_q"):
                        self.w[p + n] = up(p + n)
                    self.w[p + "ctx_o"] = pad_cols(up(p + "ctx_o"))
                    self.w[p + "ctx_kv"] = pad_cols(torch.cat([up(p + "ctx_k"),
                                                               up(p + "ctx_v")], 0))
            gate_up = torch.cat([up(p + "w_gate"), up(p + "w_up")], 1)
            down = up(p + "w_down")
            if cfg.shared_experts > 0:
                # shared experts stacked after the routed ones: experts E .. E+S-1,
                # reached by the always-on routes of llmy_moe_append_shared
                gate_up = torch.cat(
                    [gate_up, torch.cat([up(p + "w_shared_gate"), up(p + "w_shared_up")], 1)], 0)
                down = torch.cat([down, up(p + "w_shared_down")], 0)
            gate_up, down = pad_hidden(gate_up, down)
            self.w[p + "w_gate_up"] = gate_up.contiguous()
            self.w[p + "w_down"] = down.contiguous()

        # multi-stream hyper-connections: per-layer map / read / write
        # parameters in fp32, the maps' projection theta and the final
        # collapse as packed bf16 GEMM weights
        self.mhc = cfg.mhc_streams > 1
        if self.mhc:
            self.w["stream_seed"] = up("stream_seed")
            self.w["mhc_collapse"] = up("mhc_collapse")
            for p in self.prefixes():
                for n in ("mhc_map_norm", "mhc_pre_bias", "mhc_post_bias", "mhc_res_bias",
                          "mhc_alpha", "mhc_gating", "mhc_scale", "mhc_ln_w", "mhc_ln_b"):
                    self.w[p + n] = up(p + n)
                self.w[p + "mhc_theta"] = _pad_rows(up(p + "mhc_theta"), 16).contiguous()

        # Decode GEMM weights are re-laid once into the packed operand order
        # (llmy_pack_weights_bf16), so every weight byte streams as contiguous
        # 1 KiB wavefront loads; the embedding keeps a row-major copy for the
        # token lookup and a packed copy for the tied LM head.
        for name in list(self.w):
            if name.split(".")[-1] in ("wqkv", "wo", "wproj", "wout", "w_gate_up", "w_down",
                                       "ffn_gate_up", "ffn_down",
                                       "ctx_local_out", "ctx_out", "mhc_theta",
                                       "mhc_collapse", "cmp_wqkv", "cmp_wc", "cmp_wlr",
                                       "cmp_wout", "hca_lat_down", "ctx_q", "ctx_kv", "ctx_o"):
                self.w[name] = ops.pack_weights(self.w[name])
        self.w["lm_head"] = ops.pack_weights(self.w["embed"])

        # ---- state
        self.pos = torch.zeros(B, dtype=torch.int32, device=dev)
        self.state: dict = {}
        for loop in range(cfg.num_loops):
            for l, kind in enumerate(cfg.layer_kinds):
                if kind == "attn":
                    shape = (B, cfg.attn_heads, cfg.window, cfg.attn_head_dim)
                    self.state[(loop, l)] = {
                        "k": torch.zeros(shape, dtype=torch.bfloat16, device=dev),
                        "v": torch.zeros(shape, dtype=torch.bfloat16, device=dev)}
                elif kind in ("csa", "hca"):
                    # local window ring (keys, values), the memory's C slots
                    # (keys, values, tag = position + 1, 0 empty), the count of
                    # summaries a row emitted, the incomplete block's sum and count
                    cs = cfg.cmp_shape(kind)
                    Kw, W, C = cs["H"] * cs["Dh"], cs["W"], cfg.cmp_slots
                    bf = torch.bfloat16
                    self.state[(loop, l)] = {
                        "lk": torch.zeros(B, W, Kw, dtype=bf, device=dev),
                        "lv": torch.zeros(B, W, D, dtype=bf, device=dev),
                        "mk": torch.zeros(B, C, Kw, dtype=bf, device=dev),
                        "mv": torch.zeros(B, C, D, dtype=bf, device=dev),
                        "mtag": torch.zeros(B, C, dtype=torch.int32, device=dev),
                        "mcount": torch.zeros(B, dtype=torch.int32, device=dev),
                        "psum": torch.zeros(B, D, dtype=torch.float32, device=dev),
                        "pcnt": torch.zeros(B, dtype=torch.int32, device=dev)}
                    if kind == "hca" and cfg.context_router:
                        # the router's keys / values of each summary's latent,
                        # slots and tags as the memory's
                        HQ = cfg.router_heads * cfg.router_head_dim
                        self.state[(loop, l)].update({
                            "rk": torch.zeros(B, C, HQ, dtype=bf, device=dev),
                            "rv": torch.zeros(B, C, HQ, dtype=bf, device=dev),
                            "rtag": torch.zeros(B, C, dtype=torch.int32, device=dev),
                            "rcount": torch.zeros(B, dtype=torch.int32, device=dev)})
                else:
                    self.state[(loop, l)] = {
                        "S": torch.zeros(B, cfg.gdn_heads, cfg.gdn_dk, cfg.gdn_dv,
                                         dtype=torch.float32, device=dev),
                        "hist": torch.zeros(B, cfg.conv_kernel - 1, D, dtype=torch.bfloat16,
                                            device=dev)}
                if cfg.context_router:
                    # the router's last router_context latents per sequence (slot pos % W)
                    self.state[(loop, l)]["ctx_ring"] = torch.zeros(
                        B, cfg.router_context, cfg.latent_dim, dtype=torch.float32, device=dev)
        for where, prefixes in self.side.items():
            for i in range(len(prefixes)):
                self.state[(where, i)] = {
                    "S": torch.zeros(B, cfg.gdn_heads, cfg.gdn_dk, cfg.gdn_dv,
                                     dtype=torch.float32, device=dev),
                    "hist": torch.zeros(B, cfg.conv_kernel - 1, D, dtype=torch.bfloat16,
                                        device=dev)}

        # ---- activations / scratch (allocated once)
        f32, bf = torch.float32, torch.bfloat16
        Ha, hd = cfg.attn_heads, cfg.attn_head_dim
        Hg, dk, dv = cfg.gdn_heads, cfg.gdn_dk, cfg.gdn_dv
        k, E, Hf = cfg.top_k, cfg.n_experts, cfg.expert_hidden
        S = cfg.shared_experts
        kx, Ex = k + S, E + S  # routes per token and experts, shared ones included
        gdn_p = [p for p in self.prefixes() if p + "wproj" in self.w]
        side_p = self.side["stem"] + self.side["tail"]
        nproj = self.w[gdn_p[0] + "wproj"].shape[0] if gdn_p else 16
        Hf = self.w["L0.w_down"].shape[2]  # the (padded) expert hidden width
        self.buf = {
            "tokens": torch.zeros(B, dtype=torch.int32, device=dev),
            "reset": torch.zeros(B, dtype=torch.int32, device=dev),
            "x": torch.zeros(B, D, dtype=f32, device=dev),
            "h": torch.zeros(B, D, dtype=bf, device=dev),
            "qkv": torch.zeros(B, 3 * Ha * hd, dtype=bf, device=dev),
            "ao": torch.zeros(B, Ha, hd, dtype=bf, device=dev),
            "proj": torch.zeros(B, nproj, dtype=f32, device=dev),
            "go": torch.zeros(B, Hg * dv, dtype=bf, device=dev),
            "cg": torch.zeros(B, D, dtype=f32, device=dev),
            "idx": torch.zeros(B, k, dtype=torch.int32, device=dev),
            "gates": torch.zeros(B, k, dtype=f32, device=dev),
            "counts": torch.zeros(Ex, dtype=torch.int32, device=dev),
            "offsets": torch.zeros(Ex + 1, dtype=torch.int32, device=dev),
            "sorted_routes": torch.zeros(B * kx, dtype=torch.int32, device=dev),
            "route_pos": torch.zeros(B * kx, dtype=torch.int32, device=dev),
            "act": torch.zeros(B * kx, Hf, dtype=bf, device=dev),
            # the dense FFN of stem / tail blocks: its activation, and the one
            # route per token (expert 0, gate 1)
            "dact": torch.zeros(B, self.w[side_p[0] + "ffn_down"].shape[2] if side_p else 256,
                                dtype=bf, device=dev),
            "dids": torch.zeros(B, 1, dtype=torch.int32, device=dev),
            "dgates": torch.ones(B, 1, dtype=f32, device=dev),
            "y": torch.zeros(B * kx, D, dtype=f32, device=dev),
            "logits": torch.zeros(B, cfg.vocab, dtype=f32, device=dev),
            "next": torch.zeros(B, dtype=torch.int32, device=dev),
            "u": torch.zeros(B, dtype=f32, device=dev),
            "sampled": torch.zeros(B, dtype=torch.int32, device=dev),
        }
        self.graph: torch.cuda.CUDAGraph | None = None
        # CSA / HCA decode buffers: per kind the fused projection and the
        # compressor's summary row; shared branch outputs and list workspace
        cmp_kinds = sorted({k for k in cfg.layer_kinds if k in ("csa", "hca")})
        if cmp_kinds:
            ws = 16
            for kind in cmp_kinds:
                cs = cfg.cmp_shape(kind)
                Kw = cs["H"] * cs["Dh"]
                self.buf["cqkv_" + kind] = torch.zeros(B, 2 * Kw + D, dtype=bf, device=dev)
                self.buf["ckv_" + kind] = torch.zeros(B, Kw + D, dtype=bf, device=dev)
                lib = _lib_load()
                ws = max(ws, int(lib.llmy_cmp_workspace_bytes(B, cs["H"], cs["W"], 0, 1)),
                         int(lib.llmy_cmp_workspace_bytes(B, cs["H"], cfg.cmp_slots,
                                                          cs["top_k"], 1)))
            self.buf.update({"cloc": torch.zeros(B, 2 * D, dtype=bf, device=dev),
                             "cy": torch.zeros(B, D, dtype=bf, device=dev),
                             "cmean": torch.zeros(B, D, dtype=bf, device=dev),
                             "cemit": torch.zeros(B, dtype=torch.int32, device=dev),
                             "cws": torch.zeros(ws, dtype=torch.uint8, device=dev)})
        # Decode MoE: fused norm + router (W_r in LDS) and route-indexed experts
        # that derive their routes from the ids (no permutation pass) when the
        # sizes allow; else norm, router, permutation and sorted experts.
        # the fused norm + router kernel (any number of rows)
        self.fused_router_ok = E * D <= 24576 and D in (256, 512, 1024) and k <= 8
        self.fused_route = self.fused_router_ok and B * kx <= 2048
        if S > 0:
            self.buf["idx_all"] = torch.zeros(B, kx, dtype=torch.int32, device=dev)
            self.buf["gates_all"] = torch.zeros(B, kx, dtype=f32, device=dev)
        if cfg.context_router:
            if cfg.latent_dim % 64 or cfg.latent_dim > 512 or D > 1024:
                raise ValueError("the context router needs latent_dim % 64 == 0, latent_dim <= 512, "
                                 "d_model <= 1024")
            Lc = cfg.latent_dim
            self.ctx_buf = {"local": torch.zeros(B, D, dtype=f32, device=dev),
                            "lat": torch.zeros(B, Lc, dtype=f32, device=dev),
                            "ctx": torch.zeros(B, Lc, dtype=bf, device=dev),
                            "ctx_p": torch.zeros(B, round256(Lc), dtype=bf, device=dev),
                            "ctx_d": torch.zeros(B, D, dtype=bf, device=dev),
                            "ctx_c": torch.zeros(B, D, dtype=f32, device=dev),
                            "logits": torch.zeros(B, E, dtype=f32, device=dev),
                            "idx": self.buf["idx"], "gates": self.buf["gates"]}
            if "hca" in cfg.layer_kinds:
                HQ = cfg.router_heads * cfg.router_head_dim
                if HQ % 16 or cfg.router_head_dim % 8:
                    raise ValueError("the router's latent attention needs heads * head_dim % 16 "
                                     "== 0 and head_dim % 8 == 0")
                self.ctx_buf.update({"ctx_t": torch.zeros(B, D, dtype=f32, device=dev),
                                     "lq": torch.zeros(B, D, dtype=bf, device=dev),
                                     "gq": torch.zeros(B, HQ, dtype=bf, device=dev),
                                     "gattn": torch.zeros(B, HQ, dtype=bf, device=dev),
                                     "gattn_p": torch.zeros(B, round256(HQ), dtype=bf, device=dev)})
                self.buf.update({"cval": torch.zeros(B, 1, D, dtype=bf, device=dev),
                                 "clat_raw": torch.zeros(B, Lc, dtype=f32, device=dev),
                                 "clat": torch.zeros(B, Lc, dtype=bf, device=dev),
                                 "clat_p": torch.zeros(B, round256(Lc), dtype=bf, device=dev),
                                 "ckvr": torch.zeros(B, 2 * HQ, dtype=bf, device=dev)})
        # Mixer output projections (attention o, GDN out) as per-K-block
        # partial products that the fused router folds into the residual: a
        # workgroup then reads a 256-wide slice of the activations instead of
        # all of them, and no residual round trip precedes the store.
        n_parts = max(Ha * hd, Hg * dv) // 256
        self.defer_resid = (self.fused_route and B <= 64 and (Ha * hd) % 256 == 0
                            and (Hg * dv) % 256 == 0 and n_parts <= 8 and not self.mhc)
        if self.defer_resid:
            self.buf["parts"] = torch.zeros(n_parts, B, D, dtype=f32, device=dev)
        # The GDN input projection the same way: its partials are summed by
        # the GDN step kernel as it reads the row.
        self.proj_parts = B <= 64 and D % 256 == 0 and D // 256 <= 8 and cfg.has_gdn
        if self.proj_parts:
            self.buf["proj_parts"] = torch.zeros(D // 256, B, nproj, dtype=f32, device=dev)
        # ... and the attention q/k/v projection: its partials are summed (and
        # rounded to bf16, as the projection would have stored them) by the
        # attention decode kernel
        self.qkv_parts = (B <= 64 and D % 256 == 0 and D // 256 <= 8
                          and "attn" in cfg.layer_kinds)
        if self.qkv_parts:
            self.buf["qkv_parts"] = torch.zeros(D // 256, B, 3 * Ha * hd, dtype=f32, device=dev)
        self._pending: tuple | None = None
        if self.mhc:
            Sm = cfg.mhc_streams
            nt = self.w["L0.mhc_theta"].shape[0]
            self.buf.update({
                "X": torch.zeros(B, Sm, D, dtype=f32, device=dev),    # the streams
                "xb": torch.zeros(B, Sm * D, dtype=bf, device=dev),   # GEMM operands
                "raw": torch.zeros(B, nt, dtype=f32, device=dev),     # map logits
                "maps": torch.zeros(B, Sm + Sm * Sm, dtype=f32, device=dev),
                "U": torch.zeros(B, D, dtype=f32, device=dev),        # a sublayer's output
                "route_ident": torch.arange(B * kx, dtype=torch.int32, device=dev)})
        # Optional record of every MoE application's expert ids (verification
        # aid: lets a checker replay the kernel's discrete routing decisions),
        # and of the residual stream after each application.
        self.route_log: torch.Tensor | None = None
        self.x_log: torch.Tensor | None = None
        # The same for prefill: one [B*T, k] id tensor per MoE application.
        self.route_log_seq: list | None = None
        # Optional record of the CSA / HCA top-k memory selections (verification
        # aid): (core layer, positions of the selected summaries, -1 none) per
        # mixer call, [B, H, k] in decode and [B, T, H, k] in prefill.
        self.sel_log: list | None = None

    def enable_route_log(self, residuals: bool = False) -> None:
        """Record every MoE application's expert ids in ``route_log`` [apps, B, k]
        and, with ``residuals``, the residual stream after each application in
        ``x_log`` [apps, B, D] (verification aids: a checker can replay the
        discrete routing and check each application from the same input)."""
        n_apps = self.cfg.num_loops * self.cfg.n_layers
        self.route_log = torch.zeros(n_apps, self.B, self.cfg.top_k, dtype=torch.int32,
                                     device=self.dev)
        self.x_log = (torch.zeros(n_apps, self.B, self.cfg.d_model, dtype=torch.float32,
                                  device=self.dev) if residuals else None)
        self._app = 0

    def prefixes(self) -> list[str]:
        """Weight prefixes of every block: stem, core layers, tail."""
        return (self.side["stem"] + [f"L{l}." for l in range(self.cfg.n_layers)]
                + self.side["tail"])

    def _apps(self) -> list[tuple]:
        """The blocks one token passes in order, (weight prefix, kind, core
        layer or None, state): the stem, the core num_loops times (one state per
        (loop, layer)), the tail (model.py:842-909).  Stem / tail blocks have
        kind "side" (GDN mixer, dense FFN)."""
        cfg = self.cfg
        apps = [(p, "side", None, self.state[("stem", i)])
                for i, p in enumerate(self.side["stem"])]
        for loop in range(cfg.num_loops):
            for l in range(cfg.n_layers):
                apps.append((f"L{l}.", cfg.layer_kinds[l], l, self.state[(loop, l)]))
        apps += [(p, "side", None, self.state[("tail", i)])
                 for i, p in enumerate(self.side["tail"])]
        return apps

    # ------------------------------------------------------------------ blocks
    def _attn(self, l: int, st: dict, out=None, epilogue=None) -> None:
        cfg, w, b = self.cfg, self.w, self.buf
        p = f"L{l}."
        Hhd = cfg.attn_heads * cfg.attn_head_dim
        B, H, hd = self.B, cfg.attn_heads, cfg.attn_head_dim
        if self.qkv_parts:
            ops.linear(b["h"], w[p + "wqkv"], out=b["qkv_parts"], epilogue=ops.EPI_PARTIAL_F32,
                       layout=ops.LAYOUT_PACKED)
            ops.banded_attn_decode_parts(b["qkv_parts"], Hhd, 2 * Hhd, st["k"], st["v"],
                                         self.pos, cfg.attn_scale, out=b["ao"])
        else:
            ops.linear(b["h"], w[p + "wqkv"], out=b["qkv"], layout=ops.LAYOUT_PACKED)
            qkv = b["qkv"]
            q = qkv[:, :Hhd].view(B, H, hd)
            kn = qkv[:, Hhd:2 * Hhd].view(B, H, hd)
            vn = qkv[:, 2 * Hhd:].view(B, H, hd)
            ops.banded_attn_decode(q, kn, vn, st["k"], st["v"], self.pos, cfg.attn_scale,
                                   out=b["ao"])
        if self.defer_resid:
            parts = b["parts"][:Hhd // 256]
            ops.linear(b["ao"].view(B, Hhd), w[p + "wo"], out=parts,
                       epilogue=ops.EPI_PARTIAL_F32, layout=ops.LAYOUT_PACKED)
            self._pending = (parts, None)
        else:
            ops.linear(b["ao"].view(B, Hhd), w[p + "wo"], out=b["x"] if out is None else out,
                       epilogue=ops.EPI_RESID_ADD if epilogue is None else epilogue,
                       layout=ops.LAYOUT_PACKED)

    def _gdn(self, p: str, st: dict, out=None, defer: bool = True) -> None:
        """The GDN mixer of the block with weight prefix p on h; its output is
        added to x (gated by the conv), stored to ``out``, or with ``defer`` (and
        the engine's deferred residual) left as per-K-block partial products
        that the next MoE router folds in."""
        w, b = self.w, self.buf
        if self.proj_parts:
            proj = b["proj_parts"]
            ops.linear(b["h"], w[p + "wproj"], out=proj, epilogue=ops.EPI_PARTIAL_F32,
                       layout=ops.LAYOUT_PACKED)
        else:
            proj = b["proj"]
            ops.linear(b["h"], w[p + "wproj"], out=proj, epilogue=ops.EPI_STORE_F32,
                       layout=ops.LAYOUT_PACKED)
        ops.gdn_step_fused(proj, w[p + "bb"], w[p + "decay"], st["S"], out=b["go"],
                           conv=(b["h"], st["hist"], w[p + "conv"], b["cg"]))
        if self.defer_resid and defer:
            parts = b["parts"][:b["go"].shape[1] // 256]
            ops.linear(b["go"], w[p + "wout"], out=parts, epilogue=ops.EPI_PARTIAL_F32,
                       layout=ops.LAYOUT_PACKED)
            self._pending = (parts, b["cg"])
        else:
            ops.linear(b["go"], w[p + "wout"], out=b["x"] if out is None else out,
                       epilogue=ops.EPI_RESID_GATED, aux=b["cg"], layout=ops.LAYOUT_PACKED)

    def _cmp(self, l: int, st: dict, out=None, epilogue=None) -> None:
        """CSA / HCA decode (csa.py:157-259, hca.py:106-193): the q | k | v
        projection, the local window over the ring (the new key and value stored
        first), the compressor step with, for a row completing a block, its new
        summary committed to the memory, the memory branch, then
        out(local_out(local) + remote_out(memory)) into the residual."""
        cfg, w, b = self.cfg, self.w, self.buf
        p, kind = f"L{l}.", cfg.layer_kinds[l]
        cs = cfg.cmp_shape(kind)
        H, Dh, D = cs["H"], cs["Dh"], cfg.d_model
        Kw = H * Dh
        qkv = b["cqkv_" + kind]
        ops.linear(b["h"], w[p + "cmp_wqkv"], out=qkv, layout=ops.LAYOUT_PACKED)
        q, k, v = qkv[:, :Kw], qkv[:, Kw:2 * Kw], qkv[:, 2 * Kw:]
        loc = b["cloc"]
        ops.cmp_local_decode(q, k, v, st["lk"], st["lv"], self.pos, H, Dh, out=loc[:, :D],
                             workspace=b["cws"])
        ops.cmp_pool_step(b["h"], st["psum"], st["pcnt"], cs["ratio"], mean=b["cmean"],
                          emit=b["cemit"])
        ckv = b["ckv_" + kind]
        ops.linear(b["cmean"], w[p + "cmp_wc"], out=ckv, layout=ops.LAYOUT_PACKED)
        ops.cmp_commit(ckv, b["cemit"], self.pos, st["mk"], st["mv"], st["mtag"], st["mcount"])
        if "rk" in st:
            # the router's keys / values of the new summary's latent, committed
            # with the same flags (the summary values copied to a dense operand)
            ops.cmp_ring_fill(ckv[:, Kw:], self.B, 1, b["cval"])
            self._router_summary_kv(p, b["cval"].view(self.B, D), b["clat_raw"], b["clat"],
                                    b["ckvr"], b["clat_p"])
            ops.cmp_commit(b["ckvr"], b["cemit"], self.pos, st["rk"], st["rv"], st["rtag"],
                           st["rcount"])
        ops.cmp_memory_decode(q, st["mk"], st["mv"], st["mtag"], self.pos, H, Dh, cs["top_k"],
                              out=loc[:, D:], workspace=b["cws"])
        if self.sel_log is not None and cs["top_k"] > 0:
            # the list's slot indices follow its weights in the workspace
            B_, k_ = self.B, cs["top_k"]
            nl = B_ * H * k_
            il = b["cws"][:8 * nl].view(torch.int32)[nl:].view(B_, H * k_).long()
            tag = torch.gather(st["mtag"], 1, il.clamp_min(0)).view(B_, H, k_)
            self.sel_log.append((l, torch.where(il.view(B_, H, k_) >= 0, tag - 1,
                                                torch.full_like(tag, -1)).cpu()))
        ops.linear(loc, w[p + "cmp_wlr"], out=b["cy"], layout=ops.LAYOUT_PACKED)
        ops.linear(b["cy"], w[p + "cmp_wout"], out=b["x"] if out is None else out,
                   epilogue=ops.EPI_RESID_ADD if epilogue is None else epilogue,
                   layout=ops.LAYOUT_PACKED)

    def _router_summary_kv(self, p: str, vals, lat_raw=None, lat=None, out=None, lat_p=None):
        """The router's [k | v] of summary values (model.py:318-334 with
        mla_memory.py:23-24): LayerNorm(down . value) (eps 1e-5), then k | v."""
        w = self.w
        lat_raw = ops.linear(vals, w[p + "hca_lat_down"], out=lat_raw, epilogue=ops.EPI_STORE_F32,
                             layout=ops.LAYOUT_PACKED)
        lat = ops.layernorm(lat_raw, w[p + "hca_lat_ln_w"], w[p + "hca_lat_ln_b"], 1e-5, out=lat)
        lat = ops.pad_cols(lat, w[p + "ctx_kv"].shape[1], out=lat_p)
        return ops.linear(lat, w[p + "ctx_kv"], out=out, layout=ops.LAYOUT_PACKED)

    def _glob(self, l: int, st: dict) -> dict | None:
        """The context router's global branch operands of an HCA layer."""
        if "rk" not in st:
            return None
        p = f"L{l}."
        return {"q": self.w[p + "ctx_q"], "o": self.w[p + "ctx_o"], "rk": st["rk"],
                "rv": st["rv"], "rtag": st["rtag"], "heads": self.cfg.router_heads,
                "head_dim": self.cfg.router_head_dim}

    def _ctx_weights(self, p: str) -> dict:
        w = self.w
        return {n: w[p + n] for n in ("router_norm", "ctx_down", "ctx_ln_w", "ctx_ln_b",
                                       "ctx_local_out", "ctx_out", "ctx_gate", "w_router")}

    def _dense(self, p: str, next_norm=None, out=None) -> None:
        """The dense SwiGLU FFN of a stem / tail block (dense_ffn.py:14-15) on h:
        the MoE kernels over the one-expert stack with every token routed to it
        at gate 1, then added to x with the next block's pre-norm into h, or
        stored to ``out``."""
        cfg, w, b, B = self.cfg, self.w, self.buf, self.B
        y = b["y"][:B]
        ops.moe_experts_routed(b["h"], b["dids"], b["dgates"], w[p + "ffn_gate_up"],
                               w[p + "ffn_down"], act=b["dact"], y=y, layout=ops.LAYOUT_PACKED)
        if out is None:
            ops.moe_combine_norm(y, None, b["x"], b["h"], next_norm, 1, cfg.eps)
        else:
            ops.moe_combine(y, b["route_ident"][:B], B, 1, out=out, mode=ops.MOE_OUT_F32)

    def _dense_seq(self, p: str, x, h, next_norm=None, out=None) -> None:
        """``_dense`` over the B*T rows of a prefill (the grouped expert GEMMs
        with one expert)."""
        cfg, w = self.cfg, self.w
        R = h.shape[0]
        perm = ops.moe_permute(torch.zeros(R, dtype=torch.int32, device=self.dev), 1)
        gates = torch.ones(R, 1, dtype=torch.float32, device=self.dev)
        _, y = ops.moe_experts(h, perm, gates, w[p + "ffn_gate_up"], w[p + "ffn_down"],
                               layout=ops.LAYOUT_PACKED)
        if out is None:
            ops.moe_combine_norm(y, perm["route_pos"], x, h, next_norm, 1, cfg.eps)
        else:
            ops.moe_combine(y, perm["route_pos"], R, 1, out=out, mode=ops.MOE_OUT_F32)

    def _moe(self, l: int, next_norm: torch.Tensor | None, st: dict) -> None:
        """Pre-MoE norm + router + permutation, experts, then the combine fused
        with the next block's pre-norm (``next_norm``) into ``h``."""
        cfg, w, b = self.cfg, self.w, self.buf
        p = f"L{l}."
        if self.fused_route:
            # decode: router only; the experts derive their routes from the ids
            parts, gate = self._pending if self._pending is not None else (None, None)
            self._pending = None
            ops.moe_route_decode(b["x"], w[p + "ffn_norm"], w[p + "router_norm"],
                                 w[p + "w_router"], cfg.top_k, cfg.eps, bufs=b, permute=False,
                                 parts=parts, gate=gate)
        else:
            ops.rmsnorm(b["x"], w[p + "ffn_norm"], cfg.eps, out=b["h"])
            from . import _lib
            s = torch.cuda.current_stream().cuda_stream
            _lib.call("llmy_router_topk_bf16", b["h"].data_ptr(),
                      w[p + "router_norm"].data_ptr(), w[p + "w_router"].data_ptr(), None,
                      b["idx"].data_ptr(), b["gates"].data_ptr(), self.B, cfg.d_model,
                      cfg.n_experts, cfg.top_k, cfg.eps, s)
        if cfg.context_router:
            # the context-aware ids replace the plain router's (same buffers)
            ops.router_context(b["h"], self._ctx_weights(p), st["ctx_ring"], cfg.top_k,
                               pos=self.pos, eps=cfg.eps, layout=ops.LAYOUT_PACKED,
                               bufs=self.ctx_buf, glob=self._glob(l, st))
        S = cfg.shared_experts
        idx, gates = b["idx"], b["gates"]
        if S > 0:
            idx, gates = ops.moe_append_shared(idx, gates, cfg.n_experts, S,
                                               idx_out=b["idx_all"], gates_out=b["gates_all"])
        kx = cfg.top_k + S
        if not self.fused_route:
            _lib.call("llmy_moe_permute", idx.data_ptr(), self.B * kx, cfg.n_experts + S,
                      b["counts"].data_ptr(), b["offsets"].data_ptr(),
                      b["sorted_routes"].data_ptr(), b["route_pos"].data_ptr(), s)
        if self.route_log is not None:
            self.route_log[self._app].copy_(b["idx"])
        if self.fused_route:
            ops.moe_experts_routed(b["h"], idx, gates, w[p + "w_gate_up"],
                                   w[p + "w_down"], act=b["act"], y=b["y"],
                                   layout=ops.LAYOUT_PACKED)
            route_pos = None
        else:
            ops.moe_experts(b["h"], b, gates, w[p + "w_gate_up"], w[p + "w_down"],
                            act=b["act"], y=b["y"], layout=ops.LAYOUT_PACKED)
            route_pos = b["route_pos"]
        ops.moe_combine_norm(b["y"], route_pos, b["x"], b["h"], next_norm, kx, cfg.eps)
        if self.route_log is not None:
            if self.x_log is not None:
                self.x_log[self._app].copy_(b["x"])
            self._app = (self._app + 1) % self.route_log.shape[0]

    # ------------------------------------------------------------------ step
    def _step_body(self) -> None:
        if self.mhc:
            self._step_body_mhc()
            return
        cfg, w, b = self.cfg, self.w, self.buf
        apps = self._apps()
        ops.embed_norm(b["tokens"], w["embed"], w[apps[0][0] + "mix_norm"], b["x"], b["h"],
                       cfg.eps)
        for i, (p, kind, l, st) in enumerate(apps):
            nxt = w[apps[i + 1][0] + "mix_norm"] if i + 1 < len(apps) else w["final_norm"]
            if kind == "side":
                self._gdn(p, st, defer=False)
                ops.rmsnorm(b["x"], w[p + "ffn_norm"], cfg.eps, out=b["h"])
                self._dense(p, nxt)
                continue
            if kind == "attn":
                self._attn(l, st)
            elif kind in ("csa", "hca"):
                self._cmp(l, st)
            else:
                self._gdn(p, st)
            self._moe(l, nxt, st)
        ops.linear(b["h"], w["lm_head"], out=b["logits"], epilogue=ops.EPI_STORE_F32,
                   layout=ops.LAYOUT_PACKED)
        self._sample()
        self.pos.add_(1)

    # ------------------------------------------------------------------ mHC
    def _mhc_params(self, p: str) -> dict:
        return {n: self.w[p + "mhc_" + n] for n in ("pre_bias", "post_bias", "res_bias", "alpha",
                                                     "ln_w", "ln_b")}

    def _mhc_read(self, p: str, X, norm: str, raw, maps, h, xb) -> None:
        """The maps of block p's hyper-connection and the sublayer input h
        (model.py:119-123; mhc.py:156-206): RMSNorm of the flattened streams
        into bf16, the theta projection, then maps + read + LayerNorm + the
        sublayer's RMSNorm in one kernel."""
        cfg, w = self.cfg, self.w
        M = X.shape[0]
        ops.rmsnorm(X.view(M, -1), w[p + "mhc_map_norm"], ops.MHC_MAP_EPS, out=xb)
        ops.linear(xb, w[p + "mhc_theta"], out=raw, epilogue=ops.EPI_STORE_F32,
                   layout=ops.LAYOUT_PACKED)
        ops.mhc_read(X, raw, self._mhc_params(p), w[p + norm], cfg.mhc_sinkhorn_iters,
                     maps=maps, h=h, norm_eps=cfg.eps)

    def _mhc_write(self, p: str, X, U, maps) -> None:
        ops.mhc_write(X, U, maps, self.w[p + "mhc_scale"], self.w[p + "mhc_gating"])

    def _mhc_head(self, X, xb, U) -> None:
        """Collapse the streams (model.py:699-700), the final RMSNorm, the LM head."""
        w, b, M = self.w, self.buf, X.shape[0]
        ops.f32_to_bf16(X.view(M, -1), out=xb)
        ops.linear(xb, w["mhc_collapse"], out=U, epilogue=ops.EPI_STORE_F32,
                   layout=ops.LAYOUT_PACKED)
        ops.rmsnorm(U, w["final_norm"], self.cfg.eps, out=b["h"])
        ops.linear(b["h"], w["lm_head"], out=b["logits"], epilogue=ops.EPI_STORE_F32,
                   layout=ops.LAYOUT_PACKED)

    def _step_body_mhc(self) -> None:
        """The decode step with multi-stream hyper-connections: each sublayer
        reads the streams through its maps and writes its output back
        (model.py:177-264); mixer, MoE and dense FFN kernels as in the
        single-stream step, their outputs stored to U instead of added to a
        residual."""
        from . import _lib
        cfg, w, b = self.cfg, self.w, self.buf
        X, U = b["X"], b["U"]
        ops.mhc_embed(b["tokens"], w["embed"], w["stream_seed"], out=X)
        s = torch.cuda.current_stream().cuda_stream
        kx = cfg.top_k + cfg.shared_experts
        for p, kind, l, st in self._apps():
            self._mhc_read(p, X, "mix_norm", b["raw"], b["maps"], b["h"], b["xb"])
            if kind == "attn":
                self._attn(l, st, out=U, epilogue=ops.EPI_STORE_F32)
            elif kind in ("csa", "hca"):
                self._cmp(l, st, out=U, epilogue=ops.EPI_STORE_F32)
            else:
                U.zero_()
                self._gdn(p, st, out=U)
            self._mhc_write(p, X, U, b["maps"])
            self._mhc_read(p, X, "ffn_norm", b["raw"], b["maps"], b["h"], b["xb"])
            if kind == "side":
                self._dense(p, out=U)
                self._mhc_write(p, X, U, b["maps"])
                continue
            if cfg.context_router:
                ops.router_context(b["h"], self._ctx_weights(p), st["ctx_ring"], cfg.top_k,
                                   pos=self.pos, eps=cfg.eps, layout=ops.LAYOUT_PACKED,
                                   bufs=self.ctx_buf, glob=self._glob(l, st))
            else:
                _lib.call("llmy_router_topk_bf16", b["h"].data_ptr(),
                          w[p + "router_norm"].data_ptr(), w[p + "w_router"].data_ptr(), None,
                          b["idx"].data_ptr(), b["gates"].data_ptr(), self.B, cfg.d_model,
                          cfg.n_experts, cfg.top_k, cfg.eps, s)
            idx, gates = b["idx"], b["gates"]
            if cfg.shared_experts > 0:
                idx, gates = ops.moe_append_shared(idx, gates, cfg.n_experts,
                                                   cfg.shared_experts, idx_out=b["idx_all"],
                                                   gates_out=b["gates_all"])
            if self.route_log is not None:
                self.route_log[self._app].copy_(b["idx"])
                self._app = (self._app + 1) % self.route_log.shape[0]
            if self.fused_route:
                ops.moe_experts_routed(b["h"], idx, gates, w[p + "w_gate_up"],
                                       w[p + "w_down"], act=b["act"], y=b["y"],
                                       layout=ops.LAYOUT_PACKED)
                route_pos = b["route_ident"]
            else:
                _lib.call("llmy_moe_permute", idx.data_ptr(), self.B * kx,
                          cfg.n_experts + cfg.shared_experts, b["counts"].data_ptr(),
                          b["offsets"].data_ptr(), b["sorted_routes"].data_ptr(),
                          b["route_pos"].data_ptr(), s)
                ops.moe_experts(b["h"], b, gates, w[p + "w_gate_up"], w[p + "w_down"],
                                act=b["act"], y=b["y"], layout=ops.LAYOUT_PACKED)
                route_pos = b["route_pos"]
            ops.moe_combine(b["y"], route_pos, self.B, kx, out=U, mode=ops.MOE_OUT_F32)
            self._mhc_write(p, X, U, b["maps"])
        self._mhc_head(X, b["xb"], U)
        self._sample()
        self.pos.add_(1)

    def _sample(self) -> None:
        """Greedy argmax into buf["next"], and the top-p draw into buf["sampled"]
        when sampling is configured."""
        from . import _lib
        b, V = self.buf, self.cfg.vocab
        stream = torch.cuda.current_stream().cuda_stream
        _lib.call("llmy_sample_argmax_f32", b["logits"].data_ptr(), self.B, V,
                  b["next"].data_ptr(), stream)
        if self.sampling is not None:
            T, p, k = self.sampling
            _lib.call("llmy_sample_top_p_f32", b["logits"].data_ptr(), self.B, V,
                      float(T), int(k), float(p), b["u"].data_ptr(), b["sampled"].data_ptr(),
                      stream)

    def set_uniforms(self, u: torch.Tensor) -> None:
        """Per-row uniform draws in [0, 1) for the next steps' top-p sampling."""
        self.buf["u"].copy_(u.to(torch.float32).view(-1))

    def reset_rows(self, mask: torch.Tensor) -> None:
        """Rows b with mask[b] != 0 start a new sequence: their KV caches, GDN
        states, conv histories and router latent rings are zeroed and their
        next position is 0 (RecurrentState.reset_rows,
        model/recurrent_state.py:213-225, as decode_step applies it,
        model/model.py:814-822).  Kernels only, no memory set."""
        m = self.buf["reset"]
        m.copy_(torch.as_tensor(mask).to(torch.int32).view(-1))
        for st in self.state.values():
            for t in st.values():
                ops.zero_rows(t, m)
        ops.zero_rows(self.pos, m)

    def step(self, tokens: torch.Tensor | None = None, reset=None) -> torch.Tensor:
        """Decode one token for every sequence.  ``tokens`` [B] int32 (device or
        host) is copied into the static input buffer; ``reset`` [B] (optional):
        those rows start a new sequence at position 0 first (``reset_rows``).
        Returns the logits buffer."""
        if reset is not None:
            self.reset_rows(reset)
        if tokens is not None:
            self.buf["tokens"].copy_(tokens.to(torch.int32).view(-1))
        if self.graph is not None:
            self.graph.replay()
        else:
            self._step_body()
        return self.buf["logits"]

    def capture(self) -> None:
        """Capture one step (embedding .. argmax [, top-p draw], pos += 1) into a HIP graph.
        Capturing runs nothing, so the state is unchanged."""
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                self._step_body()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.graph = g

    # ------------------------------------------------------------------ prefill
    def reset(self) -> None:
        """Fresh sequences: zero every KV cache, GDN state and conv history, pos = 0
        (llmy_state_reset, llmy_cuda/src/llmy.cpp:99-114)."""
        for st in self.state.values():
            for t in st.values():
                t.zero_()
        self.pos.zero_()

    def prefill(self, tokens: torch.Tensor) -> torch.Tensor:
        """Prefill B fresh sequences with a [B, T] prompt through the sequence
        kernels and return the logits buffer [B, V] of the last position.

        The reference prefills token by token through its decode step
        (model_prefill, llmy_cuda/src/model.cpp:1955-1966); this runs every
        block once over all B*T tokens: projections as GEMMs over B*T rows,
        banded attention prefill (then the last min(T, W) K/V rows into the
        ring caches), the chunked GDN scan from the zero state with the
        sequence conv gate, and the MoE through router -> permutation ->
        grouped expert GEMMs -> combine.  Afterwards the state is the one T
        decode steps would leave, pos = T, ``buf["next"]`` holds the greedy
        next token (and ``buf["sampled"]`` the draw when sampling is set), and
        decoding continues with ``step``.  Intermediate buffers scale with
        B*T and are allocated per call."""
        cfg, w = self.cfg, self.w
        tokens = tokens.to(device=self.dev, dtype=torch.int32)
        if tokens.dim() != 2 or tokens.shape[0] != self.B or tokens.shape[1] < 1:
            raise ValueError(f"tokens must be [B={self.B}, T>=1], got {tuple(tokens.shape)}")
        B, T = tokens.shape
        R, D = B * T, cfg.d_model
        check_prompt_length(cfg, T)
        self.reset()
        if self.mhc:
            return self._prefill_mhc(tokens, B, T)
        x = torch.empty(R, D, dtype=torch.float32, device=self.dev)
        h = torch.empty(R, D, dtype=torch.bfloat16, device=self.dev)
        apps = self._apps()
        ops.embed_norm(tokens.contiguous().view(-1), w["embed"], w[apps[0][0] + "mix_norm"], x, h,
                       cfg.eps)
        for i, (p, kind, l, st) in enumerate(apps):
            nxt = w[apps[i + 1][0] + "mix_norm"] if i + 1 < len(apps) else w["final_norm"]
            if kind == "side":
                self._gdn_seq(p, st, x, h, B, T)
                ops.rmsnorm(x, w[p + "ffn_norm"], cfg.eps, out=h)
                self._dense_seq(p, x, h, nxt)
                continue
            if kind == "attn":
                self._attn_seq(l, st, x, h, B, T)
            elif kind in ("csa", "hca"):
                self._cmp_seq(l, st, x, h, B, T)
            else:
                self._gdn_seq(p, st, x, h, B, T)
            self._moe_seq(l, x, h, nxt, st, B)
        b = self.buf
        b["h"].copy_(h.view(B, T, D)[:, -1])
        ops.linear(b["h"], w["lm_head"], out=b["logits"], epilogue=ops.EPI_STORE_F32,
                   layout=ops.LAYOUT_PACKED)
        self._sample()
        self.pos.fill_(T)
        return b["logits"]

    def _prefill_mhc(self, tokens, B: int, T: int) -> torch.Tensor:
        """Prefill with multi-stream hyper-connections: the sequence kernels of
        ``prefill`` with each sublayer's output stored to U and written into the
        [B*T, S, D] streams through the layer's maps (model.py:177-264)."""
        from . import _lib
        cfg, w, b = self.cfg, self.w, self.buf
        R, D, Sm, dev = B * T, cfg.d_model, cfg.mhc_streams, self.dev
        X = ops.mhc_embed(tokens.contiguous().view(-1), w["embed"], w["stream_seed"])
        h = torch.empty(R, D, dtype=torch.bfloat16, device=dev)
        U = torch.empty(R, D, dtype=torch.float32, device=dev)
        xb = torch.empty(R, Sm * D, dtype=torch.bfloat16, device=dev)
        raw = torch.empty(R, w["L0.mhc_theta"].shape[0], dtype=torch.float32, device=dev)
        maps = torch.empty(R, Sm + Sm * Sm, dtype=torch.float32, device=dev)
        s = torch.cuda.current_stream().cuda_stream
        E, k = cfg.n_experts, cfg.top_k
        for p, kind, l, st in self._apps():
            self._mhc_read(p, X, "mix_norm", raw, maps, h, xb)
            if kind == "attn":
                self._attn_seq(l, st, U, h, B, T, epilogue=ops.EPI_STORE_F32)
            elif kind in ("csa", "hca"):
                self._cmp_seq(l, st, U, h, B, T, epilogue=ops.EPI_STORE_F32)
            else:
                U.zero_()
                self._gdn_seq(p, st, U, h, B, T)
            self._mhc_write(p, X, U, maps)
            self._mhc_read(p, X, "ffn_norm", raw, maps, h, xb)
            if kind == "side":
                self._dense_seq(p, None, h, out=U)
                self._mhc_write(p, X, U, maps)
                continue
            idx = torch.empty(R, k, dtype=torch.int32, device=dev)
            gates = torch.empty(R, k, dtype=torch.float32, device=dev)
            if cfg.context_router:
                # rows are B sequences of T tokens from position 0 (fresh state)
                idx, gates, _ = ops.router_context(h, self._ctx_weights(p), st["ctx_ring"], k,
                                                   eps=cfg.eps, layout=ops.LAYOUT_PACKED,
                                                   bufs={"idx": idx, "gates": gates},
                                                   glob=self._glob(l, st))
            else:
                _lib.call("llmy_router_topk_bf16", h.data_ptr(), w[p + "router_norm"].data_ptr(),
                          w[p + "w_router"].data_ptr(), None, idx.data_ptr(), gates.data_ptr(),
                          R, D, E, k, cfg.eps, s)
            if self.route_log_seq is not None:
                self.route_log_seq.append(idx.clone())
            Ex, kx = E, k
            if cfg.shared_experts > 0:
                idx, gates = ops.moe_append_shared(idx, gates, E, cfg.shared_experts)
                Ex, kx = E + cfg.shared_experts, k + cfg.shared_experts
            perm = ops.moe_permute(idx.view(-1), Ex)
            _, y = ops.moe_experts(h, perm, gates, w[p + "w_gate_up"], w[p + "w_down"],
                                   layout=ops.LAYOUT_PACKED)
            ops.moe_combine(y, perm["route_pos"], R, kx, out=U, mode=ops.MOE_OUT_F32)
            self._mhc_write(p, X, U, maps)
        b["X"].copy_(X.view(B, T, Sm, D)[:, -1])
        self._mhc_head(b["X"], b["xb"], b["U"])
        self._sample()
        self.pos.fill_(T)
        return b["logits"]

    def _attn_seq(self, l: int, st: dict, x, h, B: int, T: int, epilogue=None) -> None:
        cfg, w = self.cfg, self.w
        p = f"L{l}."
        H, hd = cfg.attn_heads, cfg.attn_head_dim
        Hhd, R = H * hd, B * T
        # Rows [a, b) (multiples of 16) of a packed weight are themselves the
        # packed [b - a, K] matrix, so q, k, v come from slices of wqkv.
        wqkv = w[p + "wqkv"]
        q, k, v = (ops.linear(h, wqkv[j * Hhd:(j + 1) * Hhd], layout=ops.LAYOUT_PACKED)
                   for j in range(3))
        o = ops.banded_attn_prefill(q.view(B, T, H, hd), k.view(B, T, H, hd),
                                    v.view(B, T, H, hd), cfg.window, cfg.attn_scale)
        ops.kv_cache_fill(k.view(B, T, Hhd), v.view(B, T, Hhd), st["k"], st["v"])
        ops.linear(o.view(R, Hhd), w[p + "wo"], out=x,
                   epilogue=ops.EPI_RESID_ADD if epilogue is None else epilogue,
                   layout=ops.LAYOUT_PACKED)

    def _cmp_seq(self, l: int, st: dict, x, h, B: int, T: int, epilogue=None) -> None:
        """CSA / HCA over B fresh sequences (csa.py:35-155, hca.py:32-104): the
        projection over B*T rows, the local window, the block means and their
        summaries, the memory branch, the output projections; then the state T
        decode steps would leave (ring: the last W keys / values; memory: the
        summaries with their tags; the incomplete block's sum and count)."""
        cfg, w = self.cfg, self.w
        p, kind = f"L{l}.", cfg.layer_kinds[l]
        cs = cfg.cmp_shape(kind)
        H, Dh, D, ratio = cs["H"], cs["Dh"], cfg.d_model, cs["ratio"]
        Kw, R, n = H * Dh, B * T, T // cs["ratio"]
        qkv = ops.linear(h, w[p + "cmp_wqkv"], layout=ops.LAYOUT_PACKED)
        q, k, v = qkv[:, :Kw], qkv[:, Kw:2 * Kw], qkv[:, 2 * Kw:]
        loc = torch.empty(R, 2 * D, dtype=torch.bfloat16, device=self.dev)
        ops.cmp_local_prefill(q, k, v, B, T, H, Dh, cs["W"], out=loc[:, :D])
        means = ops.cmp_pool_prefill(h, B, T, ratio, st["psum"], st["pcnt"])
        kv = (ops.linear(means, w[p + "cmp_wc"], layout=ops.LAYOUT_PACKED) if n else
              torch.empty(0, Kw + D, dtype=torch.bfloat16, device=self.dev))
        ws = (ops.cmp_workspace(R, H, max(n, 1), cs["top_k"], self.dev)
              if self.sel_log is not None and cs["top_k"] > 0 else None)
        ops.cmp_memory_prefill(q, kv[:, :Kw], kv[:, Kw:], B, T, ratio, H, Dh, cs["top_k"],
                               out=loc[:, D:], slots=cfg.cmp_slots, workspace=ws)
        if ws is not None:
            # entry i of a row is the summary at position (i + 1) ratio - 1
            nl = R * H * cs["top_k"]
            il = ws[:8 * nl].view(torch.int32)[nl:].view(B, T, H, cs["top_k"]).long()
            self.sel_log.append((l, torch.where(il >= 0, (il + 1) * ratio - 1,
                                                torch.full_like(il, -1)).cpu()))
        ops.cmp_memory_fill(kv, B, n, ratio, st["mk"], st["mv"], st["mtag"], st["mcount"])
        if "rk" in st and n:
            kvr = self._router_summary_kv(p, kv[:, Kw:].contiguous())
            ops.cmp_memory_fill(kvr, B, n, ratio, st["rk"], st["rv"], st["rtag"], st["rcount"])
        ops.cmp_ring_fill(k, B, T, st["lk"])
        ops.cmp_ring_fill(v, B, T, st["lv"])
        y1 = ops.linear(loc, w[p + "cmp_wlr"], layout=ops.LAYOUT_PACKED)
        ops.linear(y1, w[p + "cmp_wout"], out=x,
                   epilogue=ops.EPI_RESID_ADD if epilogue is None else epilogue,
                   layout=ops.LAYOUT_PACKED)

    def _gdn_seq(self, p: str, st: dict, x, h, B: int, T: int) -> None:
        """The GDN mixer of block p over B fresh sequences of T tokens, added to
        x (gated by the conv)."""
        cfg, w = self.cfg, self.w
        H, dk, dv = cfg.gdn_heads, cfg.gdn_dk, cfg.gdn_dv
        R, HV = B * T, H * dv
        proj = ops.linear(h, w[p + "wproj"], epilogue=ops.EPI_STORE_F32,
                          layout=ops.LAYOUT_PACKED)
        pp = ops.gdn_prefill_prep(proj, w[p + "bb"], w[p + "decay"], H, dk, dv)
        o = ops.gdn_prefill(pp["q"].view(B, T, H, dk), pp["k"].view(B, T, H, dk),
                            pp["v"].view(B, T, H, dv), pp["beta"].view(B, T, H),
                            pp["g"].view(B, T, H), st["S"])
        go = o.view(R, HV)
        ops.gdn_gate(go, proj, 2 * H * dk + HV, out=go)
        cg = ops.gdn_conv_gate_prefill(h.view(B, T, cfg.d_model), st["hist"], w[p + "conv"])
        ops.linear(go, w[p + "wout"], out=x, epilogue=ops.EPI_RESID_GATED,
                   aux=cg.view(R, cfg.d_model), layout=ops.LAYOUT_PACKED)

    def _moe_seq(self, l: int, x, h, next_norm, st: dict, B: int) -> None:
        """Pre-MoE norm, router + top-k, stable permutation, grouped expert
        GEMMs, then the combine fused with the next block's pre-norm into h."""
        from . import _lib
        cfg, w = self.cfg, self.w
        p = f"L{l}."
        R, D, E, k = x.shape[0], cfg.d_model, cfg.n_experts, cfg.top_k
        dev, s = self.dev, torch.cuda.current_stream().cuda_stream
        idx = torch.empty(R, k, dtype=torch.int32, device=dev)
        gates = torch.empty(R, k, dtype=torch.float32, device=dev)
        if self.fused_router_ok:
            # one launch per token: pre-MoE norm (h) + router + top-k
            ops.moe_route_decode(x, w[p + "ffn_norm"], w[p + "router_norm"], w[p + "w_router"],
                                 k, cfg.eps, bufs={"h": h, "idx": idx, "gates": gates},
                                 permute=False)
        else:
            ops.rmsnorm(x, w[p + "ffn_norm"], cfg.eps, out=h)
        if cfg.context_router:
            # rows are B sequences of T tokens from position 0 (fresh state)
            idx, gates, _ = ops.router_context(h, self._ctx_weights(p), st["ctx_ring"], k,
                                               eps=cfg.eps, layout=ops.LAYOUT_PACKED,
                                               bufs={"idx": idx, "gates": gates},
                                               glob=self._glob(l, st))
        elif not self.fused_router_ok:
            _lib.call("llmy_router_topk_bf16", h.data_ptr(), w[p + "router_norm"].data_ptr(),
                      w[p + "w_router"].data_ptr(), None, idx.data_ptr(), gates.data_ptr(), R, D,
                      E, k, cfg.eps, s)
        if self.route_log_seq is not None:
            self.route_log_seq.append(idx.clone())
        if cfg.shared_experts > 0:
            idx, gates = ops.moe_append_shared(idx, gates, E, cfg.shared_experts)
            E, k = E + cfg.shared_experts, k + cfg.shared_experts
        perm = ops.moe_permute(idx.view(-1), E)
        _, y = ops.moe_experts(h, perm, gates, w[p + "w_gate_up"], w[p + "w_down"],
                               layout=ops.LAYOUT_PACKED)
        ops.moe_combine_norm(y, perm["route_pos"], x, h, next_norm, k, cfg.eps)

    # ------------------------------------------------------------------ state io
    def load_state(self, pos: torch.Tensor, state: dict) -> None:
        """Copy a host state (the oracle's layout) into the device buffers
        (attention and GDN layers)."""
        if any(k in ("csa", "hca") for k in self.cfg.layer_kinds):
            raise NotImplementedError("load_state covers attention and GDN layers")
        self.pos.copy_(pos.to(torch.int32))
        for key, st in self.state.items():
            for name, t in st.items():
                if name == "ctx_ring":
                    # the oracle keeps the last n latents in order: slot (pos - n + i) % W
                    hist = state[key]["lat"]
                    n, W = hist.shape[1], t.shape[1]
                    for bi in range(t.shape[0]):
                        p0 = int(pos[bi])
                        for i in range(n):
                            t[bi, (p0 - n + i) % W].copy_(hist[bi, i].to(t.dtype))
                    continue
                t.copy_(state[key][name].to(t.dtype))
