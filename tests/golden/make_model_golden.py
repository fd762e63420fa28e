"""Writes tests/golden/model_golden.npz and model_golden_hca.npz: logits of the
reference's whole model, LoopedHybridMoEForCausalLM (model/model.py:379-929),
for small configs shaped like the reference's own checkpoints.  The first has
one stem and one tail block (GDN + dense SwiGLU FFN), 4 mHC streams, the
context-aware router, a GDN / CSA / GDN core looped twice, shared experts,
expert_hidden 320, latent_dim 128 and router query heads 4 x 32; the second an
HCA / GDN core with the plain router.

The weights are this build's own deterministic draw (``golden_weights``, from
``hybrid_llm_amd.config.init_weights`` plus a perturbation of the norms, biases
and gates so that their roles are pinned too), loaded into the reference model
under its state-dict names; the tests regenerate them with the same function,
so the fixture holds only the config, the token ids and the logits.  The
reference is run on the CPU in fp32: ``forward`` over a prompt with
``collect_diagnostics=False`` (the inference prefill, model.py:554-705), then,
for a few decoded tokens, ``forward`` over the prompt and the tokens so far
(the last position's logits; see ``main`` for why not ``decode_step``).

Run in the build container only (it imports the reference model from
/root/reference); the committed .npz is the fixture, the reference never
travels.

    python tests/golden/make_model_golden.py
"""
from __future__ import annotations

import os
import re
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from hybrid_llm_amd.config import HybridConfig, init_weights, weight_shapes  # noqa: E402

REF = "/root/reference"

# The golden model: the reference checkpoints' block structure at a small width.
GOLDEN = HybridConfig(
    d_model=256, layer_kinds=("gdn", "csa", "gdn"), attn_heads=0, attn_head_dim=0, window=0,
    gdn_heads=4, gdn_dk=64, gdn_dv=64, n_experts=8, top_k=4, expert_hidden=320, vocab=512,
    num_loops=2, shared_experts=2, context_router=True, latent_dim=128, router_context=8,
    router_heads=4, router_head_dim=32, mhc_streams=4, mhc_sinkhorn_iters=20,
    csa_heads=4, csa_head_dim=64, csa_window=8, csa_ratio=4, csa_top_k=3,
    stem_blocks=1, tail_blocks=1, dense_hidden=384)
# The HCA block in the whole model, with the plain router (with the context
# router the reference's Python model hands every MoE of a loop the latest HCA
# memory's latents, a rule this build does not follow; see HybridOracle).
GOLDEN_HCA = HybridConfig(
    d_model=256, layer_kinds=("hca", "gdn"), attn_heads=0, attn_head_dim=0, window=0,
    gdn_heads=4, gdn_dk=64, gdn_dv=64, n_experts=8, top_k=2, expert_hidden=256, vocab=512,
    num_loops=2, shared_experts=1, context_router=False, mhc_streams=4, mhc_sinkhorn_iters=20,
    hca_window=8, hca_ratio=4, stem_blocks=1, tail_blocks=1, dense_hidden=256)
SEED = 11
BATCH, PROMPT, DECODE = 2, 20, 4
# fixture file -> (config, weight seed)
CASES = {"model_golden.npz": (GOLDEN, SEED), "model_golden_hca.npz": (GOLDEN_HCA, SEED + 10)}


def golden_weights(cfg: HybridConfig = GOLDEN, seed: int = SEED) -> dict[str, torch.Tensor]:
    """``init_weights`` with every constant-initialised parameter perturbed
    (norm weights, biases, decay logits, router gates, mHC biases, alphas and
    gating logits), so the fixture pins what each one does."""
    w = init_weights(cfg, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    for name, shape, kind in weight_shapes(cfg):
        if kind == "normal" or kind == "seed":
            continue
        t = w[name].float()
        noise = torch.randn(shape, generator=g)
        if kind == "ones":
            t = t + 0.1 * noise
        elif kind == "zeros":
            t = 0.1 * noise
        elif kind == "decay":
            t = t + 0.5 * noise
        elif kind == "gate":       # the router's route gate: let the context matter
            t = torch.full(shape, -1.0) + 0.3 * noise
        elif kind in ("mhc_pre", "eye4"):
            t = t + 0.3 * noise
        elif kind == "alpha":      # input-dependent maps
            t = 0.5 + 0.1 * noise
        elif kind == "mhc_gate":
            t = t + 0.5 * noise
        elif kind == "collapse":
            t = t + 0.02 * noise
        w[name] = t.to(w[name].dtype)
    return w


def _ref_config(cfg: HybridConfig):
    from model.config import (AdaptiveLoopConfig, CSAConfig, DenseFFNConfig, GDNConfig,
                              HCAConfig, LoopAttnResConfig, MHCConfig, MLAConfig, MoEConfig,
                              RouterConfig, V6Config)
    return V6Config(
        vocab_size=cfg.vocab, d_model=cfg.d_model, tie_word_embeddings=True,
        physical_blocks=cfg.stem_blocks + cfg.n_layers + cfg.tail_blocks,
        stem_blocks=cfg.stem_blocks, recurrent_blocks=cfg.n_layers, tail_blocks=cfg.tail_blocks,
        num_loops=cfg.num_loops, recurrent_layout=tuple(k + "_moe" for k in cfg.layer_kinds),
        mhc=MHCConfig(enabled=True, streams=cfg.mhc_streams,
                      sinkhorn_iterations=cfg.mhc_sinkhorn_iters),
        gdn=GDNConfig(qk_heads=cfg.gdn_heads, value_heads=cfg.gdn_heads,
                      qk_head_dim=cfg.gdn_dk, value_head_dim=cfg.gdn_dv,
                      conv_kernel=cfg.conv_kernel),
        moe=MoEConfig(routed_experts=cfg.n_experts, shared_experts=cfg.shared_experts,
                      routed_top_k=cfg.top_k, expert_hidden=cfg.expert_hidden),
        mla=MLAConfig(latent_dim=cfg.latent_dim),
        router=RouterConfig(context_aware=cfg.context_router, query_heads=cfg.router_heads,
                            query_head_dim=cfg.router_head_dim,
                            local_context=cfg.router_context, use_hca_global_latents=False),
        csa=CSAConfig(temporal_compression=cfg.csa_ratio, local_window=cfg.csa_window,
                      index_heads=cfg.csa_heads, index_head_dim=cfg.csa_head_dim,
                      index_top_k=cfg.csa_top_k),
        hca=HCAConfig(temporal_compression=cfg.hca_ratio, local_window=cfg.hca_window,
                      dense_global_attention=cfg.hca_dense, global_top_k=cfg.hca_top_k),
        dense_ffn=DenseFFNConfig(hidden=cfg.dense_hidden),
        loop_attnres=LoopAttnResConfig(enabled=False),
        adaptive_loops=AdaptiveLoopConfig(enabled=False))


def load_into(model, cfg: HybridConfig, weights: dict[str, torch.Tensor]) -> list[str]:
    """Copy ``weights`` into the reference model under its state-dict names
    (the `.llmy` names with the stacked expert lists split per expert).
    Every other parameter is set to NaN; returns their names."""
    from hybrid_llm_amd.checkpoint import llmy_entries
    params = dict(model.named_parameters())
    done = set()
    for name, t in llmy_entries(cfg, weights):
        m = re.match(r"(.*\.moe\.(experts|shared))\.(gate_proj|up_proj|down_proj)\.weight$", name)
        if m:
            for e in range(t.shape[0]):
                pn = f"{m.group(1)}.{e}.{m.group(3)}.weight"
                params[pn].data.copy_(t[e].float())
                done.add(pn)
            continue
        if name not in params:
            raise KeyError(f"the reference model has no parameter {name}")
        params[name].data.copy_(t.float().reshape(params[name].shape))
        done.add(name)
    unset = sorted(set(params) - done)
    for n in unset:
        params[n].data.fill_(float("nan"))
    return unset


def main() -> None:
    sys.path.insert(0, REF)
    for fname, (cfg, seed) in CASES.items():
        write(os.path.join(HERE, fname), cfg, seed)


def write(out_path: str, cfg: HybridConfig, seed: int) -> None:
    from model.model import LoopedHybridMoEForCausalLM
    torch.manual_seed(0)
    model = LoopedHybridMoEForCausalLM(_ref_config(cfg)).eval()
    unset = load_into(model, cfg, golden_weights(cfg, seed))
    g = torch.Generator().manual_seed(seed + 2)
    prompt = torch.randint(0, cfg.vocab, (BATCH, PROMPT), generator=g)
    decode = torch.randint(0, cfg.vocab, (DECODE, BATCH), generator=g)
    with torch.no_grad():  # csa.py's checkpointed chunks refuse inference tensors
        out = model(prompt, collect_diagnostics=False)
        prefill = out.logits.float().numpy()
        # Each decoded token's logits are those of the sequence forward over
        # the prompt and the tokens so far, at its last position: the function
        # a token-by-token decode computes, and what the native engine's
        # decode does (llmy_cuda/src/model.cpp:1833-1935: the streams pass
        # from loop to loop and into the tail).  decode_step itself is not
        # used: with every row active it starts each loop, and the tail, from
        # the post-stem streams and drops the loops' output (model.py:856-872,
        # 896-905: sub_streams is never written back to streams), so its
        # logits differ from forward's by about 2% here.
        steps = []
        for t in range(DECODE):
            seq = torch.cat([prompt, decode[:t + 1].t()], dim=1)
            steps.append(model(seq, collect_diagnostics=False).logits[:, -1].float().numpy())
    if not (np.isfinite(prefill).all() and all(np.isfinite(s).all() for s in steps)):
        raise RuntimeError("non-finite logits: a used parameter was not loaded; unset: "
                           + ", ".join(unset))
    np.savez_compressed(
        out_path, prompt=prompt.numpy().astype(np.int32), decode=decode.numpy().astype(np.int32),
        prefill_logits=prefill.astype(np.float32), decode_logits=np.stack(steps).astype(np.float32),
        torch_version=np.array(torch.__version__))
    print(f"wrote {out_path}: prefill {prefill.shape}, decode {len(steps)} x {steps[0].shape}; "
          f"parameters not loaded (unused by inference): {unset}")


if __name__ == "__main__":
    main()
