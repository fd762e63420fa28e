"""GPU parity: models with CSA / HCA mixers in the Python engine against the
model oracle (oracle/model.py with oracle/compressed.py, pinned to the
reference modules), with the engine's discrete decisions replayed: decode
steps past the local window and across several emitted summaries, a captured
decode graph equal to eager bit for bit, a prefill followed by decoding, a row
reset, and the mHC stack.

Replayed decisions.  The MoE routing (route_log), and for a selective top-k
memory (CMK) the summaries each (row, head) selected (sel_log: their
positions), are handed to the oracle, which records how far each differing
choice was from its own (a near-tie of two scores within the bf16 rounding of
q).  Every step is then within rel-L2 1e-2, the bound of the other engine
tests; the mixer alone matches the oracle to 1e-6 per step
(tests/test_gpu_compressed.py checks the kernels).
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

from hybrid_llm_amd.config import C1, init_weights
from oracle.model import HybridOracle

pytestmark = pytest.mark.gpu

REL_L2 = 1e-2

# csa_top_k 16 covers every summary of these runs (<= 12 per row)
CM = replace(C1, layer_kinds=("csa", "gdn", "hca", "attn"), vocab=2048, csa_heads=4,
             csa_head_dim=64, csa_window=16, csa_ratio=4, csa_top_k=16, hca_window=12,
             hca_ratio=8, cmp_slots=64)
CMK = replace(CM, layer_kinds=("hca", "csa", "gdn"), csa_top_k=3, hca_dense=False, hca_top_k=2)
SEL_GAP = 1e-2   # a replayed top-k selection may differ only at a near-tie of scores


def _bound(cfg, errs):
    errs = np.asarray(errs)
    assert errs.max() <= REL_L2, errs


def _replay_sel(ref, eng):
    """Hand the engine's top-k memory selections of the last step to the
    oracle's mixers, in the order each mixer is called."""
    for l, pos in eng.sel_log:
        m = ref.cmp[l]
        m.forced_sel = (m.forced_sel or []) + [pos.numpy()]
    eng.sel_log.clear()


def _replay_sel_prefill(ref, eng, T):
    """The prefill's selections [B, T, H, k] per (loop, layer), as the oracle's
    token-by-token prefill calls each mixer: token by token, loops in order."""
    by_layer = {}
    for l, pos in eng.sel_log:
        by_layer.setdefault(l, []).append(pos.numpy())
    for l, entries in by_layer.items():
        ref.cmp[l].forced_sel = [e[:, t] for t in range(T) for e in entries]
    eng.sel_log.clear()


def _check_sel(ref):
    gaps = np.array([g for m in ref.cmp.values() for g in m.sel_gaps])
    total = sum(m.sel_total for m in ref.cmp.values())
    print(f"  top-k selections replayed: {gaps.size} of {total} (row, head) choices differ, "
          f"largest gap {gaps.max() if gaps.size else 0.0:.2e}", flush=True)
    assert gaps.size == 0 or np.all(np.abs(gaps) <= SEL_GAP), gaps.max()


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float(torch.linalg.norm(a - b) / torch.linalg.norm(b))


def _decode(cfg, B, steps, seed, reset_at=None, graph=False):
    from hybrid_llm_amd.engine import HybridDecoder
    w = init_weights(cfg, seed=seed)
    toks = torch.randint(0, cfg.vocab, (steps, B), generator=torch.Generator().manual_seed(seed),
                         dtype=torch.int32)
    ref = HybridOracle(cfg, w, act_bf16=True)
    st = ref.new_state(B)
    eng = HybridDecoder(cfg, w, B)
    eng.enable_route_log()
    eng.sel_log = []
    errs, outs = [], []
    for i in range(steps):
        reset = None
        if reset_at is not None and i == reset_at[0]:
            reset = torch.zeros(B, dtype=torch.int32)
            reset[reset_at[1]] = 1
        lg = eng.step(toks[i].cuda(), reset=None if reset is None else reset.cuda()).clone()
        outs.append(lg)
        ref.forced_routes = [r for r in eng.route_log.cpu().numpy()]
        _replay_sel(ref, eng)
        lr = ref.step(toks[i].numpy(), st, reset=None if reset is None else reset.numpy())
        errs.append(rel_l2(lg, lr))
    gaps = np.abs(np.array(ref.route_gaps))
    assert np.all(gaps <= 5e-3), gaps.max()
    _check_sel(ref)
    return errs, outs, toks, w


@pytest.mark.parametrize("cfg", [CM, CMK], ids=["dense", "topk"])
def test_decode_matches_oracle_and_graph(cfg):
    from hybrid_llm_amd.engine import HybridDecoder
    B, steps = 3, 40
    errs, eager, toks, w = _decode(cfg, B, steps, seed=3)
    print(f"cmp decode: worst step rel-L2 {max(errs):.2e}, median {np.median(errs):.2e}",
          flush=True)
    _bound(cfg, errs)
    g = HybridDecoder(cfg, w, B)
    g.capture()
    for i in range(steps):
        out = g.step(toks[i].cuda()).clone()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[i]), i


def test_decode_row_reset():
    errs, _, _, _ = _decode(CM, 3, 30, seed=7, reset_at=(21, 1))
    print(f"cmp decode with a reset: worst step rel-L2 {max(errs):.2e}", flush=True)
    _bound(CM, errs)


@pytest.mark.parametrize("cfg,T", [(CM, 45), (CMK, 30), (CM, 5)], ids=["dense", "topk", "short"])
def test_prefill_matches_oracle_then_decodes(cfg, T):
    from hybrid_llm_amd.engine import HybridDecoder
    w = init_weights(cfg, seed=5)
    B = 2
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(6),
                           dtype=torch.int32)
    eng = HybridDecoder(cfg, w, B)
    eng.route_log_seq = []
    eng.sel_log = []
    lg = eng.prefill(prompt.cuda()).clone()
    ref = HybridOracle(cfg, w, act_bf16=True)
    st = ref.new_state(B)
    logs = [r.view(B, T, -1).cpu().numpy() for r in eng.route_log_seq]
    ref.forced_routes = [logs[a][:, t] for t in range(T) for a in range(len(logs))]
    _replay_sel_prefill(ref, eng, T)
    out = ref.prefill(prompt.numpy(), st)
    errs = [rel_l2(lg, out[:, -1])]
    print(f"cmp prefill T={T}: last-position rel-L2 {errs[0]:.2e}", flush=True)
    eng.route_log_seq = None
    eng.enable_route_log()
    for i in range(6):
        nxt = eng.buf["next"].clone()
        lg2 = eng.step(nxt).clone()
        ref.forced_routes = [r for r in eng.route_log.cpu().numpy()]
        _replay_sel(ref, eng)
        lr2 = ref.step(nxt.cpu().numpy(), st)
        errs.append(rel_l2(lg2, lr2))
    _check_sel(ref)
    _bound(cfg, errs)


def test_mhc_with_compressed_mixers():
    cfg = replace(CM, mhc_streams=4, mhc_gating_init=0.5, num_loops=1)
    errs, _, _, _ = _decode(cfg, 2, 20, seed=11)
    print(f"mHC + cmp decode: worst step rel-L2 {max(errs):.2e}", flush=True)
    _bound(cfg, errs)


@pytest.mark.parametrize("mode", ["decode", "prefill"])
def test_context_router_global_branch(mode):
    """HCA layers with the context-aware router: the router's global branch over
    the block's summaries (context_router.py:66-68,126-127) in the Python engine
    against the model oracle (oracle.router.hca_global_context), decode steps and
    a prefill, routing replayed."""
    cfg = replace(C1, layer_kinds=("hca", "gdn", "hca"), vocab=2048, hca_window=12,
                  hca_ratio=4, cmp_slots=64, context_router=True, router_context=8,
                  route_gate_init=0.5, num_loops=1)
    if mode == "decode":
        errs, _, _, _ = _decode(cfg, 3, 24, seed=13)
        print(f"global branch decode: worst step rel-L2 {max(errs):.2e}", flush=True)
        assert max(errs) <= REL_L2, errs
        return
    from hybrid_llm_amd.engine import HybridDecoder
    w = init_weights(cfg, seed=14)
    B, T = 2, 26
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(15),
                           dtype=torch.int32)
    eng = HybridDecoder(cfg, w, B)
    eng.route_log_seq = []
    lg = eng.prefill(prompt.cuda()).clone()
    ref = HybridOracle(cfg, w, act_bf16=True)
    st = ref.new_state(B)
    logs = [r.view(B, T, -1).cpu().numpy() for r in eng.route_log_seq]
    ref.forced_routes = [logs[a][:, t] for t in range(T) for a in range(len(logs))]
    out = ref.prefill(prompt.numpy(), st)
    e = rel_l2(lg, out[:, -1])
    print(f"global branch prefill: last-position rel-L2 {e:.2e}", flush=True)
    assert e <= REL_L2, e
