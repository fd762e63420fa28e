"""Shared experts (model/layers/moe.py:185-199; llmy_cuda/src/model.cpp:
1205-1225) through the engine: every token also routed to the S shared
experts, stacked after the routed ones, at gate 1/sqrt(S), against the
oracle's sum-then-scale restatement (pinned in test_oracle_moe_attention.py).
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

from hybrid_llm_amd.config import C1, init_weights
from oracle.model import HybridOracle

pytestmark = pytest.mark.gpu

REL_L2 = 1e-2
ROUTE_GAP = 5e-3
CS = replace(C1, shared_experts=2)


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float(torch.linalg.norm(a - b) / torch.linalg.norm(b))


def test_append_shared_layout():
    from hybrid_llm_amd import ops
    T, k, E, S = 5, 2, 8, 3
    g = torch.Generator().manual_seed(0)
    idx = torch.randint(0, E, (T, k), generator=g, dtype=torch.int32)
    gates = torch.rand(T, k, generator=g)
    ia, ga = ops.moe_append_shared(idx.cuda(), gates.cuda(), E, S)
    want_i = torch.cat([idx, torch.arange(E, E + S, dtype=torch.int32).expand(T, S)], 1)
    want_g = torch.cat([gates, torch.full((T, S), np.float32(1 / np.sqrt(np.float32(S))))], 1)
    assert torch.equal(ia.cpu(), want_i)
    assert torch.equal(ga.cpu(), want_g)


@pytest.mark.parametrize("fused", [True, False])
def test_decode_with_shared_experts(fused):
    from hybrid_llm_amd.engine import HybridDecoder
    B = 3
    w = init_weights(CS, seed=0)
    ref = HybridOracle(CS, w, act_bf16=True)
    st = ref.new_state(B)
    eng = HybridDecoder(CS, w, B)
    if not fused:  # the norm -> router -> permutation -> sorted-experts path
        eng.fused_route = False
        eng.defer_resid = False
    eng.enable_route_log()
    toks = torch.randint(0, CS.vocab, (12, B), generator=torch.Generator().manual_seed(2))
    worst = 0.0
    for t in range(toks.shape[0]):
        lg = eng.step(toks[t].to(torch.int32).cuda()).clone()
        ref.forced_routes = [r for r in eng.route_log.cpu().numpy()]
        lr = ref.step(toks[t].numpy(), st)
        worst = max(worst, rel_l2(lg, lr))
    gaps = np.abs(np.array(ref.route_gaps))
    print(f"shared experts decode (fused={fused}): worst rel-L2 {worst:.2e}, "
          f"flips {gaps.size}/{ref.route_total}")
    assert worst <= REL_L2, worst
    assert gaps.size <= 0.05 * ref.route_total and np.all(gaps <= ROUTE_GAP)


def test_shared_experts_change_the_output():
    """The shared path is live: zeroing the shared experts' down projections
    changes the logits (and equals the engine without shared experts)."""
    from hybrid_llm_amd.engine import HybridDecoder
    w = init_weights(CS, seed=0)
    tok = torch.tensor([7, 8], dtype=torch.int32).cuda()
    a = HybridDecoder(CS, w, 2).step(tok).clone()
    w0 = dict(w)
    for l in range(CS.n_layers):
        w0[f"L{l}.w_shared_down"] = torch.zeros_like(w[f"L{l}.w_shared_down"])
    b = HybridDecoder(CS, w0, 2).step(tok).clone()
    plain = {k: v for k, v in w.items() if "shared" not in k}
    c = HybridDecoder(C1, plain, 2).step(tok).clone()
    assert rel_l2(a, c) > 1e-3
    assert torch.allclose(b, c, atol=1e-5, rtol=1e-5)


def test_prefill_with_shared_experts():
    from hybrid_llm_amd.engine import HybridDecoder
    B, T = 2, 40
    w = init_weights(CS, seed=0)
    tokens = torch.randint(0, CS.vocab, (B, T), generator=torch.Generator().manual_seed(3))
    eng = HybridDecoder(CS, w, B)
    eng.route_log_seq = []
    lg = eng.prefill(tokens.cuda()).clone()
    ref = HybridOracle(CS, w, act_bf16=True)
    st = ref.new_state(B)
    logs = [r.view(B, T, -1).cpu().numpy() for r in eng.route_log_seq]
    ref.forced_routes = [logs[a][:, t] for t in range(T) for a in range(len(logs))]
    lr = ref.prefill(tokens.numpy(), st)[:, -1]
    err = rel_l2(lg, lr)
    print(f"shared experts prefill: last logits rel-L2 {err:.2e}")
    assert err <= REL_L2, err
