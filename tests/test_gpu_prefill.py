"""Batched prefill of the engine (sequence kernels over a whole [B, T] prompt).

* The four glue entries against what they must equal: the KV ring fill
  against its slot rule, the GDN input preparation and output gate against
  fp32 torch, and the sequence conv gate bit for bit against T calls of the
  one-token conv gate (already pinned through the decode engine).
* The whole prefill against the oracle's token-by-token prefill
  (HybridOracle.prefill, the reference's model_prefill semantics) with the
  engine's routing replayed: last-position logits, every KV cache, GDN state
  and conv history, then decoding continued from the prefilled state.
* The prefill against the engine's own token-by-token decode of the prompt.
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

from hybrid_llm_amd.config import C1, C5, alternating, init_weights
from oracle.model import HybridOracle

pytestmark = pytest.mark.gpu

REL_L2 = 1e-2
# Model-level state after T tokens through every block and loop.  Beside the
# decode path's own deviation from the oracle (bf16 activations, GEMM order),
# each prefill block adds the sequence kernels' bf16 points: attention weights
# P in bf16 for the P.V product (as the reference's bf16 SDPA prefill does) and
# GDN q, k, v rounded to bf16 (the reference's bf16 projections); measured
# 1.1e-2 (prefill) against 0.7e-2 (decode) for the last GDN state at C5x2, T=130.
STATE_REL_L2 = 2e-2
# A routing choice may differ from the oracle's only at a near-tie.  The
# prefill's activations carry about twice the decode path's deviation (above),
# and the largest gap at a flip moves with the rounding order of the kernels:
# at C5x2, T=130 it measured 8.5e-3 and 1.06e-2 for two attention-prefill
# builds that differ only in when the softmax accumulator is rescaled (equal
# logit, KV and state errors, 18 and 16 flips of 1064).
ROUTE_GAP = 1.5e-2
ROUTE_FLIP_FRAC = 0.05


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float(torch.linalg.norm(a - b) / torch.linalg.norm(b).clamp_min(1e-30))


def _bf16_close(a, b, ulps=1):
    """|a - b| within `ulps` bf16 units of the larger magnitude (elementwise)."""
    a, b = a.float().cpu(), b.float().cpu()
    mag = torch.maximum(a.abs(), b.abs())
    return bool(((a - b).abs() <= ulps * mag * 2.0 ** -7 + 1e-30).all())


# --------------------------------------------------------------------------- glue entries
@pytest.mark.parametrize("T,W", [(5, 8), (8, 8), (37, 8), (300, 128)])
def test_kv_cache_fill(T, W):
    from hybrid_llm_amd import ops
    B, H, hd = 3, 4, 64
    g = torch.Generator().manual_seed(T)
    qkv = torch.randn(B, T, 3 * H * hd, generator=g).to(torch.bfloat16).cuda()
    k = qkv[:, :, H * hd:2 * H * hd]
    v = qkv[:, :, 2 * H * hd:]
    kc = torch.full((B, H, W, hd), 7.0, dtype=torch.bfloat16, device="cuda")
    vc = kc.clone()
    ops.kv_cache_fill(k, v, kc, vc)
    ek, ev = torch.full_like(kc.cpu(), 7.0), torch.full_like(vc.cpu(), 7.0)
    kk, vv = k.cpu().view(B, T, H, hd), v.cpu().view(B, T, H, hd)
    for t in range(max(0, T - W), T):
        ek[:, :, t % W] = kk[:, t]
        ev[:, :, t % W] = vv[:, t]
    assert torch.equal(kc.cpu(), ek) and torch.equal(vc.cpu(), ev)


@pytest.mark.parametrize("dk,dv", [(64, 64), (128, 128), (64, 128)])
def test_gdn_prefill_prep_and_gate(dk, dv):
    from hybrid_llm_amd import ops
    R, H = 77, 3
    ld = 2 * H * dk + 2 * H * dv + H
    ld += (-ld) % 16
    g = torch.Generator().manual_seed(dk + dv)
    proj = torch.randn(R, ld, generator=g)
    proj[5, :H * dk] = 0.0                      # a zero q row: the clamp keeps it finite
    bb = torch.randn(H, generator=g)
    decay = torch.randn(H, generator=g)
    out = ops.gdn_prefill_prep(proj.cuda(), bb.cuda(), decay.cuda(), H, dk, dv)
    HK, HV = H * dk, H * dv
    q = proj[:, :HK].view(R, H, dk)
    k = proj[:, HK:2 * HK].view(R, H, dk)
    qn = q * torch.rsqrt((q * q).sum(-1, keepdim=True).clamp_min(1e-12))
    kn = k * torch.rsqrt((k * k).sum(-1, keepdim=True).clamp_min(1e-12))
    assert _bf16_close(out["q"], qn) and _bf16_close(out["k"], kn)
    assert torch.equal(out["q"][5].cpu().float(), torch.zeros(H, dk))
    assert torch.equal(out["v"].cpu(), proj[:, 2 * HK:2 * HK + HV].view(R, H, dv).to(torch.bfloat16))
    beta = torch.sigmoid(proj[:, 2 * HK + 2 * HV:2 * HK + 2 * HV + H] + bb)
    torch.testing.assert_close(out["beta"].cpu(), beta, rtol=2e-6, atol=1e-7)
    torch.testing.assert_close(out["g"].cpu(), torch.sigmoid(decay).expand(R, H), rtol=2e-6,
                               atol=1e-7)
    o = torch.randn(R, HV, generator=g).to(torch.bfloat16)
    gated = ops.gdn_gate(o.cuda(), proj.cuda(), 2 * HK + HV)
    ref = o.float() * torch.sigmoid(proj[:, 2 * HK + HV:2 * HK + 2 * HV])
    assert _bf16_close(gated, ref)
    inplace = o.cuda()
    ops.gdn_gate(inplace, proj.cuda(), 2 * HK + HV, out=inplace)
    assert torch.equal(inplace.cpu(), gated.cpu())


@pytest.mark.parametrize("T", [1, 2, 3, 16, 17, 40])
def test_conv_gate_prefill_equals_steps(T):
    from hybrid_llm_amd import ops
    B, D = 2, 256
    g = torch.Generator().manual_seed(T)
    h = torch.randn(B, T, D, generator=g).to(torch.bfloat16).cuda()
    hist0 = torch.randn(B, 3, D, generator=g).to(torch.bfloat16).cuda()
    w = (0.5 * torch.randn(D, 4, generator=g)).cuda()
    hist = hist0.clone()
    got = ops.gdn_conv_gate_prefill(h, hist, w)
    hs = hist0.clone()
    steps = [ops.gdn_conv_gate(h[:, t].contiguous(), hs, w) for t in range(T)]
    assert torch.equal(got.cpu(), torch.stack(steps, 1).cpu())
    assert torch.equal(hist.cpu(), hs.cpu())


# --------------------------------------------------------------------------- model level
def _forced_oracle_prefill(ref, st, eng, tokens):
    """Oracle token-by-token prefill with the engine's prefill routing replayed:
    application a at step t uses the engine's ids of token t for application a."""
    B, T = tokens.shape
    logs = [r.view(B, T, -1).cpu().numpy() for r in eng.route_log_seq]
    ref.forced_routes = [logs[a][:, t] for t in range(T) for a in range(len(logs))]
    out = ref.prefill(tokens.numpy(), st)
    assert not ref.forced_routes
    return out


def _check_routes(ref):
    gaps = np.abs(np.array(ref.route_gaps))
    print(f"  route flips {gaps.size}/{ref.route_total}, largest gap "
          f"{gaps.max() if gaps.size else 0.0:.2e}", flush=True)
    assert gaps.size <= ROUTE_FLIP_FRAC * ref.route_total, (gaps.size, ref.route_total)
    assert np.all(gaps <= ROUTE_GAP), gaps.max()
    return gaps.size


def _compare_state(eng, st):
    worst = {}
    for key, s in eng.state.items():
        for name, t in s.items():
            r = st[key][name]
            worst[name] = max(worst.get(name, 0.0), rel_l2(t.float(), r.float()))
    return worst


@pytest.mark.parametrize("cfg_name,B,T", [("C1", 2, 200), ("C1", 1, 64), ("C5x2", 2, 130)])
def test_prefill_matches_oracle_and_continues(cfg_name, B, T):
    from hybrid_llm_amd.engine import HybridDecoder
    cfg = C1 if cfg_name == "C1" else replace(C5, layer_kinds=alternating(2))
    w = init_weights(cfg, seed=0)
    tokens = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(3))
    print(f"[prefill] {cfg_name} B={B} T={T}", flush=True)
    eng = HybridDecoder(cfg, w, B)
    eng.route_log_seq = []
    lg = eng.prefill(tokens.cuda()).clone()
    torch.cuda.synchronize()
    assert torch.equal(eng.buf["next"].cpu(), lg.argmax(-1).to(torch.int32).cpu())
    assert torch.equal(eng.pos.cpu(), torch.full((B,), T, dtype=torch.int32))

    ref = HybridOracle(cfg, w, act_bf16=True)
    st = ref.new_state(B)
    lr = _forced_oracle_prefill(ref, st, eng, tokens)[:, -1]
    err = rel_l2(lg, lr)
    sw = _compare_state(eng, st)
    print(f"  last logits rel-L2 {err:.2e}; state rel-L2 {sw}", flush=True)
    assert err <= REL_L2, err
    for name, e in sw.items():
        assert e <= STATE_REL_L2, (name, e)

    # decoding continues from the prefilled state
    eng.enable_route_log()
    nxt = eng.buf["next"].clone()
    for _ in range(3):
        lg = eng.step(nxt).clone()
        ref.forced_routes = [r for r in eng.route_log.cpu().numpy()]
        lr = ref.step(nxt.cpu().numpy(), st)
        e = rel_l2(lg, lr)
        assert e <= REL_L2, e
        nxt = eng.buf["next"].clone()
    _check_routes(ref)


def test_prefill_matches_token_by_token_decode():
    """Prefill and T decode steps of the same engine leave the same state.  Only
    the first block's K/V cache is compared: every later block sees the MoE
    routing of the blocks before it, and a near-tie decided differently by the
    two paths changes that token's whole contribution (each path is checked
    against the oracle under its own routing elsewhere)."""
    from hybrid_llm_amd.engine import HybridDecoder
    B, T = 2, 150
    w = init_weights(C1, seed=0)
    tokens = torch.randint(0, C1.vocab, (B, T), generator=torch.Generator().manual_seed(4))
    a = HybridDecoder(C1, w, B)
    a.prefill(tokens.cuda())
    b = HybridDecoder(C1, w, B)
    for t in range(T):
        b.step(tokens[:, t].cuda())
    torch.cuda.synchronize()
    assert torch.equal(a.pos.cpu(), b.pos.cpu())
    first = a.state[(0, 0)]
    for name in ("k", "v"):
        e = rel_l2(first[name].float(), b.state[(0, 0)][name].float())
        assert e <= 2e-3, (name, e)
    print("prefill vs decode state rel-L2:",
          {key: {n: round(rel_l2(t.float(), b.state[key][n].float()), 4) for n, t in s.items()}
           for key, s in a.state.items()})


def test_prefill_with_sampling_and_validation():
    from hybrid_llm_amd.engine import HybridDecoder
    B, T = 3, 20
    w = init_weights(C1, seed=0)
    eng = HybridDecoder(C1, w, B, sampling=(0.8, 0.9, 0))
    eng.set_uniforms(torch.tensor([0.1, 0.5, 0.9]))
    tokens = torch.randint(0, C1.vocab, (B, T), generator=torch.Generator().manual_seed(5))
    lg = eng.prefill(tokens.cuda())
    from oracle.sampling import top_p_sample
    want, margin = top_p_sample(lg.cpu(), 0.8, torch.tensor(0.9).item(),
                                torch.tensor([0.1, 0.5, 0.9]), return_margin=True)
    got = eng.buf["sampled"].cpu().numpy()
    # Decisions further than the kernel's cumulative-mass error (4e-6) from a
    # flip must match exactly; near-uniform random-init logits put most draws
    # within that of a step, and those may land on the neighbouring id in order.
    x = lg.cpu().double().numpy()
    for r in range(B):
        if margin[r] > 4e-6:
            assert got[r] == want[r], (r, got[r], want[r])
        else:
            order = np.lexsort((np.arange(x.shape[1]), -x[r]))
            pos = np.empty_like(order)
            pos[order] = np.arange(order.size)
            assert abs(int(pos[got[r]]) - int(pos[want[r]])) <= 1, (r, got[r], want[r])
    with pytest.raises(ValueError):
        eng.prefill(tokens[:2].cuda())
    with pytest.raises(ValueError):
        eng.prefill(tokens[:, :0].cuda())
