"""GPU parity: the context-aware router, local-context branch
(model/layers/context_router.py:59-137, mla_memory.py:18-48), against the
oracle restatement pinned in test_oracle_context_router.py.

Kernels one by one (latent encoder, window mean over a ring, logits), the
five-launch routing end to end (ids exact wherever the oracle's top-k margin
exceeds the fp32 error bound), and whole engines: decode (fused and sorted
MoE paths) and prefill against HybridOracle with replayed routing, and a
decode that continues a prefill against the oracle continuing the same
sequences.
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

from hybrid_llm_amd.config import C1, init_weights
from oracle.model import HybridOracle
from oracle.router import (context_latents, context_route_logits, context_window_mean,
                           router_topk, topk_lower_index)

pytestmark = pytest.mark.gpu

REL_L2 = 1e-2
ROUTE_GAP = 5e-3
# gate 0 -> sigmoid 1/2: the context term moves the logits well beyond noise
CC = replace(C1, context_router=True, router_context=16, route_gate_init=0.0)


def ops():
    from hybrid_llm_amd import ops as o
    return o


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float(torch.linalg.norm(a - b) / torch.linalg.norm(b))


def _layer_weights(D=256, L=256, E=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    return {"router_norm": 1 + 0.1 * torch.randn(D, generator=g),
            "ctx_down": torch.randn(L, D, generator=g) * 0.05,
            "ctx_ln_w": 1 + 0.1 * torch.randn(L, generator=g),
            "ctx_ln_b": 0.1 * torch.randn(L, generator=g),
            "ctx_local_out": (torch.randn(D, L, generator=g) * 0.05).bfloat16(),
            "ctx_out": (torch.randn(D, D, generator=g) * 0.05).bfloat16(),
            "ctx_gate": torch.tensor(0.3),
            "w_router": torch.randn(E, D, generator=g) * 0.05}


@pytest.mark.parametrize("D", [256, 512, 1024])
def test_latent_kernel(D):
    w = _layer_weights(D=D)
    rows = 37  # a ragged last workgroup of the 8-token tiles
    h = torch.randn(rows, D, generator=torch.Generator().manual_seed(1)).bfloat16()
    local, lat = ops().router_context_latent(h.cuda(), w["router_norm"].cuda(),
                                             w["ctx_down"].cuda(), w["ctx_ln_w"].cuda(),
                                             w["ctx_ln_b"].cuda())
    rl, rlat = context_latents(h.float(), w["router_norm"], w["ctx_down"], w["ctx_ln_w"],
                               w["ctx_ln_b"])
    assert rel_l2(local, rl) < 1e-6
    assert rel_l2(lat, rlat) < 1e-5
    assert float((lat.cpu() - rlat).abs().max()) < 1e-4


def test_window_prompt_then_decode():
    """A [B, T] prompt from position 0, then single tokens at ragged positions:
    every token's mean is the box mean of its sequence's last W latents."""
    B, T, W, L = 3, 70, 16, 256
    g = torch.Generator().manual_seed(2)
    lat = torch.randn(B, T + 4, L, generator=g)
    ring = torch.zeros(B, W, L, device="cuda")
    ctx = ops().router_context_window(lat[:, :T].reshape(B * T, L).cuda(), ring)
    want = context_window_mean(lat, W)
    got = ctx.view(B, T, L).float().cpu()
    # bf16 output: within one bf16 rounding of the fp64 mean
    assert torch.allclose(got, want[:, :T].bfloat16().float(), rtol=0, atol=0) or \
        float((got - want[:, :T]).abs().max()) <= float(want[:, :T].abs().max()) * 2 ** -8
    pos = torch.full((B,), T, dtype=torch.int32)
    for t in range(T, T + 4):
        c = ops().router_context_window(lat[:, t].contiguous().cuda(), ring, pos=pos.cuda())
        err = (c.float().cpu() - want[:, t]).abs().max()
        assert float(err) <= float(want[:, t].abs().max()) * 2 ** -8, t
        pos += 1
    # ragged positions: sequence b at position p_b with a ring holding its past
    p = torch.tensor([0, 5, 40], dtype=torch.int32)
    ring2 = torch.zeros(B, W, L)
    for b in range(B):
        for q in range(int(p[b])):
            ring2[b, q % W] = lat[b, q]
    cur = torch.stack([lat[b, int(p[b])] for b in range(B)])
    c = ops().router_context_window(cur.cuda(), ring2.cuda(), pos=p.cuda())
    for b in range(B):
        ref = want[b, int(p[b])]
        assert float((c[b].float().cpu() - ref).abs().max()) <= float(ref.abs().max()) * 2 ** -8


def test_logits_and_end_to_end_ids():
    D, L, E, k = 256, 256, 8, 2
    w = _layer_weights(D=D, L=L, E=E, seed=3)
    B, T, W = 4, 50, 16
    h = torch.randn(B * T, D, generator=torch.Generator().manual_seed(4)).bfloat16()
    wd = {n: t.cuda() for n, t in w.items()}
    ring = torch.zeros(B, W, L, device="cuda")
    idx, gates, logits = ops().router_context(h.cuda(), wd, ring, k)
    local, lat = context_latents(h.float(), w["router_norm"], w["ctx_down"], w["ctx_ln_w"],
                                 w["ctx_ln_b"])
    ctx = context_window_mean(lat.view(B, T, L), W).view(B * T, L)
    bf = lambda t: t.bfloat16().float()
    ref = context_route_logits(local, ctx, w["ctx_local_out"].float(), w["ctx_out"].float(),
                               w["ctx_gate"], w["w_router"], act_round=bf)
    assert rel_l2(logits, ref) < 2e-3
    # ids: exact wherever the oracle's k-th / (k+1)-th margin clears the error
    _, vals = topk_lower_index(ref, k + 1)
    margin = vals[:, k - 1] - vals[:, k]
    err = float((logits.cpu() - ref).abs().max())
    safe = margin > 4 * err
    own, _ = router_topk(ref, k)
    got = idx.cpu().numpy()
    assert safe.mean() > 0.8
    assert np.array_equal(np.sort(got[safe], 1), np.sort(own[safe], 1))
    # gates: softmax of the kernel's own top-k logits
    sel = torch.gather(logits.cpu(), 1, idx.cpu().long())
    assert torch.allclose(gates.cpu(), sel.softmax(-1), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("fused", [True, False])
def test_engine_decode_with_context_router(fused):
    from hybrid_llm_amd.engine import HybridDecoder
    B = 3
    w = init_weights(CC, seed=0)
    ref = HybridOracle(CC, w, act_bf16=True)
    st = ref.new_state(B)
    eng = HybridDecoder(CC, w, B)
    if not fused:
        eng.fused_route = False
        eng.defer_resid = False
    eng.enable_route_log()
    toks = torch.randint(0, CC.vocab, (24, B), generator=torch.Generator().manual_seed(5))
    worst = 0.0
    for t in range(toks.shape[0]):  # past router_context = 16: the ring wraps
        lg = eng.step(toks[t].to(torch.int32).cuda()).clone()
        ref.forced_routes = [r for r in eng.route_log.cpu().numpy()]
        lr = ref.step(toks[t].numpy(), st)
        worst = max(worst, rel_l2(lg, lr))
    gaps = np.abs(np.array(ref.route_gaps))
    print(f"context router decode (fused={fused}): worst rel-L2 {worst:.2e}, "
          f"flips {gaps.size}/{ref.route_total}")
    assert worst <= REL_L2, worst
    assert gaps.size <= 0.05 * ref.route_total and np.all(gaps <= ROUTE_GAP)


def test_context_changes_the_routing():
    """The context path is live: with the gate at -200 (sigmoid 0) the engine's
    logits equal the plain-router engine's on the same tensors."""
    from hybrid_llm_amd.engine import HybridDecoder
    w = init_weights(CC, seed=0)
    tok = torch.tensor([7, 8], dtype=torch.int32).cuda()
    off = dict(w)
    for l in range(CC.n_layers):
        off[f"L{l}.ctx_gate"] = torch.tensor(-200.0)
    plain = {k: v for k, v in w.items() if ".ctx_" not in k}
    a = HybridDecoder(CC, off, 2).step(tok).clone()
    b = HybridDecoder(C1, plain, 2).step(tok).clone()
    c = HybridDecoder(CC, w, 2).step(tok).clone()
    assert torch.equal(a, b)
    assert rel_l2(c, b) > 1e-4


def test_engine_prefill_then_decode_with_context_router():
    from hybrid_llm_amd.engine import HybridDecoder
    B, T = 2, 40
    w = init_weights(CC, seed=1)
    tokens = torch.randint(0, CC.vocab, (B, T), generator=torch.Generator().manual_seed(6))
    eng = HybridDecoder(CC, w, B)
    eng.route_log_seq = []
    lg = eng.prefill(tokens.cuda()).clone()
    ref = HybridOracle(CC, w, act_bf16=True)
    st = ref.new_state(B)
    logs = [r.view(B, T, -1).cpu().numpy() for r in eng.route_log_seq]
    ref.forced_routes = [logs[a][:, t] for t in range(T) for a in range(len(logs))]
    lr = ref.prefill(tokens.numpy(), st)[:, -1]
    err = rel_l2(lg, lr)
    print(f"context router prefill: last logits rel-L2 {err:.2e}")
    assert err <= REL_L2, err
    # decode continues from the prefill's ring state
    eng.enable_route_log()
    nxt = torch.randint(0, CC.vocab, (3, B), generator=torch.Generator().manual_seed(7))
    for t in range(3):
        lg = eng.step(nxt[t].to(torch.int32).cuda()).clone()
        ref.forced_routes = [r for r in eng.route_log.cpu().numpy()]
        lr = ref.step(nxt[t].numpy(), st)
        assert rel_l2(lg, lr) <= REL_L2


def test_layernorm_kernel():
    from hybrid_llm_amd import ops
    g = torch.Generator().manual_seed(21)
    x = torch.randn(37, 256, generator=g) * 3 + 1
    w, b = 1 + 0.1 * torch.randn(256, generator=g), 0.1 * torch.randn(256, generator=g)
    out = ops.layernorm(x.cuda(), w.cuda(), b.cuda(), 1e-5)
    ref = torch.nn.functional.layer_norm(x.double(), (256,), w.double(), b.double(), 1e-5)
    assert torch.allclose(out.float().cpu(), ref.float(), rtol=8e-3, atol=1e-5)


@pytest.mark.parametrize("T,C", [(1, 64), (5, 40), (1, 300)])
def test_latent_attention_kernel(T, C):
    """llmy_latent_attn_bf16 against torch SDPA with the slot visibility mask
    (1 <= tag <= position + 1), per row and head; rows with nothing visible give 0."""
    import torch.nn.functional as F
    from hybrid_llm_amd import ops
    g = torch.Generator().manual_seed(T * C)
    B, heads, hd = 3, 4, 64
    HQ = heads * hd
    q = torch.randn(B * T, HQ, generator=g).bfloat16()
    keys = torch.randn(B, C, HQ, generator=g).bfloat16()
    vals = torch.randn(B, C, HQ, generator=g).bfloat16()
    tag = torch.randint(0, 120, (B, C), generator=g, dtype=torch.int32)
    pos = torch.tensor([70, 3, 0], dtype=torch.int32)
    tag[2] = 5                                     # row 2 at position 0: nothing visible
    use_pos = T == 1
    out = ops.latent_attn(q.cuda(), keys.cuda(), vals.cuda(), tag.cuda(), heads, hd,
                          pos=pos.cuda() if use_pos else None)
    for b in range(B):
        for t in range(T):
            qp = int(pos[b]) if use_pos else t
            vis = (tag[b] >= 1) & (tag[b] <= qp + 1)
            got = out[b * T + t].float().cpu()
            if not vis.any():
                assert torch.equal(got, torch.zeros(HQ))
                continue
            qh = q[b * T + t].float().view(heads, 1, hd)
            kh = keys[b][vis].float().view(-1, heads, hd).transpose(0, 1)
            vh = vals[b][vis].float().view(-1, heads, hd).transpose(0, 1)
            ref = F.scaled_dot_product_attention(qh, kh, vh).reshape(HQ)
            assert torch.allclose(got, ref, rtol=1e-2, atol=1e-2), (b, t)
