"""Oracle pins for the context-aware router (model/layers/context_router.py:
59-137, model/layers/mla_memory.py:18-48), local-context branch.

* LayerNorm against torch.nn.functional.layer_norm.
* The window mean against the reference's own formulation: a depthwise causal
  box filter done with F.conv1d and the position rescale of
  mla_memory.py:38-48 (a library convolution, not the oracle's prefix sums);
  closed forms W = 1 (identity) and W >= T (running prefix mean).
* The decode rule (history + current latent, last W, mean;
  context_router.py:108-128) equals the prompt rule at every position.
* A planted mistake: the W+1 window of llmy_cuda's router_history_update_mean
  (model.cpp:1253-1279 averages the current latent with W history slots)
  differs from the model's W window once T > W.
* Route logits: with sigmoid(g) -> 0 they are the plain router's logits
  (pinned in test_oracle_router.py), at the op level and for a whole model.
"""
from dataclasses import replace

import numpy as np
import torch
import torch.nn.functional as F

from hybrid_llm_amd.config import C1, init_weights
from oracle.model import HybridOracle
from oracle.router import (context_latents, context_route_logits, context_window_mean, layernorm,
                           router_logits)


def _box_conv(lat: torch.Tensor, W: int) -> torch.Tensor:
    """mla_memory.py:38-48 with torch ops: pad W-1 on the left, depthwise
    conv with a 1/W kernel, then rescale position t by W / min(t+1, W)."""
    x = lat.double().transpose(1, 2)
    C = x.shape[1]
    ctx = F.conv1d(F.pad(x, (W - 1, 0)), torch.ones(C, 1, W, dtype=torch.float64) / W, groups=C)
    pos = torch.arange(lat.shape[1])
    actual = torch.minimum(pos + 1, torch.full_like(pos, W)).double()
    return (ctx * (W / actual).view(1, 1, -1)).transpose(1, 2).float()


def test_layernorm_matches_torch():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(7, 256, generator=g) * 3 + 1
    w = torch.randn(256, generator=g)
    b = torch.randn(256, generator=g)
    ref = F.layer_norm(x.double(), (256,), w.double(), b.double(), eps=1e-5).float()
    assert torch.allclose(layernorm(x, w, b), ref, rtol=1e-6, atol=1e-6)


def test_window_mean_matches_box_filter():
    g = torch.Generator().manual_seed(1)
    lat = torch.randn(3, 300, 64, generator=g)
    for W in (1, 2, 7, 128, 300, 512):
        got = context_window_mean(lat, W)
        assert torch.allclose(got, _box_conv(lat, W), rtol=1e-5, atol=1e-6), W
    assert torch.allclose(context_window_mean(lat, 1), lat)
    prefix = torch.cumsum(lat.double(), 1) / torch.arange(1, 301).double().view(1, -1, 1)
    assert torch.allclose(context_window_mean(lat, 512), prefix.float(), rtol=1e-6, atol=1e-6)


def test_decode_rule_equals_prompt_rule():
    g = torch.Generator().manual_seed(2)
    lat = torch.randn(2, 200, 32, generator=g)
    W = 50
    want = context_window_mean(lat, W)
    hist = torch.zeros(2, 0, 32)
    for t in range(200):
        hist = torch.cat([hist, lat[:, t:t + 1]], 1)[:, -W:]
        assert torch.allclose(hist.double().mean(1).float(), want[:, t], rtol=1e-6, atol=1e-6)


def test_native_w_plus_one_window_differs():
    """The planted mistake fails the pin: W history slots plus the current
    latent average W+1 latents, which the model never does."""
    g = torch.Generator().manual_seed(3)
    lat = torch.randn(1, 40, 16, generator=g)
    W = 8
    wrong = context_window_mean(lat, W + 1)
    assert torch.allclose(wrong[:, :W], context_window_mean(lat, W)[:, :W])  # same while t < W
    assert not torch.allclose(wrong[:, W:], _box_conv(lat, W)[:, W:], atol=1e-3)


def test_route_logits_reduce_to_plain_router():
    g = torch.Generator().manual_seed(4)
    D, L, E = 256, 64, 8
    h = torch.randn(5, D, generator=g).bfloat16().float()
    nw = 1 + 0.1 * torch.randn(D, generator=g)
    wr = torch.randn(E, D, generator=g) * 0.02
    local, lat = context_latents(h, nw, torch.randn(L, D, generator=g) * 0.02, torch.ones(L),
                                 torch.zeros(L))
    # LayerNorm output: zero mean and unit variance per row before the affine
    assert torch.allclose(lat.mean(-1), torch.zeros(5), atol=1e-5)
    assert torch.allclose(lat.var(-1, unbiased=False), torch.ones(5), atol=1e-3)
    wl = torch.randn(D, L, generator=g) * 0.02
    wc = torch.randn(D, D, generator=g) * 0.02
    plain = router_logits(h, wr, nw)
    off = context_route_logits(local, lat, wl, wc, torch.tensor(-200.0), wr)
    assert torch.allclose(off, plain, rtol=1e-6, atol=1e-7)
    zero_out = context_route_logits(local, lat, wl, torch.zeros(D, D), torch.tensor(1.5), wr)
    assert torch.allclose(zero_out, plain, rtol=1e-6, atol=1e-7)
    on = context_route_logits(local, lat, wl, wc, torch.tensor(1.5), wr)
    assert not torch.allclose(on, plain, atol=1e-5)
    # linear in the context term: sigmoid(g) * c enters once
    half = context_route_logits(local, lat, wl, wc * 0.5, torch.tensor(1.5), wr)
    assert torch.allclose(on - plain, 2 * (half - plain), rtol=1e-4, atol=1e-6)


def test_model_with_gate_off_equals_plain_router_model():
    cfg = replace(C1, context_router=True, route_gate_init=-200.0)
    w = init_weights(cfg, seed=0)
    plain_w = {k: v for k, v in w.items() if ".ctx_" not in k}
    a = HybridOracle(cfg, w)
    b = HybridOracle(C1, plain_w)
    sa, sb = a.new_state(2), b.new_state(2)
    # init order differs (context weights are drawn after the router's), so
    # the plain model reuses the same tensors rather than re-drawing them
    for t in ([1, 2], [3, 4], [5, 6]):
        assert torch.allclose(a.step(t, sa), b.step(t, sb), rtol=1e-5, atol=1e-6)
    assert sa[(0, 0)]["lat"].shape == (2, 3, cfg.latent_dim)
    assert np.array_equal(np.stack(a.routes), np.stack(b.routes))


def test_hca_global_context_is_layernorm_then_sdpa():
    """oracle.router.hca_global_context against nn.LayerNorm + torch's SDPA, the
    routines the reference's MLALatentMemory.encode / LatentAttention call
    (mla_memory.py:23-24,65-86), per row over that row's summaries; a row
    without summaries gives 0."""
    import torch.nn.functional as F
    from oracle.router import hca_global_context
    g = torch.Generator().manual_seed(4)
    B, D, L, heads, hd = 3, 64, 32, 4, 8
    HQ = heads * hd
    local = torch.randn(B, D, generator=g)
    values = [torch.randn(n, D, generator=g) for n in (5, 0, 9)]
    w = {n: torch.randn(s, generator=g) * 0.2 for n, s in
         (("down", (L, D)), ("q", (HQ, D)), ("k", (HQ, L)), ("v", (HQ, L)), ("o", (D, HQ)))}
    ln_w, ln_b = 1 + 0.1 * torch.randn(L, generator=g), 0.1 * torch.randn(L, generator=g)
    got = hca_global_context(local, values, w["down"], ln_w, ln_b, w["q"], w["k"], w["v"],
                             w["o"], heads, hd)
    ln = torch.nn.LayerNorm(L)
    with torch.no_grad():
        ln.weight.copy_(ln_w)
        ln.bias.copy_(ln_b)
        for b in range(B):
            if values[b].shape[0] == 0:
                assert torch.equal(got[b], torch.zeros(D))
                continue
            lat = ln(values[b] @ w["down"].t())
            q = (local[b:b + 1] @ w["q"].t()).view(1, 1, heads, hd).transpose(1, 2)
            k = (lat @ w["k"].t()).view(1, -1, heads, hd).transpose(1, 2)
            v = (lat @ w["v"].t()).view(1, -1, heads, hd).transpose(1, 2)
            o = F.scaled_dot_product_attention(q, k, v).transpose(1, 2).reshape(1, HQ)
            assert torch.allclose(got[b], (o @ w["o"].t())[0], atol=1e-5, rtol=1e-4), b
