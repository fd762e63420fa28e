"""Pins the MoE and banded-attention oracles (CPU only)."""
import numpy as np
import torch
import torch.nn.functional as F

from oracle.attention import banded_attention, banded_attention_decode
from oracle.moe import moe_grouped, moe_per_token, shared_experts, swiglu
from oracle.router import router_topk


def _experts(E, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(E, H, D, generator=g) * 0.2, torch.randn(E, H, D, generator=g) * 0.2,
            torch.randn(E, D, H, generator=g) * 0.2)


def test_grouped_moe_matches_per_token_brute_force():
    T, D, H, E, k = 13, 16, 24, 5, 2
    wg, wu, wd = _experts(E, H, D, 0)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(T, D, generator=g)
    idx, gates = router_topk(torch.randn(T, E, generator=g), k)
    a = moe_grouped(x, idx, gates, wg, wu, wd)
    b = moe_per_token(x, idx, gates, wg, wu, wd)
    assert torch.allclose(a, b, atol=1e-5, rtol=1e-5)


def test_moe_single_expert_is_dense_swiglu():
    T, D, H, E = 9, 16, 32, 4
    wg, wu, wd = _experts(E, H, D, 2)
    x = torch.randn(T, D, generator=torch.Generator().manual_seed(3))
    idx = np.full((T, 1), 2)
    out = moe_grouped(x, idx, torch.ones(T, 1), wg, wu, wd)
    assert torch.allclose(out, swiglu(x, wg[2], wu[2], wd[2]), atol=1e-6)
    # swiglu itself against the closed form silu(a)*b
    a = x @ wg[2].t()
    assert torch.allclose(swiglu(x, wg[2], wu[2], wd[2]),
                          (a * torch.sigmoid(a) * (x @ wu[2].t())) @ wd[2].t(), atol=1e-6)


def test_moe_is_token_order_invariant():
    T, D, H, E, k = 20, 8, 12, 6, 2
    wg, wu, wd = _experts(E, H, D, 4)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(T, D, generator=g)
    idx, gates = router_topk(torch.randn(T, E, generator=g), k)
    perm = torch.randperm(T, generator=g)
    a = moe_grouped(x, idx, gates, wg, wu, wd)[perm]
    b = moe_grouped(x[perm], idx[perm.numpy()], gates[perm], wg, wu, wd)
    assert torch.allclose(a, b, atol=1e-6)


def _qkv(B, T, H, hd, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, T, H, hd, generator=g) for _ in range(3)]


def test_shared_expert_closed_forms():
    """Shared experts (moe.py:185-199): one shared expert equal to routed
    expert e, on tokens routed to e alone (k = 1, gate 1), doubles that
    expert's output; S copies of one expert give sqrt(S) times it (sum of S,
    scaled by 1/sqrt(S)); and the sum is taken before the scale, over the
    experts in any order."""
    g = torch.Generator().manual_seed(11)
    T, D, H, E = 6, 32, 48, 3
    x = torch.randn(T, D, generator=g)
    wg, wu = torch.randn(E, H, D, generator=g) * 0.2, torch.randn(E, H, D, generator=g) * 0.2
    wd = torch.randn(E, D, H, generator=g) * 0.2
    e = 1
    idx = np.full((T, 1), e)
    routed = moe_grouped(x, idx, torch.ones(T, 1), wg, wu, wd)
    one = shared_experts(x, wg[e:e + 1], wu[e:e + 1], wd[e:e + 1])
    assert torch.allclose(routed + one, 2 * swiglu(x, wg[e], wu[e], wd[e]), atol=1e-5)
    S = 4
    rep = shared_experts(x, wg[e:e + 1].repeat(S, 1, 1), wu[e:e + 1].repeat(S, 1, 1),
                         wd[e:e + 1].repeat(S, 1, 1))
    assert torch.allclose(rep, np.sqrt(S) * swiglu(x, wg[e], wu[e], wd[e]), atol=1e-5)
    perm = [2, 0, 1]
    a = shared_experts(x, wg, wu, wd)
    b = shared_experts(x, wg[perm], wu[perm], wd[perm])
    brute = sum(swiglu(x, wg[s], wu[s], wd[s]).double() for s in range(E)) / np.sqrt(E)
    assert torch.allclose(a, b, atol=1e-5)
    assert torch.allclose(a.double(), brute, atol=1e-5)


def test_banded_equals_causal_sdpa_when_window_covers_sequence():
    q, k, v = _qkv(2, 37, 3, 16, 0)
    out = banded_attention(q, k, v, window=64, block=8)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2),
                                         v.transpose(1, 2), is_causal=True).transpose(1, 2)
    assert torch.allclose(out, ref, atol=1e-5)


def test_window_one_returns_values():
    q, k, v = _qkv(1, 20, 2, 8, 1)
    assert torch.allclose(banded_attention(q, k, v, window=1, block=7), v, atol=1e-6)


def test_banded_brute_force():
    B, T, H, hd, W = 1, 12, 2, 4, 5
    q, k, v = _qkv(B, T, H, hd, 2)
    out = banded_attention(q, k, v, window=W, block=5)
    for i in range(T):
        for h in range(H):
            js = [j for j in range(T) if 0 <= i - j < W]
            s = torch.stack([q[0, i, h] @ k[0, j, h] for j in js]) / hd ** 0.5
            ref = (torch.softmax(s, 0)[:, None] * v[0, js, h]).sum(0)
            assert torch.allclose(out[0, i, h], ref, atol=1e-5)


def test_decode_equals_last_row_of_prefill():
    B, T, H, hd, W = 2, 40, 3, 8, 16
    q, k, v = _qkv(B, T, H, hd, 3)
    full = banded_attention(q, k, v, window=W, block=16)
    kc = torch.zeros(B, H, W, hd)
    vc = torch.zeros(B, H, W, hd)
    for t in range(T):
        o, kc, vc = banded_attention_decode(q[:, t], k[:, t], v[:, t], kc, vc,
                                            torch.full((B,), t))
        assert torch.allclose(o, full[:, t], atol=1e-5), t


def test_moe_selected_matches_per_token_brute_force():
    from oracle.moe import moe_per_token, moe_selected_fp32
    g = torch.Generator().manual_seed(21)
    E, H, D, k = 5, 12, 16, 3
    wg = torch.randn(E, H, D, generator=g)
    wu = torch.randn(E, H, D, generator=g)
    wd = torch.randn(E, D, H, generator=g)
    x = torch.randn(1, D, generator=g)
    idx = np.array([[4, 0, 2]])
    prob = torch.tensor([[0.5, 0.3, 0.2]])
    _, ro, out = moe_selected_fp32(x.numpy(), idx, prob.numpy(),
                                   torch.cat([wg, wu], 1).numpy(), wd.numpy())
    ref = moe_per_token(x, idx, prob, wg, wu, wd)
    assert np.allclose(out, ref.numpy()[0], rtol=1e-5, atol=1e-5)
    # route_output rows are the prob-weighted expert outputs
    assert np.allclose(ro[1], 0.3 * moe_per_token(x, idx[:, 1:2], torch.ones(1, 1), wg, wu,
                                                  wd).numpy()[0], rtol=1e-5, atol=1e-5)
    # an out-of-range id contributes nothing
    _, _, out2 = moe_selected_fp32(x.numpy(), np.array([[4, 7, 2]]), prob.numpy(),
                                   torch.cat([wg, wu], 1).numpy(), wd.numpy())
    ref2 = moe_per_token(x, idx[:, [0, 2]], prob[:, [0, 2]], wg, wu, wd)
    assert np.allclose(out2, ref2.numpy()[0], rtol=1e-5, atol=1e-5)


def test_sinkhorn4_closed_forms():
    from oracle.mhc import sinkhorn4
    rng = np.random.default_rng(0)
    x = rng.normal(size=(50, 4, 4))
    assert np.allclose(sinkhorn4(x, 0), np.exp(x))                    # no iteration: exp
    assert np.allclose(sinkhorn4(np.full((1, 4, 4), 3.0), 5), 0.25)  # constant -> uniform
    d = sinkhorn4(x, 200)                                              # converged: doubly stochastic
    assert np.allclose(d.sum(-1), 1, atol=1e-9) and np.allclose(d.sum(-2), 1, atol=1e-9)
    # one iteration by hand: row softmax, then column normalisation of that
    r = np.exp(x[0]) / np.exp(x[0]).sum(-1, keepdims=True)
    assert np.allclose(sinkhorn4(x[:1], 1)[0], r / r.sum(0, keepdims=True))
    # permuting rows and columns permutes the result
    p, q = rng.permutation(4), rng.permutation(4)
    assert np.allclose(sinkhorn4(x[:, p][:, :, q], 7), sinkhorn4(x, 7)[:, p][:, :, q])
