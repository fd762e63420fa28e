"""Pins the GDN and sampling oracles (CPU only)."""
import numpy as np
import torch
import torch.nn.functional as F

from oracle.gdn import causal_conv_reset, gdn_chunked, gdn_sequential, gdn_step
from oracle.sampling import argmax, top_p_error_bound, top_p_sample


def _gdn_inputs(B, T, H, dk, dv, seed, s0_std=0.1):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, dk, generator=g), dim=-1)
    k = F.normalize(torch.randn(B, T, H, dk, generator=g), dim=-1)
    v = torch.randn(B, T, H, dv, generator=g)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    gd = torch.exp(-F.softplus(torch.randn(B, T, H, generator=g)))
    S0 = torch.randn(B, H, dk, dv, generator=g) * s0_std
    return q, k, v, beta, gd, S0


def test_beta_zero_is_pure_decay():
    q, k, v, beta, g, S0 = _gdn_inputs(2, 30, 2, 8, 4, 0)
    o, S = gdn_sequential(q, k, v, torch.zeros_like(beta), g, S0, dtype=torch.float64)
    expect = torch.prod(g.double(), dim=1)[..., None, None] * S0.double()
    assert torch.allclose(S, expect, atol=1e-12)
    # o_t = q_t^T (Gamma_t S0)
    gam = torch.cumprod(g.double(), dim=1)
    ref = torch.einsum("bthk,bhkv->bthv", q.double(), S0.double()) * gam[..., None]
    assert torch.allclose(o, ref, atol=1e-12)


def test_orthonormal_keys_overwrite_exactly():
    # g = 1, beta = 1, keys orthonormal: S = sum_i k_i v_i^T, reading q = k_i gives v_i.
    dk, dv, T = 8, 5, 8
    basis = torch.linalg.qr(torch.randn(dk, dk, generator=torch.Generator().manual_seed(1)))[0]
    k = basis.t()[None, :, None, :]                      # [1, T, 1, dk]
    v = torch.randn(1, T, 1, dv, generator=torch.Generator().manual_seed(2))
    ones = torch.ones(1, T, 1)
    _, S = gdn_sequential(k, k, v, ones, ones, torch.zeros(1, 1, dk, dv), dtype=torch.float64)
    read = torch.einsum("tk,kv->tv", k[0, :, 0].double(), S[0, 0])
    assert torch.allclose(read, v[0, :, 0].double(), atol=1e-12)
    # writing the same key again replaces (not adds) its value
    v2 = torch.randn(1, 1, 1, dv, generator=torch.Generator().manual_seed(3))
    _, S2 = gdn_sequential(k[:, :1], k[:, :1], v2, ones[:, :1], ones[:, :1], S,
                           dtype=torch.float64)
    assert torch.allclose(k[0, 0, 0].double() @ S2[0, 0], v2[0, 0, 0].double(), atol=1e-12)


def test_prediction_uses_undecayed_state():
    # Distinguishes the reference transition g*S + beta*k(v - k^T S) from
    # the textbook g*(S + beta*k(v - k^T S)): one step, hand computed.
    dk, dv = 2, 1
    S0 = torch.tensor([[[[1.0], [0.0]]]])
    k = torch.tensor([[[[1.0, 0.0]]]])
    v = torch.tensor([[[[3.0]]]])
    beta = torch.tensor([[[0.5]]])
    g = torch.tensor([[[0.25]]])
    _, S = gdn_sequential(k, k, v, beta, g, S0, dtype=torch.float64)
    # 0.25*1 + 0.5*1*(3 - 1) = 1.25
    assert abs(float(S[0, 0, 0, 0]) - 1.25) < 1e-12


def test_chunked_matches_sequential():
    for (T, C) in [(130, 64), (64, 64), (50, 16), (7, 64)]:
        q, k, v, beta, g, S0 = _gdn_inputs(2, T, 3, 16, 8, T)
        o1, S1 = gdn_sequential(q, k, v, beta, g, S0, dtype=torch.float64)
        o2, S2 = gdn_chunked(q, k, v, beta, g, S0, chunk=C)
        assert torch.allclose(o1, o2, atol=1e-10), (T, C)
        assert torch.allclose(S1, S2, atol=1e-10), (T, C)


def test_step_equals_one_token_scan():
    q, k, v, beta, g, S0 = _gdn_inputs(3, 1, 2, 8, 8, 5)
    o1, S1 = gdn_sequential(q, k, v, beta, g, S0)
    o2, S2 = gdn_step(q[:, 0], k[:, 0], v[:, 0], beta[:, 0], g[:, 0], S0)
    assert torch.equal(o1[:, 0], o2) and torch.equal(S1, S2)


def test_reset_restarts_from_zero_state():
    # A reset before token t: tokens < t are unaffected, tokens >= t equal a
    # fresh run of the suffix from S = 0 (gated_deltanet.py:138-142).
    B, T = 3, 40
    q, k, v, beta, g, S0 = _gdn_inputs(B, T, 2, 8, 6, 11, s0_std=1.0)
    reset = torch.zeros(B, T, dtype=torch.bool)
    reset[0, 17] = True
    reset[1, 0] = True
    reset[1, 25] = True                     # two resets in one row
    o, S = gdn_sequential(q, k, v, beta, g, S0, dtype=torch.float64, reset=reset)
    o_plain, S_plain = gdn_sequential(q, k, v, beta, g, S0, dtype=torch.float64)
    assert torch.allclose(o[0, :17], o_plain[0, :17], atol=1e-12)
    assert torch.equal(o[2], o_plain[2]) and torch.equal(S[2], S_plain[2])
    for b, t in [(0, 17), (1, 25)]:
        sl = slice(t, T)
        o_s, S_s = gdn_sequential(q[b:b + 1, sl], k[b:b + 1, sl], v[b:b + 1, sl],
                                  beta[b:b + 1, sl], g[b:b + 1, sl],
                                  torch.zeros_like(S0[:1]), dtype=torch.float64)
        assert torch.allclose(o[b:b + 1, sl], o_s, atol=1e-12)
        assert torch.allclose(S[b:b + 1], S_s, atol=1e-12)
    # a reset at t = 0 discards the given state for that row only
    o_z, _ = gdn_sequential(q[1:2, :25], k[1:2, :25], v[1:2, :25], beta[1:2, :25],
                            g[1:2, :25], torch.zeros_like(S0[:1]), dtype=torch.float64)
    assert torch.allclose(o[1:2, :25], o_z, atol=1e-12)
    # the step form with a per-row reset equals the one-token scan
    o1, S1 = gdn_step(q[:, 0], k[:, 0], v[:, 0], beta[:, 0], g[:, 0], S0,
                      reset=torch.tensor([True, False, True]))
    o2, S2 = gdn_sequential(q[:, :1], k[:, :1], v[:, :1], beta[:, :1], g[:, :1], S0,
                            reset=torch.tensor([[True], [False], [True]]))
    assert torch.equal(o1, o2[:, 0]) and torch.equal(S1, S2)
    assert torch.allclose(S1[0], torch.einsum("hk,hv->hkv", k[0, 0], beta[0, 0, :, None]
                                              * v[0, 0]), atol=1e-6)


def test_causal_conv_matches_library_conv_and_resets():
    B, T, D, K = 2, 23, 5, 4
    gen = torch.Generator().manual_seed(4)
    h = torch.randn(B, T, D, generator=gen, dtype=torch.float64)
    w = torch.randn(D, K, generator=gen, dtype=torch.float64)
    hist0 = torch.zeros(B, K - 1, D, dtype=torch.float64)
    out, hist = causal_conv_reset(h, hist0, w)
    # zero history = the reference's left-padded depthwise Conv1d (gated_deltanet.py:65-66)
    lib = F.conv1d(F.pad(h.transpose(1, 2), (K - 1, 0)), w[:, None, :], groups=D)
    assert torch.allclose(out, lib.transpose(1, 2), atol=1e-12)
    assert torch.equal(hist, h[:, -(K - 1):])
    # the carried history makes a split run equal the whole run
    o_a, h_a = causal_conv_reset(h[:, :9], hist0, w)
    o_b, h_b = causal_conv_reset(h[:, 9:], h_a, w)
    assert torch.allclose(torch.cat([o_a, o_b], 1), out, atol=1e-12) and torch.equal(h_b, hist)
    # a reset at t: taps never reach before t (the masked taps of :67-78)
    reset = torch.zeros(B, T, dtype=torch.bool)
    reset[0, 10] = True
    reset[1, 21] = True
    o_r, h_r = causal_conv_reset(h, torch.randn(B, K - 1, D, dtype=torch.float64,
                                                generator=gen), w, reset)
    for b, t in [(0, 10), (1, 21)]:
        o_s, h_s = causal_conv_reset(h[b:b + 1, t:], hist0[:1], w)
        assert torch.allclose(o_r[b:b + 1, t:], o_s, atol=1e-12)
        assert torch.equal(h_r[b:b + 1], h_s)
    assert torch.allclose(o_r[0, 3:10], out[0, 3:10], atol=1e-12)   # beyond the old history
    # a reset near the end leaves fewer than K-1 new tokens: the rest of the history is 0
    assert torch.equal(h_r[1, 0], torch.zeros(D, dtype=torch.float64))


def test_argmax_first_occurrence_and_nan():
    x = torch.tensor([[1.0, 5.0, 5.0, 2.0], [float("nan"), 1.0, float("nan"), 9.0],
                      [-1.0, -1.0, -3.0, -2.0]])
    assert list(argmax(x)) == [1, 0, 0]
    r = torch.randn(64, 1000, generator=torch.Generator().manual_seed(0))
    assert np.array_equal(argmax(r), torch.argmax(r, -1).numpy())


def test_top_p_closed_forms():
    g = torch.Generator().manual_seed(7)
    logits = torch.randn(16, 500, generator=g) * 2
    greedy = torch.argmax(logits, -1).numpy()
    zeros = torch.zeros(16)
    # u = 0 picks the most probable token
    assert np.array_equal(top_p_sample(logits, 0.8, 0.9, zeros), greedy)
    # p -> 0 keeps only the top token, whatever u is
    u = torch.rand(16, generator=g)
    assert np.array_equal(top_p_sample(logits, 0.8, 1e-9, u), greedy)
    # p = 1 (disabled): plain inverse CDF over the full sorted distribution
    out = top_p_sample(logits, 0.8, 1.0, u)
    for r in range(16):
        order = np.lexsort((np.arange(500), -logits[r].double().numpy()))
        p = torch.softmax(logits[r].double() / 0.8, -1).numpy()[order]
        expect = order[np.searchsorted(np.cumsum(p), float(u[r]), side="right")]
        assert out[r] == expect


def test_top_p_nucleus_matches_torch_sampler_rule():
    # The kept set is the smallest prefix reaching p; u just below the kept
    # mass boundary picks the last kept token, never one outside it.
    g = torch.Generator().manual_seed(9)
    logits = torch.randn(8, 50, generator=g)
    for r in range(8):
        sv, order = torch.sort(logits[r].double() / 0.8, descending=True, stable=True)
        p = torch.softmax(sv, -1)
        c = torch.cumsum(p, -1)
        cut = int(torch.nonzero(c >= 0.9)[0]) + 1
        got = top_p_sample(logits[r:r + 1], 0.8, 0.9, torch.tensor([0.999999]))
        assert got[0] == int(order[cut - 1])


def test_top_k_rules():
    g = torch.Generator().manual_seed(11)
    logits = torch.randn(12, 300, generator=g) * 3
    u = torch.rand(12, generator=g)
    greedy = torch.argmax(logits, -1).numpy()
    # top_k = 1 keeps only the most probable token
    assert np.array_equal(top_p_sample(logits, 0.7, 1.0, u, top_k=1), greedy)
    # top-k with the nucleus off: inverse CDF of the renormalised top-k softmax,
    # taken here through torch.topk (distinct values, so its order is unique)
    out = top_p_sample(logits, 0.7, 1.0, u, top_k=20)
    for r in range(12):
        v, i = torch.topk(logits[r].double(), 20)
        p = torch.softmax(v / 0.7, -1).numpy()
        assert out[r] == int(i[np.searchsorted(np.cumsum(p), float(u[r]), side="right")])
    # the margin is the distance of u from the CDF steps around the pick
    _, m = top_p_sample(logits[:1], 0.7, 1.0, torch.tensor([0.5]), top_k=2, return_margin=True)
    v, _ = torch.topk(logits[0].double(), 2)
    p0 = float(torch.softmax(v / 0.7, -1)[0])
    assert abs(m[0] - (abs(p0 - 0.5) if p0 > 0.5 else min(0.5 - p0, 0.5))) < 1e-12
    # ... and, with the nucleus on, from top_p around the cut: three tokens of
    # probabilities (0.5, 0.3, 0.2), p = 0.85 cuts after the second (0.8 < 0.85 <= 1.0)
    x = torch.log(torch.tensor([[0.5, 0.3, 0.2]], dtype=torch.float64))
    got, m = top_p_sample(x, 1.0, 0.85, torch.tensor([0.3]), return_margin=True)
    assert got[0] == 0 and abs(m[0] - min(0.05, 0.15, 0.5 / 0.8 - 0.3, 0.3)) < 1e-12


def test_repetition_penalty_rule():
    from oracle.sampling import repetition_penalty
    x = torch.tensor([[2.0, -2.0, 0.0, 4.0, 1.0]])
    got = repetition_penalty(x, [[0, 1, 1, 2, 7, -1, 3, 3, 3]], 2.0)
    # positive logits halve, non-positive ones double, each id once
    assert torch.equal(got, torch.tensor([[1.0, -4.0, 0.0, 2.0, 1.0]]))


def test_top_p_error_bound_covers_fp32_terms():
    """The per-row bound covers the cumulative probabilities of an fp32
    implementation (fp32 exponent and exp, exact sums), at several logit
    scales and temperatures, and is far below the flat 4e-6 margin on
    near-flat rows."""
    g = torch.Generator().manual_seed(13)
    for scale in (0.6, 2.0, 8.0, 30.0):
        for T in (0.5, 0.8, 1.3):
            x = torch.randn(8, 32000, generator=g) * scale
            bound = top_p_error_bound(x, T)
            for r in range(8):
                order = np.lexsort((np.arange(32000), -x[r].double().numpy()))
                xs = x[r].numpy()[order]
                a32 = (xs - xs[0]).astype(np.float32) / np.float32(T)   # fp32 exponent
                p32 = np.exp(a32.astype(np.float32)).astype(np.float64)  # fp32-rounded terms
                c32 = np.cumsum(p32) / p32.sum()
                a64 = (xs.astype(np.float64) - float(xs[0])) / T
                p64 = np.exp(a64)
                c64 = np.cumsum(p64) / p64.sum()
                assert np.abs(c32 - c64).max() <= bound[r], (scale, T, r)
            if scale < 1 and T == 0.8:   # the C5 sampling case
                assert bound.max() < 2e-6, bound.max()
