"""Pins oracle/compressed.py (the CSA / HCA mixers) on the CPU.

  * against tests/golden/compressed_golden.npz, written from the reference's
    own modules (model/layers/csa.py, hca.py, compressed_attention.py) by
    tests/golden/make_compressed_golden.py: the sequence forward of a 13-token
    prompt and 9 decode steps after it, for CSA (4 heads, top-2 of the
    summaries), HCA dense and HCA top-2;
  * the sequence path equals the decode path run token by token from the
    empty state (the property compressed_attention.py:161-166 states);
  * the local branch with a window covering the sequence is causal scaled
    dot-product attention (torch's SDPA), per head, heads averaged;
  * the dense memory branch is SDPA over block means visible from their last
    token on, with the means formed by an explicit loop over blocks;
  * the top-k memory branch equals a per-(token, head) brute-force selection,
    and equals the dense branch when k covers every summary;
  * a reset row continues as a fresh sequence.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.compressed import CompressedMixer, compress_sequence

GOLDEN = "tests/golden/compressed_golden.npz"
CASES = {"csa": (4, 8, 5, 4, 2), "hca": (1, 32, 5, 4, None), "hcak": (1, 32, 5, 3, 2)}


@pytest.mark.parametrize("name", sorted(CASES))
def test_matches_reference_modules(name):
    g = np.load(GOLDEN)
    H, Dh, W, r, k = CASES[name]
    w = {n: torch.from_numpy(g[f"{name}.{n}"]) for n in CompressedMixer.NAMES}
    m = CompressedMixer(w, "", H, Dh, W, r, k)
    h = torch.from_numpy(g[f"{name}.h"])
    B, T, _ = h.shape
    out, st, _ = m.forward(h)
    assert torch.allclose(out, torch.from_numpy(g[f"{name}.seq_out"]), atol=1e-6, rtol=1e-5)
    xs = torch.from_numpy(g[f"{name}.xs"])
    for i in range(xs.shape[0]):
        y = m.step(xs[i], st, torch.full((B,), T + i))
        assert torch.allclose(y, torch.from_numpy(g[f"{name}.step_out"][i]), atol=1e-6,
                              rtol=1e-5), i


def _mixer(H, Dh, D, W, r, k, seed, zero=()):
    gen = torch.Generator().manual_seed(seed)
    Kw = H * Dh
    shapes = {"cmp_wq": (Kw, D), "cmp_wk": (Kw, D), "cmp_wv": (D, D), "cmp_wlo": (D, D),
              "cmp_wro": (D, D), "cmp_wout": (D, D), "cmp_wck": (Kw, D), "cmp_wcv": (D, D)}
    w = {n: torch.randn(s, generator=gen) / math.sqrt(D) for n, s in shapes.items()}
    for n in zero:
        w[n] = torch.zeros_like(w[n])
    return CompressedMixer(w, "", H, Dh, W, r, k)


@pytest.mark.parametrize("H,Dh,k", [(4, 8, 3), (1, 32, None), (2, 16, 1)])
def test_sequence_equals_steps(H, Dh, k):
    D, W, r, B, T = 32, 6, 3, 3, 20
    m = _mixer(H, Dh, D, W, r, k, seed=H + Dh)
    h = torch.randn(B, T, D, generator=torch.Generator().manual_seed(1))
    out, st, _ = m.forward(h)
    st2 = m.new_state(B, D)
    ys = torch.stack([m.step(h[:, t], st2, torch.full((B,), t)) for t in range(T)], 1)
    assert torch.allclose(ys, out, atol=1e-5, rtol=1e-5)
    # the state a sequence leaves continues like the stepped one
    x = torch.randn(B, D, generator=torch.Generator().manual_seed(2))
    assert torch.allclose(m.step(x, st, torch.full((B,), T)), m.step(x, st2, torch.full((B,), T)),
                          atol=1e-5, rtol=1e-5)
    assert torch.equal(st["pcnt"], st2["pcnt"]) and torch.allclose(st["psum"], st2["psum"],
                                                                    atol=1e-5)


@pytest.mark.parametrize("H,Dh", [(1, 32), (4, 8)])
def test_local_branch_is_causal_sdpa(H, Dh):
    D, B, T = 32, 2, 11
    m = _mixer(H, Dh, D, T + 3, 4, None, seed=5)
    h = torch.randn(B, T, D, generator=torch.Generator().manual_seed(6))
    _, _, parts = m.forward(h)
    w = m.w
    q = (h @ w["cmp_wq"].t()).view(B, T, H, Dh).transpose(1, 2)
    kk = (h @ w["cmp_wk"].t()).view(B, T, H, Dh).transpose(1, 2)
    v = (h @ w["cmp_wv"].t())[:, None].expand(B, H, T, D)
    ref = F.scaled_dot_product_attention(q, kk, v, is_causal=True).mean(1)
    assert torch.allclose(parts["local"], ref, atol=1e-5, rtol=1e-4)


def test_compress_sequence_block_loop():
    h = torch.randn(2, 23, 8, generator=torch.Generator().manual_seed(7))
    means, pos, tail, cnt = compress_sequence(h, 5)
    for i in range(4):
        assert torch.allclose(means[:, i], h[:, 5 * i:5 * i + 5].sum(1) / 5, atol=1e-6)
        assert int(pos[i]) == 5 * i + 4
    assert cnt == 3 and torch.allclose(tail, h[:, 20:].sum(1), atol=1e-6)


def test_dense_memory_is_masked_sdpa():
    D, B, T, r = 32, 2, 17, 4
    m = _mixer(1, D, D, 3, r, None, seed=8)
    h = torch.randn(B, T, D, generator=torch.Generator().manual_seed(9))
    _, _, parts = m.forward(h)
    w = m.w
    means = torch.stack([h[:, r * i:r * i + r].mean(1) for i in range(T // r)], 1)
    mk, mv = means @ w["cmp_wck"].t(), means @ w["cmp_wcv"].t()
    q = h @ w["cmp_wq"].t()
    vis = torch.tensor([[r * i + r - 1 <= t for i in range(T // r)] for t in range(T)])
    ref = F.scaled_dot_product_attention(q[:, None], mk[:, None], mv[:, None],
                                         attn_mask=vis)[:, 0]
    rows = vis.any(1)                      # queries before the first block end see nothing
    assert torch.allclose(parts["remote"][:, rows], ref[:, rows], atol=1e-5, rtol=1e-4)
    assert torch.equal(parts["remote"][:, ~rows], torch.zeros_like(parts["remote"][:, ~rows]))


@pytest.mark.parametrize("k", [1, 2, 5])
def test_topk_memory_brute_force(k):
    H, Dh, D, B, T, r = 3, 8, 24, 2, 22, 2
    m = _mixer(H, Dh, D, 3, r, k, seed=10 + k)
    h = torch.randn(B, T, D, generator=torch.Generator().manual_seed(11))
    _, _, parts = m.forward(h)
    q = (h @ m.w["cmp_wq"].t()).view(B, T, H, Dh)
    mk = parts["mk"].view(B, -1, H, Dh)
    mv = parts["mv"]
    for b in range(B):
        for t in range(T):
            acc = torch.zeros(D, dtype=torch.float64)
            nvis = (t + 1) // r
            for hh in range(H):
                sc = [(float(q[b, t, hh] @ mk[b, i, hh]) / math.sqrt(Dh), i) for i in range(nvis)]
                top = sorted(sc, key=lambda x: -x[0])[:k]
                if not top:
                    continue
                mx = max(s for s, _ in top)
                ws = [math.exp(s - mx) for s, _ in top]
                for (s, i), wv in zip(top, ws):
                    acc += wv / sum(ws) * mv[b, i].double()
            assert torch.allclose(parts["remote"][b, t], (acc / H).float(), atol=1e-5), (b, t)
    # k covering every summary is the dense branch
    dense = _mixer(H, Dh, D, 3, r, None, seed=10 + k)
    wide = _mixer(H, Dh, D, 3, r, T, seed=10 + k)
    assert torch.allclose(dense.forward(h)[0], wide.forward(h)[0], atol=1e-6)


def test_reset_row_continues_as_fresh_sequence():
    H, Dh, D, W, r, B = 2, 8, 16, 4, 3, 3
    m = _mixer(H, Dh, D, W, r, 2, seed=12)
    gen = torch.Generator().manual_seed(13)
    st = m.new_state(B, D)
    for t in range(10):
        m.step(torch.randn(B, D, generator=gen), st, torch.full((B,), t))
    m.reset_rows(st, torch.tensor([False, True, False]))
    fresh = m.new_state(1, D)
    pos = torch.tensor([10, 0, 10])
    for i in range(8):
        x = torch.randn(B, D, generator=gen)
        y = m.step(x, st, pos + i)
        yf = m.step(x[1:2], fresh, torch.tensor([i]))
        assert torch.allclose(y[1:2], yf, atol=1e-6), i


def test_forced_selection_replay():
    """Forcing a mixer's top-k memory selection (the replay of the engine's
    choice): forcing the selection a brute-force sort makes gives the unforced
    output and records no gap; forcing another set changes the output and
    records the score gap between the k-th best and the forced set's lowest."""
    H, Dh, D, W, r, k = 2, 8, 16, 4, 2, 2
    m = _mixer(H, Dh, D, W, r, k, seed=21)
    gen = torch.Generator().manual_seed(22)
    B, steps = 2, 9
    xs = torch.randn(steps, B, D, generator=gen)
    st_a, st_b = m.new_state(B, D), m.new_state(B, D)
    for i in range(steps):
        pos = torch.full((B,), i)
        ya = m.step(xs[i], st_a, pos)
        # the brute-force top-k positions of the memory after this step's emit
        q = m._proj(xs[i])[0]
        mpos_next = torch.cat([st_b["mpos"], torch.where(
            st_b["pcnt"] + 1 >= r, pos, torch.full_like(pos, -1))[:, None]], 1)
        mk_next = torch.cat([st_b["mk"], m._summaries(
            (st_b["psum"] + xs[i]) / (st_b["pcnt"] + 1).float()[:, None])[0][:, None]], 1)
        forced = np.full((B, H, k), -1)
        for b in range(B):
            for h in range(H):
                vis = [(float(q[b, h * Dh:(h + 1) * Dh] @ mk_next[b, j, h * Dh:(h + 1) * Dh]), j)
                       for j in range(mk_next.shape[1]) if 0 <= mpos_next[b, j] <= i]
                best = sorted(vis, key=lambda t: (-t[0], t[1]))[:k]
                for n, (_, j) in enumerate(best):
                    forced[b, h, n] = int(mpos_next[b, j])
        m.forced_sel = [forced]
        yb = m.step(xs[i], st_b, pos)
        assert torch.allclose(ya, yb, atol=1e-6), i
    assert m.sel_gaps == [] and m.sel_total == steps * B * H
    # force the lowest-scoring visible summary instead: a different output, one
    # positive gap per (row, head) whose choice changed
    q = m._proj(xs[0])[0]
    m.forced_sel = [np.zeros((B, H, 1), dtype=np.int64) + r - 1]   # the first summary only
    y_forced = m.step(xs[0], st_b, torch.full((B,), steps))
    y_own = m.step(xs[0], st_a, torch.full((B,), steps))
    assert not torch.allclose(y_forced, y_own)
    assert len(m.sel_gaps) > 0 and all(g > 0 for g in m.sel_gaps)
