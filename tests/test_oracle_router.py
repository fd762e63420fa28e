"""Pins the router / permutation oracle (CPU only)."""
import itertools

import numpy as np
import torch

from oracle.router import moe_permute, rmsnorm, router_logits, router_topk, topk_lower_index


def brute_topk(row, k):
    """Exhaustive: the k-subset, ordered, that a (value desc, index asc) rule picks."""
    n = len(row)
    best = None
    for combo in itertools.permutations(range(n), k):
        key = [(-(np.inf if np.isnan(row[i]) else row[i]), i) for i in combo]
        rest = [i for i in range(n) if i not in combo]
        ok = key == sorted(key) and all(
            (-(np.inf if np.isnan(row[j]) else row[j]), j) > key[-1] for j in rest)
        if ok:
            best = list(combo)
    return best


def test_topk_matches_brute_force_with_ties_and_nan():
    rng = np.random.default_rng(0)
    for trial in range(60):
        n = int(rng.integers(2, 7))
        k = int(rng.integers(1, n + 1))
        row = rng.choice([-1.0, 0.0, -0.0, 0.5, 0.5, 2.0, np.nan], size=n).astype(np.float32)
        idx, vals = topk_lower_index(torch.from_numpy(row[None]), k)
        assert list(idx[0]) == brute_topk(list(row), k), (row, k)


def test_ties_go_to_lower_index():
    logits = torch.tensor([[1.0, 3.0, 3.0, 0.5, 3.0]])
    idx, _ = topk_lower_index(logits, 3)
    assert list(idx[0]) == [1, 2, 4]
    idx, _ = topk_lower_index(torch.tensor([[0.0, -0.0, 0.0]]), 2)
    assert list(idx[0]) == [0, 1]


def test_gates_are_softmax_of_selected_and_sum_to_one():
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(50, 24, generator=g)
    idx, gates = router_topk(logits, 2)
    assert torch.allclose(gates.sum(-1), torch.ones(50), atol=1e-6)
    v = torch.gather(logits, 1, torch.from_numpy(idx))
    assert torch.all(v[:, 0] >= v[:, 1])
    ref = torch.exp(v - v[:, :1]) / torch.exp(v - v[:, :1]).sum(-1, keepdim=True)
    assert torch.allclose(gates, ref, atol=1e-7)
    # k = E: gates equal the softmax over all logits, in sorted order
    idx, gates = router_topk(logits, 24)
    full = torch.softmax(logits, -1)
    assert torch.allclose(gates, torch.gather(full, 1, torch.from_numpy(idx)), atol=1e-6)


def test_router_logits_closed_form():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(7, 32, generator=g)
    w = torch.randn(5, 32, generator=g)
    nw = torch.rand(32, generator=g) + 0.5
    ref = np.stack([[sum(float(xi) / np.sqrt(np.mean(x[t].double().numpy() ** 2) + 1e-6)
                         * float(nw[d]) * float(w[e, d]) for d, xi in enumerate(x[t]))
                     for e in range(5)] for t in range(7)])
    assert np.allclose(router_logits(x, w, nw).numpy(), ref, atol=1e-5)
    assert torch.allclose(router_logits(x, w), x @ w.t())
    # RMSNorm output has unit mean square with unit weight
    assert torch.allclose(rmsnorm(x, None).pow(2).mean(-1), torch.ones(7), atol=1e-4)


def test_permutation_is_stable_counting_sort():
    rng = np.random.default_rng(3)
    for n, E in [(0, 4), (1, 1), (17, 3), (8192, 24), (300, 256)]:
        ids = rng.integers(0, E, size=n)
        p = moe_permute(ids, E)
        assert p["counts"].sum() == n
        assert np.array_equal(p["counts"], np.bincount(ids, minlength=E))
        assert p["offsets"][0] == 0 and p["offsets"][-1] == n
        assert np.array_equal(np.diff(p["offsets"]), p["counts"])
        sr = p["sorted_routes"]
        assert np.array_equal(np.sort(sr), np.arange(n))       # bijection
        assert np.array_equal(p["route_pos"][sr], np.arange(n))  # inverse
        for e in range(E):
            seg = sr[p["offsets"][e]:p["offsets"][e + 1]]
            assert np.all(ids[seg] == e)
            assert np.all(np.diff(seg) > 0)                     # ascending r inside e
        assert np.array_equal(sr, torch.argsort(torch.from_numpy(ids), stable=True).numpy())
