"""GPU parity: router top-k, permutation and greedy argmax (exact)."""
import numpy as np
import pytest
import torch

from oracle.router import moe_permute, router_logits, router_topk
from oracle.sampling import argmax as argmax_ref

pytestmark = pytest.mark.gpu


def ops():
    from hybrid_llm_amd import ops as o
    return o


def _c2_router_inputs(T=4096, D=1024, E=24, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, D, generator=g).to(torch.bfloat16)
    w = torch.randn(E, D, generator=g) * 0.02
    return x, w


@pytest.mark.parametrize("T,D,E,k", [(4096, 1024, 24, 2), (64, 1024, 24, 2), (5, 256, 8, 2),
                                     (33, 512, 256, 8), (1, 64, 1, 1), (100, 2048, 70, 32)])
def test_topk_from_logits_exact(T, D, E, k):
    g = torch.Generator().manual_seed(T + E)
    logits = torch.randn(T, E, generator=g)
    # plant exact ties and a NaN row so the tie rule is exercised
    logits[0, : min(E, 4)] = 1.5
    if T > 2:
        logits[2, E // 2] = float("nan")
    idx, gates = ops().router_topk_from_logits(logits.cuda(), k)
    ref_idx, ref_gates = router_topk(logits, k)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    ok = ~torch.isnan(ref_gates).any(-1)
    assert torch.allclose(gates.cpu()[ok], ref_gates[ok], atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("with_norm", [False, True])
def test_router_fused_c2(with_norm):
    x, w = _c2_router_inputs()
    nw = (torch.rand(1024, generator=torch.Generator().manual_seed(3)) + 0.5) if with_norm else None
    idx, gates, logits = ops().router_topk(x.cuda(), w.cuda(), 2,
                                           None if nw is None else nw.cuda(), return_logits=True)
    ref_logits = router_logits(x.float(), w, nw)
    assert torch.allclose(logits.cpu(), ref_logits, atol=2e-5, rtol=1e-5)
    # Exact on the kernel's own logits (same-input rule) ...
    ref_idx, ref_gates = router_topk(logits.cpu(), 2)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    assert torch.allclose(gates.cpu(), ref_gates, atol=1e-6)
    # ... and exact against the fp32 oracle logits wherever the top-k margin
    # exceeds the logit error bound (near-ties may flip by design of fp32).
    oi, _ = router_topk(ref_logits, 3)
    v = torch.gather(ref_logits, 1, torch.from_numpy(oi))
    margin = (v[:, 1] - v[:, 2]).numpy()
    safe = margin > 1e-4
    assert safe.mean() > 0.99
    assert np.array_equal(idx.cpu().numpy()[safe], oi[safe, :2])


def test_router_deterministic():
    x, w = _c2_router_inputs(T=1024)
    a = ops().router_topk(x.cuda(), w.cuda(), 2, return_logits=True)
    b = ops().router_topk(x.cuda(), w.cuda(), 2, return_logits=True)
    for p, q in zip(a, b):
        assert torch.equal(p, q)


@pytest.mark.parametrize("n,E", [(8192, 24), (128, 24), (0, 24), (1, 1), (65, 3), (20000, 256),
                                 (777, 1000),
                                 # more than 16 chunks per wave (held + reloaded chunks)
                                 (20000, 24), (4097, 64), (3000, 7),
                                 # one expert, just past one wave's limit, long lists
                                 (5000, 1), (2049, 24), (50000, 2), (65536, 64)])
def test_permute_exact(n, E):
    g = torch.Generator().manual_seed(n + E)
    ids = torch.randint(0, E, (n,), generator=g, dtype=torch.int32)
    got = ops().moe_permute(ids.cuda(), E)
    ref = moe_permute(ids.numpy(), E)
    assert np.array_equal(got["counts"].cpu().numpy(), ref["counts"])
    assert np.array_equal(got["offsets"].cpu().numpy(), ref["offsets"])
    assert np.array_equal(got["sorted_routes"].cpu().numpy(), ref["sorted_routes"])
    assert np.array_equal(got["route_pos"].cpu().numpy(), ref["route_pos"])


@pytest.mark.parametrize("n,E", [(8192, 24), (3000, 64), (500, 5), (20000, 256)])
def test_permute_skips_out_of_range_ids(n, E):
    """Ids outside [0, E) are not placed: the valid routes are counted and
    sorted stably by expert exactly as if the others were absent."""
    g = torch.Generator().manual_seed(7 * n + E)
    ids = torch.randint(-2, E + 2, (n,), generator=g, dtype=torch.int32)
    got = ops().moe_permute(ids.cuda(), E)
    ok = ((ids >= 0) & (ids < E)).numpy()
    valid = np.nonzero(ok)[0]
    ref = moe_permute(ids.numpy()[valid], E)
    nv = valid.size
    assert np.array_equal(got["counts"].cpu().numpy(), ref["counts"])
    assert np.array_equal(got["offsets"].cpu().numpy(), ref["offsets"])
    assert np.array_equal(got["sorted_routes"].cpu().numpy()[:nv], valid[ref["sorted_routes"]])
    assert np.array_equal(got["route_pos"].cpu().numpy()[valid], ref["route_pos"])


def test_permute_skewed_all_one_expert():
    ids = torch.full((8192,), 5, dtype=torch.int32)
    got = ops().moe_permute(ids.cuda(), 24)
    assert np.array_equal(got["sorted_routes"].cpu().numpy(), np.arange(8192))


@pytest.mark.parametrize("R,V", [(64, 32000), (1, 32000), (3, 7), (8, 100003)])
def test_argmax_exact(R, V):
    g = torch.Generator().manual_seed(R * V)
    logits = torch.randn(R, V, generator=g)
    logits[0, V // 3] = logits[0].max() + 1
    logits[0, V // 2] = logits[0, V // 3]          # tie: lower index wins
    if R > 1:
        logits[1, V - 1] = float("nan")
    got = ops().argmax(logits.cuda()).cpu().numpy()
    assert np.array_equal(got, argmax_ref(logits))
