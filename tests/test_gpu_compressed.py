"""GPU parity: the compressed-memory (CSA / HCA) kernels against oracle/compressed.py.

Attention branches: the local window and the memory summaries, dense and
top-k, prefill and decode, at CSA-like (16 heads x 128) and HCA-like (one head
of width d_model) shapes, against the oracle's head-mean probabilities applied
in fp64 to the same bf16 operands.  Outputs are bf16: rel-L2 <= 5e-3 and
max-abs <= 3e-2 (a top-k boundary swap between two scores equal to fp32
accumulation order moves one head's weight; it stays inside both bounds).
Compressor and state kernels (block means, the decode running sum, the
commit, ring and memory fills) are checked exactly or to one bf16 rounding.
"""
import math

import pytest
import torch

from oracle.compressed import band_visible, head_mean_probs, head_scores

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS = 5e-3, 2e-2


def ops():
    from hybrid_llm_amd import ops as o
    return o


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float(torch.linalg.norm(a - b) / torch.linalg.norm(b).clamp_min(1e-30))


def _close(got, ref):
    got, ref = got.float().cpu(), ref.float().cpu()
    assert rel_l2(got, ref) <= REL_L2, rel_l2(got, ref)
    assert float((got - ref).abs().max()) <= MAX_ABS, float((got - ref).abs().max())


def _bf(*shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).bfloat16()


LOCAL = [  # B, T, H, Dh, Dv, W
    (2, 100, 4, 128, 256, 37),
    (1, 300, 16, 128, 1024, 128),
    (2, 200, 1, 512, 512, 64),
    (1, 70, 1, 1024, 1024, 128),
    (3, 5, 2, 64, 64, 8),
]


@pytest.mark.parametrize("B,T,H,Dh,Dv,W", LOCAL)
def test_local_prefill(B, T, H, Dh, Dv, W):
    print(f"local prefill B={B} T={T} H={H} Dh={Dh} Dv={Dv} W={W}", flush=True)
    g = torch.Generator().manual_seed(T + H + Dh)
    Kw = H * Dh
    qkv = _bf(B * T, 2 * Kw + Dv, gen=g)       # one fused projection: column slices
    q, k, v = qkv[:, :Kw], qkv[:, Kw:2 * Kw], qkv[:, 2 * Kw:]
    d = qkv.cuda()
    out = ops().cmp_local_prefill(d[:, :Kw], d[:, Kw:2 * Kw], d[:, 2 * Kw:], B, T, H, Dh, W)
    torch.cuda.synchronize()
    P = head_mean_probs(head_scores(q.float().view(B, T, Kw), k.float().view(B, T, Kw), H, Dh),
                        band_visible(T, W)[None].expand(B, T, T))
    ref = (P.double() @ v.double().view(B, T, Dv)).view(B * T, Dv)
    _close(out, ref)


MEMORY = [  # B, T, ratio, H, Dh, Dv, top_k
    (2, 100, 4, 4, 64, 256, 3),
    (1, 512, 4, 16, 128, 1024, 32),
    (2, 300, 32, 1, 512, 512, 0),
    (1, 256, 8, 1, 1024, 1024, 4),
    (2, 40, 4, 2, 64, 64, 0),
    (2, 3, 4, 2, 64, 64, 2),          # no summary yet
    (1, 2048, 4, 8, 64, 128, 32),     # 512 summaries: the lane-maximum prefilter
    (1, 4096, 4, 4, 64, 64, 32),      # 1024 summaries, the bench's selection size
]


def _mem_ref(q, mk, mv, B, T, ratio, H, Dh, top_k):
    n = T // ratio
    Kw, Dv = H * Dh, mv.shape[1]
    if n == 0:
        return torch.zeros(B * T, Dv, dtype=torch.float64)
    pos = torch.arange(n) * ratio + ratio - 1
    vis = (pos[None, :] <= torch.arange(T)[:, None])[None].expand(B, T, n)
    P = head_mean_probs(head_scores(q.float().view(B, T, Kw), mk.float().view(B, n, Kw), H, Dh),
                        vis, top_k or None)
    return (P.double() @ mv.double().view(B, n, Dv)).view(B * T, Dv)


@pytest.mark.parametrize("B,T,ratio,H,Dh,Dv,top_k", MEMORY)
def test_memory_prefill(B, T, ratio, H, Dh, Dv, top_k):
    print(f"memory prefill B={B} T={T} r={ratio} H={H} Dh={Dh} Dv={Dv} k={top_k}", flush=True)
    g = torch.Generator().manual_seed(T + ratio + top_k)
    Kw, n = H * Dh, T // ratio
    q = _bf(B * T, Kw, gen=g)
    kv = _bf(max(B * n, 1), Kw + Dv, gen=g)[:B * n]
    d = kv.cuda()
    out = ops().cmp_memory_prefill(q.cuda(), d[:, :Kw], d[:, Kw:], B, T, ratio, H, Dh, top_k)
    torch.cuda.synchronize()
    _close(out, _mem_ref(q, kv[:, :Kw], kv[:, Kw:], B, T, ratio, H, Dh, top_k))


@pytest.mark.parametrize("T,ratio,top_k,levels", [(2048, 4, 32, 3), (2048, 4, 16, 9), (1024, 2, 5, 2)])
def test_memory_prefill_topk_ties(T, ratio, top_k, levels):
    """Scores drawn from a few levels, so many summaries tie at the top-k
    boundary (and the prefilter's survivors can pass 64, the all-key path):
    the selection must keep the lowest indices among equal scores, which the
    output shows, since every summary's value row differs."""
    print(f"memory prefill ties T={T} r={ratio} k={top_k} levels={levels}", flush=True)
    g = torch.Generator().manual_seed(T + top_k + levels)
    B, H, Dh, Dv = 1, 2, 64, 64
    Kw, n = H * Dh, T // ratio
    # q . k takes (levels) distinct values per head: k rows are one of a few
    # fixed directions, q rows one shared direction per head
    base = torch.randn(levels, Kw, generator=g)
    pick = torch.randint(0, levels, (B * n,), generator=g)
    mk = (base[pick] * 0.5).bfloat16()
    q = (torch.randn(1, Kw, generator=g).expand(B * T, Kw) * 0.5).bfloat16().contiguous()
    mv = _bf(B * n, Dv, gen=g)
    kv = torch.cat([mk, mv], 1).cuda()
    out = ops().cmp_memory_prefill(q.cuda(), kv[:, :Kw], kv[:, Kw:], B, T, ratio, H, Dh, top_k)
    torch.cuda.synchronize()
    _close(out, _mem_ref(q, mk, mv, B, T, ratio, H, Dh, top_k))


@pytest.mark.parametrize("T,ratio,C,top_k", [(100, 4, 4, 3), (100, 4, 4, 0), (300, 32, 3, 0)])
def test_memory_prefill_ring_window(T, ratio, C, top_k):
    """With slots = C below the prompt's T / ratio summaries, query t sees only
    the last C summaries emitted up to it: the brute-force reference with that
    window, and the decode kernel over a C-slot memory filled with the first
    (t + 1) // ratio summaries, which is the token-by-token decode's state."""
    B, H, Dh, Dv = 1, 2, 64, 128
    print(f"memory prefill ring window T={T} r={ratio} C={C} k={top_k}", flush=True)
    g = torch.Generator().manual_seed(T + C + top_k)
    Kw, n = H * Dh, T // ratio
    q = _bf(B * T, Kw, gen=g)
    kv = _bf(B * n, Kw + Dv, gen=g)
    d = kv.cuda()
    out = ops().cmp_memory_prefill(q.cuda(), d[:, :Kw], d[:, Kw:], B, T, ratio, H, Dh, top_k,
                                   slots=C)
    torch.cuda.synchronize()
    i = torch.arange(n)
    t = torch.arange(T)[:, None]
    vis = ((i * ratio + ratio - 1)[None] <= t) & (i[None] >= (t + 1) // ratio - C)
    P = head_mean_probs(head_scores(q.float().view(B, T, Kw), kv[:, :Kw].float().view(B, n, Kw),
                                    H, Dh), vis[None], top_k or None)
    _close(out, (P.double() @ kv[:, Kw:].double().view(B, n, Dv)).view(B * T, Dv))
    for tq in [0, ratio - 1, C * ratio - 1, C * ratio, T // 2, T - 1]:
        cnt = (tq + 1) // ratio
        mk = torch.zeros(B, C, Kw, dtype=torch.bfloat16, device="cuda")
        mv = torch.zeros(B, C, Dv, dtype=torch.bfloat16, device="cuda")
        mtag = torch.zeros(B, C, dtype=torch.int32, device="cuda")
        mcount = torch.zeros(B, dtype=torch.int32, device="cuda")
        ops().cmp_memory_fill(d[:cnt], B, cnt, ratio, mk, mv, mtag, mcount)
        dec = ops().cmp_memory_decode(q[tq:tq + 1].cuda(), mk, mv, mtag,
                                      torch.tensor([tq], dtype=torch.int32, device="cuda"), H, Dh,
                                      top_k)
        torch.cuda.synchronize()
        assert float((dec.float() - out[tq:tq + 1].float()).abs().max()) <= 1e-2, tq


# B * H >= 512 (the last case) takes the one-kernel scores + list form
@pytest.mark.parametrize("B,H,Dh,Dv,W", [(8, 16, 128, 1024, 128), (4, 1, 1024, 1024, 128),
                                         (3, 2, 64, 128, 7), (32, 16, 128, 256, 128)])
def test_local_decode(B, H, Dh, Dv, W):
    print(f"local decode B={B} H={H} Dh={Dh} Dv={Dv} W={W}", flush=True)
    g = torch.Generator().manual_seed(B * W + Dh)
    Kw = H * Dh
    pos = torch.tensor(([0, 3, W - 1, W, 5 * W + 2, 2 * W - 1, 17, 1000] * ((B + 7) // 8))[:B],
                       dtype=torch.int32)
    ring_k, ring_v = _bf(B, W, Kw, gen=g), _bf(B, W, Dv, gen=g)
    q = _bf(B, Kw, gen=g)
    kvn = _bf(B, Kw + Dv, gen=g)
    rk, rv = ring_k.clone().cuda(), ring_v.clone().cuda()
    d = kvn.cuda()
    out = ops().cmp_local_decode(q.cuda(), d[:, :Kw], d[:, Kw:], rk, rv, pos.cuda(), H, Dh)
    torch.cuda.synchronize()
    # reference: keys max(0, p-W+1)..p, the current one from k_new
    ref = torch.zeros(B, Dv, dtype=torch.float64)
    for b in range(B):
        p = int(pos[b])
        keys = list(range(max(0, p - W + 1), p + 1))
        K = torch.stack([kvn[b, :Kw] if j == p else ring_k[b, j % W] for j in keys]).float()
        V = torch.stack([kvn[b, Kw:] if j == p else ring_v[b, j % W] for j in keys]).float()
        P = head_mean_probs(head_scores(q[b:b + 1, None].float(), K[None], H, Dh),
                            torch.ones(1, 1, len(keys), dtype=torch.bool))
        ref[b] = (P.double() @ V.double())[0, 0]
        # the ring now holds the new key / value at slot p % W, other slots unchanged
        assert torch.equal(rk[b, p % W].cpu(), kvn[b, :Kw]) and torch.equal(rv[b, p % W].cpu(),
                                                                            kvn[b, Kw:])
        others = [s for s in range(W) if s != p % W]
        assert torch.equal(rk[b, others].cpu(), ring_k[b, others])
    _close(out, ref)


# B * H >= 512 (the last two cases) takes the one-kernel scores + list form
@pytest.mark.parametrize("B,C,H,Dh,Dv,top_k", [(8, 256, 16, 128, 1024, 32), (4, 64, 1, 1024, 1024, 0),
                                               (3, 40, 2, 64, 128, 5), (2, 300, 1, 512, 512, 8),
                                               (32, 256, 16, 128, 256, 32),
                                               (64, 100, 8, 64, 128, 0)])
def test_memory_decode(B, C, H, Dh, Dv, top_k):
    print(f"memory decode B={B} C={C} H={H} Dh={Dh} Dv={Dv} k={top_k}", flush=True)
    g = torch.Generator().manual_seed(C + H + top_k)
    Kw = H * Dh
    mk, mv = _bf(B, C, Kw, gen=g), _bf(B, C, Dv, gen=g)
    pos = torch.randint(50, 400, (B,), generator=g, dtype=torch.int32)
    # tags: empty (0), visible (1..pos+1) and a few from later positions (invisible)
    tag = torch.randint(0, 450, (B, C), generator=g, dtype=torch.int32)
    tag[:, :3] = 0
    q = _bf(B, Kw, gen=g)
    out = ops().cmp_memory_decode(q.cuda(), mk.cuda(), mv.cuda(), tag.cuda(), pos.cuda(), H, Dh,
                                  top_k)
    torch.cuda.synchronize()
    vis = ((tag >= 1) & (tag <= pos[:, None] + 1))[:, None]
    P = head_mean_probs(head_scores(q[:, None].float(), mk.float(), H, Dh), vis, top_k or None)
    ref = (P.double() @ mv.double())[:, 0]
    _close(out, ref)
    # no visible slot gives 0
    out0 = ops().cmp_memory_decode(q.cuda(), mk.cuda(), mv.cuda(), torch.zeros_like(tag).cuda(),
                                   pos.cuda(), H, Dh, top_k)
    assert torch.equal(out0.cpu(), torch.zeros(B, Dv, dtype=torch.bfloat16))


@pytest.mark.parametrize("T,ratio", [(37, 4), (64, 32), (3, 4), (96, 32)])
def test_pool_prefill(T, ratio):
    B, D = 3, 256
    g = torch.Generator().manual_seed(T * ratio)
    h = _bf(B * T, D, gen=g)
    psum = torch.full((B, D), 7.0).cuda()
    pcnt = torch.full((B,), 9, dtype=torch.int32).cuda()
    means = ops().cmp_pool_prefill(h.cuda(), B, T, ratio, psum, pcnt)
    n = T // ratio
    hf = h.float().view(B, T, D)
    ref = hf[:, :n * ratio].reshape(B, n, ratio, D).double().mean(2)
    assert means.shape == (B * n, D)
    assert torch.allclose(means.float().cpu().view(B, n, D), ref.float(), rtol=8e-3, atol=1e-6)
    assert torch.allclose(psum.cpu(), hf[:, n * ratio:].sum(1), atol=1e-4)
    assert torch.equal(pcnt.cpu(), torch.full((B,), T - n * ratio, dtype=torch.int32))


def test_pool_step_commit_and_fill():
    B, D, Kw, C, ratio = 4, 256, 128, 6, 3
    g = torch.Generator().manual_seed(3)
    psum = torch.zeros(B, D).cuda()
    pcnt = torch.tensor([0, 1, 2, 0], dtype=torch.int32).cuda()
    mk = torch.zeros(B, C, Kw, dtype=torch.bfloat16).cuda()
    mv = torch.zeros(B, C, D, dtype=torch.bfloat16).cuda()
    mtag = torch.zeros(B, C, dtype=torch.int32).cuda()
    mcount = torch.zeros(B, dtype=torch.int32).cuda()
    ref_sum, ref_cnt = torch.zeros(B, D, dtype=torch.float64), pcnt.cpu().long().clone()
    entries = [[] for _ in range(B)]
    for step in range(10):
        h = _bf(B, D, gen=g)
        pos = torch.full((B,), 20 + step, dtype=torch.int32)
        mean, emit = ops().cmp_pool_step(h.cuda(), psum, pcnt, ratio)
        ref_sum += h.double()
        ref_cnt += 1
        done = ref_cnt >= ratio
        assert torch.allclose(mean.float().cpu(), (ref_sum / ref_cnt[:, None]).float(), rtol=8e-3,
                              atol=1e-6)
        assert torch.equal(emit.cpu().bool(), done)
        kv = _bf(B, Kw + D, gen=g)
        ops().cmp_commit(kv.cuda(), emit, pos.cuda(), mk, mv, mtag, mcount)
        for b in range(B):
            if done[b]:
                entries[b].append((kv[b], 20 + step))
        ref_sum[done] = 0
        ref_cnt[done] = 0
        assert torch.equal(pcnt.cpu().long(), ref_cnt)
    for b in range(B):
        assert int(mcount[b]) == len(entries[b])
        for i, (row, p) in enumerate(entries[b]):
            s = i % C
            if i < len(entries[b]) - C:
                continue           # overwritten by a later summary
            assert torch.equal(mk[b, s].cpu(), row[:Kw]) and torch.equal(mv[b, s].cpu(), row[Kw:])
            assert int(mtag[b, s]) == p + 1
    # prefill fill: the last min(n, C) summaries into slots i % C
    n = 9
    kv = _bf(B * n, Kw + D, gen=g)
    mk.zero_(), mv.zero_(), mtag.zero_(), mcount.zero_()
    ops().cmp_memory_fill(kv.cuda(), B, n, ratio, mk, mv, mtag, mcount)
    for b in range(B):
        assert int(mcount[b]) == n
        for i in range(n - C, n):
            assert torch.equal(mk[b, i % C].cpu(), kv[b * n + i, :Kw])
            assert torch.equal(mv[b, i % C].cpu(), kv[b * n + i, Kw:])
            assert int(mtag[b, i % C]) == (i + 1) * ratio
    # ring fill: the last min(T, W) rows into slots t % W
    T, W = 11, 4
    src = _bf(B * T, 2 * Kw, gen=g)
    ring = torch.zeros(B, W, Kw, dtype=torch.bfloat16).cuda()
    ops().cmp_ring_fill(src.cuda()[:, Kw:], B, T, ring)
    for b in range(B):
        for t in range(T - W, T):
            assert torch.equal(ring[b, t % W].cpu(), src[b * T + t, Kw:])
