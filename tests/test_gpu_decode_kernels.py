"""GPU parity of the decode-path kernels against the CPU oracle / fp32 torch.

Tolerances (north star): bf16 outputs max-abs 2e-2 and rel-L2 1e-2; the fp32
GDN state rel-L2 1e-4; indices and permutations exact.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.attention import banded_attention_decode
from oracle.gdn import gdn_step as gdn_step_ref
from oracle.moe import moe_grouped
from oracle.router import moe_permute, rmsnorm, router_logits, router_topk

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2, STATE_REL_L2 = 2e-2, 1e-2, 1e-4


def ops():
    from hybrid_llm_amd import ops as o
    return o


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float(torch.linalg.norm(a - b) / torch.linalg.norm(b).clamp_min(1e-30))


def close_bf16(got, ref):
    got = got.float().cpu()
    assert float((got - ref).abs().max()) <= MAX_ABS, float((got - ref).abs().max())
    assert rel_l2(got, ref) <= REL_L2, rel_l2(got, ref)


def _bf(t):
    return t.to(torch.bfloat16)


# ---------------------------------------------------------------- linear
@pytest.mark.parametrize("M,N,K", [(64, 3072, 1024), (64, 1024, 1024), (1, 4112, 1024),
                                   (5, 32000, 1024), (64, 1040, 256), (130, 512, 512),
                                   (17, 16, 2048),
                                   # M >= 256: MFMA tiles, incl. partial m/n tiles
                                   (256, 1024, 1024), (300, 4112, 1024), (1000, 1040, 256),
                                   (257, 16, 512), (4096, 1024, 1024),
                                   # wide tiles with a narrow column tail (16 / 64 columns)
                                   # run as two launches; an 80-column tail stays in one
                                   (4096, 4112, 1024), (4000, 4160, 256), (4096, 4176, 256)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
@pytest.mark.parametrize("layout", [0, 1])
def test_linear_epilogues(M, N, K, epi, layout):
    g = torch.Generator().manual_seed(M * N + K + epi)
    x = _bf(torch.randn(M, K, generator=g))
    w = _bf(torch.randn(N, K, generator=g) * 0.02)
    ref = x.float() @ w.float().t()
    wg = w.cuda() if layout == 0 else ops().pack_weights(w.cuda())
    if epi == 0:
        out = ops().linear(x.cuda(), wg, epilogue=0, layout=layout)
        close_bf16(out, ref)
        return
    if epi == 1:
        out = ops().linear(x.cuda(), wg, epilogue=1, layout=layout)
        assert torch.allclose(out.cpu(), ref, atol=1e-4, rtol=1e-4)
        return
    base = torch.randn(M, N, generator=g)
    aux = torch.rand(M, N, generator=g)
    out = base.clone().cuda()
    ops().linear(x.cuda(), wg, out=out, epilogue=epi, aux=aux.cuda() if epi == 3 else None,
                 layout=layout)
    expect = base + (ref * aux if epi == 3 else ref)
    assert torch.allclose(out.cpu(), expect, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("M,N,K", [(64, 1024, 1024), (64, 1024, 2048), (1, 4112, 256),
                                   (37, 1040, 512)])
@pytest.mark.parametrize("layout", [0, 1])
def test_linear_partial_products(M, N, K, layout):
    """Epilogue 4: slice s is the product over the K block [256s, 256s+256),
    and folding the slices in order is the residual-add epilogue bit for bit
    (both sum the same 256-wide block products in K order)."""
    g = torch.Generator().manual_seed(M + N + K)
    x = _bf(torch.randn(M, K, generator=g))
    w = _bf(torch.randn(N, K, generator=g) * 0.02)
    wg = w.cuda() if layout == 0 else ops().pack_weights(w.cuda())
    parts = ops().linear(x.cuda(), wg, epilogue=ops().EPI_PARTIAL_F32, layout=layout)
    assert parts.shape == (K // 256, M, N)
    for s in range(K // 256):
        ref = x[:, 256 * s:256 * s + 256].float() @ w[:, 256 * s:256 * s + 256].float().t()
        assert torch.allclose(parts[s].cpu(), ref, atol=1e-4, rtol=1e-4), s
    base = torch.randn(M, N, generator=g).cuda()
    want = base.clone()
    ops().linear(x.cuda(), wg, out=want, epilogue=ops().EPI_RESID_ADD, layout=layout)
    folded = parts[0].clone()
    for s in range(1, K // 256):
        folded += parts[s]
    assert torch.equal(base + folded, want)


def test_pack_layout_closed_form():
    # tile j, lane l, element e of block (nb, kb) = W[16nb + l%16][256kb + 32j + 8(l//16) + e]
    N, K = 32, 512
    w = torch.arange(N * K, dtype=torch.float32).view(N, K)
    w = (w % 251).to(torch.bfloat16)
    p = ops().pack_weights(w.cuda()).cpu().view(N // 16, K // 256, 8, 64, 8)
    for nb in range(N // 16):
        for kb in range(K // 256):
            for j in range(8):
                for lane in (0, 5, 17, 63):
                    row = 16 * nb + lane % 16
                    col = 256 * kb + 32 * j + 8 * (lane // 16)
                    assert torch.equal(p[nb, kb, j, lane], w[row, col:col + 8])
    assert torch.equal(torch.sort(p.flatten().float()).values, torch.sort(w.flatten().float()).values)


def test_linear_empty_and_deterministic():
    x = _bf(torch.randn(64, 1024)).cuda()
    w = _bf(torch.randn(3072, 1024) * 0.02).cuda()
    a = ops().linear(x, w, epilogue=1)
    b = ops().linear(x, w, epilogue=1)
    assert torch.equal(a, b)
    ops().linear(x[:0], w, epilogue=1)


# ---------------------------------------------------------------- MoE
def _c2_weights(E=24, D=1024, H=2048, seed=0):
    g = torch.Generator().manual_seed(seed)
    wg = _bf(torch.randn(E, H, D, generator=g) * 0.02)
    wu = _bf(torch.randn(E, H, D, generator=g) * 0.02)
    wd = _bf(torch.randn(E, D, H, generator=g) * 0.02)
    wr = torch.randn(E, D, generator=g) * 0.02
    return wg, wu, wd, wr


@pytest.mark.parametrize("T,layout", [(64, 0), (64, 1), (1, 1), (300, 1), (4096, 0), (4096, 1)])
def test_moe_layer_c2(T, layout):
    wg, wu, wd, wr = _c2_weights()
    x = _bf(torch.randn(T, 1024, generator=torch.Generator().manual_seed(T)))
    wgu, wdn = torch.cat([wg, wu], 1).cuda(), wd.cuda()
    if layout == 1:
        wgu, wdn = ops().pack_weights(wgu), ops().pack_weights(wdn)
    res = ops().moe_forward(x.cuda(), wr.cuda(), wgu, wdn, 2, layout=layout)
    idx = res["idx"].cpu().numpy()
    logits = router_logits(x.float(), wr)
    ref_idx, _ = router_topk(logits, 2)
    # indices exact wherever the oracle's own top-2/top-3 margin is not a near tie
    v = torch.sort(logits, dim=-1, descending=True).values
    safe = ((v[:, 1] - v[:, 2]) > 1e-4).numpy()
    assert np.array_equal(idx[safe], ref_idx[safe])
    perm = moe_permute(idx.reshape(-1), 24)
    for key in ("counts", "offsets", "sorted_routes", "route_pos"):
        assert np.array_equal(res["perm"][key].cpu().numpy(), perm[key]), key
    # the output on the kernel's own routing, oracle math in fp32
    ref = moe_grouped(x.float(), idx, res["gates"].cpu(), wg, wu, wd,
                      act_round=lambda t: t.to(torch.bfloat16).float())
    close_bf16(res["out"], ref)


def test_moe_all_routes_to_one_expert():
    wg, wu, wd, _ = _c2_weights(E=4, D=256, H=512, seed=3)
    T, k = 200, 2
    x = _bf(torch.randn(T, 256, generator=torch.Generator().manual_seed(4)))
    idx = torch.full((T, k), 2, dtype=torch.int32)
    idx[:, 1] = 1
    gates = torch.full((T, k), 0.5)
    perm = ops().moe_permute(idx.view(-1).cuda(), 4)
    act, y = ops().moe_experts(x.cuda(), perm, gates.cuda(), torch.cat([wg, wu], 1).cuda(),
                               wd.cuda())
    out = ops().moe_combine(y, perm["route_pos"], T, k)
    ref = moe_grouped(x.float(), idx.numpy(), gates, wg, wu, wd,
                      act_round=lambda t: t.to(torch.bfloat16).float())
    close_bf16(out, ref)


# ---------------------------------------------------------------- attention decode
@pytest.mark.parametrize("B,H,W,hd,fill", [(64, 16, 2048, 64, "full"), (4, 4, 128, 64, "ragged"),
                                           (3, 2, 256, 128, "ragged"), (2, 2, 96, 64, "ragged")])
def test_attn_decode(B, H, W, hd, fill):
    g = torch.Generator().manual_seed(B * W + hd)
    q = _bf(torch.randn(B, H, hd, generator=g))
    kn = _bf(torch.randn(B, H, hd, generator=g))
    vn = _bf(torch.randn(B, H, hd, generator=g))
    kc = _bf(torch.randn(B, H, W, hd, generator=g))
    vc = _bf(torch.randn(B, H, W, hd, generator=g))
    if fill == "full":
        pos = torch.full((B,), W, dtype=torch.int32)        # cache full: ring wraps
    else:
        pos = torch.tensor([0, 1, W - 1, W, 3 * W + 5, W // 2][:B], dtype=torch.int32)
        # slots past pos are garbage in a real cache: plant NaN there
        for b in range(B):
            if int(pos[b]) + 1 < W:
                kc[b, :, int(pos[b]) + 1:] = float("nan")
                vc[b, :, int(pos[b]) + 1:] = float("nan")
    kcg, vcg = kc.cuda(), vc.cuda()
    out = ops().banded_attn_decode(q.cuda(), kn.cuda(), vn.cuda(), kcg, vcg, pos.cuda())
    ref, kref, vref = banded_attention_decode(q, kn, vn, kc, vc, pos.long())
    close_bf16(out, ref)
    assert torch.equal(kcg.cpu().view(torch.int16), kref.view(torch.int16))
    assert torch.equal(vcg.cpu().view(torch.int16), vref.view(torch.int16))


def test_attn_decode_from_fused_projection_view():
    B, H, hd, W = 8, 4, 64, 64
    g = torch.Generator().manual_seed(11)
    qkv = _bf(torch.randn(B, 3 * H * hd, generator=g))
    kc = _bf(torch.randn(B, H, W, hd, generator=g))
    vc = _bf(torch.randn(B, H, W, hd, generator=g))
    pos = torch.arange(B, dtype=torch.int32) * 9
    q, kn, vn = (qkv[:, i * H * hd:(i + 1) * H * hd].view(B, H, hd) for i in range(3))
    qg = qkv.cuda()
    qq, kk, vv = (qg[:, i * H * hd:(i + 1) * H * hd].view(B, H, hd) for i in range(3))
    out = ops().banded_attn_decode(qq, kk, vv, kc.cuda(), vc.cuda(), pos.cuda())
    ref, _, _ = banded_attention_decode(q, kn, vn, kc, vc, pos.long())
    close_bf16(out, ref)


@pytest.mark.parametrize("B,H,hd,W,P", [(64, 16, 64, 2048, 4), (5, 3, 128, 100, 2),
                                        (1, 2, 64, 16, 1), (7, 4, 64, 64, 8)])
def test_attn_decode_from_partial_products(B, H, hd, W, P):
    # q/k/v as per-K-block partial products [P, B, 3 H hd]: the kernel sums the
    # slices in order and rounds to bf16, so the step equals the bf16 entry
    # point on that sum bit for bit (output and both caches)
    g = torch.Generator().manual_seed(B * 31 + P)
    Hhd = H * hd
    parts = torch.randn(P, B, 3 * Hhd, generator=g) / P ** 0.5  # sums of unit variance
    acc = parts[0].clone()
    for s in range(1, P):
        acc += parts[s]
    qkv = acc.to(torch.bfloat16)
    kc = _bf(torch.randn(B, H, W, hd, generator=g))
    vc = _bf(torch.randn(B, H, W, hd, generator=g))
    pos = torch.randint(0, 3 * W, (B,), generator=g, dtype=torch.int32)
    q, kn, vn = (qkv[:, i * Hhd:(i + 1) * Hhd].reshape(B, H, hd).contiguous() for i in range(3))
    kc1, vc1, kc2, vc2 = kc.cuda(), vc.cuda(), kc.cuda(), vc.cuda()
    out1 = ops().banded_attn_decode(q.cuda(), kn.cuda(), vn.cuda(), kc1, vc1, pos.cuda())
    out2 = ops().banded_attn_decode_parts(parts.cuda(), Hhd, 2 * Hhd, kc2, vc2, pos.cuda())
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc2.view(torch.int16))
    ref, _, _ = banded_attention_decode(q, kn, vn, kc, vc, pos.long())
    close_bf16(out2, ref)


def test_attn_decode_parts_after_projection():
    # the engine's path: linear(..., EPI_PARTIAL_F32) then the parts entry
    # equals the bf16 projection then the bf16 entry, bit for bit
    B, H, hd, W, D = 64, 16, 64, 256, 1024
    g = torch.Generator().manual_seed(5)
    x = _bf(torch.randn(B, D, generator=g)).cuda()
    w = ops().pack_weights(_bf(torch.randn(3 * H * hd, D, generator=g) * 0.03).cuda())
    kc = _bf(torch.randn(B, H, W, hd, generator=g)).cuda()
    vc = _bf(torch.randn(B, H, W, hd, generator=g)).cuda()
    pos = torch.randint(0, 2 * W, (B,), generator=g, dtype=torch.int32).cuda()
    qkv = ops().linear(x, w, layout=ops().LAYOUT_PACKED)
    q, kn, vn = (qkv[:, i * H * hd:(i + 1) * H * hd].view(B, H, hd) for i in range(3))
    kc1, vc1 = kc.clone(), vc.clone()
    out1 = ops().banded_attn_decode(q, kn, vn, kc1, vc1, pos)
    parts = ops().linear(x, w, epilogue=ops().EPI_PARTIAL_F32, layout=ops().LAYOUT_PACKED)
    out2 = ops().banded_attn_decode_parts(parts, H * hd, 2 * H * hd, kc, vc, pos)
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    assert torch.equal(kc1.view(torch.int16), kc.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc.view(torch.int16))


# ---------------------------------------------------------------- GDN step
@pytest.mark.parametrize("B,H,d,with_gate", [(64, 16, 128, False), (64, 16, 64, True),
                                             (3, 2, 64, False)])
def test_gdn_step(B, H, d, with_gate):
    g = torch.Generator().manual_seed(B + d)
    q = _bf(F.normalize(torch.randn(B, H, d, generator=g), dim=-1))
    k = _bf(F.normalize(torch.randn(B, H, d, generator=g), dim=-1))
    v = _bf(torch.randn(B, H, d, generator=g))
    beta = torch.sigmoid(torch.randn(B, H, generator=g))
    gd = torch.exp(-F.softplus(torch.randn(B, H, generator=g)))
    gate = _bf(torch.rand(B, H, d, generator=g)) if with_gate else None
    S0 = torch.randn(B, H, d, d, generator=g) * 0.1
    S = S0.cuda()
    out = ops().gdn_step(q.cuda(), k.cuda(), v.cuda(), beta.cuda(), gd.cuda(), S,
                         None if gate is None else gate.cuda())
    o_ref, S_ref = gdn_step_ref(q.float(), k.float(), v.float(), beta, gd, S0,
                                None if gate is None else gate.float())
    assert rel_l2(S, S_ref) <= STATE_REL_L2
    close_bf16(out, o_ref)


def test_gdn_step_fused_projection():
    B, H, d = 16, 4, 64
    g = torch.Generator().manual_seed(5)
    ld = 4 * H * d + H + 12  # padded row
    proj = torch.randn(B, ld, generator=g)
    bb = torch.randn(H, generator=g) * 0.1
    decay = torch.full((H,), 2.0)
    S0 = torch.randn(B, H, d, d, generator=g) * 0.1
    S = S0.cuda()
    out = ops().gdn_step_fused(proj.cuda(), bb.cuda(), decay.cuda(), S)
    HK = H * d
    q = proj[:, :HK].view(B, H, d)
    k = proj[:, HK:2 * HK].view(B, H, d)
    v = proj[:, 2 * HK:3 * HK].view(B, H, d)
    gate = torch.sigmoid(proj[:, 3 * HK:4 * HK]).view(B, H, d)
    beta = torch.sigmoid(proj[:, 4 * HK:4 * HK + H] + bb)
    q = q * torch.rsqrt((q * q).sum(-1, keepdim=True).clamp_min(1e-12))
    k = k * torch.rsqrt((k * k).sum(-1, keepdim=True).clamp_min(1e-12))
    o_ref, S_ref = gdn_step_ref(q, k, v, beta, torch.sigmoid(decay).expand(B, H), S0, gate)
    assert rel_l2(S, S_ref) <= STATE_REL_L2
    close_bf16(out.view(B, H, d), o_ref)


@pytest.mark.parametrize("nparts", [2, 4, 8])
def test_gdn_step_fused_partial_products(nparts):
    """Projection slices [P, B, ld] are summed in slice order by the step:
    the same outputs and state as the step on the summed row, bit for bit."""
    B, H, d = 64, 16, 64
    g = torch.Generator().manual_seed(nparts)
    ld = 4 * H * d + H + 16
    parts = (torch.randn(nparts, B, ld, generator=g) * 0.5).cuda()
    bb = (torch.randn(H, generator=g) * 0.1).cuda()
    decay = torch.randn(H, generator=g).cuda()
    S0 = (torch.randn(B, H, d, d, generator=g) * 0.1).cuda()
    summed = parts[0].clone()
    for p in range(1, nparts):
        summed += parts[p]
    S1, S2 = S0.clone(), S0.clone()
    o1 = ops().gdn_step_fused(parts, bb, decay, S1)
    o2 = ops().gdn_step_fused(summed, bb, decay, S2)
    assert torch.equal(o1, o2) and torch.equal(S1, S2)


# ---------------------------------------------------------------- glue
def test_rmsnorm_embed_conv():
    g = torch.Generator().manual_seed(8)
    x = torch.randn(64, 1024, generator=g) * 3
    w = torch.rand(1024, generator=g) + 0.5
    close_bf16(ops().rmsnorm(x.cuda(), w.cuda()), rmsnorm(x, w))
    table = _bf(torch.randn(1000, 256, generator=g))
    tok = torch.randint(0, 1000, (33,), generator=g, dtype=torch.int32)
    assert torch.equal(ops().embed(tok.cuda(), table.cuda()).cpu(), table[tok.long()].float())
    B, D = 5, 256
    h = _bf(torch.randn(B, D, generator=g))
    hist = _bf(torch.randn(B, 3, D, generator=g))
    cw = torch.randn(D, 4, generator=g) * 0.3
    hg = hist.cuda()
    out = ops().gdn_conv_gate(h.cuda(), hg, cw.cuda())
    win = torch.cat([hist.float(), h.float()[:, None]], 1)
    ref = torch.sigmoid((win * cw.t()[None]).sum(1))
    assert torch.allclose(out.cpu(), ref, atol=1e-6)
    assert torch.equal(hg.cpu().view(torch.int16), win[:, 1:].to(torch.bfloat16).view(torch.int16))


# ---------------------------------------------------------------- fused decode kernels
@pytest.mark.parametrize("T,D,E,k", [(64, 1024, 24, 2), (1, 256, 8, 2), (200, 512, 40, 4),
                                     # sequences: the 32-token block kernel (fp32 MFMA logits)
                                     (4096, 1024, 24, 2), (300, 256, 8, 2), (512, 512, 32, 4),
                                     (260, 512, 40, 2)])
def test_moe_route_decode_equals_unfused(T, D, E, k):
    g = torch.Generator().manual_seed(T + D)
    x = (torch.randn(T, D, generator=g) * 2).cuda()
    fw = (torch.rand(D, generator=g) + 0.5).cuda()
    rw = (torch.rand(D, generator=g) + 0.5).cuda()
    wr = (torch.randn(E, D, generator=g) * 0.02).cuda()
    fused = ops().moe_route_decode(x, fw, rw, wr, k)
    h2 = ops().rmsnorm(x, fw)
    assert torch.equal(fused["h"], h2)
    idx, gates, lg = ops().router_topk(h2, wr, k, rw, return_logits=True)
    # the two kernels sum the logits in different orders: ids must agree
    # wherever the k-th / (k+1)-th gap is above fp32 rounding noise
    srt = torch.sort(lg, -1, descending=True).values
    ok = ((srt[:, k - 1] - srt[:, k]) > 1e-5) if k < E else torch.ones(T, dtype=torch.bool, device=lg.device)
    assert ok.float().mean() > 0.95
    assert torch.equal(fused["idx"][ok], idx[ok])
    assert torch.allclose(fused["gates"][ok], gates[ok], atol=1e-5)
    # the permutation is a function of the fused ids: compare with the standalone kernel
    perm = ops().moe_permute(fused["idx"].view(-1), E)
    for key in ("counts", "offsets", "sorted_routes", "route_pos"):
        assert torch.equal(fused[key], perm[key]), key
    # and against the oracle: exact ids wherever the oracle margin is not a near tie
    logits = router_logits(h2.float().cpu(), wr.cpu(), rw.cpu())
    ref_idx, _ = router_topk(logits, k)
    srt = torch.sort(logits, -1, descending=True).values
    safe = ((srt[:, k - 1] - srt[:, k]) > 1e-4).numpy() if k < E else np.ones(T, bool)
    assert np.array_equal(fused["idx"].cpu().numpy()[safe], ref_idx[safe])


@pytest.mark.parametrize("nparts,gated", [(4, False), (4, True), (1, False), (8, True)])
def test_moe_route_decode_folds_partials(nparts, gated):
    """x += sum_p parts[p] (p ascending; gated: one fma per element with the
    gate), written back to x, then the same norm/router as on the folded x."""
    T, D, E, k = 64, 1024, 24, 2
    g = torch.Generator().manual_seed(nparts * 2 + gated)
    x0 = (torch.randn(T, D, generator=g) * 2).cuda()
    parts = (torch.randn(nparts, T, D, generator=g) * 0.5).cuda()
    gate = torch.rand(T, D, generator=g).cuda() if gated else None
    fw = (torch.rand(D, generator=g) + 0.5).cuda()
    rw = (torch.rand(D, generator=g) + 0.5).cuda()
    wr = (torch.randn(E, D, generator=g) * 0.02).cuda()
    acc = parts[0].clone()
    for p in range(1, nparts):
        acc += parts[p]
    if gated:
        want = (acc.double() * gate.double() + x0.double()).float().cpu()
    else:
        want = (x0 + acc).cpu()
    x = x0.clone()
    got = ops().moe_route_decode(x, fw, rw, wr, k, parts=parts, gate=gate)
    if gated:
        # fma rounds once: within one fp32 ulp of the exactly rounded value
        assert torch.allclose(x.cpu(), want, rtol=2 ** -23, atol=1e-30)
    else:
        assert torch.equal(x.cpu(), want)
    ref = ops().moe_route_decode(x.clone(), fw, rw, wr, k)
    for key in ("h", "idx", "gates", "counts", "offsets", "sorted_routes", "route_pos"):
        assert torch.equal(got[key], ref[key]), key


@pytest.mark.parametrize("D", [256, 1024])
def test_embed_norm_and_combine_norm(D):
    g = torch.Generator().manual_seed(D)
    B, k, V = 64, 2, 1000
    table = _bf(torch.randn(V, D, generator=g)).cuda()
    tok = torch.randint(0, V, (B,), generator=g, dtype=torch.int32).cuda()
    w = (torch.rand(D, generator=g) + 0.5).cuda()
    x = torch.empty(B, D, device="cuda")
    h = torch.empty(B, D, dtype=torch.bfloat16, device="cuda")
    ops().embed_norm(tok, table, w, x, h)
    assert torch.equal(x, ops().embed(tok, table))
    assert torch.equal(h, ops().rmsnorm(x, w))
    y = torch.randn(B * k, D, generator=g).cuda()
    rp = torch.randperm(B * k, generator=g).to(torch.int32).cuda()
    x0 = x.clone()
    ops().moe_combine_norm(y, rp, x, h, w, k)
    ref = x0.clone()
    ops().moe_combine(y, rp, B, k, out=ref, mode=2)
    assert torch.equal(x, ref)
    assert torch.equal(h, ops().rmsnorm(ref, w))
    x1 = x.clone()
    ops().moe_combine_norm(y, rp, x, None, None, k)   # no norm requested
    ops().moe_combine(y, rp, B, k, out=x1, mode=2)
    assert torch.equal(x, x1)


def test_gdn_step_with_fused_conv_gate():
    B, H, d, D = 8, 16, 64, 1024
    g = torch.Generator().manual_seed(9)
    proj = torch.randn(B, 4 * H * d + H, generator=g).cuda()
    bb = (torch.randn(H, generator=g) * 0.1).cuda()
    decay = torch.full((H,), 2.0).cuda()
    S = (torch.randn(B, H, d, d, generator=g) * 0.1).cuda()
    h = _bf(torch.randn(B, D, generator=g)).cuda()
    hist = _bf(torch.randn(B, 3, D, generator=g)).cuda()
    cw = (torch.randn(D, 4, generator=g) * 0.3).cuda()
    S2, hist2 = S.clone(), hist.clone()
    cg = torch.empty(B, D, device="cuda")
    o1 = ops().gdn_step_fused(proj, bb, decay, S, conv=(h, hist, cw, cg))
    o2 = ops().gdn_step_fused(proj, bb, decay, S2)
    cg2 = ops().gdn_conv_gate(h, hist2, cw)
    assert torch.equal(o1, o2) and torch.equal(S, S2)
    assert torch.equal(hist, hist2)
    assert torch.allclose(cg, cg2, atol=1e-6)


@pytest.mark.parametrize("T,E,D,H", [(64, 24, 512, 512), (1, 8, 512, 512), (300, 24, 512, 512),
                                     # C5 decode shape: down K = 2048 is two pieces per wave
                                     (64, 24, 1024, 2048),
                                     # down K = 1024 and 4096: one and four pieces per wave
                                     (48, 12, 512, 1024), (32, 8, 256, 4096),
                                     # about 16 routes per expert: several 16-route chunks
                                     (64, 8, 512, 512), (20, 24, 256, 512)])
def test_moe_routed_equals_sorted(T, E, D, H):
    """Route-indexed experts (no permutation) match the sorted path row for
    row: y_routed[r] vs y_sorted[route_pos[r]].  At decode sizes (T*k <= 16*E)
    both run the same weight-streaming configuration and agree bit for bit;
    above that the sorted path runs the tiled MFMA GEMMs (another summation
    order), so the rows agree to bf16/fp32 rounding."""
    wg, wu, wd, wr = _c2_weights(E=E, D=D, H=H, seed=T)
    x = _bf(torch.randn(T, D, generator=torch.Generator().manual_seed(T))).cuda()
    wgu = ops().pack_weights(torch.cat([wg, wu], 1).cuda())
    wdn = ops().pack_weights(wd.cuda())
    idx, gates = ops().router_topk(x, wr.cuda(), 2)
    perm = ops().moe_permute(idx.view(-1), E)
    act_s, y_s = ops().moe_experts(x, perm, gates, wgu, wdn, layout=1)
    act_r, y_r = ops().moe_experts_routed(x, idx, gates, wgu, wdn, layout=1)
    rp = perm["route_pos"].long()
    xs = torch.randn(T, D, device="cuda")
    xr = xs.clone()
    ops().moe_combine_norm(y_s, perm["route_pos"], xs, None, None, 2)
    ops().moe_combine_norm(y_r, None, xr, None, None, 2)
    if T * 2 <= 16 * E:
        assert torch.equal(y_r, y_s[rp])
        assert torch.equal(act_r, act_s[rp])
        assert torch.equal(xs, xr)
    else:
        assert (act_r.float() - act_s[rp].float()).abs().max() <= 2e-2 * act_s.float().abs().max()
        assert rel_l2(y_r, y_s[rp]) <= 1e-2
        assert rel_l2(xr, xs) <= 1e-3
