"""GPU parity: per-sequence GDN resets (a new document starting inside a batch
row or inside a prompt) against the sequential oracle with its reset mask.

The reference zeroes the recurrent carry where reset_mask is set
(model/layers/gated_deltanet.py:138-142) and masks conv taps that would
cross the reset (gated_deltanet.py:56-78).  Tolerances as for the plain
kernels: fp32 state rel-L2 1e-4; bf16 outputs max-abs 2e-2, rel-L2 1e-2.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle.gdn import causal_conv_reset, gdn_sequential
from oracle.gdn import gdn_step as gdn_step_ref

pytestmark = pytest.mark.gpu

STATE_REL_L2, MAX_ABS, REL_L2 = 1e-4, 2e-2, 1e-2


def ops():
    from hybrid_llm_amd import ops as o
    return o


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float(torch.linalg.norm(a - b) / torch.linalg.norm(b).clamp_min(1e-30))


def _inputs(B, T, H, d, seed, s0=0.5):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, d, generator=g), dim=-1).to(torch.bfloat16)
    k = F.normalize(torch.randn(B, T, H, d, generator=g), dim=-1).to(torch.bfloat16)
    v = torch.randn(B, T, H, d, generator=g).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    gd = torch.exp(-F.softplus(torch.randn(B, T, H, generator=g) - 2.0))   # slow decay
    S0 = torch.randn(B, H, d, d, generator=g) * s0
    return q, k, v, beta, gd, S0


def _prefill(q, k, v, beta, gd, S0, reset):
    S = S0.clone().cuda()
    out = ops().gdn_prefill(q.cuda(), k.cuda(), v.cuda(), beta.cuda(), gd.cuda(), S,
                            reset=None if reset is None else reset.cuda())
    torch.cuda.synchronize()
    return out.float().cpu(), S.cpu()


def _check(out, S, o_ref, S_ref):
    assert rel_l2(S, S_ref) <= STATE_REL_L2, rel_l2(S, S_ref)
    assert float((out - o_ref).abs().max()) <= MAX_ABS
    assert rel_l2(out, o_ref) <= REL_L2, rel_l2(out, o_ref)


# (row, position) resets: mid-chunk, on a chunk boundary, at t = 0, two in one
# chunk, adjacent, the last token; one row never resets.
CASES = {
    "mixed": (4, 200, 2, 64, [(0, 17), (1, 64), (1, 0), (2, 100), (2, 101), (2, 120),
                              (3, 199)]),
    "d128": (3, 150, 2, 128, [(0, 63), (0, 65), (2, 1), (2, 128)]),
    "short": (2, 5, 3, 64, [(0, 2), (1, 4)]),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_prefill_reset_matches_sequential(name):
    B, T, H, d, pts = CASES[name]
    print(f"prefill reset case {name}", flush=True)
    q, k, v, beta, gd, S0 = _inputs(B, T, H, d, T + d)
    reset = torch.zeros(B, T, dtype=torch.int32)
    for b, t in pts:
        reset[b, t] = 1
    o_ref, S_ref = gdn_sequential(q.float(), k.float(), v.float(), beta, gd, S0, reset=reset)
    out, S = _prefill(q, k, v, beta, gd, S0, reset)
    _check(out, S, o_ref, S_ref)
    # rows without a reset are bitwise what the plain entry computes
    out0, S_0 = _prefill(q, k, v, beta, gd, S0, None)
    free = [b for b in range(B) if not reset[b].any()]
    for b in free:
        assert torch.equal(out[b], out0[b]) and torch.equal(S[b], S_0[b])


def test_prefill_dense_random_resets():
    B, T, H, d = 3, 300, 2, 128
    q, k, v, beta, gd, S0 = _inputs(B, T, H, d, 77)
    reset = (torch.rand(B, T, generator=torch.Generator().manual_seed(3)) < 0.08).to(torch.int32)
    o_ref, S_ref = gdn_sequential(q.float(), k.float(), v.float(), beta, gd, S0, reset=reset)
    out, S = _prefill(q, k, v, beta, gd, S0, reset)
    _check(out, S, o_ref, S_ref)


def test_prefill_zero_mask_equals_plain_entry():
    q, k, v, beta, gd, S0 = _inputs(2, 130, 2, 64, 5)
    out1, S1 = _prefill(q, k, v, beta, gd, S0, torch.zeros(2, 130, dtype=torch.int32))
    out2, S2 = _prefill(q, k, v, beta, gd, S0, None)
    assert torch.equal(out1, out2) and torch.equal(S1, S2)


def test_prefill_reset_then_continue():
    """A prompt split in two prefill calls with a reset inside the second part
    equals one call over the whole prompt (the state carries across calls)."""
    B, T, H, d = 2, 180, 2, 64
    q, k, v, beta, gd, S0 = _inputs(B, T, H, d, 21)
    reset = torch.zeros(B, T, dtype=torch.int32)
    reset[0, 150] = 1
    reset[1, 70] = 1
    whole, Sw = _prefill(q, k, v, beta, gd, S0, reset)
    S = S0.clone().cuda()
    parts = []
    for a, b in [(0, 100), (100, T)]:
        sl = slice(a, b)
        parts.append(ops().gdn_prefill(q[:, sl].contiguous().cuda(), k[:, sl].contiguous().cuda(),
                                       v[:, sl].contiguous().cuda(), beta[:, sl].contiguous().cuda(),
                                       gd[:, sl].contiguous().cuda(), S,
                                       reset=reset[:, sl].contiguous().cuda()).float().cpu())
    o_ref, S_ref = gdn_sequential(q.float(), k.float(), v.float(), beta, gd, S0, reset=reset)
    _check(torch.cat(parts, 1), S.cpu(), o_ref, S_ref)
    _check(whole, Sw, o_ref, S_ref)


def test_step_reset_rows():
    B, H, d = 8, 4, 128
    g = torch.Generator().manual_seed(12)
    q = F.normalize(torch.randn(B, H, d, generator=g), dim=-1).to(torch.bfloat16)
    k = F.normalize(torch.randn(B, H, d, generator=g), dim=-1).to(torch.bfloat16)
    v = torch.randn(B, H, d, generator=g).to(torch.bfloat16)
    gate = torch.rand(B, H, d, generator=g).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, H, generator=g))
    gd = torch.exp(-F.softplus(torch.randn(B, H, generator=g)))
    S0 = torch.randn(B, H, d, d, generator=g) * 0.5
    reset = torch.tensor([1, 0, 0, 1, 1, 0, 1, 0], dtype=torch.int32)
    S = S0.clone().cuda()
    out = ops().gdn_step(q.cuda(), k.cuda(), v.cuda(), beta.cuda(), gd.cuda(), S, gate.cuda(),
                         reset=reset.cuda())
    o_ref, S_ref = gdn_step_ref(q.float(), k.float(), v.float(), beta, gd, S0, gate.float(),
                                reset=reset.bool())
    assert rel_l2(S, S_ref) <= STATE_REL_L2
    assert float((out.float().cpu() - o_ref).abs().max()) <= MAX_ABS
    # equals the plain step on a state whose reset rows were cleared
    S2 = S0.clone()
    S2[reset.bool()] = 0
    S2 = S2.cuda()
    out2 = ops().gdn_step(q.cuda(), k.cuda(), v.cuda(), beta.cuda(), gd.cuda(), S2, gate.cuda())
    assert torch.equal(out.cpu(), out2.cpu()) and torch.equal(S.cpu(), S2.cpu())


def test_step_fused_reset_clears_state_and_conv_history():
    B, H, d, D = 8, 16, 64, 1024
    g = torch.Generator().manual_seed(19)
    proj = torch.randn(B, 4 * H * d + H, generator=g).cuda()
    bb = (torch.randn(H, generator=g) * 0.1).cuda()
    decay = torch.full((H,), 2.0).cuda()
    S = (torch.randn(B, H, d, d, generator=g) * 0.5).cuda()
    h = torch.randn(B, D, generator=g).to(torch.bfloat16).cuda()
    hist = torch.randn(B, 3, D, generator=g).to(torch.bfloat16).cuda()
    cw = (torch.randn(D, 4, generator=g) * 0.3).cuda()
    reset = torch.tensor([0, 1, 1, 0, 0, 0, 1, 0], dtype=torch.int32)
    S2, hist2 = S.clone(), hist.clone()
    S2[reset.bool().cuda()] = 0
    hist2[reset.bool().cuda()] = 0
    cg = torch.empty(B, D, device="cuda")
    cg2 = torch.empty(B, D, device="cuda")
    o1 = ops().gdn_step_fused(proj, bb, decay, S, conv=(h, hist, cw, cg), reset=reset.cuda())
    o2 = ops().gdn_step_fused(proj, bb, decay, S2, conv=(h, hist2, cw, cg2))
    assert torch.equal(o1, o2) and torch.equal(S, S2)
    assert torch.equal(hist, hist2) and torch.equal(cg, cg2)


@pytest.mark.parametrize("T", [1, 3, 17, 64])
def test_conv_gate_prefill_reset(T):
    B, D = 3, 512
    g = torch.Generator().manual_seed(40 + T)
    h = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    hist0 = torch.randn(B, 3, D, generator=g).to(torch.bfloat16)
    w = 0.5 * torch.randn(D, 4, generator=g)
    reset = torch.zeros(B, T, dtype=torch.int32)
    reset[0, 0] = 1                      # the whole history is discarded
    reset[1, T // 2] = 1
    reset[1, T - 1] = 1                  # a reset on the last token: history keeps one token
    hist = hist0.clone().cuda()
    got = ops().gdn_conv_gate_prefill(h.cuda(), hist, w.cuda(), reset=reset.cuda())
    conv, hist_ref = causal_conv_reset(h.float(), hist0.float(), w, reset)
    assert torch.allclose(got.cpu(), torch.sigmoid(conv), atol=1e-6)
    assert torch.equal(hist.cpu().float(), hist_ref)
    # token by token through the decode conv, clearing the history at each reset
    hs = hist0.clone().cuda()
    steps = []
    for t in range(T):
        hs[reset[:, t].bool().cuda()] = 0
        steps.append(ops().gdn_conv_gate(h[:, t].contiguous().cuda(), hs, w.cuda()))
    assert torch.equal(got.cpu(), torch.stack(steps, 1).cpu())
    assert torch.equal(hist.cpu(), hs.cpu())
    # an all-zero mask is the plain entry, bitwise
    h1, h2 = hist0.clone().cuda(), hist0.clone().cuda()
    a = ops().gdn_conv_gate_prefill(h.cuda(), h1, w.cuda(), reset=torch.zeros_like(reset).cuda())
    b = ops().gdn_conv_gate_prefill(h.cuda(), h2, w.cuda())
    assert torch.equal(a.cpu(), b.cpu()) and torch.equal(h1.cpu(), h2.cpu())
