"""GPU parity: banded causal attention prefill (MFMA) against the oracle.

Tolerance (north star, bf16 outputs): max-abs 2e-2, rel-L2 1e-2.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle.attention import banded_attention

pytestmark = pytest.mark.gpu


def ops():
    from hybrid_llm_amd import ops as o
    return o


def _qkv(B, T, H, hd, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, T, H, hd, generator=g).to(torch.bfloat16) for _ in range(3)]


def _check(out, ref):
    out = out.float().cpu()
    err = (out - ref).abs().max().item()
    rel = (torch.linalg.norm((out - ref).double()) / torch.linalg.norm(ref.double())).item()
    assert err <= 2e-2, err
    assert rel <= 1e-2, rel


@pytest.mark.parametrize("B,T,H,hd,W", [(1, 64, 1, 64, 16), (2, 300, 3, 64, 128),
                                        (1, 257, 2, 128, 64), (2, 130, 2, 64, 1),
                                        (1, 200, 2, 64, 1000), (1, 1024, 4, 64, 512),
                                        (3, 97, 1, 64, 33)])
def test_prefill_matches_oracle(B, T, H, hd, W):
    q, k, v = _qkv(B, T, H, hd, B * T + W)
    out = ops().banded_attn_prefill(q.cuda(), k.cuda(), v.cuda(), W)
    ref = banded_attention(q.float(), k.float(), v.float(), W)
    _check(out, ref)


def test_prefill_window_covering_sequence_is_causal_sdpa():
    q, k, v = _qkv(1, 333, 2, 64, 7)
    out = ops().banded_attn_prefill(q.cuda(), k.cuda(), v.cuda(), 333)
    ref = F.scaled_dot_product_attention(q.float().transpose(1, 2), k.float().transpose(1, 2),
                                         v.float().transpose(1, 2), is_causal=True).transpose(1, 2)
    _check(out, ref)


def test_prefill_c3_shape():
    """B=4, T=8192, H=16, hd=64, W=512."""
    q, k, v = _qkv(4, 8192, 16, 64, 3)
    out = ops().banded_attn_prefill(q.cuda(), k.cuda(), v.cuda(), 512)
    ref = banded_attention(q.float(), k.float(), v.float(), 512, block=512)
    _check(out, ref)


def test_prefill_deterministic_and_decode_consistent():
    """Prefill row t equals a decode step at position t over the same window."""
    B, T, H, hd, W = 2, 150, 2, 64, 64
    q, k, v = _qkv(B, T, H, hd, 11)
    a = ops().banded_attn_prefill(q.cuda(), k.cuda(), v.cuda(), W)
    b2 = ops().banded_attn_prefill(q.cuda(), k.cuda(), v.cuda(), W)
    assert torch.equal(a, b2)
    kc = torch.zeros(B, H, W, hd, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    for t in range(T):
        pos = torch.full((B,), t, dtype=torch.int32, device="cuda")
        od = ops().banded_attn_decode(q[:, t].cuda(), k[:, t].cuda(), v[:, t].cuda(), kc, vc, pos)
    assert (od.float() - a[:, T - 1].float()).abs().max().item() <= 2e-2
