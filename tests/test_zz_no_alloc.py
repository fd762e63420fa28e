"""The no-allocation GDN prefill entry (llmy_gdn_prefill_bf16_noalloc) against
the workspace entry it mirrors (llmy_gdn_prefill_bf16).

Both run the same kernels on the same inputs, so outputs and final states
must be equal bit for bit.  Two calls in a row per head size, the second with
a smaller input, so the second call reads the fixed workspace the first one
left behind.  Sizes past the fixed 64 MiB workspace are rejected with
hipErrorOutOfMemory before anything runs; a bad head size with
hipErrorInvalidValue.
"""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

OUT_OF_MEMORY = 2   # hipErrorOutOfMemory
INVALID_VALUE = 1   # hipErrorInvalidValue


def _lib():
    from hybrid_llm_amd import _lib as L
    return L.load()


def _inputs(B, T, H, d, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, d, device="cuda", generator=g), dim=-1).bfloat16()
    k = F.normalize(torch.randn(B, T, H, d, device="cuda", generator=g), dim=-1).bfloat16()
    v = torch.randn(B, T, H, d, device="cuda", generator=g).bfloat16()
    beta = torch.sigmoid(torch.randn(B, T, H, device="cuda", generator=g))
    gd = torch.exp(-F.softplus(torch.randn(B, T, H, device="cuda", generator=g)))
    S0 = torch.randn(B, H, d, d, device="cuda", generator=g) * 0.1
    return q, k, v, beta, gd, S0


def _ptrs(*ts):
    return [t.data_ptr() for t in ts]


@pytest.mark.parametrize("d,sizes", [(128, [(2, 1000, 8), (1, 300, 4)]),
                                     (64, [(4, 777, 16), (1, 65, 2)])])
def test_noalloc_matches_workspace_entry(d, sizes):
    lib = _lib()
    stream = torch.cuda.current_stream().cuda_stream
    for n, (B, T, H) in enumerate(sizes):
        print(f"[no-alloc] d={d} call {n}: B={B} T={T} H={H}", flush=True)
        q, k, v, beta, gd, S0 = _inputs(B, T, H, d, seed=10 * d + n)
        nb = int(lib.llmy_gdn_prefill_workspace_bytes(B, T, H, d, d))
        assert 0 < nb <= 64 << 20
        ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
        S_ref, S_new = S0.clone(), S0.clone()
        out_ref = torch.empty(B, T, H, d, dtype=torch.bfloat16, device="cuda")
        out_new = torch.full_like(out_ref, float("nan"))
        st = lib.llmy_gdn_prefill_bf16(*_ptrs(q, k, v, beta, gd, S_ref, out_ref, ws), nb,
                                       B, T, H, d, d, stream)
        assert st == 0, st
        st = lib.llmy_gdn_prefill_bf16_noalloc(*_ptrs(q, k, v, beta, gd, S_new, out_new),
                                               B, T, H, d, d, stream)
        assert st == 0, st
        torch.cuda.synchronize()
        assert torch.equal(out_new, out_ref)
        assert torch.equal(S_new, S_ref)
        assert not torch.equal(S_new, S0)


def test_noalloc_rejects_before_running():
    lib = _lib()
    stream = torch.cuda.current_stream().cuda_stream
    t = torch.zeros(64, device="cuda")  # any valid, aligned device buffer: nothing is launched
    p = t.data_ptr()
    # 832 chunks of 64 tokens x heads at dk = dv = 128: 68.4 MB of workspace
    B, T, H = 1, 64 * 52, 16
    assert lib.llmy_gdn_prefill_workspace_bytes(B, T, H, 128, 128) > 64 << 20
    assert lib.llmy_gdn_prefill_bf16_noalloc(p, p, p, p, p, p, p, B, T, H, 128, 128,
                                             stream) == OUT_OF_MEMORY
    assert lib.llmy_gdn_prefill_bf16_noalloc(p, p, p, p, p, p, p, 1, 64, 2, 96, 96,
                                             stream) == INVALID_VALUE
    assert lib.llmy_gdn_prefill_bf16_noalloc(None, p, p, p, p, p, p, 1, 64, 2, 64, 64,
                                             stream) == INVALID_VALUE
    assert lib.llmy_gdn_prefill_bf16_noalloc(p, p, p, p, p, p, p, 0, 64, 2, 64, 64, stream) == 0
    torch.cuda.synchronize()
    assert torch.count_nonzero(t) == 0
