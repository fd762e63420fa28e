"""GPU parity: the reference ABI's fp32 operator hooks, bound the way the
reference caller binds them (a fresh ctypes.CDLL of the library with the
argtypes of sample_standalone.py:2499-2508, raw pointers, c_int32 sizes)."""
import ctypes

import numpy as np
import pytest
import torch

from oracle.mhc import sinkhorn4
from oracle.moe import moe_selected_fp32

pytestmark = pytest.mark.gpu


def _hook(symbol):
    from hybrid_llm_amd import _lib
    lib = ctypes.CDLL(str(_lib.library_path()))
    sig = {
        "llmy_mhc_sinkhorn4": [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                               ctypes.c_void_p],
        "llmy_moe_selected_fp32": [*([ctypes.c_void_p] * 8), ctypes.c_int32, ctypes.c_int32,
                                   ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p],
    }[symbol]
    fn = getattr(lib, symbol)
    fn.argtypes = sig
    fn.restype = ctypes.c_int32
    return fn


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _run_moe(x, idx, prob, gate_up, down):
    E, H2, D = gate_up.shape
    H = H2 // 2
    k = idx.shape[1]
    act = torch.empty(k, H, device="cuda")
    ro = torch.empty(k, D, device="cuda")
    out = torch.empty(1, D, device="cuda")
    st = _hook("llmy_moe_selected_fp32")(
        _p(x), _p(idx), _p(prob), _p(gate_up), _p(down), _p(act), _p(ro), _p(out), D, H, E, k,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0
    torch.cuda.synchronize()
    return act.cpu().numpy(), ro.cpu().numpy(), out.cpu().numpy()[0]


@pytest.mark.parametrize("D,H,E,k", [(1024, 2048, 24, 2), (256, 512, 8, 2), (100, 50, 3, 3),
                                     (64, 16, 1, 1), (1024, 2048, 24, 8)])
def test_moe_selected_fp32(D, H, E, k):
    g = torch.Generator().manual_seed(D + H + k)
    x = torch.randn(1, D, generator=g)
    gate_up = torch.randn(E, 2 * H, D, generator=g) * 0.02
    down = torch.randn(E, D, H, generator=g) * 0.02
    idx = torch.randint(0, E, (1, k), generator=g, dtype=torch.int64)
    prob = torch.softmax(torch.randn(1, k, generator=g), -1)
    act, ro, out = _run_moe(x.cuda(), idx.cuda(), prob.cuda(), gate_up.cuda(), down.cuda())
    ra, rr, rout = moe_selected_fp32(x.numpy(), idx.numpy(), prob.numpy(), gate_up.numpy(),
                                     down.numpy())
    for got, ref in ((act, ra), (ro, rr), (out, rout)):
        assert np.abs(got - ref).max() <= 1e-5 + 1e-4 * np.abs(ref).max()


def test_moe_selected_out_of_range_id_contributes_zero():
    g = torch.Generator().manual_seed(1)
    D, H, E = 128, 64, 4
    x = torch.randn(1, D, generator=g)
    gate_up = torch.randn(E, 2 * H, D, generator=g) * 0.05
    down = torch.randn(E, D, H, generator=g) * 0.05
    idx = torch.tensor([[2, 9, -1]])
    prob = torch.tensor([[0.6, 0.3, 0.1]])
    act, ro, out = _run_moe(x.cuda(), idx.cuda(), prob.cuda(), gate_up.cuda(), down.cuda())
    assert not act[1:].any() and not ro[1:].any()
    _, _, rout = moe_selected_fp32(x.numpy(), idx.numpy(), prob.numpy(), gate_up.numpy(),
                                   down.numpy())
    assert np.allclose(out, rout, rtol=1e-4, atol=1e-6)


def test_moe_selected_rejects_bad_arguments_before_launch():
    fn = _hook("llmy_moe_selected_fp32")
    t = torch.zeros(4, device="cuda")
    args = [_p(t)] * 8
    assert fn(*args, 0, 8, 2, 1, None) == 1
    assert fn(None, *args[1:], 4, 8, 2, 1, None) == 1


@pytest.mark.parametrize("n,iters", [(1, 0), (1000, 20), (4097, 3), (64, 1)])
def test_sinkhorn4(n, iters):
    g = torch.Generator().manual_seed(n + iters)
    x = torch.randn(n, 4, 4, generator=g) * 2
    src = x.cuda()
    out = torch.empty_like(src)
    st = _hook("llmy_mhc_sinkhorn4")(_p(src), _p(out), n, iters,
                                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0
    ref = sinkhorn4(x.numpy(), iters)
    assert np.allclose(out.cpu().numpy(), ref, rtol=2e-5, atol=1e-6)
    # the reference's own status rules: empty or negative arguments are rejected
    fn = _hook("llmy_mhc_sinkhorn4")
    assert fn(_p(src), _p(out), 0, iters, None) == 1
    assert fn(_p(src), _p(out), n, -1, None) == 1
