"""Pins the mHC oracle (oracle/mhc.py): the reference module's own outputs on
seeded inputs (tests/golden/mhc_golden.npz, written by make_mhc_golden.py from
model/layers/mhc.py) and closed forms."""
import os

import numpy as np
import torch

from oracle.mhc import mhc_maps, mhc_read, mhc_write, sinkhorn4, sinkhorn_t

GOLD = os.path.join(os.path.dirname(__file__), "golden", "mhc_golden.npz")


def _g():
    z = np.load(GOLD)
    return {k: torch.from_numpy(np.asarray(z[k])) for k in z.files}


def test_maps_read_write_match_reference_module():
    g = _g()
    pre, post, res = mhc_maps(g["streams"], g["theta"], g["map_norm_w"], g["pre_bias"],
                              g["post_bias"], g["res_bias"], g["alpha"], int(g["iters"]),
                              float(g["map_norm_eps"][0]))
    assert torch.allclose(pre, g["pre"], atol=1e-6)
    assert torch.allclose(post, g["post"], atol=1e-6)
    assert torch.allclose(res, g["residual"], atol=1e-6)
    read = mhc_read(g["streams"], g["pre"], g["ln_w"], g["ln_b"], float(g["ln_eps"][0]))
    assert torch.allclose(read, g["read"], atol=1e-5)
    out = mhc_write(g["streams"], g["update"], g["post"], g["residual"], g["scale"],
                    g["gating_logit"])
    assert torch.allclose(out, g["write"], atol=1e-5)


def test_closed_forms():
    S, D = 4, 8
    gen = torch.Generator().manual_seed(3)
    X = torch.randn(5, S, D, generator=gen)
    # zero projection: the maps are the biases' own functions
    pb, qb = torch.randn(S, generator=gen), torch.randn(S, generator=gen)
    rb = torch.randn(S, S, generator=gen)
    pre, post, res = mhc_maps(X, torch.zeros(2 * S + S * S, S * D), torch.ones(S * D), pb, qb, rb,
                              torch.full((3,), 0.5), 10)
    assert torch.allclose(pre, torch.sigmoid(pb).expand(5, S))
    assert torch.allclose(post, 2 * torch.sigmoid(qb).expand(5, S))
    assert torch.allclose(res[0].double(), torch.from_numpy(sinkhorn4(rb.numpy(), 10)), atol=1e-6)
    assert torch.allclose(res.sum(-2), torch.ones(5, S), atol=1e-5)        # columns sum to 1
    # read with one-hot pre picks a stream; LayerNorm of it
    onehot = torch.zeros(5, S)
    onehot[:, 2] = 1
    r = mhc_read(X, onehot, torch.ones(D), torch.zeros(D))
    ref = (X[:, 2] - X[:, 2].mean(-1, keepdim=True)) / torch.sqrt(
        X[:, 2].var(-1, unbiased=False, keepdim=True) + 1e-5)
    assert torch.allclose(r, ref, atol=1e-5)
    # write with R = I, post = 0, gating logit +inf-like: X + scale * X
    w = mhc_write(X, torch.randn(5, D, generator=gen), torch.zeros(5, S), torch.eye(S).expand(5, S, S),
                  torch.full((S, D), 2.0), torch.tensor([50.0]))
    assert torch.allclose(w, 3 * X, atol=1e-5)
    assert torch.allclose(sinkhorn_t(rb, 0), rb.exp())
