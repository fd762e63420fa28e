"""Writes tests/golden/mhc_golden.npz: inputs and outputs of the reference's
MultiStreamHyperConnection (model/layers/mhc.py:156-231) on small seeded
inputs, for pinning oracle/mhc.py.  Run in the build container only (it
imports the reference module from /root/reference); the committed .npz is the
fixture, the reference never travels.

    python tests/golden/make_mhc_golden.py
"""
import importlib.util
import os

import numpy as np
import torch

REF = "/root/reference/model/layers/mhc.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mhc_golden.npz")


def main():
    spec = importlib.util.spec_from_file_location("ref_mhc", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    torch.manual_seed(0)
    S, D, iters, B, T = 4, 32, 10, 2, 3
    m = mod.MultiStreamHyperConnection(D, S, iters, 0.01)
    g = torch.Generator().manual_seed(1)
    with torch.no_grad():   # non-trivial values for every parameter
        m.theta.weight.copy_(torch.randn(m.theta.weight.shape, generator=g) * 0.05)
        m.mapping_norm.weight.copy_(1 + 0.1 * torch.randn(S * D, generator=g))
        m.stream_norm.weight.copy_(1 + 0.1 * torch.randn(D, generator=g))
        m.stream_norm.bias.copy_(0.1 * torch.randn(D, generator=g))
        m.stream_scale.copy_(1 + 0.1 * torch.randn(S, D, generator=g))
        m.pre_bias.add_(0.2 * torch.randn(S, generator=g))
        m.post_bias.add_(0.2 * torch.randn(S, generator=g))
        m.residual_bias.add_(0.5 * torch.randn(S, S, generator=g))
        m.alpha_pre.fill_(0.7)
        m.alpha_post.fill_(0.4)
        m.alpha_residual.fill_(0.9)
        m.gating_logit.fill_(0.3)
    m.train(False)
    m._static_inference = False       # the dynamic (input-dependent) maps
    streams = torch.randn(B, T, S, D, generator=g)
    update = torch.randn(B, T, D, generator=g)
    with torch.no_grad():
        maps = m.compute_mappings(streams)
        read = m.read(streams, maps)
        write = m.write(streams, update, maps)
    np.savez(OUT,
             S=S, D=D, iters=iters,
             theta=m.theta.weight.detach().numpy(), map_norm_w=m.mapping_norm.weight.detach().numpy(),
             ln_w=m.stream_norm.weight.detach().numpy(), ln_b=m.stream_norm.bias.detach().numpy(),
             scale=m.stream_scale.detach().numpy(), pre_bias=m.pre_bias.detach().numpy(),
             post_bias=m.post_bias.detach().numpy(), res_bias=m.residual_bias.detach().numpy(),
             alpha=np.array([0.7, 0.4, 0.9], dtype=np.float32),
             gating_logit=np.array([0.3], dtype=np.float32),
             map_norm_eps=np.array([m.mapping_norm.eps if m.mapping_norm.eps is not None
                                    else torch.finfo(torch.float32).eps], dtype=np.float64),
             ln_eps=np.array([m.stream_norm.eps], dtype=np.float64),
             streams=streams.numpy(), update=update.numpy(),
             pre=maps.pre.numpy(), post=maps.post.numpy(), residual=maps.residual.numpy(),
             read=read.numpy(), write=write.numpy())
    print("wrote", OUT)


if __name__ == "__main__":
    main()
