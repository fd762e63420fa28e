"""Writes tests/golden/compressed_golden.npz: inputs and outputs of the
reference's CompressedSelectiveAttention (model/layers/csa.py:16-259) and
HierarchicalCompressedAttention (model/layers/hca.py:15-193) on small seeded
inputs: the sequence forward of a prompt, then decode steps driven the way the
reference block drives them (model/model.py:290-347: the memory reserved as a
writable cache, the last window - 1 inputs as the local history).  For pinning
oracle/compressed.py.  Run in the build container only (it loads the
reference modules from /root/reference); the committed .npz is the fixture,
the reference never travels.

    python tests/golden/make_compressed_golden.py
"""
import importlib.util
import os
import sys
import types

import numpy as np
import torch

REF = "/root/reference/model"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "compressed_golden.npz")


def _load():
    """The three layer modules and the state module under a stand-in package
    name, so their relative imports resolve without the package's __init__."""
    pkg = types.ModuleType("refmodel")
    pkg.__path__ = [REF]
    sub = types.ModuleType("refmodel.layers")
    sub.__path__ = [REF + "/layers"]
    sys.modules["refmodel"], sys.modules["refmodel.layers"] = pkg, sub
    mods = {}
    for name, path in [("refmodel.recurrent_state", REF + "/recurrent_state.py"),
                       ("refmodel.layers.compressed_attention",
                        REF + "/layers/compressed_attention.py"),
                       ("refmodel.layers.csa", REF + "/layers/csa.py"),
                       ("refmodel.layers.hca", REF + "/layers/hca.py")]:
        spec = importlib.util.spec_from_file_location(name, path)
        mod = importlib.util.module_from_spec(spec)
        sys.modules[name] = mod
        spec.loader.exec_module(mod)
        mods[name.split(".")[-1]] = mod
    return mods


def _weights(m, kind):
    """The mixer's eight matrices under the oracle's names."""
    remote = m.remote_out if kind == "csa" else m.global_out
    return {"cmp_wq": m.query.weight, "cmp_wk": m.key.weight, "cmp_wv": m.value.weight,
            "cmp_wlo": m.local_out.weight, "cmp_wro": remote.weight, "cmp_wout": m.out.weight,
            "cmp_wck": m.compressor.key.weight, "cmp_wcv": m.compressor.value.weight}


def _run(mods, m, kind, B, T, steps, D, W, seed):
    MemoryState = mods["recurrent_state"].MemoryState
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(B, T, D, generator=g)
    xs = torch.randn(steps, B, 1, D, generator=g)
    out = {}
    with torch.no_grad():
        y, comp, _ = m(h, return_stats=False)
        out["seq_out"] = y
        mem = MemoryState(comp.keys, comp.values, comp.positions, comp.segment_ids,
                          pending_sum=comp.pending_sum, pending_count=comp.pending_count,
                          pending_segment_ids=comp.pending_segment_ids)
        hist = h[:, -(W - 1):]
        valid = torch.ones(hist.shape[:2], dtype=torch.bool)
        ys = []
        for i in range(steps):
            active = mem.keys.shape[1] if mem.length is None else int(mem.length)
            mem.reserve(max(256, active + 1))
            yi, _, _ = m.forward_step(xs[i], memory=mem, local_history=hist,
                                      local_history_valid=valid,
                                      position=torch.full((B,), T + i, dtype=torch.long))
            ys.append(yi[:, 0])
            hist = torch.cat([hist, xs[i]], 1)[:, -(W - 1):]
            valid = torch.ones(hist.shape[:2], dtype=torch.bool)
        out["step_out"] = torch.stack(ys)
    out["h"], out["xs"] = h, xs[:, :, 0]
    for n, t in _weights(m, kind).items():
        out[n] = t
    return out


def main():
    mods = _load()
    D, W, B, T, steps = 32, 5, 2, 13, 9
    torch.manual_seed(0)
    cases = {
        "csa": mods["csa"].CompressedSelectiveAttention(D, compression=4, local_window=W,
                                                         index_heads=4, index_head_dim=8,
                                                         top_k=2),
        "hca": mods["hca"].HierarchicalCompressedAttention(D, compression=4, local_window=W,
                                                            dense_global_attention=True),
        "hcak": mods["hca"].HierarchicalCompressedAttention(D, compression=3, local_window=W,
                                                             dense_global_attention=False,
                                                             global_top_k=2),
    }
    data = {}
    for i, (name, m) in enumerate(cases.items()):
        m.train(False)
        kind = "csa" if name == "csa" else "hca"
        for k, v in _run(mods, m, kind, B, T, steps, D, W, 10 + i).items():
            data[f"{name}.{k}"] = v.detach().float().numpy()
    np.savez_compressed(OUT, **data)
    print("wrote", OUT, sorted(data))


if __name__ == "__main__":
    main()
