"""GPU parity for models shaped like the reference's checkpoints
(tests/golden/make_model_golden.py): stem and tail blocks (GDN + dense SwiGLU
FFN), 4 mHC streams with the context-aware router, GDN / CSA and HCA / GDN
cores, shared experts, expert_hidden 320 (zero-padded to 512 inside the
engine), latent_dim 128 and router query heads 4 x 32 (zero-padded GEMM
inputs).

The Python engine's prefill and decode logits are checked against the oracle
with the engine's routing replayed (rel-L2 1e-2, the bf16 bound), and the
oracle is pinned to the reference model's own logits by
tests/test_oracle_model_golden.py; the engine is also compared with those
reference fp32 logits directly (rel-L2 1e-2 and max-abs 2e-2; measured about
1.7e-3 and 2.4e-3).  A captured decode step equals eager bit for
bit, and the native engine (llmy_load of a `.llmy` file written from the
config) equals the Python engine bit for bit.
"""
import ctypes as C
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

from make_model_golden import CASES, golden_weights  # noqa: E402
from oracle.model import HybridOracle  # noqa: E402

pytestmark = pytest.mark.gpu

REL_L2 = 1e-2   # the bf16 bounds of the path: rel-L2 1e-2, max-abs 2e-2
MAX_ABS = 2e-2


def rel_l2(a, b):
    a, b = torch.as_tensor(a).double().cpu(), torch.as_tensor(b).double().cpu()
    return float(torch.linalg.norm(a - b) / torch.linalg.norm(b))


def _fixture(fname):
    cfg, seed = CASES[fname]
    return cfg, golden_weights(cfg, seed), np.load(os.path.join(HERE, "golden", fname))


@pytest.mark.parametrize("fname", sorted(CASES))
def test_python_engine_matches_oracle_and_reference(fname):
    from hybrid_llm_amd.engine import HybridDecoder
    cfg, w, z = _fixture(fname)
    prompt = torch.from_numpy(z["prompt"])
    B, T = prompt.shape
    print(f"[golden] {fname}: prefill {T} + decode {z['decode'].shape[0]}, B={B}", flush=True)
    eng = HybridDecoder(cfg, w, B)
    eng.route_log_seq = []
    lg = eng.prefill(prompt.cuda()).clone()
    ref = HybridOracle(cfg, w, act_bf16=True)
    st = ref.new_state(B)
    logs = [r.view(B, T, -1).cpu().numpy() for r in eng.route_log_seq]
    ref.forced_routes = [logs[a][:, t] for t in range(T) for a in range(len(logs))]
    out = ref.prefill(prompt.numpy(), st)
    e_ora = rel_l2(lg, out[:, -1])
    e_ref = rel_l2(lg, z["prefill_logits"][:, -1])
    m_ref = float((lg.cpu() - torch.from_numpy(z["prefill_logits"][:, -1])).abs().max())
    print(f"[golden] prefill rel-L2 vs oracle {e_ora:.2e}, vs reference fp32 {e_ref:.2e} "
          f"(max-abs {m_ref:.2e})", flush=True)
    assert e_ora <= REL_L2, e_ora
    assert e_ref <= REL_L2 and m_ref <= MAX_ABS, (e_ref, m_ref)
    eng.route_log_seq = None
    eng.enable_route_log()
    for t in range(z["decode"].shape[0]):
        tok = torch.from_numpy(z["decode"][t])
        lg = eng.step(tok.cuda()).clone()
        ref.forced_routes = [r for r in eng.route_log.cpu().numpy()]
        lr = ref.step(tok.numpy(), st)
        e_ora, e_ref = rel_l2(lg, lr), rel_l2(lg, z["decode_logits"][t])
        m_ref = float((lg.cpu() - torch.from_numpy(z["decode_logits"][t])).abs().max())
        print(f"[golden] decode {t}: rel-L2 vs oracle {e_ora:.2e}, vs reference {e_ref:.2e}",
              flush=True)
        assert e_ora <= REL_L2, (t, e_ora)
        assert e_ref <= REL_L2 and m_ref <= MAX_ABS, (t, e_ref, m_ref)
    gaps = np.abs(np.array(ref.route_gaps))
    assert gaps.size == 0 or np.all(gaps <= 5e-3), gaps.max()


def test_golden_decode_graph_equals_eager():
    from hybrid_llm_amd.engine import HybridDecoder
    cfg, w, z = _fixture("model_golden.npz")
    prompt = torch.from_numpy(z["prompt"]).cuda()
    B = prompt.shape[0]
    a, g = HybridDecoder(cfg, w, B), HybridDecoder(cfg, w, B)
    a.prefill(prompt)
    g.prefill(prompt)
    g.capture()
    for t in range(z["decode"].shape[0]):
        tok = torch.from_numpy(z["decode"][t]).cuda()
        la = a.step(tok).clone()
        lgr = g.step(tok).clone()
        torch.cuda.synchronize()
        assert torch.equal(la, lgr), t


@pytest.mark.parametrize("fname", sorted(CASES))
def test_native_engine_matches_python_engine(fname, tmp_path):
    """llmy_load of a `.llmy` file written from the golden config (stem and
    tail blocks, mHC, the context router, padded widths): prefill and
    graph-replayed decode logits equal the Python engine's bit for bit."""
    from hybrid_llm_amd import _lib
    from hybrid_llm_amd.checkpoint import save_llmy
    from hybrid_llm_amd.engine import HybridDecoder
    lib = _lib.load()
    lib.llmy_load.argtypes = [C.c_char_p]
    lib.llmy_load.restype = C.c_void_p
    lib.llmy_free.argtypes = [C.c_void_p]
    lib.llmy_state_free.argtypes = [C.c_void_p]
    cfg, w, z = _fixture(fname)
    path = tmp_path / "golden.llmy"
    save_llmy(path, cfg, w)
    prompt = torch.from_numpy(z["prompt"])
    B, T = prompt.shape
    print(f"[golden] native {fname}: prefill {T} + decode, B={B}", flush=True)
    m = lib.llmy_load(str(path).encode())
    assert m, lib.llmy_last_error()
    try:
        s = lib.llmy_state_new_batch(m, B)
        assert s
        out = torch.zeros(B, cfg.vocab, device="cuda")
        assert lib.llmy_prefill_batch(m, s, prompt.cuda().data_ptr(), T, out.data_ptr()) == 0
        py = HybridDecoder(cfg, w, B)
        assert torch.equal(out, py.prefill(prompt.cuda()))
        for t in range(z["decode"].shape[0]):
            tok = torch.from_numpy(z["decode"][t]).to(torch.int32).contiguous()
            assert lib.llmy_decode_batch(m, s, tok.data_ptr(), None, 0, out.data_ptr()) == 0
            assert torch.equal(out, py.step(tok.cuda())), t
        lib.llmy_state_free(s)
    finally:
        lib.llmy_free(m)
