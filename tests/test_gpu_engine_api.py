"""The native engine behind the reference's engine API (llmy_load, state
handles, llmy_prefill, llmy_decode, llmy_sample), bound exactly as
llmy_cuda/python/sample.py:104-175 binds it.

The engine runs the same kernels in the same order as
hybrid_llm_amd.engine.HybridDecoder, so its logits must equal the Python
engine's bit for bit; the Python engine is pinned against the oracle in
test_gpu_engine.py and test_gpu_prefill.py.  Loop control is checked against
the oracle directly.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from hybrid_llm_amd.checkpoint import save_llmy
from hybrid_llm_amd.config import C1, init_weights

pytestmark = pytest.mark.gpu


def _bind(lib):
    """The reference binding's signatures (llmy_cuda/python/sample.py:110-170)."""
    lib.llmy_load.argtypes = [C.c_char_p]
    lib.llmy_load.restype = C.c_void_p
    lib.llmy_free.argtypes = [C.c_void_p]
    lib.llmy_vocab_size.argtypes = [C.c_void_p]
    lib.llmy_vocab_size.restype = C.c_int32
    lib.llmy_num_loops.argtypes = [C.c_void_p]
    lib.llmy_num_loops.restype = C.c_int32
    lib.llmy_max_loops.argtypes = [C.c_void_p]
    lib.llmy_max_loops.restype = C.c_int32
    lib.llmy_set_num_loops.argtypes = [C.c_void_p, C.c_int32]
    lib.llmy_state_new.argtypes = [C.c_void_p]
    lib.llmy_state_new.restype = C.c_void_p
    lib.llmy_state_free.argtypes = [C.c_void_p]
    lib.llmy_prefill.argtypes = [C.c_void_p, C.c_void_p, C.POINTER(C.c_int32), C.c_int32,
                                 C.POINTER(C.c_float)]
    lib.llmy_prefill.restype = None
    lib.llmy_decode.argtypes = [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                                C.POINTER(C.c_float)]
    lib.llmy_decode.restype = None
    lib.llmy_last_executed_loops.argtypes = [C.c_void_p]
    lib.llmy_last_executed_loops.restype = C.c_int32
    return lib


@pytest.fixture(scope="module")
def c1_file(tmp_path_factory):
    w = init_weights(C1, seed=0)
    path = tmp_path_factory.mktemp("engine") / "c1.llmy"
    save_llmy(path, C1, w)
    return path, w


@pytest.fixture(scope="module")
def lib():
    from hybrid_llm_amd import _lib
    return _bind(_lib.load())


def test_prefill_and_decode_match_python_engine(lib, c1_file):
    from hybrid_llm_amd.engine import HybridDecoder
    path, w = c1_file
    prompt = torch.randint(0, C1.vocab, (40,), generator=torch.Generator().manual_seed(7))
    print("[engine-api] C1 prefill 40 + decode 6", flush=True)
    m = lib.llmy_load(str(path).encode())
    assert m, lib.llmy_last_error()
    try:
        assert lib.llmy_vocab_size(m) == C1.vocab
        assert lib.llmy_num_loops(m) == C1.num_loops == lib.llmy_max_loops(m)
        s = lib.llmy_state_new(m)
        assert s
        V = C1.vocab
        out = (C.c_float * V)()
        toks = (C.c_int32 * 40)(*prompt.tolist())
        lib.llmy_prefill(m, s, toks, 40, out)
        assert lib.llmy_last_status() == 0, lib.llmy_last_error()
        native = [np.frombuffer(out, dtype=np.float32).copy()]
        py = HybridDecoder(C1, w, 1)
        ref = [py.prefill(prompt.view(1, -1).cuda())[0].cpu().numpy().copy()]
        tok = int(np.argmax(native[0]))
        for step in range(6):
            lib.llmy_decode(m, s, tok, 40 + step, 0, out)
            assert lib.llmy_last_status() == 0, lib.llmy_last_error()
            native.append(np.frombuffer(out, dtype=np.float32).copy())
            ref.append(py.step(torch.tensor([tok], dtype=torch.int32).cuda())[0].cpu().numpy().copy())
            tok = int(np.argmax(native[-1]))
        for a, b in zip(native, ref):
            assert np.array_equal(a, b)
        assert lib.llmy_last_executed_loops(s) == C1.num_loops
        lib.llmy_state_free(s)
    finally:
        lib.llmy_free(m)


def test_batched_api_and_device_logits(lib, c1_file):
    from hybrid_llm_amd.engine import HybridDecoder
    path, w = c1_file
    B, T = 3, 24
    prompt = torch.randint(0, C1.vocab, (B, T), generator=torch.Generator().manual_seed(8),
                           dtype=torch.int32)
    m = lib.llmy_load(str(path).encode())
    assert m
    try:
        s = lib.llmy_state_new_batch(m, B)
        assert s
        out = torch.zeros(B, C1.vocab, device="cuda")    # device-resident logits
        toks = prompt.cuda()                              # device-resident tokens
        assert lib.llmy_prefill_batch(m, s, toks.data_ptr(), T, out.data_ptr()) == 0
        py = HybridDecoder(C1, w, B)
        assert torch.equal(out, py.prefill(prompt.cuda()))
        nxt = torch.zeros(B, dtype=torch.int32)
        assert lib.llmy_greedy_tokens(s, nxt.data_ptr()) == 0
        assert torch.equal(nxt, py.buf["next"].cpu())
        for _ in range(3):
            assert lib.llmy_decode_batch(m, s, nxt.data_ptr(), None, 0, out.data_ptr()) == 0
            assert torch.equal(out, py.step(nxt.cuda()))
            assert lib.llmy_greedy_tokens(s, nxt.data_ptr()) == 0
        # reset, then a decode from position 0 equals a fresh engine's first step
        lib.llmy_state_reset(s)
        first = torch.tensor([5, 6, 7], dtype=torch.int32)
        pos = torch.zeros(B, dtype=torch.int32)
        assert lib.llmy_decode_batch(m, s, first.data_ptr(), pos.data_ptr(), 0, out.data_ptr()) == 0
        py2 = HybridDecoder(C1, w, B)
        assert torch.equal(out, py2.step(first.cuda()))
        lib.llmy_state_free(s)
    finally:
        lib.llmy_free(m)


def test_loop_control(lib, c1_file):
    """num_loops = 1 runs the first loop only: bitwise the Python engine of
    the one-loop model (loops share weights), and that engine against the
    oracle's one-loop step with its routing replayed, every token within the
    stated tolerance.  After llmy_set_num_loops(1) the prefill runs one loop
    and an explicit decode num_loops of 2 is capped at 1 (the reference
    overwrites cfg.num_loops: llmy.cpp:66-69, model.cpp:1824-1825,1964)."""
    from dataclasses import replace
    from hybrid_llm_amd.engine import HybridDecoder
    from oracle.model import HybridOracle
    path, w = c1_file
    m = lib.llmy_load(str(path).encode())
    assert m
    try:
        s = lib.llmy_state_new(m)
        out = (C.c_float * C1.vocab)()
        one = HybridDecoder(replace(C1, num_loops=1), w, 1)
        one.enable_route_log()
        ref = HybridOracle(C1, w, act_bf16=True)
        st = ref.new_state(1)
        for i, tok in enumerate([11, 22, 33, 44]):
            lib.llmy_decode(m, s, tok, i, 1, out)            # one loop of two
            assert lib.llmy_last_executed_loops(s) == 1
            got = torch.from_numpy(np.frombuffer(out, dtype=np.float32).copy())
            assert torch.equal(got, one.step(torch.tensor([tok], dtype=torch.int32).cuda())[0].cpu())
            ref.forced_routes = [r for r in one.route_log.cpu().numpy()[:C1.n_layers]]
            want = ref.step([tok], st, num_loops=1)[0]
            assert not ref.forced_routes
            err = float(torch.linalg.norm(got.double() - want.double()) / torch.linalg.norm(want.double()))
            assert err <= 1e-2, (i, err)
        lib.llmy_set_num_loops(m, 1)
        assert lib.llmy_num_loops(m) == 1
        lib.llmy_decode(m, s, 55, 4, 0, out)                # default is now one loop
        assert lib.llmy_last_executed_loops(s) == 1
        # prefill after set_num_loops(1): one loop, bitwise the one-loop engine
        prompt = torch.randint(0, C1.vocab, (12,), generator=torch.Generator().manual_seed(9))
        toks = (C.c_int32 * 12)(*prompt.tolist())
        lib.llmy_prefill(m, s, toks, 12, out)
        assert lib.llmy_last_status() == 0, lib.llmy_last_error()
        assert lib.llmy_last_executed_loops(s) == 1
        one2 = HybridDecoder(replace(C1, num_loops=1), w, 1)
        want = one2.prefill(prompt.view(1, -1).cuda())[0].cpu()
        assert torch.equal(torch.from_numpy(np.frombuffer(out, dtype=np.float32).copy()), want)
        # an explicit num_loops above the set count is capped at it
        lib.llmy_decode(m, s, 66, 12, 2, out)
        assert lib.llmy_last_executed_loops(s) == 1
        want = one2.step(torch.tensor([66], dtype=torch.int32).cuda())[0].cpu()
        assert torch.equal(torch.from_numpy(np.frombuffer(out, dtype=np.float32).copy()), want)
        lib.llmy_state_free(s)
    finally:
        lib.llmy_free(m)


def test_errors_are_reported_not_thrown(lib, tmp_path):
    bad = tmp_path / "x.llmy"
    bad.write_bytes(b"LLMY" + b"\0" * 8)
    assert lib.llmy_load(str(bad).encode()) is None
    assert lib.llmy_last_status() != 0 and lib.llmy_last_error()
    assert lib.llmy_state_new_batch(None, 2) is None


def test_shared_experts_match_python_engine(lib, tmp_path):
    """A checkpoint with shared experts (moe.shared_experts=2): the native
    engine stacks them after the routed experts exactly as the Python engine
    does, so prefill and decode logits agree bit for bit, on the fused decode
    router (B=2) and the sorted prefill path."""
    from dataclasses import replace
    from hybrid_llm_amd.engine import HybridDecoder
    cfg = replace(C1, shared_experts=2)
    w = init_weights(cfg, seed=1)
    path = tmp_path / "shared.llmy"
    save_llmy(path, cfg, w)
    B, T = 2, 20
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(9),
                           dtype=torch.int32)
    print("[engine-api] shared experts: prefill 20 + decode 3, B=2", flush=True)
    m = lib.llmy_load(str(path).encode())
    assert m, lib.llmy_last_error()
    try:
        s = lib.llmy_state_new_batch(m, B)
        assert s
        out = torch.zeros(B, cfg.vocab, device="cuda")
        assert lib.llmy_prefill_batch(m, s, prompt.cuda().data_ptr(), T, out.data_ptr()) == 0
        py = HybridDecoder(cfg, w, B)
        assert torch.equal(out, py.prefill(prompt.cuda()))
        nxt = torch.zeros(B, dtype=torch.int32)
        for _ in range(3):
            assert lib.llmy_greedy_tokens(s, nxt.data_ptr()) == 0
            assert lib.llmy_decode_batch(m, s, nxt.data_ptr(), None, 0, out.data_ptr()) == 0
            assert torch.equal(out, py.step(nxt.cuda()))
        lib.llmy_state_free(s)
    finally:
        lib.llmy_free(m)


def test_state_reset_rows_matches_python_engine(lib, tmp_path):
    """llmy_state_reset_rows (RecurrentState.reset_rows before decode_step,
    model/model.py:814-822) with the context router on, so the latent ring is
    reset too: the next decodes (positions NULL: the reset row restarts at 0)
    equal the Python engine's reset_rows + step bit for bit."""
    from dataclasses import replace
    from hybrid_llm_amd.engine import HybridDecoder
    cfg = replace(C1, context_router=True, router_context=8, route_gate_init=0.0)
    w = init_weights(cfg, seed=3)
    path = tmp_path / "ctx_reset.llmy"
    save_llmy(path, cfg, w)
    B, T = 3, 12
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(13),
                           dtype=torch.int32)
    print("[engine-api] reset rows: prefill 12 + decode 4 with a reset, B=3", flush=True)
    m = lib.llmy_load(str(path).encode())
    assert m, lib.llmy_last_error()
    try:
        s = lib.llmy_state_new_batch(m, B)
        assert s
        out = torch.zeros(B, cfg.vocab, device="cuda")
        assert lib.llmy_prefill_batch(m, s, prompt.cuda().data_ptr(), T, out.data_ptr()) == 0
        py = HybridDecoder(cfg, w, B)
        assert torch.equal(out, py.prefill(prompt.cuda()))
        mask = torch.tensor([0, 1, 1], dtype=torch.int32)
        nxt = torch.zeros(B, dtype=torch.int32)
        for i in range(4):
            assert lib.llmy_greedy_tokens(s, nxt.data_ptr()) == 0
            if i == 1:
                assert lib.llmy_state_reset_rows(s, mask.data_ptr()) == 0       # host mask
                py.reset_rows(mask.cuda())
            if i == 3:
                dmask = torch.tensor([1, 0, 0], dtype=torch.int32, device="cuda")
                assert lib.llmy_state_reset_rows(s, dmask.data_ptr()) == 0      # device mask
                py.reset_rows(dmask)
            assert lib.llmy_decode_batch(m, s, nxt.data_ptr(), None, 0, out.data_ptr()) == 0
            assert torch.equal(out, py.step(nxt.cuda())), i
        assert py.pos.cpu().tolist() == [1, 3, 3]
        assert lib.llmy_state_reset_rows(None, mask.data_ptr()) == 1
        lib.llmy_state_free(s)
    finally:
        lib.llmy_free(m)


def test_mhc_matches_python_engine(lib, tmp_path):
    """A 4-stream mHC model (model/layers/mhc.py in the block of model.py:
    177-264): llmy_mhc_streams reports 4, and the native engine's prefill and
    graph-replayed decode logits equal the Python engine's bit for bit."""
    from dataclasses import replace
    from hybrid_llm_amd.engine import HybridDecoder
    cfg = replace(C1, layer_kinds=("attn", "gdn"), mhc_streams=4, mhc_gating_init=0.5)
    w = init_weights(cfg, seed=7)
    path = tmp_path / "mhc.llmy"
    save_llmy(path, cfg, w)
    B, T = 2, 24
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(14),
                           dtype=torch.int32)
    print("[engine-api] mHC: prefill 24 + decode 3, B=2", flush=True)
    m = lib.llmy_load(str(path).encode())
    assert m, lib.llmy_last_error()
    try:
        lib.llmy_mhc_streams.argtypes = [C.c_void_p]
        lib.llmy_mhc_streams.restype = C.c_int32
        assert lib.llmy_mhc_streams(m) == 4
        s = lib.llmy_state_new_batch(m, B)
        assert s
        out = torch.zeros(B, cfg.vocab, device="cuda")
        assert lib.llmy_prefill_batch(m, s, prompt.cuda().data_ptr(), T, out.data_ptr()) == 0
        py = HybridDecoder(cfg, w, B)
        assert torch.equal(out, py.prefill(prompt.cuda()))
        nxt = torch.zeros(B, dtype=torch.int32)
        for _ in range(3):
            assert lib.llmy_greedy_tokens(s, nxt.data_ptr()) == 0
            assert lib.llmy_decode_batch(m, s, nxt.data_ptr(), None, 0, out.data_ptr()) == 0
            assert torch.equal(out, py.step(nxt.cuda()))
        lib.llmy_state_free(s)
    finally:
        lib.llmy_free(m)


def test_context_router_matches_python_engine(lib, tmp_path):
    """router.context_aware=1 (local latent window of 8 tokens, latent 256):
    the native engine's prefill and decode logits equal the Python engine's
    bit for bit; the prompt is longer than the window, so the ring wraps."""
    from dataclasses import replace
    from hybrid_llm_amd.engine import HybridDecoder
    cfg = replace(C1, context_router=True, router_context=8, route_gate_init=0.0)
    w = init_weights(cfg, seed=2)
    path = tmp_path / "ctx.llmy"
    save_llmy(path, cfg, w)
    B, T = 2, 20
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(10),
                           dtype=torch.int32)
    print("[engine-api] context router: prefill 20 + decode 3, B=2", flush=True)
    m = lib.llmy_load(str(path).encode())
    assert m, lib.llmy_last_error()
    try:
        s = lib.llmy_state_new_batch(m, B)
        assert s
        out = torch.zeros(B, cfg.vocab, device="cuda")
        assert lib.llmy_prefill_batch(m, s, prompt.cuda().data_ptr(), T, out.data_ptr()) == 0
        py = HybridDecoder(cfg, w, B)
        assert torch.equal(out, py.prefill(prompt.cuda()))
        nxt = torch.zeros(B, dtype=torch.int32)
        for _ in range(3):
            assert lib.llmy_greedy_tokens(s, nxt.data_ptr()) == 0
            assert lib.llmy_decode_batch(m, s, nxt.data_ptr(), None, 0, out.data_ptr()) == 0
            assert torch.equal(out, py.step(nxt.cuda()))
        lib.llmy_state_free(s)
    finally:
        lib.llmy_free(m)


@pytest.mark.parametrize("mhc", [1, 4])
def test_cmp_matches_python_engine(lib, tmp_path, mhc):
    """CSA and HCA mixers (model/layers/csa.py, hca.py; .llmy names of
    llmy_cuda/src/model.cpp:132-160): the native engine's prefill, graph-replayed
    decode (past the local window, across emitted summaries) and a row reset
    equal the Python engine's bit for bit, single-stream and with 4 mHC streams."""
    from dataclasses import replace
    from hybrid_llm_amd.engine import HybridDecoder
    cfg = replace(C1, layer_kinds=("csa", "gdn", "hca", "attn"), csa_heads=4, csa_head_dim=64,
                  csa_window=16, csa_ratio=4, csa_top_k=3, hca_window=12, hca_ratio=8,
                  hca_dense=mhc == 1, hca_top_k=2, cmp_slots=64, mhc_streams=mhc,
                  mhc_gating_init=0.5)
    w = init_weights(cfg, seed=17)
    path = tmp_path / "cmp.llmy"
    save_llmy(path, cfg, w)
    B, T = 3, 21
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(18),
                           dtype=torch.int32)
    print(f"[engine-api] CSA/HCA (mhc {mhc}): prefill 21 + decode 14 with a reset, B=3",
          flush=True)
    m = lib.llmy_load(str(path).encode())
    assert m, lib.llmy_last_error()
    try:
        s = lib.llmy_state_new_batch(m, B)
        assert s
        out = torch.zeros(B, cfg.vocab, device="cuda")
        assert lib.llmy_prefill_batch(m, s, prompt.cuda().data_ptr(), T, out.data_ptr()) == 0
        py = HybridDecoder(cfg, w, B)
        assert torch.equal(out, py.prefill(prompt.cuda()))
        mask = torch.tensor([0, 1, 0], dtype=torch.int32)
        nxt = torch.zeros(B, dtype=torch.int32)
        for i in range(14):
            assert lib.llmy_greedy_tokens(s, nxt.data_ptr()) == 0
            if i == 5:
                assert lib.llmy_state_reset_rows(s, mask.data_ptr()) == 0
                py.reset_rows(mask.cuda())
            assert lib.llmy_decode_batch(m, s, nxt.data_ptr(), None, 0, out.data_ptr()) == 0
            assert torch.equal(out, py.step(nxt.cuda())), i
        lib.llmy_state_free(s)
    finally:
        lib.llmy_free(m)


def test_context_router_global_branch_matches_python_engine(lib, tmp_path):
    """HCA blocks with the context-aware router (the global branch over the
    block's summaries, .llmy names moe.router.latent_attention.* and
    hca_latent.*, llmy_cuda/src/model.cpp:98-104,234): the native engine's
    prefill and graph-replayed decodes equal the Python engine's bit for bit."""
    from dataclasses import replace
    from hybrid_llm_amd.engine import HybridDecoder
    cfg = replace(C1, layer_kinds=("hca", "gdn", "hca"), hca_window=12, hca_ratio=4,
                  cmp_slots=64, context_router=True, router_context=8, route_gate_init=0.5)
    w = init_weights(cfg, seed=19)
    path = tmp_path / "hca_ctx.llmy"
    save_llmy(path, cfg, w)
    B, T = 2, 18
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(20),
                           dtype=torch.int32)
    print("[engine-api] HCA + context router: prefill 18 + decode 9, B=2", flush=True)
    m = lib.llmy_load(str(path).encode())
    assert m, lib.llmy_last_error()
    try:
        s = lib.llmy_state_new_batch(m, B)
        assert s
        out = torch.zeros(B, cfg.vocab, device="cuda")
        assert lib.llmy_prefill_batch(m, s, prompt.cuda().data_ptr(), T, out.data_ptr()) == 0
        py = HybridDecoder(cfg, w, B)
        assert torch.equal(out, py.prefill(prompt.cuda()))
        nxt = torch.zeros(B, dtype=torch.int32)
        for i in range(9):
            assert lib.llmy_greedy_tokens(s, nxt.data_ptr()) == 0
            assert lib.llmy_decode_batch(m, s, nxt.data_ptr(), None, 0, out.data_ptr()) == 0
            assert torch.equal(out, py.step(nxt.cuda())), i
        lib.llmy_state_free(s)
    finally:
        lib.llmy_free(m)
