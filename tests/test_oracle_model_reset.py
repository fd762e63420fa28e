"""Pins the model oracle's per-row reset (RecurrentState.reset_rows,
model/recurrent_state.py:213-225, applied by decode_step before a token whose
reset_mask is set, model/model.py:814-822) on the CPU: a reset row continues
exactly as a fresh sequence would, and the other rows as if nothing happened.
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

from hybrid_llm_amd.config import HybridConfig, alternating, init_weights
from oracle.model import HybridOracle

TINY = HybridConfig(d_model=256, layer_kinds=alternating(2), attn_heads=4, attn_head_dim=64,
                    window=4, gdn_heads=4, gdn_dk=64, gdn_dv=64, n_experts=4, top_k=2,
                    expert_hidden=256, vocab=512, num_loops=2)

SEQ = [[3, 7, 11], [5, 9, 13], [17, 19, 23], [29, 31, 37], [41, 43, 47], [53, 59, 61]]


@pytest.mark.parametrize("ctx", [False, True])
def test_reset_row_equals_fresh_sequence(ctx):
    cfg = replace(TINY, context_router=True, router_context=3, route_gate_init=0.0) if ctx else TINY
    w = init_weights(cfg, seed=1)
    ref = HybridOracle(cfg, w)
    st = ref.new_state(3)
    for t in SEQ[:5]:                     # past the window and the latent ring
        ref.step(t, st)
    reset = np.array([False, True, False])
    after = [[2, 4, 6], [8, 10, 12], [14, 16, 18]]
    got = [ref.step(after[0], st, reset=reset)] + [ref.step(t, st) for t in after[1:]]
    assert int(st["pos"][1]) == 3 and int(st["pos"][0]) == 8

    # row 1 = a fresh single sequence fed the tokens after the reset
    fresh = HybridOracle(cfg, w)
    sf = fresh.new_state(1)
    want1 = [fresh.step([t[1]], sf) for t in after]
    # rows 0 and 2 = the same batch without any reset
    plain = HybridOracle(cfg, w)
    sp = plain.new_state(3)
    for t in SEQ[:5]:
        plain.step(t, sp)
    want = [plain.step(t, sp) for t in after]
    for i in range(len(after)):
        assert torch.allclose(got[i][1], want1[i][0], rtol=1e-5, atol=1e-5), i
        assert torch.allclose(got[i][[0, 2]], want[i][[0, 2]], rtol=1e-5, atol=1e-5), i
    # and the reset row differs from the no-reset run (the reset did something)
    assert float((got[0][1] - want[0][1]).abs().max()) > 1e-2


def test_reset_all_rows_equals_new_state():
    w = init_weights(TINY, seed=2)
    ref = HybridOracle(TINY, w)
    st = ref.new_state(2)
    for t in SEQ[:3]:
        ref.step(t[:2], st)
    a = ref.step([1, 2], st, reset=[1, 1])
    st2 = ref.new_state(2)
    b = ref.step([1, 2], st2)
    assert torch.equal(a, b)
