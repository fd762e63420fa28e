"""The whole-model oracle against the reference model's own logits
(tests/golden/model_golden*.npz, written by tests/golden/make_model_golden.py
from model/model.py:LoopedHybridMoEForCausalLM in fp32): stem and tail blocks
with the dense SwiGLU FFN, mHC around every sublayer, the context-aware router,
CSA / HCA / GDN core blocks looped twice, shared experts and the reference
checkpoints' widths (expert_hidden 320, latent_dim 128, router heads 4 x 32).
The prompt's logits at every position and the decoded tokens' logits (the
sequence forward's last position) are compared."""
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

from make_model_golden import CASES, golden_weights  # noqa: E402
from oracle.model import HybridOracle  # noqa: E402


def _rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("fname", sorted(CASES))
def test_oracle_matches_reference_model(fname):
    cfg, seed = CASES[fname]
    z = np.load(os.path.join(HERE, "golden", fname))
    ora = HybridOracle(cfg, golden_weights(cfg, seed))
    st = ora.new_state(z["prompt"].shape[0])
    pre = ora.prefill(z["prompt"], st).numpy()
    ref = z["prefill_logits"]
    assert _rel(pre, ref) < 1e-5 and np.abs(pre - ref).max() < 1e-4
    for t in range(z["decode"].shape[0]):
        lg = ora.step(z["decode"][t], st).numpy()
        ref = z["decode_logits"][t]
        assert _rel(lg, ref) < 1e-5 and np.abs(lg - ref).max() < 1e-4, t


def test_golden_is_sensitive_to_the_stem_and_tail():
    """A plain mistake in the composition fails the fixture: dropping the
    tail block's FFN moves the logits far past the tolerance."""
    cfg, seed = CASES["model_golden.npz"]
    z = np.load(os.path.join(HERE, "golden", "model_golden.npz"))
    ora = HybridOracle(cfg, golden_weights(cfg, seed))
    ora._dense = lambda p, h2: (torch.zeros_like(h2) if p.startswith("T")
                                else HybridOracle._dense(ora, p, h2))
    st = ora.new_state(z["prompt"].shape[0])
    pre = ora.prefill(z["prompt"][:, :4], st).numpy()
    assert _rel(pre, z["prefill_logits"][:, :4]) > 1e-3
