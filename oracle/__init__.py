"""CPU oracle for the LLMY hybrid-block inference hot path.

TEST INFRASTRUCTURE ONLY.  This package restates the reference's algorithms
(StillPillWill/Hybrid_LLM, cited file:line in each function) in plain PyTorch
on the CPU (fp32, fp64 where stated) and numpy (integer work).  It is imported
only by ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py``, and only as the checker or the timed CPU baseline.  The product
path (``hybrid_llm_amd``) never imports it and has no CPU fallback.

How each function is pinned (so that a plausible mistake fails a check) is
listed in the docstrings and exercised by ``tests/test_oracle_*.py``:

* router / permutation: brute force on tiny inputs, invariants, library
  routines (stable argsort).
* MoE: per-token brute force vs grouped form; dense-SwiGLU special case.
* banded attention: W >= T equals causal SDPA; W = 1 gives o = v; brute force.
* GDN: closed forms (beta = 0 decay; orthonormal-key overwrite); chunked form
  equals the sequential recurrence; T = 1 equals the step.
* sampling: torch.argmax; top-p closed forms (u = 0, p -> 0, p = 1).
"""
