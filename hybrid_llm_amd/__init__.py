"""MI355X-native hybrid-block inference hot path of LLMY (StillPillWill/Hybrid_LLM).

Host code is Python on PyTorch-ROCm; the compute is hand-written gfx950 HIP
kernels in ``libllmy.so`` reached through the C ABI of ``include/llmy.h``.
"""
from .config import C1, C5, HybridConfig, init_weights  # noqa: F401

__all__ = ["C1", "C5", "HybridConfig", "init_weights"]
