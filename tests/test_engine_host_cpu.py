"""Host-side checks of the engines that need no GPU: the prompt lengths the
compressed-memory prefill refuses before any kernel runs, and the padding of
expert / dense hidden widths and GEMM input widths to the kernels' multiple
of 256 (exact by construction: zero rows and columns)."""
from dataclasses import replace

import pytest
import torch

from hybrid_llm_amd.config import C1
from hybrid_llm_amd.engine import check_prompt_length, pad_cols, pad_hidden

CSA = replace(C1, layer_kinds=("csa", "gdn"), csa_ratio=4, cmp_slots=8)
HCA = replace(C1, layer_kinds=("hca", "gdn"), hca_ratio=8, cmp_slots=8, context_router=True)


def test_prompt_limits():
    check_prompt_length(CSA, 4 * 4000 + 3)           # 4000 summaries: fine
    with pytest.raises(ValueError, match="4000"):
        check_prompt_length(CSA, 4 * 4001)
    check_prompt_length(HCA, 8 * 8 + 7)              # 8 summaries = the ring: fine
    with pytest.raises(ValueError, match="decode_slots"):
        check_prompt_length(HCA, 8 * 9)
    check_prompt_length(replace(HCA, context_router=False), 8 * 9)   # no router memory


def test_pad_hidden_is_exact():
    g = torch.Generator().manual_seed(0)
    E, H, D = 3, 320, 256
    gu = torch.randn(E, 2 * H, D, generator=g)
    dn = torch.randn(E, D, H, generator=g)
    gp, dp = pad_hidden(gu, dn)
    assert gp.shape == (E, 1024, D) and dp.shape == (E, D, 512)
    x = torch.randn(5, D, generator=g, dtype=torch.float64)
    for e in range(E):
        ref = (torch.nn.functional.silu(x @ gu[e, :H].double().t()) * (x @ gu[e, H:].double().t())
               ) @ dn[e].double().t()
        a = torch.nn.functional.silu(x @ gp[e, :512].double().t()) * (x @ gp[e, 512:].double().t())
        assert torch.equal(a[:, H:], torch.zeros(5, 512 - H, dtype=torch.float64))
        assert torch.allclose(a @ dp[e].double().t(), ref, rtol=1e-12, atol=1e-12)
    assert pad_cols(torch.ones(4, 128)).shape == (4, 256)
    assert torch.equal(pad_cols(torch.ones(4, 128))[:, 128:], torch.zeros(4, 128))
    w = torch.ones(4, 512)
    assert pad_cols(w) is w
