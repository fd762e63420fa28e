"""C-ABI checks that run without a GPU: the library loads, exports every
symbol include/llmy.h declares, and rejects bad arguments before launching
(the reference convention, llmy_cuda/src/llmy.cpp:216-217,230-233)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from hybrid_llm_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
INVALID = 1  # hipErrorInvalidValue


def declared_symbols() -> list[str]:
    text = (ROOT / "include" / "llmy.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(llmy_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "llmy_router_topk_bf16" in syms and len(syms) >= 5


def test_library_exports_every_declared_symbol(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), f"{name} declared in llmy.h but not exported"


def test_binding_covers_every_declared_symbol():
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_abi_version(lib):
    assert lib.llmy_abi_version() >= 1


FAKE = 0x10000  # non-null, 256-byte aligned; never dereferenced (validation fails first)


@pytest.mark.parametrize("args", [
    # null x
    (None, None, FAKE, None, FAKE, FAKE, 4, 64, 8, 2, 1e-6, None),
    # D not a multiple of 4
    (FAKE, None, FAKE, None, FAKE, FAKE, 4, 62, 8, 2, 1e-6, None),
    # k > E
    (FAKE, None, FAKE, None, FAKE, FAKE, 4, 64, 8, 9, 1e-6, None),
    # E too large
    (FAKE, None, FAKE, None, FAKE, FAKE, 4, 64, 300, 2, 1e-6, None),
    # negative T
    (FAKE, None, FAKE, None, FAKE, FAKE, -1, 64, 8, 2, 1e-6, None),
    # misaligned router weights
    (FAKE, None, FAKE + 4, None, FAKE, FAKE, 4, 64, 8, 2, 1e-6, None),
])
def test_router_rejects_bad_arguments(lib, args):
    assert lib.llmy_router_topk_bf16(*args) == INVALID


def test_empty_token_axis_is_noop(lib):
    assert lib.llmy_router_topk_bf16(FAKE, None, FAKE, None, FAKE, FAKE, 0, 64, 8, 2, 1e-6,
                                     None) == 0
    assert lib.llmy_sample_argmax_f32(FAKE, 0, 10, FAKE, None) == 0


def test_permute_and_argmax_reject_bad_arguments(lib):
    assert lib.llmy_moe_permute(None, 8, 4, FAKE, FAKE, FAKE, FAKE, None) == INVALID
    assert lib.llmy_moe_permute(FAKE, 8, 0, FAKE, FAKE, FAKE, FAKE, None) == INVALID
    assert lib.llmy_sample_argmax_f32(FAKE, 4, 0, FAKE, None) == INVALID
    assert lib.llmy_sample_argmax_f32(None, 4, 10, FAKE, None) == INVALID
    assert lib.llmy_router_topk_logits_f32(FAKE, FAKE, FAKE, 4, 8, 0, None) == INVALID


def test_call_raises_on_status():
    with pytest.raises(_lib.LlmyError):
        _lib.call("llmy_sample_argmax_f32", None, 4, 10, FAKE, None)


def test_sampling_entries_reject_bad_arguments(lib):
    top_p = lib.llmy_sample_top_p_f32
    assert top_p(FAKE, 4, 32769, 0.8, 0, 0.9, FAKE, FAKE, None) == INVALID   # V > 32768
    assert top_p(FAKE, 4, 0, 0.8, 0, 0.9, FAKE, FAKE, None) == INVALID       # empty vocab
    assert top_p(FAKE, -1, 10, 0.8, 0, 0.9, FAKE, FAKE, None) == INVALID
    assert top_p(FAKE, 4, 10, 0.8, 0, 0.9, None, FAKE, None) == INVALID      # u missing
    assert top_p(None, 4, 10, 0.8, 0, 0.9, FAKE, FAKE, None) == INVALID
    assert top_p(FAKE, 0, 10, 0.8, 0, 0.9, None, None, None) == 0            # no rows: no-op
    pen = lib.llmy_repetition_penalty_f32
    assert pen(FAKE, 4, 10, FAKE, 3, 0.0, None) == INVALID                   # penalty <= 0
    assert pen(FAKE, 4, 10, FAKE, -1, 1.3, None) == INVALID
    assert pen(FAKE, 4, (1 << 18) + 1, FAKE, 3, 1.3, None) == INVALID
    assert pen(None, 4, 10, None, 0, 1.3, None) == 0                          # nothing listed
    assert pen(None, 4, 10, None, 3, 1.0, None) == 0                          # penalty 1: no-op


def test_reference_op_hooks_reject_bad_arguments(lib):
    moe = lib.llmy_moe_selected_fp32
    ptrs = [FAKE] * 8
    assert moe(None, *ptrs[1:], 16, 8, 2, 1, None) == INVALID
    for bad in ((0, 8, 2, 1), (16, 0, 2, 1), (16, 8, 0, 1), (16, 8, 2, 0)):
        assert moe(*ptrs, *bad, None) == INVALID
    sk = lib.llmy_mhc_sinkhorn4
    assert sk(None, FAKE, 4, 20, None) == INVALID
    assert sk(FAKE, FAKE, 0, 20, None) == INVALID
    assert sk(FAKE, FAKE, 4, -1, None) == INVALID


def test_prefill_glue_rejects_bad_arguments(lib):
    fill = lib.llmy_kv_cache_fill_bf16
    assert fill(FAKE, FAKE, 256, FAKE, FAKE, 2, 10, 4, 64, 0, None) == INVALID     # W = 0
    assert fill(FAKE, FAKE, 255, FAKE, FAKE, 2, 10, 4, 64, 8, None) == INVALID     # ld < H*hd
    assert fill(FAKE, FAKE, 256, FAKE, FAKE, 2, 10, 4, 60, 8, None) == INVALID     # hd % 8
    assert fill(None, FAKE, 256, FAKE, FAKE, 2, 10, 4, 64, 8, None) == INVALID
    assert fill(None, None, 256, None, None, 2, 0, 4, 64, 8, None) == 0            # T = 0
    prep = lib.llmy_gdn_prefill_prep_f32
    ptrs = [FAKE] * 7
    assert prep(FAKE, 800, *ptrs, 4, 2, 96, 64, None) == INVALID                   # dk
    assert prep(FAKE, 100, *ptrs, 4, 2, 64, 64, None) == INVALID                   # ld too small
    assert prep(None, 800, *ptrs, 4, 2, 64, 64, None) == INVALID
    assert prep(None, 800, *([None] * 7), 0, 2, 64, 64, None) == 0
    gate = lib.llmy_gdn_gate_bf16
    assert gate(FAKE, FAKE, 512, 256, FAKE, 4, 100, None) == INVALID              # HV % 8
    assert gate(FAKE, FAKE, 300, 256, FAKE, 4, 128, None) == INVALID              # ld < off+HV
    assert gate(FAKE, FAKE, 512, 2, FAKE, 4, 128, None) == INVALID                # off % 4
    conv = lib.llmy_gdn_conv_gate_prefill
    assert conv(FAKE, FAKE, FAKE, FAKE, 2, 10, 256, 3, None) == INVALID           # kernel != 4
    assert conv(None, FAKE, FAKE, FAKE, 2, 10, 256, 4, None) == INVALID
    assert conv(None, None, None, None, 2, 0, 256, 4, None) == 0


def test_partial_products_and_fold_reject_bad_arguments(lib):
    lin = lib.llmy_linear_bf16
    assert lin(FAKE, FAKE, FAKE, None, 65, 1024, 1024, 4, 1, None) == INVALID    # M > 64
    assert lin(FAKE, FAKE, FAKE, None, 64, 1024, 1024, 5, 1, None) == INVALID    # epilogue
    route = lib.llmy_moe_route_decode
    rest = [FAKE] * 6 + [None] * 4  # ffn_w .. gates, then no permutation
    assert route(FAKE, FAKE, 9, None, *rest, 64, 1024, 24, 2, 1e-6, None) == INVALID  # nparts
    assert route(FAKE, None, 0, FAKE, *rest, 64, 1024, 24, 2, 1e-6, None) == INVALID  # gate alone
    assert route(FAKE, None, 4, None, *rest, 64, 1024, 24, 2, 1e-6, None) == INVALID  # parts NULL


def test_gdn_step_partial_slices_reject_bad_arguments(lib):
    f = lib.llmy_gdn_step_fused_f32
    tail = [FAKE, FAKE, FAKE, FAKE, None, None, None, None, 0, 4, 64, 16, 64, 64, None]
    assert f(FAKE, 4112, 0, *tail) == INVALID     # nparts < 1
    assert f(FAKE, 4112, 9, *tail) == INVALID     # nparts > 8
    assert f(FAKE, 4000, 4, *tail) == INVALID     # ld below the row


def test_context_router_entries_reject_bad_arguments(lib):
    """Checked before any launch (no GPU needed): shapes outside the kernels'
    range, missing pointers, misaligned rows; an empty token axis is a no-op."""
    lat = lib.llmy_router_context_latent_f32
    ok = (FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE)
    assert lat(*ok, 0, 1024, 256, 1e-6, 1e-5, None) == 0                    # no rows
    assert lat(*ok, 4, 300, 256, 1e-6, 1e-5, None) == INVALID               # D not 256 n (n <= 4)
    assert lat(*ok, 4, 2048, 256, 1e-6, 1e-5, None) == INVALID
    assert lat(*ok, 4, 1024, 100, 1e-6, 1e-5, None) == INVALID              # L % 64
    assert lat(*ok, 4, 1024, 1024, 1e-6, 1e-5, None) == INVALID             # L > 512
    assert lat(None, *ok[1:], 4, 1024, 256, 1e-6, 1e-5, None) == INVALID
    assert lat(*ok[:6], None, 4, 1024, 256, 1e-6, 1e-5, None) == INVALID
    assert lat(FAKE, FAKE, FAKE + 4, *ok[3:], 4, 1024, 256, 1e-6, 1e-5, None) == INVALID
    win = lib.llmy_router_context_window
    assert win(FAKE, FAKE, None, FAKE, 0, 5, 8, 256, None) == 0               # no sequences
    assert win(FAKE, FAKE, None, FAKE, 2, 0, 8, 256, None) == 0               # no tokens
    assert win(FAKE, FAKE, None, FAKE, 2, 5, 0, 256, None) == INVALID         # window < 1
    assert win(None, FAKE, None, FAKE, 2, 5, 8, 256, None) == INVALID
    assert win(FAKE, FAKE, None, FAKE, 70000, 5, 8, 256, None) == INVALID     # grid y limit
    lg = lib.llmy_router_context_logits_f32
    assert lg(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 1024, 24, None) == 0
    assert lg(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 1000, 24, None) == INVALID
    assert lg(FAKE, FAKE, None, FAKE, FAKE, 4, 1024, 24, None) == INVALID     # no gate
    assert lg(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 1024, 0, None) == INVALID
    shared = lib.llmy_moe_append_shared
    assert shared(FAKE, FAKE, FAKE, FAKE, 4, 2, 8, 0, None) == INVALID         # S = 0
    assert shared(FAKE, FAKE, FAKE, FAKE, 4, 0, 8, 2, None) == INVALID         # k = 0


def test_gdn_prefill_noalloc_rejects_before_any_device_call(lib):
    """Argument checks and the fixed-workspace limit run before the library
    touches a device (so they answer here, without a GPU)."""
    f = lib.llmy_gdn_prefill_bf16_noalloc
    ptrs = [FAKE] * 7
    assert f(*ptrs, 1, 64, 2, 96, 96, None) == INVALID                            # head size
    assert f(None, *ptrs[1:], 1, 64, 2, 64, 64, None) == INVALID
    assert f(*([None] * 7), 0, 64, 2, 64, 64, None) == 0                          # B = 0
    # 816 chunks x 82 KB at dk = dv = 128: beyond the 64 MiB workspace; 800 fit
    assert f(*ptrs, 1, 64 * 51, 16, 128, 128, None) == 2                         # hipErrorOutOfMemory
    assert lib.llmy_gdn_prefill_workspace_bytes(1, 64 * 51, 16, 128, 128) > 64 << 20
    assert lib.llmy_gdn_prefill_workspace_bytes(1, 64 * 50, 16, 128, 128) <= 64 << 20
