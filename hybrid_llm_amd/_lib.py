"""ctypes binding of libllmy.so (the C ABI declared in include/llmy.h).

Mirrors the reference binding style (llmy_cuda/python/sample.py:104-175:
``ctypes.CDLL`` + explicit argtypes/restype).  The library is looked up in
``$LLMY_LIBRARY`` or next to this file; a missing library raises — there is
no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

_P = C.c_void_p
_I = C.c_int32
_F = C.c_float
_I64 = C.c_int64
_U64P = C.POINTER(C.c_uint64)

# name -> (restype, argtypes); one entry per declaration in include/llmy.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "llmy_abi_version": (_I, []),
    "llmy_router_topk_bf16": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P]),
    "llmy_router_topk_logits_f32": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "llmy_moe_permute": (_I, [_P, _I, _I, _P, _P, _P, _P, _P]),
    "llmy_sample_argmax_f32": (_I, [_P, _I, _I, _P, _P]),
    "llmy_moe_selected_fp32": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "llmy_mhc_sinkhorn4": (_I, [_P, _P, _I, _I, _P]),
    "llmy_sample_top_p_f32": (_I, [_P, _I, _I, _F, _I, _F, _P, _P, _P]),
    "llmy_repetition_penalty_f32": (_I, [_P, _I, _I, _P, _I, _F, _P]),
    "llmy_linear_bf16": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "llmy_pack_weights_bf16": (_I, [_P, _P, _I64, _I, _I, _P]),
    "llmy_moe_experts_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "llmy_moe_combine": (_I, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "llmy_moe_experts_routed_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                                          _P]),
    "llmy_banded_attn_prefill_bf16": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P]),
    "llmy_banded_attn_decode_bf16": (_I, [_P, _P, _P, _I64, _I64, _P, _P, _P, _P, _I, _I, _I,
                                          _I, _F, _P]),
    "llmy_banded_attn_decode_parts_bf16": (_I, [_P, _I, _I64, _I64, _I, _I, _P, _P, _P, _P, _I,
                                                _I, _I, _I, _F, _P]),
    "llmy_gdn_prefill_workspace_bytes": (C.c_int64, [_I, _I, _I, _I, _I]),
    "llmy_gdn_prefill_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I, _I, _I, _I, _I, _P]),
    "llmy_gdn_prefill_bf16_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "llmy_gdn_step_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "llmy_gdn_step_fused_f32": (_I, [_P, _I64, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I,
                                     _I, _I, _I, _P]),
    "llmy_embed_norm_bf16": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _F, _P]),
    "llmy_moe_combine_norm": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _F, _P]),
    "llmy_moe_route_decode": (_I, [_P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I,
                                   _I, _I, _I, _F, _P]),
    "llmy_gdn_conv_gate": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "llmy_moe_append_shared": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "llmy_router_context_latent_f32": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _F,
                                            _P]),
    "llmy_router_context_window": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "llmy_router_context_logits_f32": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "llmy_kv_cache_fill_bf16": (_I, [_P, _P, _I64, _P, _P, _I, _I, _I, _I, _I, _P]),
    "llmy_gdn_prefill_prep_f32": (_I, [_P, _I64, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I,
                                       _P]),
    "llmy_gdn_gate_bf16": (_I, [_P, _P, _I64, _I, _P, _I, _I, _P]),
    "llmy_gdn_conv_gate_prefill": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "llmy_gdn_prefill_reset_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I, _I, _I,
                                         _I, _I, _P]),
    "llmy_gdn_step_reset_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "llmy_gdn_step_fused_reset_f32": (_I, [_P, _I64, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                           _I, _I, _I, _I, _I, _I, _P]),
    "llmy_gdn_conv_gate_prefill_reset": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "llmy_zero_rows": (_I, [_P, _I64, _I, _P, _P]),
    "llmy_mhc_embed": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "llmy_mhc_read": (_I, [_P, _P, _I64, _P, _P, _P, _P, _I, _P, _P, _F, _P, _F, _P, _P,
                           _I, _I, _I, _P]),
    "llmy_mhc_write": (_I, [_P, _P, _I64, _P, _P, _P, _I, _I, _I, _P]),
    "llmy_f32_to_bf16": (_I, [_P, _P, _I64, _P]),
    "llmy_pad_cols_bf16": (_I, [_P, _P, _I, _I, _I, _P]),
    "llmy_layernorm_f32_bf16": (_I, [_P, _P, _P, _P, _I, _I, _F, _P]),
    "llmy_latent_attn_bf16": (_I, [_P, _I64, _P, _P, _P, _P, _P, _I64, _I, _I, _I, _I, _I, _F,
                                   _P]),
    "llmy_cmp_workspace_bytes": (C.c_int64, [_I, _I, _I, _I, _I]),
    "llmy_cmp_local_prefill_bf16": (_I, [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I, _I, _I, _I,
                                         _I, _I, _F, _P, _I64, _P]),
    "llmy_cmp_memory_prefill_bf16": (_I, [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I, _I, _I,
                                          _I, _I, _I, _I, _I, _I, _F, _P, _I64, _P]),
    "llmy_cmp_local_decode_bf16": (_I, [_P, _I64, _P, _P, _I64, _P, _P, _P, _P, _I64, _I, _I, _I,
                                        _I, _I, _F, _P, _I64, _P]),
    "llmy_cmp_memory_decode_bf16": (_I, [_P, _I64, _P, _P, _P, _P, _P, _I64, _I, _I, _I, _I, _I,
                                         _I, _F, _P, _I64, _P]),
    "llmy_cmp_pool_prefill_bf16": (_I, [_P, _I64, _P, _P, _P, _I, _I, _I, _I, _P]),
    "llmy_cmp_pool_step_bf16": (_I, [_P, _I64, _P, _P, _P, _P, _I, _I, _I, _P]),
    "llmy_cmp_commit_bf16": (_I, [_P, _I64, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "llmy_cmp_memory_fill_bf16": (_I, [_P, _I64, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "llmy_cmp_ring_fill_bf16": (_I, [_P, _I64, _P, _I, _I, _I, _I, _P]),
    # engine handles (the reference binding's argtypes, llmy_cuda/python/sample.py:110-170)
    "llmy_load": (_P, [C.c_char_p]),
    "llmy_free": (None, [_P]),
    "llmy_vocab_size": (_I, [_P]),
    "llmy_d_model": (_I, [_P]),
    "llmy_num_loops": (_I, [_P]),
    "llmy_max_loops": (_I, [_P]),
    "llmy_mhc_streams": (_I, [_P]),
    "llmy_set_num_loops": (None, [_P, _I]),
    "llmy_set_fixed_loops": (None, [_P, _I]),
    "llmy_state_new": (_P, [_P]),
    "llmy_state_free": (None, [_P]),
    "llmy_state_reset": (None, [_P]),
    "llmy_prefill": (None, [_P, _P, C.POINTER(C.c_int32), _I, C.POINTER(C.c_float)]),
    "llmy_decode": (None, [_P, _P, _I, _I, _I, C.POINTER(C.c_float)]),
    "llmy_sample": (_I, [C.POINTER(C.c_float), _I, _F, _I, _F, _F, C.POINTER(C.c_int32), _I,
                         C.POINTER(C.c_uint64)]),
    "llmy_last_executed_loops": (_I, [_P]),
    "llmy_sync": (None, []),
    "llmy_state_new_batch": (_P, [_P, _I]),
    "llmy_prefill_batch": (_I, [_P, _P, _P, _I, _P]),
    "llmy_decode_batch": (_I, [_P, _P, _P, _P, _I, _P]),
    "llmy_greedy_tokens": (_I, [_P, _P]),
    "llmy_state_reset_rows": (_I, [_P, _P]),
    "llmy_last_status": (_I, []),
    "llmy_last_error": (C.c_char_p, []),
    "llmy_checkpoint_describe": (_I, [C.c_char_p, C.c_char_p, _I64]),
    "llmy_rmsnorm_f32_bf16": (_I, [_P, _P, _P, _I, _I, _F, _P]),
    "llmy_embed_bf16": (_I, [_P, _P, _P, _I, _I, _I, _P]),
}

_LIB: C.CDLL | None = None


def library_path() -> Path:
    env = os.environ.get("LLMY_LIBRARY")
    if env:
        return Path(env)
    return Path(__file__).resolve().parent / "libllmy.so"


def load() -> C.CDLL:
    """Load libllmy.so once and bind every exported signature."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"libllmy.so not found at {path}; build it with `python -m hybrid_llm_amd._build` "
            "(or __graft_entry__.build()). There is no CPU fallback.")
    lib = C.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError = library/ABI mismatch
        fn.restype = restype
        fn.argtypes = argtypes
    _LIB = lib
    return lib


class LlmyError(RuntimeError):
    def __init__(self, fn: str, code: int):
        super().__init__(f"{fn} failed with hipError {code}"
                         + (" (invalid argument)" if code == 1 else ""))
        self.code = code


def call(name: str, *args) -> None:
    """Call an entry point and raise LlmyError on a nonzero status
    (the reference caller's rule, sample_standalone.py:3059-3063)."""
    code = int(getattr(load(), name)(*args))
    if code != 0:
        raise LlmyError(name, code)
