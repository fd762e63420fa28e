"""`.llmy` v1 checkpoint files for the hybrid block stack: writer and reader.

The container is the reference engine's flat format
(llmy_cuda/tools/convert_checkpoint.py:1-31,42-47,205-236 writes it,
llmy_cuda/src/checkpoint.cpp:103-170 parses it):

    offset 0   magic "LLMY"
    4          u32 version = 1
    8          u32 cfg_len, then cfg_len bytes of UTF-8 `key=value` lines
    ...        u32 n_tensors, then n_tensors index entries of 108 bytes:
               <I 64s I I 4I Q Q> = name_len, name (NUL padded), dtype
               (0 f32, 1 f16, 2 bf16), ndim, shape[4], offset, nbytes
    data_start the first multiple of 4096 after the index; each entry's
               offset is relative to it

Tensor names and config keys follow the reference model's where the concept
is the same (`embed_tokens.weight`, `recurrent_core.<i>.mixer_norm.weight`,
GDN `q_proj/k_proj/v_proj/gate_proj/beta_proj/out_proj/conv/decay_logit`,
MoE `router.norm/router.logits` and expert stacks `[E, H, D]`; `gdn.*` and
`moe.*` keys; CSA / HCA `query/key/value/local_out/remote_out|global_out/out`
and `compressor.key/value`, `csa.*` / `hca.*` keys).  The banded attention
mixer of this block stack has no reference counterpart with the same weights,
so its layout entry is `attn` and its keys are `attn.heads`, `attn.head_dim`,
`attn.window`.  `memory.decode_slots` (the CSA / HCA decode memory's slots per
row) is this engine's key; the reference reader ignores unknown keys.

The native loader `llmy_load` (hybrid_llm_amd/csrc/engine.cpp) reads the same
files; this module writes them from `config.init_weights`-style dicts and
reads them back for tests.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np
import torch

from .config import HybridConfig

MAGIC = b"LLMY"
VERSION = 1
INDEX_ENTRY = struct.Struct("<I64sII4IQQ")
assert INDEX_ENTRY.size == 108
DATA_ALIGN = 4096
DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
DTYPE_OF = {v: k for k, v in DTYPES.items()}
ITEMSIZE = {0: 4, 1: 2, 2: 2}

_GDN = {"wq": "q_proj.weight", "wk": "k_proj.weight", "wv": "v_proj.weight",
        "wg": "gate_proj.weight", "wb": "beta_proj.weight", "bb": "beta_proj.bias",
        "wout": "out_proj.weight", "conv": "conv.weight", "decay": "decay_logit"}
_ATTN = {"wq": "q.weight", "wk": "k.weight", "wv": "v.weight", "wo": "o.weight"}
# CSA / HCA (model/layers/csa.py:21-29, hca.py:24-30; llmy_cuda/src/model.cpp:132-160):
# remote_out is CSA's name, global_out HCA's
_CMP = {"cmp_wq": "query.weight", "cmp_wk": "key.weight", "cmp_wv": "value.weight",
        "cmp_wlo": "local_out.weight", "cmp_wout": "out.weight",
        "cmp_wck": "compressor.key.weight", "cmp_wcv": "compressor.value.weight"}
_BLOCK = {"mix_norm": "mixer_norm.weight", "ffn_norm": "ffn_norm.weight",
          "router_norm": "moe.router.norm.weight", "w_router": "moe.router.logits.weight",
          "w_gate": "moe.experts.gate_proj.weight", "w_up": "moe.experts.up_proj.weight",
          "w_down": "moe.experts.down_proj.weight",
          "w_shared_gate": "moe.shared.gate_proj.weight",
          "w_shared_up": "moe.shared.up_proj.weight",
          "w_shared_down": "moe.shared.down_proj.weight",
          "ctx_down": "moe.router.latent_memory.down.weight",
          "ctx_ln_w": "moe.router.latent_memory.norm.weight",
          "ctx_ln_b": "moe.router.latent_memory.norm.bias",
          "ctx_local_out": "moe.router.local_context_out.weight",
          "ctx_out": "moe.router.context_out.weight",
          "ctx_gate": "moe.router.route_gate",
          # the router's global branch (context_router.py:24; mla_memory.py:55-63)
          # and the HCA block's summary latents (model.py:117; mla_memory.py:17-21)
          "ctx_q": "moe.router.latent_attention.q.weight",
          "ctx_k": "moe.router.latent_attention.k.weight",
          "ctx_v": "moe.router.latent_attention.v.weight",
          "ctx_o": "moe.router.latent_attention.o.weight",
          "hca_lat_down": "hca_latent.down.weight", "hca_lat_ln_w": "hca_latent.norm.weight",
          "hca_lat_ln_b": "hca_latent.norm.bias"}


# mHC parameters (model/layers/mhc.py:63-84; the names llmy_cuda/src/model.cpp:34-63
# reads); the three alpha scalars are one [3] tensor here (mhc_alpha)
_MHC = {"mhc_map_norm": "mhc.mapping_norm.weight", "mhc_theta": "mhc.theta.weight",
        "mhc_pre_bias": "mhc.pre_bias", "mhc_post_bias": "mhc.post_bias",
        "mhc_res_bias": "mhc.residual_bias", "mhc_gating": "mhc.gating_logit",
        "mhc_scale": "mhc.stream_scale", "mhc_ln_w": "mhc.stream_norm.weight",
        "mhc_ln_b": "mhc.stream_norm.bias"}
_MHC_ALPHA = ("mhc.alpha_pre", "mhc.alpha_post", "mhc.alpha_residual")
# the dense SwiGLU FFN of a stem / tail block (model/layers/dense_ffn.py:9-11;
# llmy_cuda/src/model.cpp:81-87 reads these names)
_DENSE = {"ffn_gate": "ffn.gate_proj.weight", "ffn_up": "ffn.up_proj.weight",
          "ffn_down": "ffn.down_proj.weight"}
_SIDE = {"S": "stem", "T": "tail"}


def file_name(cfg: HybridConfig, key: str) -> str:
    """The `.llmy` tensor name of a `config.weight_shapes` key (mhc_alpha maps
    to the three names of _MHC_ALPHA, handled by the writer and reader)."""
    if key == "embed":
        return "embed_tokens.weight"
    if key == "final_norm":
        return "final_norm.weight"
    if key == "stream_seed":
        return "stream_seed"
    if key == "mhc_collapse":
        return "mhc_collapse.weight"
    layer, short = key.split(".", 1)
    l = int(layer[1:])
    if layer[0] in _SIDE:
        # stem.<i> / tail.<i> blocks (model.py:391-394,411-414): GDN mixer,
        # norms, hyper-connection and dense FFN
        p = f"{_SIDE[layer[0]]}.{l}."
        if short in _DENSE:
            return p + _DENSE[short]
        if short in _MHC:
            return p + _MHC[short]
        if short in ("mix_norm", "ffn_norm"):
            return p + _BLOCK[short]
        return p + "mixer." + _GDN[short]
    p = f"recurrent_core.{l}."
    if short in _BLOCK:
        return p + _BLOCK[short]
    if short in _MHC:
        return p + _MHC[short]
    kind = cfg.layer_kinds[l]
    if kind in ("csa", "hca"):
        if short == "cmp_wro":
            return p + "mixer." + ("remote_out.weight" if kind == "csa" else "global_out.weight")
        return p + "mixer." + _CMP[short]
    table = _ATTN if kind == "attn" else _GDN
    return p + "mixer." + table[short]


def config_text(cfg: HybridConfig) -> str:
    keys = {
        "vocab_size": cfg.vocab, "d_model": cfg.d_model, "num_loops": cfg.num_loops,
        "stem_blocks": cfg.stem_blocks, "tail_blocks": cfg.tail_blocks,
        "dense_ffn.hidden": cfg.dense_hidden,
        "physical_blocks": cfg.stem_blocks + cfg.n_layers + cfg.tail_blocks,
        "recurrent_blocks": cfg.n_layers,
        "recurrent_layout": ",".join(cfg.layer_kinds), "mhc.enabled": int(cfg.mhc_streams > 1),
        "mhc.streams": cfg.mhc_streams, "mhc.sinkhorn_iterations": cfg.mhc_sinkhorn_iters,
        "attn.heads": cfg.attn_heads, "attn.head_dim": cfg.attn_head_dim,
        "attn.window": cfg.window,
        "gdn.qk_heads": cfg.gdn_heads, "gdn.value_heads": cfg.gdn_heads,
        "gdn.qk_head_dim": cfg.gdn_dk, "gdn.value_head_dim": cfg.gdn_dv,
        "gdn.conv_kernel": cfg.conv_kernel,
        "moe.routed_experts": cfg.n_experts, "moe.routed_top_k": cfg.top_k,
        "moe.expert_hidden": cfg.expert_hidden, "moe.shared_experts": cfg.shared_experts,
        "router.context_aware": int(cfg.context_router),
        "router.local_context": cfg.router_context, "mla.latent_dim": cfg.latent_dim,
        "router.query_heads": cfg.router_heads, "router.query_head_dim": cfg.router_head_dim,
        "rms_norm_eps": repr(float(cfg.eps)),
        "csa.temporal_compression": cfg.csa_ratio, "csa.local_window": cfg.csa_window,
        "csa.index_heads": cfg.csa_heads, "csa.index_head_dim": cfg.csa_head_dim,
        "csa.index_top_k": cfg.csa_top_k, "hca.temporal_compression": cfg.hca_ratio,
        "hca.local_window": cfg.hca_window, "hca.dense_global_attention": int(cfg.hca_dense),
        "hca.global_top_k": cfg.hca_top_k, "memory.decode_slots": cfg.cmp_slots,
    }
    return "".join(f"{k}={keys[k]}\n" for k in sorted(keys))


def config_from_text(text: str) -> HybridConfig:
    kv = dict(line.split("=", 1) for line in text.splitlines() if "=" in line)
    # every core block carries a MoE: "gdn_moe" and "gdn" name the same block
    kinds = tuple(k[:-4] if k.endswith("_moe") else k for k in kv["recurrent_layout"].split(","))
    _refuse_unsupported(kv, kinds)
    if kv.get("gdn.qk_heads") != kv.get("gdn.value_heads"):
        raise ValueError("GDN q/k and value head counts must match")
    return HybridConfig(
        d_model=int(kv["d_model"]), layer_kinds=kinds, attn_heads=int(kv.get("attn.heads", 0)),
        attn_head_dim=int(kv.get("attn.head_dim", 0)), window=int(kv.get("attn.window", 0)),
        gdn_heads=int(kv["gdn.qk_heads"]), gdn_dk=int(kv["gdn.qk_head_dim"]),
        gdn_dv=int(kv["gdn.value_head_dim"]), n_experts=int(kv["moe.routed_experts"]),
        top_k=int(kv["moe.routed_top_k"]), expert_hidden=int(kv["moe.expert_hidden"]),
        vocab=int(kv["vocab_size"]), num_loops=int(kv["num_loops"]),
        conv_kernel=int(kv.get("gdn.conv_kernel", 4)), eps=float(kv.get("rms_norm_eps", 1e-6)),
        shared_experts=int(kv.get("moe.shared_experts", 0)),
        # absent keys take the reference defaults (llmy_cuda/include/config.h:60-66)
        context_router=_parse_bool(kv.get("router.context_aware", "1")),
        router_context=int(kv.get("router.local_context", 128)),
        latent_dim=int(kv.get("mla.latent_dim", 256)),
        router_heads=int(kv.get("router.query_heads", 4)),
        router_head_dim=int(kv.get("router.query_head_dim", 64)),
        # CSA / HCA keys with the reference defaults (llmy_cuda/include/config.h:41-51)
        csa_ratio=int(kv.get("csa.temporal_compression", 4)),
        csa_window=int(kv.get("csa.local_window", 128)),
        csa_heads=int(kv.get("csa.index_heads", 16)),
        csa_head_dim=int(kv.get("csa.index_head_dim", 128)),
        csa_top_k=int(kv.get("csa.index_top_k", 32)),
        hca_ratio=int(kv.get("hca.temporal_compression", 32)),
        hca_window=int(kv.get("hca.local_window", 128)),
        hca_dense=_parse_bool(kv.get("hca.dense_global_attention", "1")),
        hca_top_k=int(kv.get("hca.global_top_k", 32)),
        cmp_slots=int(kv.get("memory.decode_slots", 256)),
        stem_blocks=int(kv.get("stem_blocks", 0)), tail_blocks=int(kv.get("tail_blocks", 0)),
        dense_hidden=int(kv.get("dense_ffn.hidden", 3584)),
        **_mhc_from(kv))


def _refuse_unsupported(kv: dict, kinds: tuple) -> None:
    """Config keys that change the reference model's math in ways this block
    stack does not run are refused with a message rather than ignored."""
    def on(key, dflt):
        return _parse_bool(kv.get(key, dflt))
    if on("loop_attnres.enabled", "0"):
        raise ValueError("loop_attnres.enabled: the loop-attention residual (model/loop_memory.py) "
                         "is not part of this block stack")
    if on("adaptive_loops.enabled", "0"):
        raise ValueError("adaptive_loops.enabled: learned halting (model.py:521-538) is not part "
                         "of this block stack; run a fixed loop count")
    if not on("mhc.shared_across_loops", "1"):
        raise ValueError("mhc.shared_across_loops = 0: per-loop block copies (model.py:397-408) "
                         "are not part of this block stack")
    if not on("mhc.preserve_streams_across_loop_boundary", "1"):
        raise ValueError("mhc.preserve_streams_across_loop_boundary = 0: the per-loop stream reset "
                         "(model.py:634-635) is not part of this block stack")
    if ("hca" in kinds and on("router.context_aware", "1")
            and not on("router.use_hca_global_latents", "1")):
        # both reference implementations build the router without this key
        # (model/model.py:112-117, llmy_cuda/src/config.cpp) and always attend
        # to the HCA summaries, so a file that turns it off asks for math that
        # neither reference runs
        raise ValueError("router.use_hca_global_latents = 0 with HCA blocks: the reference "
                         "models ignore this key and always use the HCA global branch")
    if int(kv.get("physical_blocks", -1)) not in (-1, int(kv.get("stem_blocks", 0)) + len(kinds)
                                                  + int(kv.get("tail_blocks", 0))):
        raise ValueError("physical_blocks must equal stem + recurrent + tail blocks")


def _mhc_from(kv: dict) -> dict:
    """mhc.* keys with the reference's defaults (llmy_cuda/include/config.h:27-29):
    streams read through the maps when mhc.enabled, else one stream."""
    if _parse_bool(kv.get("mhc.enabled", "1")):
        s = int(kv.get("mhc.streams", 4))
        if s not in (2, 4):
            raise ValueError("mhc.streams must be 2 or 4")
        return {"mhc_streams": s, "mhc_sinkhorn_iters": int(kv.get("mhc.sinkhorn_iterations", 20))}
    if int(kv.get("mhc.streams", 1)) != 1:
        raise ValueError("streams without mHC maps (mhc.enabled = 0, mhc.streams > 1) are not "
                         "part of this block stack")
    return {"mhc_streams": 1}


def _parse_bool(s: str) -> bool:
    """The reference's boolean config values (llmy_cuda/src/config.cpp:18-22)."""
    if s in ("1", "true", "True", "yes"):
        return True
    if s in ("0", "false", "False", "no"):
        return False
    raise ValueError(f"expected bool, got: {s}")


def llmy_entries(cfg: HybridConfig, weights: dict[str, torch.Tensor]) -> list:
    """(file name, tensor) of every weight in a `.llmy` file, sorted by name:
    the reference's state-dict names and shapes with expert lists stacked
    (the depthwise conv as nn.Conv1d's [D, 1, K], the mHC alphas and gating
    logit as 0-d tensors)."""
    from .config import weight_shapes
    entries = []
    for key, shape, _ in weight_shapes(cfg):
        t = weights[key].detach().to("cpu").contiguous()
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"{key}: shape {tuple(t.shape)} != {shape}")
        if key.endswith(".conv"):
            t = t.view(shape[0], 1, shape[1])
        if key.endswith(".mhc_alpha"):  # three 0-d parameters in the reference
            pre = file_name(cfg, key.replace("mhc_alpha", "mhc_map_norm")).rsplit("mhc.", 1)[0]
            entries += [(pre + n, t[i].reshape(())) for i, n in enumerate(_MHC_ALPHA)]
            continue
        if key.endswith(".mhc_gating"):
            t = t.reshape(())
        entries.append((file_name(cfg, key), t))
    entries.sort(key=lambda e: e[0])
    return entries


def save_llmy(path: str | Path, cfg: HybridConfig, weights: dict[str, torch.Tensor]) -> None:
    """Write ``weights`` (keys of `config.weight_shapes`) as a `.llmy` v1 file."""
    entries = llmy_entries(cfg, weights)
    cfg_b = config_text(cfg).encode()
    head = MAGIC + struct.pack("<II", VERSION, len(cfg_b)) + cfg_b + struct.pack("<I", len(entries))
    index_end = len(head) + INDEX_ENTRY.size * len(entries)
    data_start = (index_end + DATA_ALIGN - 1) // DATA_ALIGN * DATA_ALIGN
    index, blobs, off = [], [], 0
    for name, t in entries:
        if t.dtype not in DTYPES:
            raise ValueError(f"{name}: unsupported dtype {t.dtype}")
        blob = t.view(torch.uint8).numpy().tobytes() if t.dtype == torch.bfloat16 else t.numpy().tobytes()
        nb = name.encode()
        if len(nb) > 63 or t.dim() > 4:
            raise ValueError(f"{name}: name longer than 63 bytes or more than 4 dims")
        shape4 = list(t.shape) + [0] * (4 - t.dim())
        index.append(INDEX_ENTRY.pack(len(nb), nb.ljust(64, b"\0"), DTYPES[t.dtype], t.dim(),
                                      *shape4, off, len(blob)))
        blobs.append(blob)
        off += len(blob)
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"".join(index))
        f.write(b"\0" * (data_start - index_end))
        for blob in blobs:
            f.write(blob)


def read_llmy(path: str | Path) -> tuple[str, dict[str, torch.Tensor]]:
    """(config text, {name: tensor}) of a `.llmy` v1 file, with the bounds
    checks of the native reader."""
    data = Path(path).read_bytes()
    if data[:4] != MAGIC:
        raise ValueError("not an .llmy file (bad magic)")
    version, cfg_len = struct.unpack_from("<II", data, 4)
    if version != VERSION:
        raise ValueError(f"unsupported .llmy version {version}")
    p = 12 + cfg_len
    text = data[12:p].decode()
    (n,) = struct.unpack_from("<I", data, p)
    p += 4
    index_end = p + n * INDEX_ENTRY.size
    if index_end > len(data):
        raise ValueError("truncated index")
    data_start = (index_end + DATA_ALIGN - 1) // DATA_ALIGN * DATA_ALIGN
    out = {}
    for i in range(n):
        nl, name, dt, nd, s0, s1, s2, s3, off, nbytes = INDEX_ENTRY.unpack_from(data, p + i * 108)
        if nl > 63 or nd > 4:
            raise ValueError("bad index entry (name length or rank)")
        name = name[:nl].decode()
        shape = (s0, s1, s2, s3)[:nd]
        if dt not in DTYPE_OF or nbytes != int(np.prod(shape, dtype=np.int64)) * ITEMSIZE[dt]:
            raise ValueError(f"{name}: bad dtype or size")
        if data_start + off + nbytes > len(data):
            raise ValueError(f"{name}: payload out of the file")
        raw = torch.frombuffer(bytearray(data[data_start + off:data_start + off + nbytes]),
                               dtype=torch.uint8)
        out[name] = raw.view(DTYPE_OF[dt]).view(shape)
    return text, out


def load_weights(path: str | Path) -> tuple[HybridConfig, dict[str, torch.Tensor]]:
    """Config and `config.weight_shapes`-keyed weights of a `.llmy` file."""
    from .config import weight_shapes
    text, tensors = read_llmy(path)
    cfg = config_from_text(text)
    w = {}
    for key, shape, _ in weight_shapes(cfg):
        if key.endswith(".mhc_alpha"):
            pre = file_name(cfg, key.replace("mhc_alpha", "mhc_map_norm")).rsplit("mhc.", 1)[0]
            w[key] = torch.stack([tensors[pre + n].reshape(()) for n in _MHC_ALPHA])
            continue
        w[key] = tensors[file_name(cfg, key)].reshape(shape)
    return cfg, w
