"""`.llmy` v1 files and the engine API pieces that need no GPU.

* The writer's byte layout against the format of
  llmy_cuda/tools/convert_checkpoint.py:1-31 (magic, version, config,
  108-byte `<I 64s I I 4I Q Q>` index entries, 4 KiB-aligned data start).
* The native parser (llmy_checkpoint_describe) agrees with the writer on the
  config and every tensor, and rejects corrupt files.
* llmy_sample (the reference's CPU sampler) against hand-computed cases and
  the oracle's sampling rule.
* llmy_load without a GPU fails with NULL and a message, never a crash.
"""
import ctypes as C
import struct

import numpy as np
import pytest
import torch

from hybrid_llm_amd import _lib
from hybrid_llm_amd.checkpoint import (INDEX_ENTRY, config_from_text, config_text, file_name,
                                       load_weights, read_llmy, save_llmy)
from hybrid_llm_amd.config import C1, HybridConfig, alternating, init_weights, weight_shapes

TINY = HybridConfig(d_model=256, layer_kinds=alternating(2), attn_heads=4, attn_head_dim=64,
                    window=16, gdn_heads=4, gdn_dk=64, gdn_dv=64, n_experts=4, top_k=2,
                    expert_hidden=256, vocab=512, num_loops=2)


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


@pytest.fixture(scope="module")
def tiny_file(tmp_path_factory):
    path = tmp_path_factory.mktemp("ck") / "tiny.llmy"
    w = init_weights(TINY, seed=3)
    save_llmy(path, TINY, w)
    return path, w


def test_byte_layout(tiny_file):
    path, w = tiny_file
    data = path.read_bytes()
    assert data[:4] == b"LLMY"
    version, cfg_len = struct.unpack_from("<II", data, 4)
    assert version == 1
    text = data[12:12 + cfg_len].decode()
    assert text == config_text(TINY)
    (n,) = struct.unpack_from("<I", data, 12 + cfg_len)
    assert n == len(weight_shapes(TINY))
    index = 16 + cfg_len
    data_start = -(-(index + 108 * n) // 4096) * 4096
    names, expect_off = [], 0
    for i in range(n):
        nl, name, dt, nd, *rest = INDEX_ENTRY.unpack_from(data, index + 108 * i)
        shape, off, nbytes = rest[:4], rest[4], rest[5]
        assert 0 < nl <= 63 and name[nl:] == b"\0" * (64 - nl)
        assert off == expect_off and data_start + off + nbytes <= len(data)
        expect_off += nbytes
        names.append(name[:nl].decode())
    assert names == sorted(names)
    # one payload checked byte for byte: the first GDN beta bias (fp32 zeros)
    # and the embedding (bf16 words)
    _, tensors = read_llmy(path)
    assert torch.equal(tensors["embed_tokens.weight"], w["embed"])
    assert tensors["recurrent_core.1.mixer.conv.weight"].shape == (256, 1, 4)


def test_roundtrip_and_names(tiny_file):
    path, w = tiny_file
    cfg, back = load_weights(path)
    assert cfg == TINY
    for key, t in w.items():
        assert torch.equal(back[key], t), key
    assert file_name(C1, "L0.wq") == "recurrent_core.0.mixer.q.weight"
    assert file_name(C1, "L1.wq") == "recurrent_core.1.mixer.q_proj.weight"
    assert file_name(C1, "L1.bb") == "recurrent_core.1.mixer.beta_proj.bias"
    assert file_name(C1, "L3.w_down") == "recurrent_core.3.moe.experts.down_proj.weight"
    assert config_from_text(config_text(C1)) == C1


def _describe(lib, path):
    buf = C.create_string_buffer(1 << 20)
    st = lib.llmy_checkpoint_describe(str(path).encode(), buf, len(buf))
    return st, buf.value.decode()


def test_native_parser_agrees(lib, tiny_file):
    path, _ = tiny_file
    st, text = _describe(lib, path)
    assert st == 0, lib.llmy_last_error()
    cfg_part, tensor_part = text.split("--\n")
    assert cfg_part == config_text(TINY)
    _, tensors = read_llmy(path)
    lines = [l.split() for l in tensor_part.strip().splitlines()]
    assert [l[0] for l in lines] == sorted(tensors)
    for name, dt, nd, d0, d1, d2, d3, nb in lines:
        t = tensors[name]
        assert int(nd) == t.dim() and [int(x) for x in (d0, d1, d2, d3)][:t.dim()] == list(t.shape)
        assert int(nb) == t.numel() * t.element_size()
        assert int(dt) == {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[t.dtype]


def test_shared_experts_roundtrip(lib, tmp_path):
    """Shared experts travel as moe.shared.{gate,up,down}_proj.weight, stacked
    [S, H, D] / [S, D, H] (model/layers/moe.py:110), with moe.shared_experts=S
    in the config; both parsers read them back unchanged."""
    from dataclasses import replace
    cfg = replace(TINY, shared_experts=2)
    w = init_weights(cfg, seed=4)
    path = tmp_path / "shared.llmy"
    save_llmy(path, cfg, w)
    back_cfg, back = load_weights(path)
    assert back_cfg == cfg and "moe.shared_experts=2\n" in config_text(cfg)
    for key, t in w.items():
        assert torch.equal(back[key], t), key
    assert file_name(cfg, "L0.w_shared_down") == "recurrent_core.0.moe.shared.down_proj.weight"
    assert back["L1.w_shared_gate"].shape == (2, 256, 256)
    st, text = _describe(lib, path)
    assert st == 0, lib.llmy_last_error()
    names = [l.split()[0] for l in text.split("--\n")[1].strip().splitlines()]
    assert sum(".moe.shared." in n for n in names) == 3 * cfg.n_layers


def test_context_router_roundtrip(lib, tmp_path):
    """Context-aware router weights under the reference's names
    (llmy_cuda/src/model.cpp:89-116), the route gate as a 0-d tensor, and the
    three config keys; an absent router.context_aware reads as true, the
    reference default (llmy_cuda/include/config.h:63)."""
    from dataclasses import replace
    cfg = replace(TINY, context_router=True, router_context=32)
    w = init_weights(cfg, seed=5)
    assert w["L0.ctx_gate"].shape == () and float(w["L0.ctx_gate"]) == pytest.approx(-4.59512)
    path = tmp_path / "ctx.llmy"
    save_llmy(path, cfg, w)
    back_cfg, back = load_weights(path)
    assert back_cfg == cfg
    for key, t in w.items():
        assert torch.equal(back[key], t), key
    text = config_text(cfg)
    assert "router.context_aware=1\n" in text and "router.local_context=32\n" in text
    assert "mla.latent_dim=256\n" in text
    assert file_name(cfg, "L1.ctx_gate") == "recurrent_core.1.moe.router.route_gate"
    assert file_name(cfg, "L0.ctx_down") == "recurrent_core.0.moe.router.latent_memory.down.weight"
    st, desc = _describe(lib, path)
    assert st == 0, lib.llmy_last_error()
    gate_lines = [l for l in desc.split("--\n")[1].splitlines() if l.endswith("route_gate 0 0 0 0 0 4")
                  or ".route_gate " in l]
    assert len(gate_lines) == cfg.n_layers and all(l.split()[2] == "0" for l in gate_lines)
    plain = "".join(l + "\n" for l in config_text(TINY).splitlines()
                    if not l.startswith("router.context_aware"))
    assert config_from_text(plain).context_router
    assert not config_from_text(config_text(TINY)).context_router
    with pytest.raises(ValueError):
        config_from_text(config_text(TINY).replace("router.context_aware=0", "router.context_aware=2"))


def test_mhc_roundtrip(lib, tmp_path):
    """mHC parameters under the reference's names (llmy_cuda/src/model.cpp:34-63,
    178-180): per block mhc.theta / mapping_norm / biases / stream_scale /
    stream_norm, the alphas and the gating logit as 0-d tensors, stream_seed
    and mhc_collapse.weight; config keys mhc.enabled / streams /
    sinkhorn_iterations with the reference's defaults when absent
    (llmy_cuda/include/config.h:27-29)."""
    from dataclasses import replace
    cfg = replace(TINY, mhc_streams=4, mhc_sinkhorn_iters=10)
    w = init_weights(cfg, seed=6)
    path = tmp_path / "mhc.llmy"
    save_llmy(path, cfg, w)
    back_cfg, back = load_weights(path)
    assert back_cfg == cfg
    for key, t in w.items():
        assert torch.equal(back[key], t), key
    text = config_text(cfg)
    assert "mhc.enabled=1\n" in text and "mhc.streams=4\n" in text
    assert file_name(cfg, "L1.mhc_theta") == "recurrent_core.1.mhc.theta.weight"
    assert file_name(cfg, "mhc_collapse") == "mhc_collapse.weight"
    st, desc = _describe(lib, path)
    assert st == 0, lib.llmy_last_error()
    lines = desc.split("--\n")[1].splitlines()
    names = {l.split()[0]: l.split() for l in lines}
    for n in ("alpha_pre", "alpha_post", "alpha_residual", "gating_logit"):
        assert names[f"recurrent_core.0.mhc.{n}"][2] == "0"          # 0-d
    assert "stream_seed" in names and "mhc_collapse.weight" in names
    # defaults: no mhc keys -> 4 streams, 20 iterations; enabled=0 -> one stream
    bare = "".join(l + "\n" for l in config_text(TINY).splitlines() if not l.startswith("mhc."))
    c0 = config_from_text(bare)
    assert c0.mhc_streams == 4 and c0.mhc_sinkhorn_iters == 20
    assert config_from_text(config_text(TINY)).mhc_streams == 1
    with pytest.raises(ValueError):
        config_from_text(config_text(TINY).replace("mhc.streams=1", "mhc.streams=4"))


@pytest.mark.parametrize("damage", ["magic", "version", "truncate_index", "payload", "name_len",
                                    "shape"])
def test_native_parser_rejects_corrupt_files(lib, tiny_file, tmp_path, damage):
    path, _ = tiny_file
    data = bytearray(path.read_bytes())
    cfg_len = struct.unpack_from("<I", data, 8)[0]
    first = 16 + cfg_len
    if damage == "magic":
        data[:4] = b"LLMZ"
    elif damage == "version":
        struct.pack_into("<I", data, 4, 2)
    elif damage == "truncate_index":
        data = data[:first + 50]
    elif damage == "payload":
        struct.pack_into("<Q", data, first + 92, len(data))  # offset past the end
    elif damage == "name_len":
        struct.pack_into("<I", data, first, 64)
    elif damage == "shape":
        struct.pack_into("<I", data, first + 76, 7)  # shape no longer matches nbytes
    bad = tmp_path / "bad.llmy"
    bad.write_bytes(bytes(data))
    st, _ = _describe(lib, bad)
    assert st != 0
    assert lib.llmy_last_status() != 0 and lib.llmy_last_error()
    with pytest.raises(ValueError):
        read_llmy(bad)


def test_load_without_gpu_fails_cleanly(lib, tiny_file):
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the GPU tests cover llmy_load")
    path, _ = tiny_file
    assert lib.llmy_load(str(path).encode()) is None
    assert lib.llmy_last_status() != 0 and lib.llmy_last_error()
    assert lib.llmy_load(b"/nonexistent.llmy") is None


def _sample(lib, logits, T, k, p, rep=1.0, recent=(), seed=1337):
    x = np.ascontiguousarray(np.asarray(logits, dtype=np.float32))
    rec = (C.c_int32 * max(len(recent), 1))(*recent)
    rng = C.c_uint64(seed)
    tok = lib.llmy_sample(x.ctypes.data_as(C.POINTER(C.c_float)), x.size, T, k, p, rep, rec,
                          len(recent), C.byref(rng))
    return tok, rng.value


def _xorshift(r):
    m = (1 << 64) - 1
    r ^= (r << 13) & m
    r ^= r >> 7
    r ^= (r << 17) & m
    return r


def test_sampler_rules(lib):
    x = np.array([0.5, 3.0, 3.0, -1.0, 2.0], np.float32)
    # greedy: ties to the lower id
    assert _sample(lib, x, 0.0, 0, 0.9)[0] == 1
    # top_k = 1 returns the top id for any temperature
    assert _sample(lib, x, 0.7, 1, 1.0)[0] == 1
    # the generator advances exactly one xorshift64 step per draw
    assert _sample(lib, x, 0.7, 0, 0.9, seed=99)[1] == _xorshift(99)
    # the draw: first id in order whose running probability exceeds u
    r = _xorshift(1337)
    u = (r >> 11) / 2.0 ** 53
    order = [1, 2, 4, 0, 3]
    e = np.exp((x[order] - x.max()) / np.float32(0.7)).astype(np.float64)
    cdf = np.cumsum(e / e.sum())
    want = order[int(np.searchsorted(cdf, u, side="right"))]
    assert _sample(lib, x, 0.7, 0, 1.0)[0] == want
    # repetition penalty divides positive logits, multiplies negative ones
    assert _sample(lib, x, 0.0, 0, 1.0, rep=2.0, recent=(1, 2))[0] == 4


def test_sampler_matches_oracle_rule(lib):
    from oracle.sampling import top_p_sample
    g = np.random.default_rng(0)
    agree = 0
    for trial in range(40):
        x = g.standard_normal(300).astype(np.float32) * 2
        seed = 1000 + trial
        tok, _ = _sample(lib, x, 0.8, 0, 0.9, seed=seed)
        u = (_xorshift(seed) >> 11) / 2.0 ** 53
        # the C sampler caps top-k at 256 (llmy.cpp:139)
        ref, margin = top_p_sample(torch.from_numpy(x[None]), 0.8, float(np.float32(0.9)),
                                   torch.tensor([u]), top_k=256, return_margin=True)
        if margin[0] > 1e-5:
            assert tok == int(ref[0]), trial
            agree += 1
    assert agree >= 30


def test_cmp_roundtrip(lib, tmp_path):
    """CSA / HCA mixers under the reference's names (model/layers/csa.py:21-29,
    hca.py:24-30; llmy_cuda/src/model.cpp:132-160): mixer.query / key / value /
    local_out / out, remote_out (CSA) or global_out (HCA), compressor.key /
    value; csa.* / hca.* keys with the reference defaults when absent
    (llmy_cuda/include/config.h:41-51); the reference's "<kind>_moe" layout
    entries."""
    from dataclasses import replace
    cfg = replace(TINY, layer_kinds=("csa", "gdn", "hca"), csa_heads=2, csa_head_dim=64,
                  csa_window=8, csa_ratio=4, csa_top_k=5, hca_window=6, hca_ratio=8,
                  hca_dense=False, hca_top_k=3, cmp_slots=32)
    w = init_weights(cfg, seed=8)
    path = tmp_path / "cmp.llmy"
    save_llmy(path, cfg, w)
    back_cfg, back = load_weights(path)
    assert back_cfg == cfg
    for key, t in w.items():
        assert torch.equal(back[key], t), key
    assert file_name(cfg, "L0.cmp_wro") == "recurrent_core.0.mixer.remote_out.weight"
    assert file_name(cfg, "L2.cmp_wro") == "recurrent_core.2.mixer.global_out.weight"
    assert file_name(cfg, "L2.cmp_wck") == "recurrent_core.2.mixer.compressor.key.weight"
    assert file_name(cfg, "L0.cmp_wq") == "recurrent_core.0.mixer.query.weight"
    st, desc = _describe(lib, path)
    assert st == 0, lib.llmy_last_error()
    names = {l.split()[0] for l in desc.split("--\n")[1].splitlines()}
    for n in ("query", "key", "value", "local_out", "remote_out", "out", "compressor.key",
              "compressor.value"):
        assert f"recurrent_core.0.mixer.{n}.weight" in names
    assert "recurrent_core.2.mixer.global_out.weight" in names
    # the reference's layout spelling and defaults
    text = config_text(cfg).replace("recurrent_layout=csa,gdn,hca",
                                    "recurrent_layout=csa_moe,gdn_moe,hca_moe")
    bare = "".join(l + "\n" for l in text.splitlines()
                   if not l.startswith(("csa.", "hca.", "memory.")))
    c0 = config_from_text(bare)
    assert c0.layer_kinds == ("csa", "gdn", "hca")
    assert (c0.csa_ratio, c0.csa_window, c0.csa_heads, c0.csa_head_dim, c0.csa_top_k) == \
        (4, 128, 16, 128, 32)
    assert (c0.hca_ratio, c0.hca_window, c0.hca_dense, c0.hca_top_k, c0.cmp_slots) == \
        (32, 128, True, 32, 256)


def test_stem_tail_roundtrip(lib, tmp_path):
    """Stem and tail blocks under the reference's names (stem.<i>. / tail.<i>.
    mixer_norm, ffn_norm, mixer.<GDN>, ffn.gate_proj / up_proj / down_proj,
    mhc.*: model/model.py:391-394,411-414; llmy_cuda/src/model.cpp:81-87,
    205-250) and the keys stem_blocks / tail_blocks / dense_ffn.hidden /
    physical_blocks; the native parser accepts the file."""
    from dataclasses import replace
    cfg = replace(TINY, stem_blocks=1, tail_blocks=2, dense_hidden=320, mhc_streams=4,
                  expert_hidden=320)
    w = init_weights(cfg, seed=9)
    path = tmp_path / "side.llmy"
    save_llmy(path, cfg, w)
    back_cfg, back = load_weights(path)
    assert back_cfg == cfg
    for key, t in w.items():
        assert torch.equal(back[key], t), key
    assert file_name(cfg, "S0.ffn_gate") == "stem.0.ffn.gate_proj.weight"
    assert file_name(cfg, "T1.ffn_down") == "tail.1.ffn.down_proj.weight"
    assert file_name(cfg, "T0.wq") == "tail.0.mixer.q_proj.weight"
    assert file_name(cfg, "S0.mix_norm") == "stem.0.mixer_norm.weight"
    assert file_name(cfg, "S0.mhc_theta") == "stem.0.mhc.theta.weight"
    text = config_text(cfg)
    for kv in ("stem_blocks=1", "tail_blocks=2", "dense_ffn.hidden=320", "physical_blocks=5"):
        assert kv + "\n" in text
    st, desc = _describe(lib, path)
    assert st == 0, lib.llmy_last_error()
    names = {l.split()[0] for l in desc.split("--\n")[1].splitlines()}
    assert {"stem.0.ffn.up_proj.weight", "tail.1.mixer.conv.weight",
            "tail.1.mhc.alpha_pre"} <= names


@pytest.mark.parametrize("key,value", [
    ("loop_attnres.enabled", "true"), ("adaptive_loops.enabled", "1"),
    ("mhc.shared_across_loops", "false"), ("mhc.preserve_streams_across_loop_boundary", "0"),
    ("physical_blocks", "7")])
def test_unsupported_keys_are_refused(lib, tmp_path, key, value):
    """Config keys that change the reference model's math in ways this block
    stack does not run are refused by both readers, with a message, rather
    than ignored (model/config.py:14-15,80-102; model.py:397-408,634-635)."""
    lines = [l for l in config_text(TINY).splitlines() if not l.startswith(key + "=")]
    text = "".join(l + "\n" for l in lines + [f"{key}={value}"])
    with pytest.raises(ValueError, match=key.split(".")[0]):
        config_from_text(text)
    # the same file written with that config text, for the native reader
    from hybrid_llm_amd import checkpoint as ck
    path = tmp_path / "k.llmy"
    orig = ck.config_text
    try:
        ck.config_text = lambda cfg: text
        save_llmy(path, TINY, init_weights(TINY, seed=3))
    finally:
        ck.config_text = orig
    st, _ = _describe(lib, path)
    assert st != 0
    assert key.split(".")[0].encode() in lib.llmy_last_error() or b"physical" in lib.llmy_last_error()


def test_hca_global_latents_off_is_refused():
    """router.use_hca_global_latents = 0 with HCA blocks and the context router:
    both reference implementations ignore the key, so a file asking for it is
    refused; without HCA blocks (the reference training config) it is inert."""
    from dataclasses import replace
    cfg = replace(TINY, layer_kinds=("hca", "gdn"), context_router=True)
    text = config_text(cfg) + "router.use_hca_global_latents=false\n"
    with pytest.raises(ValueError, match="use_hca_global_latents"):
        config_from_text(text)
    plain = config_text(replace(TINY, context_router=True)) + "router.use_hca_global_latents=0\n"
    assert config_from_text(plain).context_router
