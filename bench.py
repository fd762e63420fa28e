"""Headline benchmark: bs=64 hybrid-MoE decode step on one MI355X.

A step is one decode token for all 64 sequences through the full stack —
embedding, 12 layers (6 banded-attention + 6 GDN, each with a 24-expert
SwiGLU MoE) looped twice, final norm, tied LM head and greedy argmax — with
the KV caches pre-filled to the 2048-token window and random fp32 GDN states,
captured once into a HIP graph and replayed.  Inputs and state are resident
in HBM before the timed region.  Weights are random N(0, 0.02) drawn on the
GPU from seed 0 (synthetic; no checkpoint).

Also reported on the same JSON line:
  roofline      the dominant kernel of the step, timed alone with HIP events
                on its own stream over rotated state buffers, against the
                HBM peak (8 TB/s);
  cpu_baseline  the oracle (fp32 PyTorch restatement of the reference math)
                on the host cores, on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-iters", type=int, default=50)
    return ap.parse_args()


def fill_state(eng, gen):
    import torch
    cfg = eng.cfg
    eng.pos.fill_(cfg.window)
    for st in eng.state.values():
        if "k" in st:
            st["k"].normal_(0.0, 1.0, generator=gen)
            st["v"].normal_(0.0, 1.0, generator=gen)
        else:
            st["S"].normal_(0.0, 0.1, generator=gen)
            st["hist"].normal_(0.0, 1.0, generator=gen)
    torch.cuda.synchronize()


def time_attn_decode(cfg, B, iters, gen):
    """Average duration of llmy_banded_attn_decode_bf16 at the C5 shape, HIP
    events on the launch stream, rotating 3 cache sets (1.6 GB) so the
    256 MB Infinity Cache cannot serve the window."""
    import torch
    from hybrid_llm_amd import _lib
    H, hd, W = cfg.attn_heads, cfg.attn_head_dim, cfg.window
    sets = []
    for _ in range(3):
        kc = torch.empty(B, H, W, hd, dtype=torch.bfloat16, device="cuda").normal_(generator=gen)
        vc = torch.empty_like(kc).normal_(generator=gen)
        qkv = torch.empty(B, 3 * H * hd, dtype=torch.bfloat16, device="cuda").normal_(generator=gen)
        sets.append((kc, vc, qkv))
    pos = torch.full((B,), W, dtype=torch.int32, device="cuda")
    out = torch.empty(B, H, hd, dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream

    def launch(i):
        kc, vc, qkv = sets[i % 3]
        Hhd = H * hd
        p = qkv.data_ptr()
        _lib.call("llmy_banded_attn_decode_bf16", p, p + 2 * Hhd, p + 4 * Hhd, 3 * Hhd, 3 * Hhd,
                  kc.data_ptr(), vc.data_ptr(), pos.data_ptr(), out.data_ptr(), B, H, hd, W,
                  cfg.attn_scale, sp)

    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for i in range(5):
            launch(i)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(iters):
            launch(i)
        end.record(stream)
    end.synchronize()
    us = start.elapsed_time(end) * 1e3 / iters
    # algorithmic bytes: K and V windows read, new K/V written, q/k/v/out rows
    bytes_ = 2 * B * H * W * hd * 2 + 2 * B * H * hd * 2 + 4 * B * H * hd * 2
    del sets
    torch.cuda.empty_cache()
    return us, bytes_


def cpu_baseline(B, seconds_budget=30.0):
    """Oracle (fp32 torch on the host) on a bounded sample: one decode step of
    a C5-shaped slice — one attention + one GDN layer with their MoEs, one
    loop, batch 64, 2048-token window — scaled to the full step (12 such
    layer pairs plus the LM head, which is timed separately)."""
    import torch
    from dataclasses import replace
    from hybrid_llm_amd.config import C5, alternating, init_weights
    from oracle.model import HybridOracle

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    cfg = replace(C5, layer_kinds=alternating(2), num_loops=1)
    w = init_weights(cfg, seed=0)
    ora = HybridOracle(cfg, w, act_bf16=False)
    st = ora.new_state(B)
    g = torch.Generator().manual_seed(2)
    st["pos"].fill_(cfg.window)
    for key, s in st.items():
        if key == "pos":
            continue
        for name, t in s.items():
            t.normal_(0.0, 0.1 if name == "S" else 1.0, generator=g)
    tokens = torch.randint(0, cfg.vocab, (B,), generator=g)
    ora.step(tokens, st)  # warmup
    t0 = time.perf_counter()
    ora.step(tokens, st)
    t_pair = time.perf_counter() - t0
    # the sample's step includes one LM head; the full step has 12 pairs + 1 head
    hf = torch.randn(B, cfg.d_model, generator=g)
    t0 = time.perf_counter()
    _ = hf @ ora.w["embed"].t()
    t_head = time.perf_counter() - t0
    t_full = 12 * (t_pair - t_head) + t_head
    return {"value": B / t_full, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": (f"oracle fp32 decode step of 1 attention + 1 GDN layer (+MoE) at batch {B},"
                       f" window 2048, timed {t_pair:.2f}s; scaled x12 layer pairs + LM head")}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1"}))
        sys.exit(2)
    import torch
    from hybrid_llm_amd.config import C5, init_weights
    from hybrid_llm_amd.engine import HybridDecoder

    cfg = C5
    B = 64
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    t0 = time.time()
    weights = init_weights(cfg, seed=0, device=dev)
    eng = HybridDecoder(cfg, weights, B, device=dev)
    del weights
    torch.cuda.empty_cache()
    fill_state(eng, gen)
    tokens = torch.randint(0, cfg.vocab, (B,), device=dev, generator=gen, dtype=torch.int64)
    eng.buf["tokens"].copy_(tokens.to(torch.int32))
    eng.capture()
    print(f"[bench] setup {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        eng.graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        eng.graph.replay()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt * 1e3 / args.steps
    value = B / (ms / 1e3)
    print(f"[bench] {ms:.3f} ms/step, {value:.0f} tok/s", file=sys.stderr, flush=True)

    del eng
    torch.cuda.empty_cache()
    us, bytes_ = time_attn_decode(cfg, B, args.kernel_iters, gen)
    achieved = bytes_ / (us * 1e-6) / 1e9
    roofline = {"kernel": "attn_decode_kernel<64>", "bound": "hbm", "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": None, "avg_us": round(us, 2), "bytes_per_launch": bytes_}
    print(f"[bench] attn decode {us:.1f} us, {achieved:.0f} GB/s", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(B)
        print(f"[bench] cpu baseline {cpu['value']:.2f} tok/s", file=sys.stderr, flush=True)

    line = {"metric": "decode tok/s @bs64 (hybrid-MoE decode step, BASELINE config 5)",
            "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "C5 full hybrid-MoE decode step, bs64",
                       "d_model": cfg.d_model, "layers": cfg.n_layers, "loops": cfg.num_loops,
                       "experts": cfg.n_experts, "top_k": cfg.top_k, "window": cfg.window,
                       "global_batch": B, "parallelism": "single GPU"},
            "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
