"""Headline benchmark: bs=64 hybrid-MoE decode step on one MI355X.

A step is one decode token for all 64 sequences through the full stack —
embedding, 12 layers (6 banded-attention + 6 GDN, each with a 24-expert
SwiGLU MoE) looped twice, final norm, tied LM head, greedy argmax and a
temperature-0.8 / top-p-0.9 draw from a fixed per-row uniform — with the KV
caches pre-filled to the 2048-token window and random fp32 GDN states,
captured once into a HIP graph and replayed.  Inputs and state are resident
in HBM before the timed region.  Weights are random N(0, 0.02) drawn on the
GPU from seed 0 (synthetic; no checkpoint).

Also reported on the same JSON line:
  roofline      the dominant kernel of the step (banded attention decode),
                timed alone over rotated cache sets with one pair of HIP
                events on its launch stream around the timed region's
                launches (``avg_us`` = elapsed / launches; the mean and median
                of per-launch event pairs are reported beside it), against
                the HBM peak (8 TB/s); ``traffic`` is its
                HBM bytes per launch from two rocprofv3 --pmc runs (FETCH_SIZE,
                WRITE_SIZE) of this script's --pmc-child mode, each scaled by
                the counter's reading for a plain copy of known size;
  kernels       the other hot-path kernels the metric names (MoE, attention,
                GDN; decode and prefill), each timed the same way against the
                HBM or bf16-MFMA peak;
  cpu_baseline  the oracle (fp32 PyTorch restatement of the reference math)
                on the host cores, on the same workload (the full C5 step at
                batch 64): 1 warmup + median of 3 steps.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0   # dense bf16 MFMA
METRIC = "decode tok/s @bs64 + per-kernel % of HBM/MFMA roofline (MoE, attn, GDN)"
SAMPLING = (0.8, 0.9, 0)         # temperature, top_p, top_k (0 = off)
COPY_BYTES = 1 << 29             # calibration copy: 512 MiB read + 512 MiB written


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 --pmc runs (e.g. when already under a profiler)")
    ap.add_argument("--no-kernels", action="store_true", help="skip the per-kernel table")
    ap.add_argument("--kernel-iters", type=int, default=100)
    ap.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--only", default=None,
                    help="comma-separated kernel-table rows to run alone (after a 512 MiB "
                         "device copy that calibrates HBM counters), e.g. attn_prefill; "
                         "prints those rows as JSON and exits")
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


_SLEEP_MS_PER_MCYCLE = None


def _sleep_rate():
    """Milliseconds of ``torch.cuda._sleep(1_000_000)`` on this GPU (event-timed once)."""
    global _SLEEP_MS_PER_MCYCLE
    if _SLEEP_MS_PER_MCYCLE is None:
        import torch
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(100_000)
        a.record()
        torch.cuda._sleep(1_000_000)
        b.record()
        b.synchronize()
        _SLEEP_MS_PER_MCYCLE = max(a.elapsed_time(b), 1e-3)
    return _SLEEP_MS_PER_MCYCLE


def event_time(launch, iters, warm=10):
    """Duration (us) of ``launch(i)`` on a stream of its own: each of ``iters``
    launches (after ``warm`` untimed ones) is bracketed by its own pair of HIP
    events recorded on that stream.  A sleep kernel queued ahead of the timed
    launches keeps the GPU busy while the host enqueues them (sized from the
    host time of the warmup launches), so the launches run back to back and
    each pair measures device time, not the Python wrapper's launch gaps.
    Returns (mean, median) over the launches."""
    import torch
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        t0 = time.perf_counter()
        for i in range(warm):
            launch(i)
        host_ms = (time.perf_counter() - t0) * 1e3 / max(warm, 1)
        stream.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(iters)]
        sleep_ms = min(2.0 + 2.0 * host_ms * iters, 2000.0)
        torch.cuda._sleep(int(sleep_ms / _sleep_rate() * 1e6))
        for i, (a, b) in enumerate(ev):
            a.record(stream)
            launch(warm + i)
            b.record(stream)
    ev[-1][1].synchronize()
    us = sorted(a.elapsed_time(b) * 1e3 for a, b in ev)
    mid = len(us) // 2
    median = us[mid] if len(us) % 2 else 0.5 * (us[mid - 1] + us[mid])
    return sum(us) / len(us), median


def region_time(launch, iters, warm=10):
    """Average duration (us) of ``launch(i)`` over one timed region: ``iters``
    launches back to back on a stream of their own between a single pair of HIP
    events (after ``warm`` untimed launches and a sleep kernel that keeps the GPU
    busy while the host enqueues them), divided by ``iters``.  Unlike
    event_time, no event is recorded between the launches."""
    import torch
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        t0 = time.perf_counter()
        for i in range(warm):
            launch(i)
        host_ms = (time.perf_counter() - t0) * 1e3 / max(warm, 1)
        stream.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        sleep_ms = min(2.0 + 2.0 * host_ms * iters, 2000.0)
        torch.cuda._sleep(int(sleep_ms / _sleep_rate() * 1e6))
        a.record(stream)
        for i in range(iters):
            launch(warm + i)
        b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) * 1e3 / iters


def attn_decode_sets(cfg, B, gen):
    """3 rotated cache sets (1.6 GB) so the 256 MB Infinity Cache cannot serve
    the window between launches."""
    import torch
    H, hd, W = cfg.attn_heads, cfg.attn_head_dim, cfg.window
    sets = []
    for _ in range(3):
        kc = torch.empty(B, H, W, hd, dtype=torch.bfloat16, device="cuda").normal_(generator=gen)
        vc = torch.empty_like(kc).normal_(generator=gen)
        # q/k/v as the decode step hands them over: the projection's partial
        # products, 4 fp32 slices (d_model / 256) of [B, 3 H hd]
        parts = torch.empty(cfg.d_model // 256, B, 3 * H * hd, device="cuda").normal_(
            generator=gen)
        sets.append((kc, vc, parts))
    return sets


def attn_decode_launcher(cfg, B, sets):
    import torch
    from hybrid_llm_amd import _lib
    H, hd, W = cfg.attn_heads, cfg.attn_head_dim, cfg.window
    pos = torch.full((B,), W, dtype=torch.int32, device="cuda")
    out = torch.empty(B, H, hd, dtype=torch.bfloat16, device="cuda")

    def launch(i):
        kc, vc, parts = sets[i % 3]
        Hhd = H * hd
        _lib.call("llmy_banded_attn_decode_parts_bf16", parts.data_ptr(), parts.shape[0],
                  parts.stride(0), parts.stride(1), Hhd, 2 * Hhd, kc.data_ptr(), vc.data_ptr(),
                  pos.data_ptr(), out.data_ptr(), B, H, hd, W, cfg.attn_scale,
                  torch.cuda.current_stream().cuda_stream)
    return launch


def attn_decode_bytes(cfg, B):
    """Algorithmic bytes of one decode launch as the step runs it: the K and V
    windows read, the new K/V rows written (bf16), the q/k/v partial products
    read (d_model / 256 fp32 slices) and the output written (bf16)."""
    H, hd, W = cfg.attn_heads, cfg.attn_head_dim, cfg.window
    P = cfg.d_model // 256
    return 2 * B * H * W * hd * 2 + 2 * B * H * hd * 2 + P * 3 * B * H * hd * 4 + B * H * hd * 2


def step_bytes(cfg, B: int) -> dict:
    """Algorithmic HBM bytes of one decode step (every weight, cache and state
    byte the step must move once), by component; experts count the expected
    number of distinct experts hit by B*top_k routes drawn over E."""
    E, k, D, H = cfg.n_experts, cfg.top_k, cfg.d_model, cfg.expert_hidden
    apps = cfg.num_loops * cfg.n_layers
    n_attn = cfg.num_loops * sum(1 for kd in cfg.layer_kinds if kd == "attn")
    n_gdn = apps - n_attn
    Ha, hd, W = cfg.attn_heads, cfg.attn_head_dim, cfg.window
    Hg, dk, dv = cfg.gdn_heads, cfg.gdn_dk, cfg.gdn_dv
    distinct = E * (1.0 - (1.0 - k / E) ** B)
    parts = {
        "experts": apps * distinct * 3 * H * D * 2,
        "attn_projections": n_attn * 4 * D * Ha * hd * 2,
        "gdn_projections": n_gdn * ((2 * Hg * dk + 2 * Hg * dv + Hg) * D + D * Hg * dv) * 2,
        "kv_reads": n_attn * 2 * B * Ha * W * hd * 2,
        "kv_writes": n_attn * 2 * B * Ha * hd * 2,
        "gdn_state": n_gdn * 2 * B * Hg * dk * dv * 4,
        "router": apps * E * D * 4,
        "lm_head": cfg.vocab * D * 2,
        "logits": 2 * B * cfg.vocab * 4,
    }
    parts["total"] = sum(parts.values())
    return parts


def time_attn_decode(cfg, B, iters, gen):
    import torch
    sets = attn_decode_sets(cfg, B, gen)
    launch = attn_decode_launcher(cfg, B, sets)
    t = event_time(launch, iters)
    region = region_time(launch, iters)
    del sets
    torch.cuda.empty_cache()
    return t, region, attn_decode_bytes(cfg, B)


# --------------------------------------------------------------------------- HBM traffic
def copy_calibration():
    """Three plain device copies of COPY_BYTES: a counter run divides a kernel's
    FETCH_SIZE / WRITE_SIZE by these launches' reading per byte copied."""
    import torch
    gen = torch.Generator(device="cuda").manual_seed(1)
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device="cuda").normal_(generator=gen)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


def pmc_child():
    """Run under ``rocprofv3 --pmc``: a plain device copy of COPY_BYTES (the
    calibration), then the dominant kernel at the bench shape."""
    import torch
    from hybrid_llm_amd.config import C5
    torch.cuda.set_device(0)
    gen = torch.Generator(device="cuda").manual_seed(0)
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device="cuda").normal_(generator=gen)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()
    sets = attn_decode_sets(C5, 64, gen)
    launch = attn_decode_launcher(C5, 64, sets)
    for i in range(9):
        launch(i)
    torch.cuda.synchronize()
    print("[pmc-child] done", flush=True)


def _pmc_run(counter, outdir):
    """One rocprofv3 pass collecting ``counter``; returns {kernel name: [values]}."""
    cmd = ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", outdir, "-o", "pmc",
           "--", sys.executable, os.path.abspath(__file__), "--pmc-child"]
    subprocess.run(cmd, check=True, timeout=240, stdout=subprocess.DEVNULL,
                   stderr=subprocess.DEVNULL, cwd=ROOT)
    per: dict[str, dict[int, float]] = {}
    for path in glob.glob(os.path.join(outdir, "**", "*counter_collection.csv"), recursive=True):
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                d = per.setdefault(row["Kernel_Name"], {})
                key = int(row["Dispatch_Id"])
                d[key] = d.get(key, 0.0) + float(row["Counter_Value"])
    return {k: [v[i] for i in sorted(v)] for k, v in per.items()}


def measure_traffic():
    """HBM bytes per launch of the decode attention kernel: FETCH_SIZE and
    WRITE_SIZE (KiB per dispatch) each divided by the same counter's reading
    per byte of a plain 512 MiB device copy.  Runs before this process touches
    the GPU; any failure yields None."""
    if shutil.which("rocprofv3") is None:
        return None
    out = {}
    try:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            with tempfile.TemporaryDirectory(prefix="llmy_pmc_") as d:
                per = _pmc_run(counter, d)
            copy = [v for k, vals in per.items() if "copy" in k.lower() for v in vals]
            attn = [v for k, vals in per.items() if "attn_decode_kernel" in k for v in vals]
            if not copy or len(attn) < 4:
                return None
            factor = (sum(copy) / len(copy)) * 1024.0 / COPY_BYTES
            attn = attn[3:]  # the first launches warm the caches' tags
            out[counter] = {"kib_per_launch": sum(attn) / len(attn), "copy_factor": factor}
    except (subprocess.SubprocessError, OSError, ValueError, KeyError):
        return None
    fetch = out["FETCH_SIZE"]["kib_per_launch"] * 1024.0 / out["FETCH_SIZE"]["copy_factor"]
    write = out["WRITE_SIZE"]["kib_per_launch"] * 1024.0 / out["WRITE_SIZE"]["copy_factor"]
    return {"bytes": fetch + write, "fetch_bytes": fetch, "write_bytes": write,
            "fetch_copy_factor": out["FETCH_SIZE"]["copy_factor"],
            "write_copy_factor": out["WRITE_SIZE"]["copy_factor"]}


# --------------------------------------------------------------------------- kernel table
MALL_BYTES = 256 << 20   # Infinity Cache: rotated input sets must exceed it


def n_sets(bytes_per_set: float, minimum: int = 3) -> int:
    """Number of rotated input sets whose total exceeds the Infinity Cache."""
    return max(minimum, int(MALL_BYTES // max(bytes_per_set, 1)) + 1)


KERNEL_ROWS = ("hbm_copy", "mfma_gemm", "moe_decode_experts", "lm_head", "gdn_decode_step", "gdn_decode_step_c4",
               "sample_argmax", "sample_top_p", "moe_prefill_layer", "moe_prefill_experts",
               "dense_prefill_gemm", "attn_prefill", "gdn_prefill", "csa_decode", "hca_decode",
               "csa_prefill", "hca_prefill")


def kernel_table(cfg, B, gen, iters, only=None):
    """Per-kernel roofline fractions for the kernels the metric names.  Every
    row: HIP events around each launch on the launch stream, 10 warmup
    launches, mean and median over ``iters``; bandwidth-bound rows rotate
    input sets totalling more than the 256 MB Infinity Cache.  ``only``: the
    row names to run (each row sets up its own inputs)."""
    import torch
    import torch.nn.functional as F
    from hybrid_llm_amd import _lib, ops
    rows = {}

    def hbm(name, t, bytes_, workload):
        us, med = t
        gbs = bytes_ / (us * 1e-6) / 1e9
        rows[name] = {"workload": workload, "bound": "hbm", "avg_us": round(us, 2),
                      "median_us": round(med, 2), "bytes": round(bytes_),
                      "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(gbs / HBM_PEAK_GBS, 4)}

    def mfma(name, t, flops, workload):
        us, med = t
        tf = flops / (us * 1e-6) / 1e12
        rows[name] = {"workload": workload, "bound": "mfma", "avg_us": round(us, 2),
                      "median_us": round(med, 2), "flops": round(flops),
                      "achieved": round(tf, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                      "unit": "TFLOP/s", "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)}

    def latency(name, t, workload):
        us, med = t
        rows[name] = {"workload": workload, "bound": "latency", "avg_us": round(us, 2),
                      "median_us": round(med, 2)}

    D, E, Hf, k = cfg.d_model, cfg.n_experts, cfg.expert_hidden, cfg.top_k
    Hg, dk, dv = cfg.gdn_heads, cfg.gdn_dk, cfg.gdn_dv
    V = cfg.vocab
    it_mfma = max(10, iters // 5)
    strm = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    def hbm_copy():
        # the practical ceiling of a read + write stream: a plain 512 MiB device
        # copy (torch), bytes = read + written; 2 rotated source buffers
        n = COPY_BYTES // 4
        srcs = [torch.empty(n, device="cuda").normal_(generator=gen) for _ in range(2)]
        dst = torch.empty(n, device="cuda")
        t = event_time(lambda i: dst.copy_(srcs[i % 2]), max(10, iters // 5))
        hbm("hbm_copy", t, 2 * COPY_BYTES, "torch device copy of 512 MiB (read + write)")

    def mfma_gemm():
        # the practical ceiling of a bf16 MFMA stream on this box: a library
        # GEMM (torch.matmul -> hipBLASLt) of random bf16 operands, 8192^3
        # (random operands draw more power than constant ones; the clock, and
        # with it the matrix rate, drops to match)
        n = 8192
        a = torch.randn(n, n, device="cuda", generator=gen).bfloat16()
        bt = torch.randn(n, n, device="cuda", generator=gen).bfloat16()
        c = torch.empty(n, n, device="cuda", dtype=torch.bfloat16)
        t = event_time(lambda i: torch.matmul(a, bt, out=c), max(10, iters // 10))
        mfma("mfma_gemm", t, 2 * n ** 3, "hipBLASLt bf16 GEMM (torch.matmul), random operands, "
             "M=N=K=8192: the practical MFMA ceiling")

    def moe_decode_experts():
        # one C5 MoE application at decode: packed expert weights (302 MB per
        # set, 3 rotated sets); bytes = weights of the experts the routes touch
        wsets = [(ops.pack_weights((torch.randn(E, 2 * Hf, D, device="cuda", generator=gen)
                                    * 0.02).bfloat16()),
                  ops.pack_weights((torch.randn(E, D, Hf, device="cuda", generator=gen)
                                    * 0.02).bfloat16())) for _ in range(3)]
        x = torch.randn(B, D, device="cuda", generator=gen)
        wr = torch.randn(E, D, device="cuda", generator=gen) * 0.02
        ones = torch.ones(D, device="cuda")
        bufs = ops.moe_route_decode(x, ones, ones, wr, k)
        act = torch.empty(B * k, Hf, dtype=torch.bfloat16, device="cuda")
        y = torch.empty(B * k, D, device="cuda")
        n_active = int((bufs["counts"] > 0).sum())
        t = event_time(lambda i: ops.moe_experts_routed(bufs["h"], bufs["idx"], bufs["gates"],
                                                        *wsets[i % 3], act=act, y=y,
                                                        layout=ops.LAYOUT_PACKED), iters)
        hbm("moe_decode_experts", t, n_active * 3 * Hf * D * 2 + B * D * 2 + B * k * D * 4,
            f"T={B}, D={D}, E={E}, top-{k}, H={Hf}; {n_active} experts active, 3 weight sets")

    def lm_head():
        # the tied LM head of the decode step: [B, D] bf16 x packed [V, D] -> fp32 logits
        wb = V * D * 2
        ns = n_sets(wb)
        heads = [ops.pack_weights((torch.randn(V, D, device="cuda", generator=gen) * 0.02)
                                  .bfloat16()) for _ in range(ns)]
        hx = torch.randn(B, D, device="cuda", generator=gen).bfloat16()
        lo = torch.empty(B, V, device="cuda")
        t = event_time(lambda i: ops.linear(hx, heads[i % ns], out=lo, epilogue=ops.EPI_STORE_F32,
                                            layout=ops.LAYOUT_PACKED), iters)
        hbm("lm_head", t, wb + B * D * 2 + B * V * 4,
            f"B={B} rows x [{V}, {D}] packed bf16 weights -> fp32 logits, {ns} rotated weight sets")

    def gdn_decode_step():
        # the fused step of the engine at the C5 head shape (dk = dv = 64):
        # projection row in, conv gate, state in place
        nproj = 2 * Hg * dk + Hg * dv + D + Hg
        sb = B * Hg * dk * dv * 4
        ns = n_sets(sb)
        Ss = [torch.randn(B, Hg, dk, dv, device="cuda", generator=gen) * 0.1 for _ in range(ns)]
        proj = torch.randn(B, nproj, device="cuda", generator=gen)
        go = torch.empty(B, Hg * dv, dtype=torch.bfloat16, device="cuda")
        zb, dec = torch.zeros(Hg, device="cuda"), torch.full((Hg,), 2.0, device="cuda")
        t = event_time(lambda i: ops.gdn_step_fused(proj, zb, dec, Ss[i % ns], out=go), iters)
        hbm("gdn_decode_step", t, 2 * sb + B * nproj * 4 + B * Hg * dv * 2,
            f"C5 shape: B={B}, H={Hg}, dk=dv={dk}, fp32 state, {ns} rotated states "
            f"({ns * sb / 1e6:.0f} MB)")

    def gdn_decode_step_c4():
        # BASELINE config 4's decode variant: B=64, H=16, dk = dv = 128
        # (134 MB of state read + written)
        B4, H4, d4 = 64, 16, 128
        sb = B4 * H4 * d4 * d4 * 4
        ns = n_sets(sb)
        Ss = [torch.randn(B4, H4, d4, d4, device="cuda", generator=gen) * 0.1 for _ in range(ns)]
        q4 = F.normalize(torch.randn(B4, H4, d4, device="cuda", generator=gen), dim=-1).bfloat16()
        k4 = F.normalize(torch.randn(B4, H4, d4, device="cuda", generator=gen), dim=-1).bfloat16()
        v4 = torch.randn(B4, H4, d4, device="cuda", generator=gen).bfloat16()
        b4 = torch.sigmoid(torch.randn(B4, H4, device="cuda", generator=gen))
        g4 = torch.exp(-F.softplus(torch.randn(B4, H4, device="cuda", generator=gen)))
        o4 = torch.empty(B4, H4, d4, dtype=torch.bfloat16, device="cuda")
        t = event_time(lambda i: ops.gdn_step(q4, k4, v4, b4, g4, Ss[i % ns], out=o4), iters)
        hbm("gdn_decode_step_c4", t, 2 * sb + 4 * B4 * H4 * d4 * 2 + 2 * B4 * H4 * 4,
            f"C4 decode: B={B4}, H={H4}, dk=dv={d4}, fp32 state, {ns} rotated states "
            f"({ns * sb / 1e6:.0f} MB)")

    def _logit_sets():
        ns = n_sets(B * V * 4)
        return ns, [torch.randn(B, V, device="cuda", generator=gen) * 0.6 for _ in range(ns)]

    def sample_argmax():
        ns, lsets = _logit_sets()
        so = torch.empty(B, dtype=torch.int32, device="cuda")
        t = event_time(lambda i: _lib.call("llmy_sample_argmax_f32", lsets[i % ns].data_ptr(), B,
                                           V, so.data_ptr(), strm()), iters)
        latency("sample_argmax", t, f"greedy argmax over [{B}, {V}] fp32, {ns} rotated logit sets")

    def sample_top_p():
        ns, lsets = _logit_sets()
        us_ = torch.rand(B, device="cuda", generator=gen)
        so = torch.empty(B, dtype=torch.int32, device="cuda")
        t = event_time(lambda i: _lib.call("llmy_sample_top_p_f32", lsets[i % ns].data_ptr(), B,
                                           V, SAMPLING[0], SAMPLING[2], SAMPLING[1],
                                           us_.data_ptr(), so.data_ptr(), strm()), iters)
        latency("sample_top_p", t, f"T={SAMPLING[0]}, top-p={SAMPLING[1]} draw over [{B}, {V}] "
                                   f"fp32, {ns} rotated logit sets")

    T2 = 4096

    def _moe_prefill_inputs():
        # C2 (T=4096) with the engine's packed expert weights, 2 rotated sets
        x2 = torch.randn(T2, D, device="cuda", generator=gen).bfloat16()
        wr2 = torch.randn(E, D, device="cuda", generator=gen) * 0.02
        esets = [(ops.pack_weights((torch.randn(E, 2 * Hf, D, device="cuda", generator=gen)
                                    * 0.02).bfloat16()),
                  ops.pack_weights((torch.randn(E, D, Hf, device="cuda", generator=gen)
                                    * 0.02).bfloat16())) for _ in range(2)]
        return x2, wr2, esets

    def moe_prefill_layer():
        x2, wr2, esets = _moe_prefill_inputs()
        t = event_time(lambda i: ops.moe_forward(x2, wr2, *esets[i % 2], k,
                                                 layout=ops.LAYOUT_PACKED), it_mfma)
        mfma("moe_prefill_layer", t, 2 * T2 * k * (D * 2 * Hf + Hf * D),
             f"C2: T={T2}, D={D}, E={E}, top-{k}, H={Hf} (router+permute+experts+combine), "
             f"packed weights, 2 weight sets")

    def moe_prefill_experts():
        x2, wr2, esets = _moe_prefill_inputs()
        idx2, gates2 = ops.router_topk(x2, wr2, k)
        perm2 = ops.moe_permute(idx2.view(-1), E)
        act2 = torch.empty(T2 * k, Hf, dtype=torch.bfloat16, device="cuda")
        y2 = torch.empty(T2 * k, D, device="cuda")
        t = event_time(lambda i: ops.moe_experts(x2, perm2, gates2, *esets[i % 2], act=act2, y=y2,
                                                 layout=ops.LAYOUT_PACKED), it_mfma)
        mfma("moe_prefill_experts", t, 2 * T2 * k * (D * 2 * Hf + Hf * D),
             f"C2 grouped GEMMs only: {T2 * k} routes, gate_up+SwiGLU then down, packed "
             f"weights, 2 weight sets")

    def dense_prefill_gemm():
        # the C5 GDN input projection over 4096 tokens
        nprj = 2 * Hg * dk + 2 * Hg * dv + Hg
        nprj += (-nprj) % 16
        xs = torch.randn(4096, D, device="cuda", generator=gen).bfloat16()
        wps = [ops.pack_weights((torch.randn(nprj, D, device="cuda", generator=gen) * 0.02)
                                .bfloat16()) for _ in range(2)]
        po = torch.empty(4096, nprj, device="cuda")
        t = event_time(lambda i: ops.linear(xs, wps[i % 2], out=po, epilogue=ops.EPI_STORE_F32,
                                            layout=ops.LAYOUT_PACKED), it_mfma)
        mfma("dense_prefill_gemm", t, 2 * 4096 * nprj * D,
             f"C5 GDN projection over 4096 tokens: M=4096, N={nprj}, K={D}, packed weights")

    def attn_prefill():
        Bq, Tq, Hq, hq, Wq = 4, 8192, 16, 64, 512
        qkv = [torch.randn(Bq, Tq, Hq, hq, device="cuda", generator=gen).bfloat16()
               for _ in range(3)]
        ao = torch.empty_like(qkv[0])
        t = event_time(lambda i: ops.banded_attn_prefill(*qkv, Wq, out=ao), it_mfma)
        pairs = sum(min(t_ + 1, Wq) for t_ in range(Tq))
        mfma("attn_prefill", t, 4 * Bq * Hq * hq * pairs,
             f"C3: B={Bq}, T={Tq}, H={Hq}, hd={hq}, window={Wq}")

    def gdn_prefill():
        # C4: chunked gated delta rule
        Bg, Tg, Hg4, d4 = 8, 4096, 16, 128
        gq = F.normalize(torch.randn(Bg, Tg, Hg4, d4, device="cuda", generator=gen),
                         dim=-1).bfloat16()
        gk = F.normalize(torch.randn(Bg, Tg, Hg4, d4, device="cuda", generator=gen),
                         dim=-1).bfloat16()
        gv = torch.randn(Bg, Tg, Hg4, d4, device="cuda", generator=gen).bfloat16()
        gb = torch.sigmoid(torch.randn(Bg, Tg, Hg4, device="cuda", generator=gen))
        gg = torch.exp(-F.softplus(torch.randn(Bg, Tg, Hg4, device="cuda", generator=gen)))
        gS = torch.zeros(Bg, Hg4, d4, d4, device="cuda")
        go4 = torch.empty(Bg, Tg, Hg4, d4, dtype=torch.bfloat16, device="cuda")
        nb = int(_lib.load().llmy_gdn_prefill_workspace_bytes(Bg, Tg, Hg4, d4, d4))
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
        t = event_time(lambda i: ops.gdn_prefill(gq, gk, gv, gb, gg, gS, out=go4, workspace=ws),
                       10, warm=2)
        bytes4 = 4 * Bg * Tg * Hg4 * d4 * 2 + 2 * Bg * Tg * Hg4 * 4 + 2 * Bg * Hg4 * d4 * d4 * 4
        hbm("gdn_prefill", t, bytes4, f"C4: B={Bg}, T={Tg}, H={Hg4}, dk=dv={d4}, chunk 64")

    # CSA / HCA mixers at the reference's defaults (model/config.py:56-70):
    # d_model 1024, local window 128; CSA 16 index heads x 128, ratio 4, top-32;
    # HCA one head of 1024, ratio 32, dense; 256 memory slots per row
    def cmp_shape(kind):
        return ((16, 128, 4, 32) if kind == "csa" else (1, D, 32, 0))

    def cmp_decode(kind):
        # local window + memory branch for B rows; rings and memories full
        # (every slot visible); bytes = the window's and the memory's keys and
        # values read once per row (the branches' algorithmic reads)
        H, Dh, ratio, top_k = cmp_shape(kind)
        Kw, W, C = H * Dh, 128, 256
        per_set = B * (W + C) * (Kw + D) * 2
        nsets = max(2, -(-300_000_000 // per_set))
        sets = []
        for _ in range(nsets):
            sets.append({"lk": torch.randn(B, W, Kw, device="cuda", generator=gen).bfloat16(),
                         "lv": torch.randn(B, W, D, device="cuda", generator=gen).bfloat16(),
                         "mk": torch.randn(B, C, Kw, device="cuda", generator=gen).bfloat16(),
                         "mv": torch.randn(B, C, D, device="cuda", generator=gen).bfloat16()})
        tag = torch.arange(1, C + 1, device="cuda", dtype=torch.int32).repeat(B, 1)
        pos = torch.full((B,), 5000, dtype=torch.int32, device="cuda")
        qkv = torch.randn(B, 2 * Kw + D, device="cuda", generator=gen).bfloat16()
        loc = torch.empty(B, 2 * D, dtype=torch.bfloat16, device="cuda")
        ws = ops.cmp_workspace(B, H, C, top_k, "cuda", decode=True)
        wsl = ops.cmp_workspace(B, H, W, 0, "cuda", decode=True)

        def launch(i):
            st = sets[i % nsets]
            ops.cmp_local_decode(qkv[:, :Kw], qkv[:, Kw:2 * Kw], qkv[:, 2 * Kw:], st["lk"],
                                 st["lv"], pos, H, Dh, out=loc[:, :D], workspace=wsl)
            ops.cmp_memory_decode(qkv[:, :Kw], st["mk"], st["mv"], tag, pos, H, Dh, top_k,
                                  out=loc[:, D:], workspace=ws)
        t = event_time(launch, iters)
        hbm(f"{kind}_decode", t, per_set,
            f"{kind.upper()} decode branches: B={B}, heads={H} x {Dh}, d_model={D}, "
            f"window={W}, {C} memory slots, top_k={top_k or 'dense'}")

    def cmp_prefill(kind):
        # local + memory branches over one fresh 4096-token sequence; FLOPs =
        # scores and weighted sums over the candidates each query sees
        H, Dh, ratio, top_k = cmp_shape(kind)
        Kw, W, Bq, Tq = H * Dh, 128, 1, 4096
        n = Tq // ratio
        qkv = torch.randn(Bq * Tq, 2 * Kw + D, device="cuda", generator=gen).bfloat16()
        kv = torch.randn(Bq * n, Kw + D, device="cuda", generator=gen).bfloat16()
        loc = torch.empty(Bq * Tq, 2 * D, dtype=torch.bfloat16, device="cuda")
        wsl = ops.cmp_workspace(Bq * Tq, H, W, 0, "cuda")
        wsm = ops.cmp_workspace(Bq * Tq, H, n, top_k, "cuda")

        def launch(i):
            ops.cmp_local_prefill(qkv[:, :Kw], qkv[:, Kw:2 * Kw], qkv[:, 2 * Kw:], Bq, Tq, H, Dh,
                                  W, out=loc[:, :D], workspace=wsl)
            ops.cmp_memory_prefill(qkv[:, :Kw], kv[:, :Kw], kv[:, Kw:], Bq, Tq, ratio, H, Dh,
                                   top_k, out=loc[:, D:], workspace=wsm)
        t = event_time(launch, it_mfma)
        band = sum(min(t_ + 1, W) for t_ in range(Tq))
        vis = sum(min(n, (t_ + 1) // ratio) for t_ in range(Tq))
        sel = sum(min(top_k, (t_ + 1) // ratio) for t_ in range(Tq)) * H if top_k else vis
        flops = 2 * Bq * (band * (Kw + D) + vis * Kw + sel * D)
        mfma(f"{kind}_prefill", t, flops,
             f"{kind.upper()} prefill branches: B={Bq}, T={Tq}, heads={H} x {Dh}, "
             f"d_model={D}, window={W}, ratio={ratio}, top_k={top_k or 'dense'}")

    fns = {"hbm_copy": hbm_copy, "mfma_gemm": mfma_gemm, "moe_decode_experts": moe_decode_experts, "lm_head": lm_head,
           "gdn_decode_step": gdn_decode_step,
           "gdn_decode_step_c4": gdn_decode_step_c4, "sample_argmax": sample_argmax,
           "sample_top_p": sample_top_p, "moe_prefill_layer": moe_prefill_layer,
           "moe_prefill_experts": moe_prefill_experts, "dense_prefill_gemm": dense_prefill_gemm,
           "attn_prefill": attn_prefill, "gdn_prefill": gdn_prefill,
           "csa_decode": lambda: cmp_decode("csa"), "hca_decode": lambda: cmp_decode("hca"),
           "csa_prefill": lambda: cmp_prefill("csa"), "hca_prefill": lambda: cmp_prefill("hca")}
    for name in KERNEL_ROWS:
        if only is None or name in only:
            fns[name]()
            torch.cuda.empty_cache()
    return rows


def model_flops_per_token(cfg, T):
    """Dense-equivalent FLOPs per prompt token of a [B, T] prefill: every
    projection, banded attention over the average window of a T-token
    prompt, the GDN recurrence (6 dk dv per head), router and top-k
    experts; the LM head of the last position is left out."""
    D, Hhd = cfg.d_model, cfg.attn_heads * cfg.attn_head_dim
    Hg, dk, dv = cfg.gdn_heads, cfg.gdn_dk, cfg.gdn_dv
    keys = sum(min(t + 1, cfg.window) for t in range(T)) / T
    attn = 2 * 4 * D * Hhd + 4 * Hhd * keys
    nproj = 2 * Hg * dk + 2 * Hg * dv + Hg
    gdn = 2 * (D * nproj + Hg * dv * D) + 6 * Hg * dk * dv
    moe = 2 * D * cfg.n_experts + 2 * cfg.top_k * 3 * D * cfg.expert_hidden
    per_loop = sum((attn if kind == "attn" else gdn) + moe for kind in cfg.layer_kinds)
    return per_loop * cfg.num_loops


def engine_prefill(cfg, gen, Bp=8, Tp=512, iters=5):
    """Whole-model prefill of Bp fresh sequences of Tp prompt tokens through
    HybridDecoder.prefill (embedding to the last position's logits and
    greedy token)."""
    import torch
    from hybrid_llm_amd.config import init_weights
    from hybrid_llm_amd.engine import HybridDecoder
    weights = init_weights(cfg, seed=1, device="cuda")
    eng = HybridDecoder(cfg, weights, Bp, device="cuda")
    del weights
    toks = torch.randint(0, cfg.vocab, (Bp, Tp), device="cuda", generator=gen)
    eng.prefill(toks)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        eng.prefill(toks)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / iters
    del eng
    torch.cuda.empty_cache()
    tok_s = Bp * Tp / (ms / 1e3)
    tf = model_flops_per_token(cfg, Tp) * tok_s / 1e12
    return {"workload": f"C5 model prefill, {Bp} fresh sequences x {Tp} tokens (to last logits)",
            "bound": "mfma", "ms": round(ms, 3), "tok_s": round(tok_s, 1),
            "achieved": round(tf, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
            "flops_per_token": round(model_flops_per_token(cfg, Tp))}


def _cpu_model_name() -> str:
    """The host CPU's model name, as ``lscpu`` prints it (from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline(B):
    """The oracle (fp32 PyTorch restatement of the reference math) on the host
    cores, on the full C5 decode step at batch B: all 12 layers looped twice,
    2048-token windows pre-filled, the LM head and the top-p draw.  One warmup
    step, then the median of three timed steps (wall clock).  Needs about
    22 GB of host memory (fp32 weights 7.6 GB, KV caches 12.9 GB)."""
    import torch
    from hybrid_llm_amd.config import C5, init_weights
    from oracle.model import HybridOracle
    from oracle.sampling import top_p_sample

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    cfg = C5
    t_setup = time.perf_counter()
    w = init_weights(cfg, seed=0)
    ora = HybridOracle(cfg, w, act_bf16=False)
    del w
    st = ora.new_state(B)
    g = torch.Generator().manual_seed(2)
    st["pos"].fill_(cfg.window)
    for key, s in st.items():
        if key == "pos":
            continue
        for name, t in s.items():
            if t.numel():
                t.normal_(0.0, 0.1 if name == "S" else 1.0, generator=g)
    tokens = torch.randint(0, cfg.vocab, (B,), generator=g)
    u = torch.rand(B, generator=g)
    t_setup = time.perf_counter() - t_setup

    def step():
        t0 = time.perf_counter()
        logits = ora.step(tokens, st)
        top_p_sample(logits, SAMPLING[0], SAMPLING[1], u, top_k=SAMPLING[2])
        return time.perf_counter() - t0

    step()  # warmup
    times = sorted(step() for _ in range(3))
    t_step = times[1]
    del ora, st
    return {"value": B / t_step, "unit": "tok/s", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model_name(), "torch": torch.__version__,
            "step_s": [round(x, 3) for x in times],
            "sample": (f"oracle fp32 decode step of the full C5 model (12 layers x 2 loops, "
                       f"24-expert MoEs, batch {B}, 2048-token windows, LM head, top-p draw): "
                       f"1 warmup + median of 3 steps = {t_step:.2f} s/step on {threads} threads "
                       f"(setup {t_setup:.0f} s untimed)")}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU (one MI355X per box); "
                                   "--gpus must be 1"}))
        sys.exit(2)
    if args.pmc_child:
        pmc_child()
        return
    if args.only:
        only = [r.strip() for r in args.only.split(",") if r.strip()]
        unknown = [r for r in only if r not in KERNEL_ROWS]
        if unknown:
            print(json.dumps({"error": f"unknown rows {unknown}; rows: {list(KERNEL_ROWS)}"}))
            sys.exit(2)
        import torch
        from hybrid_llm_amd.config import C5
        torch.cuda.set_device(0)
        gen = torch.Generator(device="cuda").manual_seed(0)
        copy_calibration()
        rows = kernel_table(C5, 64, gen, args.kernel_iters, only=only)
        print(json.dumps(rows))
        return
    # the counter passes run as child processes before this process touches the GPU
    traffic = None if args.no_traffic else measure_traffic()
    if traffic is not None:
        print(f"[bench] attn decode traffic {traffic['bytes'] / 1e6:.1f} MB/launch",
              file=sys.stderr, flush=True)
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
    eng = HybridDecoder(cfg, weights, B, device=dev, sampling=SAMPLING)
    del weights
    torch.cuda.empty_cache()
    fill_state(eng, gen)
    tokens = torch.randint(0, cfg.vocab, (B,), device=dev, generator=gen, dtype=torch.int64)
    eng.buf["tokens"].copy_(tokens.to(torch.int32))
    eng.set_uniforms(torch.rand(B, device=dev, generator=gen))
    eng.capture()
    print(f"[bench] setup {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        eng.graph.replay()
    # the timed region: exactly `steps` replays between two synchronisations;
    # a pair of HIP events on the replay stream brackets each one as well
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in ev:
        a.record(stream)
        eng.graph.replay()
        b.record(stream)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt * 1e3 / args.steps
    value = B / (ms / 1e3)
    ev_ms = sorted(a.elapsed_time(b) for a, b in ev)
    mid = len(ev_ms) // 2
    ev_median = ev_ms[mid] if len(ev_ms) % 2 else 0.5 * (ev_ms[mid - 1] + ev_ms[mid])
    print(f"[bench] {ms:.3f} ms/step, {value:.0f} tok/s (event median {ev_median:.3f} ms)",
          file=sys.stderr, flush=True)

    del eng
    torch.cuda.empty_cache()
    (us_pl, us_med), us, bytes_ = time_attn_decode(cfg, B, args.kernel_iters, gen)
    achieved = bytes_ / (us * 1e-6) / 1e9
    roofline = {"kernel": "attn_decode_kernel<64, true>", "bound": "hbm", "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": None if traffic is None else round(traffic["bytes"]),
                "avg_us": round(us, 2), "timing": "one event pair over the timed region / launches",
                "per_launch_event_avg_us": round(us_pl, 2), "per_launch_event_median_us": round(us_med, 2),
                "bytes_per_launch": bytes_}
    if traffic is not None:
        roofline["traffic_detail"] = {k: (round(v, 4) if "factor" in k else round(v))
                                      for k, v in traffic.items() if k != "bytes"}
    print(f"[bench] attn decode {us:.1f} us, {achieved:.0f} GB/s", file=sys.stderr, flush=True)

    kernels = None
    if not args.no_kernels:
        kernels = kernel_table(cfg, B, gen, args.kernel_iters)
        for name, r in kernels.items():
            if "frac" in r:
                print(f"[bench] {name}: {r['avg_us']} us, {r['achieved']} {r['unit']} "
                      f"({100 * r['frac']:.1f}%)", file=sys.stderr, flush=True)
            else:
                print(f"[bench] {name}: {r['avg_us']} us", file=sys.stderr, flush=True)
        kernels["engine_prefill"] = engine_prefill(cfg, gen)
        r = kernels["engine_prefill"]
        print(f"[bench] engine_prefill: {r['ms']} ms, {r['tok_s']:.0f} tok/s, "
              f"{r['achieved']} TFLOP/s ({100 * r['frac']:.1f}%)", file=sys.stderr, flush=True)

    sb = step_bytes(cfg, B)
    step_gbs = sb["total"] / (ms * 1e-3) / 1e9
    step_rf = {"bound": "hbm", "bytes_per_step": round(sb["total"]), "achieved": round(step_gbs, 1),
               "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(step_gbs / HBM_PEAK_GBS, 4),
               "ms_at_peak": round(sb["total"] / (HBM_PEAK_GBS * 1e9) * 1e3, 4)}
    print(f"[bench] step {sb['total'] / 1e9:.2f} GB: {step_gbs:.0f} GB/s "
          f"({100 * step_rf['frac']:.1f}% of peak)", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(B)
        print(f"[bench] cpu baseline {cpu['value']:.2f} tok/s", file=sys.stderr, flush=True)

    line = {"metric": METRIC,
            "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 4),
            "ms_per_step_event_median": round(ev_median, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "C5 full hybrid-MoE decode step, bs64 (greedy + top-p draw)",
                       "d_model": cfg.d_model, "layers": cfg.n_layers, "loops": cfg.num_loops,
                       "experts": cfg.n_experts, "top_k": cfg.top_k, "window": cfg.window,
                       "vocab": cfg.vocab, "sampling": {"temperature": SAMPLING[0],
                                                        "top_p": SAMPLING[1]},
                       "global_batch": B, "parallelism": "single GPU"},
            "roofline": roofline, "step_roofline": step_rf, "kernels": kernels,
            "cpu_baseline": cpu}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
