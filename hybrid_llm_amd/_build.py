"""Build libllmy.so (all HIP kernels + the C ABI) for gfx950 with hipcc.

Every ``csrc/*.hip`` / ``csrc/*.cpp`` file is compiled to an object in
``hybrid_llm_amd/_build/`` and linked into ``hybrid_llm_amd/libllmy.so``.
The library is built in-tree so it travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libllmy.so"
INCLUDE = ROOT / "include"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming packed fp32 VALU ops
# (the host pass warns that it does not know the feature; that is expected).
COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(INCLUDE), "-I", str(CSRC),
    # streamed operands (weights, KV windows) use non-temporal loads
    "-DLLMY_NT=1",
]

_NOISE = "is not a recognized feature for this target"


def _filter(text: str) -> str:
    return "\n".join(l for l in text.splitlines() if _NOISE not in l)


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


# Per-source additions.  attn_prefill: the output accumulators are rescaled by
# VALU between MFMAs, so they stay in VGPRs (the default AGPR form moves every
# one out and back; measured 12% faster, same results).
FILE_FLAGS = {
    "attn_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    # gdn_chunk: the scan prefetches the next chunk's operands at the top of a
    # chunk so the loads run behind its MFMAs; machine sinking would move them
    # down next to their first use (the LDS stash at the chunk's end).
    "gdn_chunk.hip": ["-mllvm", "-disable-machine-sink"],
}


def _compile(src: Path) -> tuple[Path, str]:
    obj = BUILD / (src.stem + ".o")
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [HIPCC, *COMMON_FLAGS, *FILE_FLAGS.get(src.name, []), *lang, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{_filter(proc.stderr)}")
    return obj, _filter(proc.stderr)


def _stale(objs_srcs, headers) -> bool:
    if not LIB.exists():
        return True
    lib_m = LIB.stat().st_mtime
    newest = max([p.stat().st_mtime for p in headers] + [s.stat().st_mtime for s in objs_srcs])
    return newest > lib_m


def build(force: bool = True, jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every kernel source and link libllmy.so; returns the path."""
    srcs = sources()
    headers = list(CSRC.glob("*.hpp")) + list(INCLUDE.glob("*.h"))
    if not force and not _stale(srcs, headers):
        return LIB
    BUILD.mkdir(exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 1, len(srcs))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(_compile, srcs))
    for obj, warn in results:
        if warn.strip() and verbose:
            print(warn, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    # -z defs: an unresolved symbol fails the link instead of the first dlopen
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs",
           *[str(o) for o, _ in results], "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{_filter(proc.stderr)}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    force = "--incremental" not in sys.argv
    print(build(force=force, verbose="-v" in sys.argv))
