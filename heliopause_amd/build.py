"""Build libhp_hip.so (the gfx950 runner) in-tree with hipcc.

Every source is compiled for gfx950 only.  Packed-fp32 instructions are
disabled (``-packed-fp32-ops``) and FP contraction is off so the f32 tails
keep the reference's rounding.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libhp_hip.so"
NAPI_SRC = PKG / "napi" / "hp_hip_napi.c"
NAPI_ADDON = PKG / "napi" / "hp_hip.node"
NODE_INCLUDE = Path(os.environ.get("NODE_INCLUDE", "/usr/include/node"))
SOURCES = ["q8k.hip", "kquant_matvec.hip", "kquant_wide.hip", "kquant_mfma.hip", "kquant_prefill.hip", "repack.hip", "topk.hip",
           "geglu.hip", "gguf.hip", "sample.hip", "decode_layer.hip", "attn_prefill.hip", "decode_fused.hip",
           "capi.hip"]

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{PKG.parent / 'include'}",
]


def _compile(src: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass does not know the packed-fp32 feature; drop that note
    noise = "is not a recognized feature for this target"
    lines = [ln for ln in (r.stderr or "").splitlines() if noise not in ln]
    if lines:
        sys.stderr.write("\n".join(lines) + "\n")
    return obj


def build(jobs: int | None = None) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = [s for s in SOURCES if (CSRC / s).exists()]
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


SYNTH_SRC = CSRC / "hp_synth.c"
SYNTH_LIB = PKG / "libhp_synth.so"


def build_synth() -> Path:
    """The host-side SplitMix64 stream of the synthetic workloads
    (heliopause_amd/libhp_synth.so; plain C, no GPU code)."""
    cc = os.environ.get("CC", shutil.which("gcc") or "cc")
    tmp = SYNTH_LIB.with_suffix(".so.tmp")
    cmd = [cc, "-O2", "-fPIC", "-shared", "-std=c11", "-Wall", "-Wextra", "-pthread", str(SYNTH_SRC), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"synthetic-stream build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, SYNTH_LIB)
    return SYNTH_LIB


def build_napi() -> Path | None:
    """Node N-API addon over libhp_hip.so (heliopause_amd/napi/hp_hip.node).

    Plain C against node_api.h; it links the runner with an rpath of its
    parent directory, so the two files travel together.  Returns None (and
    says so) when the Node headers are not installed.
    """
    if not (NODE_INCLUDE / "node_api.h").exists():
        sys.stderr.write(f"node_api.h not found under {NODE_INCLUDE}; N-API addon not built\n")
        return None
    cc = os.environ.get("CC", shutil.which("gcc") or "cc")
    tmp = NAPI_ADDON.with_suffix(".node.tmp")
    cmd = [cc, "-O2", "-fPIC", "-shared", "-std=c11", "-Wall", "-Wextra", "-Wno-unused-parameter",
           f"-I{NODE_INCLUDE}", f"-I{PKG.parent / 'include'}", str(NAPI_SRC), "-o", str(tmp),
           f"-L{PKG}", "-lhp_hip", "-Wl,-rpath,$ORIGIN/.."]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"N-API addon build failed:\n{r.stdout}\n{r.stderr}")
    if r.stderr.strip():
        sys.stderr.write(r.stderr)
    os.replace(tmp, NAPI_ADDON)
    return NAPI_ADDON


if __name__ == "__main__":
    print(build())
    print(build_synth())
    print(build_napi())
