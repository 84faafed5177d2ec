"""Build the gfx950 HIP library ``delta_amd/_delta_hip.so`` with hipcc.

Usage: ``python -m delta_amd.build`` (also called by ``__graft_entry__.build()``).
The library is built in-tree so it travels with the source tree; it is
git-ignored.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "_delta_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
SOURCES = ["capi.hip", "paged_decode.hip", "page_score.hip", "page_select.hip",
           "page_metadata.hip", "kv_rope.hip", "step_utils.hip",
           "skinny_gemm.hip", "prefill.hip"]

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
    "--offload-arch=gfx950",
    # Packed fp32 instructions off (v_pk_{add,mul,fma}_f32 are avoided on this pool).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def build(verbose: bool = False, extra_flags=None) -> Path:
    """Compile every HIP source into one shared library; returns its path."""
    srcs = [str(CSRC / s) for s in SOURCES]
    fd, tmp = tempfile.mkstemp(prefix=".delta_hip.", suffix=".so.tmp", dir=str(PKG_DIR))
    os.close(fd)
    cmd = [hipcc(), *HIPCC_FLAGS, *(extra_flags or []), "-o", tmp, *srcs]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only target feature: harmless.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        try:
            os.unlink(tmp)
        except OSError:
            pass
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    build_probe(verbose)
    return LIB_PATH


PROBE_SOURCES = ["probe_gather.hip"]
PROBE_PATH = PKG_DIR / "_delta_probe.so"


def build_probe(verbose: bool = False) -> Path:
    """The measurement probe bench.py loads beside the library (``_delta_probe.so``)."""
    fd, tmp = tempfile.mkstemp(prefix=".delta_probe.", suffix=".so.tmp", dir=str(PKG_DIR))
    os.close(fd)
    cmd = [hipcc(), *HIPCC_FLAGS, "-o", tmp, *[str(CSRC / s) for s in PROBE_SOURCES]]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        try:
            os.unlink(tmp)
        except OSError:
            pass
        raise RuntimeError(f"hipcc failed on the probe ({proc.returncode}):\n{proc.stderr}")
    os.replace(tmp, PROBE_PATH)
    return PROBE_PATH


if __name__ == "__main__":
    p = build(verbose=True)
    print(p)
