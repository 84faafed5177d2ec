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
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "_delta_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
SOURCES = ["capi.hip", "paged_decode.hip", "page_score.hip", "page_select.hip",
           "page_metadata.hip", "kv_rope.hip", "step_utils.hip",
           "skinny_gemm.hip", "prefill.hip"]

COMPILE_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "--offload-arch=gfx950",
    # Packed fp32 instructions off (v_pk_{add,mul,fma}_f32 are avoided on this pool).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]
LINK_FLAGS = ["-shared", "-fPIC", "--offload-arch=gfx950"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


# hipcc's host pass warns about the device-only target feature: harmless.
_NOISE = "is not a recognized feature for this target"


def _run(cmd, verbose: bool, what: str) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in proc.stderr.splitlines() if _NOISE not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {what} ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, extra_flags=None, jobs: int = 0) -> Path:
    """Compile every HIP source (one object each, ``jobs`` at a time; default: one per CPU up
    to 8) and link them into one shared library; returns its path."""
    jobs = jobs or min(8, len(SOURCES), os.cpu_count() or 1)
    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix="delta_hip_build.") as tmpdir:
        objs = [os.path.join(tmpdir, Path(s).stem + ".o") for s in SOURCES]
        cmds = [[cc, *COMPILE_FLAGS, *(extra_flags or []), "-c", str(CSRC / s), "-o", o]
                for s, o in zip(SOURCES, objs)]
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            futs = [pool.submit(_run, cmd, verbose, s) for cmd, s in zip(cmds, SOURCES)]
            for f in futs:
                f.result()
        fd, tmp = tempfile.mkstemp(prefix=".delta_hip.", suffix=".so.tmp", dir=str(PKG_DIR))
        os.close(fd)
        try:
            _run([cc, *LINK_FLAGS, "-o", tmp, *objs], verbose, "the link")
        except Exception:
            os.unlink(tmp)
            raise
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    p = build(verbose=True)
    print(p)
