# -*- coding: utf-8 -*-
"""Build ``librvc_hip.so`` in-tree with hipcc for gfx950.

``python -m rvc_hip.build`` (with ``rvc-vulkan_amd`` on ``sys.path``) or
``build()`` from Python.  Always recompiles; the output lands next to this
file, where ``rvc_hip._hip`` looks for it.
"""

from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)
CSRC = os.path.join(PKG_ROOT, "csrc")
OUT = os.path.join(HERE, "librvc_hip.so")

# -packed-fp32-ops is disabled for device code: packed FP32 VALU forms are
# kept out of every kernel (hipcc's host pass warns that it does not know the
# feature; that is expected).
HIP_FLAGS = [
    "-O3", "-std=c++17", "--offload-arch=gfx950", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC", ""), "/opt/rocm/bin/hipcc", shutil.which("hipcc") or ""):
        if cand and os.path.isfile(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip"))) + sorted(glob.glob(os.path.join(CSRC, "*.cpp")))


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in (proc.stdout + proc.stderr).splitlines() if noise not in ln]
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs[-60:]))
    if verbose and msgs:
        print("\n".join(msgs))


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every source to an object in parallel (a temporary folder),
    then link the shared library."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor

    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    compile_flags = [f for f in HIP_FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="rvc_hip_build_") as tmpdir:
        objs = [os.path.join(tmpdir, os.path.basename(src) + ".o") for src in srcs]
        with ThreadPoolExecutor(jobs) as ex:
            for f in [ex.submit(_run, [hipcc(), *compile_flags, "-c", src, "-o", obj], verbose)
                      for src, obj in zip(srcs, objs)]:
                f.result()
        tmp = OUT + ".tmp"
        _run([hipcc(), "--offload-arch=gfx950", "-fPIC", "-shared", "-o", tmp, *objs], verbose)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
