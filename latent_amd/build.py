"""Build liblatent_hip.so (gfx950) in-tree with hipcc.

    python latent_amd/build.py

(Run as a script: importing the package would load the library being rebuilt.)

The library links only against the HIP runtime; no torch headers.  When the
Python binding loads it after `import torch`, the dynamic linker binds it to
the HIP runtime torch already loaded (same SONAME), so torch's streams and
device pointers are valid in it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
SOURCES = ["codec.hip", "expert.hip", "moe.hip", "moe_fused.hip", "noalloc.hip", "prefill.hip", "route.hip", "rows.hip", "stream.hip"]
LIB = PKG / "liblatent_hip.so"
ARCH = os.environ.get("LATENT_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    # Keep the compiler from forming packed-FP32 (v_pk_*_f32) instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def build(verbose: bool = False) -> Path:
    """Compile every source and link the shared library; always rebuilds."""
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    cc = hipcc()
    cmds, objs = [], []
    for src in SOURCES:
        obj = objdir / (Path(src).stem + ".o")
        cmds.append([cc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(str(obj))
    # One compiler process per source, at most `jobs` at a time.
    jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        for cmd in cmds:
            if verbose:
                print(" ".join(cmd), flush=True)
        for result in pool.map(lambda c: subprocess.run(c, capture_output=True, text=True), cmds):
            sys.stderr.write(result.stderr)
            if result.returncode != 0:
                raise subprocess.CalledProcessError(result.returncode, result.args, result.stdout, result.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
