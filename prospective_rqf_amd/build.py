"""Build ``librqf_hip.so`` (the C-ABI scan library) for gfx950 with hipcc.

Usage: ``python -m prospective_rqf_amd.build`` (or ``__graft_entry__.build()``).
The library is built in-tree so it travels with the source tree; it is
git-ignored.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_NAME = "librqf_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["selective.hip", "timeinv.hip", "btf.hip", "multiosc.hip", "proj.hip"]
ARCH = os.environ.get("RQF_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm")


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=fast",
        # Keep the compiler from emitting packed-fp32 VALU instructions.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-command-line-argument",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
    ]


def build(verbose: bool = False) -> str:
    """Compile every HIP source (concurrently) and link the shared library;
    returns its path."""
    build_dir = os.path.join(PKG_DIR, "_objs")
    os.makedirs(build_dir, exist_ok=True)
    cc = hipcc()
    objs = [os.path.join(build_dir, src.replace(".hip", ".o")) for src in SOURCES]
    cmds = [[cc, *compile_flags(), "-c", os.path.join(CSRC, src), "-o", obj]
            for src, obj in zip(SOURCES, objs)]
    if verbose:
        for cmd in cmds:
            print(" ".join(cmd), flush=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(cmds)) as pool:
        for done in pool.map(lambda c: subprocess.run(c, capture_output=True, text=True), cmds):
            sys.stderr.write(done.stderr)
            if done.returncode:
                raise subprocess.CalledProcessError(done.returncode, done.args)
    tmp = LIB_PATH + ".tmp"
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
