"""In-tree build of the gfx950 HIP library ``lib/libtqk.so``.

Each ``csrc/*.hip`` translation unit is compiled for gfx950 only and linked
into one shared library that exports the C ABI declared in ``include/tqk.h``.
The encode and block units are built with ``-ffp-contract=off`` and correctly
rounded division/sqrt: their results must match NumPy bit for bit.
"""

from __future__ import annotations

import os
import shutil
import subprocess

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))  # turboquant-pro_amd/
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
LIB_DIR = os.path.join(PKG_ROOT, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libtqk.so")
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # packed FP32 VALU forms are kept out of every kernel of this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(REPO_ROOT, "include"),
]
PER_UNIT = {
    "tqk_encode.hip": ["-ffp-contract=off"],
    "tqk_block.hip": ["-ffp-contract=off"],
    "tqk_decode.hip": [],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def build(verbose: bool = False) -> str:
    """Compile every HIP unit and link ``lib/libtqk.so``; returns its path."""
    os.makedirs(LIB_DIR, exist_ok=True)
    objs = []
    cc = hipcc()
    procs = []
    for unit, extra in PER_UNIT.items():
        src = os.path.join(CSRC, unit)
        obj = os.path.join(LIB_DIR, unit.replace(".hip", ".o"))
        cmd = [cc, *COMMON, *extra, "-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd)))
        objs.append(obj)
    for cmd, p in procs:  # the units compile side by side
        if p.wait() != 0:
            raise subprocess.CalledProcessError(p.returncode, cmd)
    tmp = LIB_PATH + ".tmp"
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    for o in objs:
        os.remove(o)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
