"""Builds libquipsharp_hip.so (gfx950) from quipsharp_amd/csrc with hipcc.

    python -m quipsharp_amd.build        # or quipsharp_amd.build.build()

Each .hip file compiles to an object in quipsharp_amd/_build/, then one
shared library is linked in the package directory so it travels with the
source tree.  Code whose results must match the reference bit for bit
(codebook encode/decode, Walsh-Hadamard) is compiled with
-ffp-contract=off; packed fp32 instructions are disabled everywhere.
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libquipsharp_hip.so")
ARCH = os.environ.get("QS_OFFLOAD_ARCH", "gfx950")

COMMON = ["-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wall", "-Wno-unused-function", "-I", os.path.join(HERE, "..", "include")]
EXACT = {"qs_codebook.hip", "qs_transform.hip"}


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    flags = list(COMMON)
    flags.append("-ffp-contract=off" if os.path.basename(src) in EXACT else "-ffp-contract=fast")
    cmd = [hipcc()] + flags + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
