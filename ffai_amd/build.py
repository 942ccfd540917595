"""Build the gfx950 attention library in-tree: ffai_amd/libffai_attn.so.

One hipcc invocation compiles the kernels (attn_kernels.hip) and the C ABI (attn_api.cpp) for
gfx950 only. Packed-FP32 VALU instructions are disabled for all device code.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libffai_attn.so")
SOURCES = [os.path.join(CSRC, "attn_kernels.hip"), os.path.join(CSRC, "attn_api.cpp")]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build ffai_amd)")


def flags() -> list[str]:
    return [
        "-O3", "-std=c++17", "-fPIC", "-shared",
        f"--offload-arch={ARCH}",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(ROOT, "include"),
        "-Wall", "-Wno-unused-function",
    ]


def build(verbose: bool = False) -> str:
    """Compile every source into LIB_PATH (always recompiles). Returns the library path."""
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc()] + flags()
    # hipcc compiles .cpp as host C++ unless told otherwise; the API file calls the HIP runtime
    # only, so it is fine either way, but force HIP language for the .hip source.
    cmd += ["-x", "hip", SOURCES[0], "-x", "hip", SOURCES[1], "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
