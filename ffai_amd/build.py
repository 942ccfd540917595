"""Build the gfx950 attention library in-tree: ffai_amd/libffai_attn.so.

hipcc compiles the kernel instantiations (fwd_bf16.hip, fwd_f16.hip, fwd_f32.hip, decode.hip,
decode_f16.hip, decode_vec.hip),
the decode-state kernels and their C ABI (kv_cache.hip), the decoder GEMVs (gemv.hip), the
launch-floor probes (probe.hip), the launch dispatch (attn_launch.hip), the attention C ABI
(attn_api.cpp) and the encoder attention block around hipBLASLt (encoder_attn.cpp) for gfx950
only, in parallel, then links them into one shared library. Packed-FP32 VALU instructions are
disabled for all device code.
"""

from __future__ import annotations

import json
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libffai_attn.so")
BUILD_DIR = os.path.join(HERE, "_build")
SOURCES = [os.path.join(CSRC, n) for n in
           ("fwd_bf16.hip", "fwd_f16.hip", "fwd_f32.hip", "decode.hip", "decode_f16.hip",
            "decode_vec.hip",
            "kv_cache.hip", "gemv.hip", "probe.hip", "attn_launch.hip", "attn_api.cpp",
            "encoder_attn.cpp")]
LIBS = ["-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build ffai_amd)")


def flags() -> list[str]:
    return [
        "-O3", "-std=c++17", "-fPIC",
        f"--offload-arch={ARCH}",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # No NaN is ever produced or consumed in the kernels (masked scores are -inf, never
        # NaN): let maxima skip IEEE NaN quieting (otherwise every fmaxf operand is canonicalised
        # first). Device code only: the host-side argument checks must still see a NaN as NaN.
        "-Xarch_device", "-fno-honor-nans", "-Xarch_device", "-mno-amdgpu-ieee",
        "-I", os.path.join(ROOT, "include"),
        "-Wall", "-Wno-unused-function",
    ]


# Per-kernel register, scratch and occupancy figures the compiler reports, written at every
# build (kernel name -> {"vgprs", "agprs", "scratch", "occupancy", "vgpr_spill", "sgpr_spill"}).
# The fused kernels sit at their register budget, where a small change of the code can make the
# compiler spill to scratch: correct results, several times slower. A CPU test reads this file.
RESOURCES_PATH = os.path.join(BUILD_DIR, "resource_usage.json")
_REMARK = "-Rpass-analysis=kernel-resource-usage"
_FIELDS = {"VGPRs": "vgprs", "AGPRs": "agprs", "ScratchSize [bytes/lane]": "scratch",
           "Occupancy [waves/SIMD]": "occupancy", "VGPRs Spill": "vgpr_spill",
           "SGPRs Spill": "sgpr_spill"}


def _resources(stderr: str) -> dict:
    """The compiler's kernel-resource-usage remarks of one compile, by kernel."""
    out, cur = {}, None
    for line in stderr.splitlines():
        if "remark:" not in line or _REMARK not in line:
            continue
        body = line.split("remark:", 1)[1].replace(f"[{_REMARK}]", "").strip()
        key, _, val = body.partition(":")
        key, val = key.strip(), val.strip()
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None and key in _FIELDS:
            try:
                cur[_FIELDS[key]] = int(val)
            except ValueError:
                pass
    return out


def _run(cmd: list[str], verbose: bool) -> dict:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l and "remark:" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    return _resources(res.stderr)


# The diagnostic library: the attention sources compiled with FFAI_STAMPS, so that the fused and
# decode kernels record their phase times (bench.py --legs stamps). The product library's code
# is unaffected; nothing but that benchmark leg loads this one.
STAMPS_LIB_PATH = os.path.join(HERE, "libffai_attn_stamps.so")
STAMPS_SOURCES = [os.path.join(CSRC, n) for n in
                  ("fwd_bf16.hip", "fwd_f16.hip", "fwd_f32.hip", "decode.hip", "decode_f16.hip",
                   "decode_vec.hip", "attn_launch.hip", "attn_api.cpp")]


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every source (always) into objects in parallel, then link LIB_PATH and the
    diagnostic STAMPS_LIB_PATH."""
    from concurrent.futures import ThreadPoolExecutor

    os.makedirs(BUILD_DIR, exist_ok=True)
    cc = hipcc()
    objs, sobjs, cmds = [], [], []
    for src in SOURCES:
        obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
        objs.append(obj)
        cmds.append([cc] + flags() + [_REMARK, "-c", "-x", "hip", src, "-o", obj])
    for src in STAMPS_SOURCES:
        obj = os.path.join(BUILD_DIR, "stamps_" + os.path.basename(src) + ".o")
        sobjs.append(obj)
        cmds.append([cc] + flags() + ["-DFFAI_STAMPS", _REMARK, "-c", "-x", "hip", src, "-o",
                                      obj])
    jobs = jobs or min(len(cmds), max(1, min(os.cpu_count() or 1, 8)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        usage = {}
        for c, r in zip(cmds, ex.map(lambda c: _run(c, verbose), cmds)):
            # the diagnostic library's kernels under their own names: its timings are only
            # representative while it too keeps the register budget
            tag = "stamps:" if "-DFFAI_STAMPS" in c else ""
            usage.update({tag + k: v for k, v in r.items()})
    with open(RESOURCES_PATH, "w") as f:
        json.dump(usage, f, indent=0, sort_keys=True)
    for path, os_ in ((LIB_PATH, objs), (STAMPS_LIB_PATH, sobjs)):
        tmp = path + ".tmp"
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + os_ + LIBS, verbose)
        os.replace(tmp, path)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
