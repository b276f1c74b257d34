"""Build libfemto_attn.so for gfx950 with hipcc (in-tree).

    python nano-vllm-practice_amd/build.py            # build
    python nano-vllm-practice_amd/build.py --verbose  # print the hipcc line

The library lands in ``femtovllm/_lib/libfemto_attn.so`` next to the Python
package that loads it.  Code objects are pinned to code-object version 5 so
the HIP runtime bundled with PyTorch-ROCm 7.0 loads them, and packed-fp32
instruction selection is disabled for the device pass.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OUT_DIR = os.path.join(HERE, "femtovllm", "_lib")
LIB = os.path.join(OUT_DIR, "libfemto_attn.so")

SOURCES = ["femto_attn_api.hip", "paged_decode.hip", "paged_prefill.hip", "kv_cache_write.hip", "qk_norm_rope.hip", "varlen_metadata.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libfemto_attn.so)")


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", INCLUDE, "-I", CSRC,
           *[os.path.join(CSRC, s) for s in SOURCES], "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(
        line for line in (res.stdout + res.stderr).splitlines()
        if "packed-fp32-ops" not in line  # host pass does not know the device feature
    )
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{errs}")
    if verbose and errs.strip():
        print(errs, flush=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
