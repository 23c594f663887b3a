"""Builds the gfx950 HIP library ``dsalt_amd/libdsalt_amd.so`` from ``dsalt_amd/csrc``.

Usage: ``python -m dsalt_amd.build`` (also called by ``__graft_entry__.build()``).
Every call recompiles.  The library exports the C ABI of ``include/dsalt_amd.h`` and
links nothing but the HIP runtime.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libdsalt_amd.so")
ARCH = "gfx950"

SOURCES = {
    # selection follows a fixed fp64 arithmetic order shared with the oracle:
    # no contraction into fused multiply-adds there
    "select.hip": ["-ffp-contract=off"],
    "attn_fwd.hip": [],
    "attn_bwd.hip": [],
    # the rotation rounds every product and sum to the tensor type: no fused multiply-adds
    "rope.hip": ["-ffp-contract=off"],
    # products rounded to the tensor type one operation at a time, as the torch expression
    "ffn.hip": ["-ffp-contract=off"],
    "probs.hip": [],
    "ce.hip": [],
    "capi.hip": [],
    "timing.hip": [],
}


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def common_flags() -> list[str]:
    return [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-mcode-object-version=5",
            "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
            # packed fp32 instructions are kept out of all generated code
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _compile(src: str, extra: list[str]) -> str:
    out = os.path.join(OBJ, src.replace(".hip", ".o"))
    cmd = [hipcc()] + common_flags() + extra + ["-c", os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return out


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=4) as ex:
        objs = list(ex.map(lambda kv: _compile(*kv), SOURCES.items()))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
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
