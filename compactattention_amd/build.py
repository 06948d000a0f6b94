"""Builds libcompactattn_hip.so (gfx950) in-tree with hipcc.

Run as ``python -m compactattention_amd.build``; ``__graft_entry__.build()`` calls
:func:`build`.  Flags:
  -ffp-contract=off   no implicit fused multiply-adds: the bit-reproducible kernels spell
                      every fma out, so their fp32 results follow one fixed order;
  -packed-fp32-ops    (disabled) keeps the compiler from emitting packed fp32 VALU ops.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libcompactattn_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["ca_api.hip", "ca_select.hip", "ca_score_token.hip", "ca_attn.hip", "ca_model.hip"]
HEADERS = ["ca_common.h", "ca_kernels.h"]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return path


def command(out: str = LIB_PATH) -> list:
    return [
        hipcc(),
        "--offload-arch=gfx950",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-o", out,
    ] + [os.path.join(CSRC, s) for s in SOURCES]


def build(verbose: bool = False) -> str:
    tmp = LIB_PATH + ".tmp"
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with exit code {res.returncode}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
