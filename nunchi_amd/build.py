"""Build libseoul_hip.so in-tree with hipcc for gfx950.

    python -m nunchi_amd.build        (or __graft_entry__.build())
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libseoul_hip.so")
SOURCES = ["csrc/sh_kernels.hip", "csrc/sh_voice.hip", "csrc/sh_prefill.hip", "csrc/sh_noalloc.hip", "csrc/sh_codec.hip",
           "csrc/sh_ears.hip", "csrc/sh_calib.hip", "csrc/sh_engine.cpp", "csrc/sh_codec_host.cpp", "csrc/sh_ears_host.cpp",
           "csrc/sh_voice_host.cpp", "csrc/sh_prefill_host.cpp", "csrc/gguf_file.cpp", "csrc/sh_file.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # every fused multiply-add is written out in the source, so op order does not depend on the compiler
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]


def build(verbose: bool = False) -> str:
    srcs = [os.path.join(HERE, s) for s in SOURCES]
    tmp = LIB + f".tmp{os.getpid()}"
    cmd = [HIPCC, *FLAGS, "-I", os.path.join(ROOT, "include"), "-o", tmp, *srcs]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building libseoul_hip.so")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
