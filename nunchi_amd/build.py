"""Build libseoul_hip.so in-tree with hipcc for gfx950.

    python -m nunchi_amd.build        (or __graft_entry__.build())

Each source is compiled to its own object in parallel (the device code of one file never calls another file's device
code, so no relocatable device code is needed), then the objects are linked into the library.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libseoul_hip.so")
SOURCES = ["csrc/sh_kernels.hip", "csrc/sh_voice.hip", "csrc/sh_prefill.hip", "csrc/sh_noalloc.hip", "csrc/sh_codec.hip",
           "csrc/sh_ears.hip", "csrc/sh_calib.hip", "csrc/sh_engine.cpp", "csrc/sh_codec_host.cpp", "csrc/sh_ears_host.cpp",
           "csrc/sh_voice_host.cpp", "csrc/sh_prefill_host.cpp", "csrc/gguf_file.cpp", "csrc/sh_file.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # every fused multiply-add is written out in the source, so op order does not depend on the compiler
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]


def _jobs() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16, len(SOURCES)))


def build(verbose: bool = False) -> str:
    inc = ["-I", os.path.join(ROOT, "include")]
    tmpdir = tempfile.mkdtemp(prefix="sh_build_")
    try:
        def compile_one(src: str) -> str:
            obj = os.path.join(tmpdir, os.path.basename(src) + ".o")
            cmd = [HIPCC, *FLAGS, *inc, "-c", "-o", obj, os.path.join(HERE, src)]
            if verbose:
                print(" ".join(cmd), flush=True)
            r = subprocess.run(cmd, capture_output=True, text=True)
            if r.returncode != 0:
                sys.stderr.write(r.stdout + r.stderr)
                raise RuntimeError(f"hipcc failed on {src}")
            return obj

        with ThreadPoolExecutor(max_workers=_jobs()) as ex:
            objs = list(ex.map(compile_one, SOURCES))
        tmp = LIB + f".tmp{os.getpid()}"
        cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError("hipcc failed linking libseoul_hip.so")
        os.replace(tmp, LIB)
    finally:
        shutil.rmtree(tmpdir, ignore_errors=True)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
