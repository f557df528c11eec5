"""bench.py's host side without a GPU: the one-GPU guard, the kernel kinds it names, the CPU description."""
import os
import re
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_every_kernel_kind_bench_names_exists():
    import nunchi_amd
    src = open(os.path.join(ROOT, "bench.py")).read()
    kinds = set(re.findall(r"bench_(?:step_)?kernel\(\"(\w+)\"", src))
    assert kinds, "bench.py names no kernel kind"
    assert kinds <= set(nunchi_amd.Brain.KERNELS), kinds - set(nunchi_amd.Brain.KERNELS)


def test_cpu_info_describes_the_affinity_mask():
    import bench
    info = bench.cpu_info()
    assert info["logical_cpus"] == len(os.sched_getaffinity(0))
    assert info["smt_width"] >= 1
    assert info["physical_cores"] is None or 1 <= info["physical_cores"] <= info["logical_cpus"]


def test_layer_tables_are_the_seoul_layer():
    import bench
    # q, k, v, o, gate, up, down of a hidden-2048, 32/8 x 64 head, FFN-8192 layer
    assert bench.LAYER_TABLES == ((2048, 2048), (512, 2048), (512, 2048), (2048, 2048), (8192, 2048), (8192, 2048),
                                  (2048, 8192))
    assert sum(r * c // 32 * 18 for r, c in bench.LAYER_TABLES) == 34209792
    w, x = bench.layer_weights()
    assert [a.size for a in w] == [r * c // 32 for r, c in bench.LAYER_TABLES]
    assert x.shape == (2, 8192) and np.isfinite(x).all()
