"""Writes the small golden fixtures under tests/golden/ from the oracle (the CPU restatement of imi's arithmetic):
int8 cut vectors with ties and edge blocks, a 64 x 512 Q4_0 GEMV in both cut modes, and the first positions of the
tiny synthetic brain. Regenerate with:  python tests/golden/make_golden.py"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from nunchi_amd import synth  # noqa: E402


def main():
    rng = np.random.default_rng(2026)
    x = (rng.standard_normal(32 * 16) * 3).astype(np.float32)
    x[:32] = 0.0
    x[32:64] = np.float32(0.5) * np.arange(32, dtype=np.float32)
    x[64:96] = np.float32(127.0) * np.linspace(-1, 1, 32, dtype=np.float32)
    x[96:128] = np.float32(1e-30) * np.arange(32, dtype=np.float32)
    q, d, s = oracle.cut(x)
    np.savez(os.path.join(HERE, "cut32.npz"), x=x, q=q, d=d, s=s)

    rows, cols = 64, 512
    blk = synth.q4_0_random(np.random.default_rng(7), rows, cols)
    xv = rng.standard_normal((2, cols)).astype(np.float32)
    y, _ = oracle.Q4Table(blk, rows, cols).gemv(xv)
    y8, _ = oracle.Q4x8Table(blk, rows, cols).gemv(xv[0])
    np.savez(os.path.join(HERE, "gemv_64x512.npz"), q4_0=blk.view(np.uint8).reshape(-1), x=xv, y=y, y_q4x8=y8)

    path = synth.write_brain("/tmp/golden_tiny.gguf", synth.TINY, seed=0)
    eng = oracle.Engine(path, threads=2, n_ctx=16)
    toks = np.array([3, 141, 59, 26, 535, 897], np.int32)
    hid, lg = [], []
    for t in toks:
        h, l = eng.step(int(t))
        hid.append(h)
        lg.append(l)
    np.savez(os.path.join(HERE, "tiny_steps.npz"), tokens=toks, hidden=np.array(hid), logits=np.array(lg),
             best=np.array([oracle.top(l) for l in lg], np.int32))
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
