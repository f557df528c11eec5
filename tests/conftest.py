import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path through the C ABI)")
    config.addinivalue_line("markers", "slow: full Seoul-sized case (seconds to minutes)")


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    d = os.environ.get("NUNCHI_MODEL_DIR") or str(tmp_path_factory.mktemp("models"))
    os.environ["NUNCHI_MODEL_DIR"] = d
    return d


@pytest.fixture(scope="session")
def tiny_model(model_dir):
    from nunchi_amd import synth
    return synth.cached("brain", synth.TINY, 0, model_dir)


@pytest.fixture(scope="session")
def mid_model(model_dir):
    """Seoul widths (n_embd 2048, 32/8 heads x 64, FFN 8192) with 4 layers and a small word table: exercises every
    kernel at its real per-layer shape while the CPU oracle still steps in milliseconds."""
    from nunchi_amd import synth
    shape = synth.BrainShape(n_layer=4, attn_layers=(1, 3), n_vocab=4096)
    return synth.cached("brain", shape, 7, model_dir)


@pytest.fixture(scope="session")
def tiny_voice(model_dir):
    from nunchi_amd import synth
    return synth.cached("voice", synth.TINY_VOICE, 1, model_dir)


def rel(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.sqrt(((a - b) ** 2).sum() / ((b ** 2).sum() + 1e-30)))


def q4_random(rows, cols, seed):
    from nunchi_amd import synth
    return synth.q4_0_random(np.random.default_rng(seed), rows, cols)
