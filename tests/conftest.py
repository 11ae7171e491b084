import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "index-tts-25-metal_amd"
for p in (str(PKG), str(ROOT / "oracle"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")


@pytest.fixture(scope="session")
def itts():
    import itts_gpt

    return itts_gpt


@pytest.fixture(scope="session")
def oracle():
    import oracle as orc

    return orc


@pytest.fixture(scope="session")
def small_weights(itts):
    """2-layer model at the real widths; LayerNorm parameters randomised so gamma/beta are exercised."""
    return itts.make_synthetic_weights(layers=2, seed=11, ln_random=True)


@pytest.fixture(scope="session")
def full_weights(itts):
    """The 24-layer d=1280 GPT, FP32 N(0, 0.02), gamma=1, beta=0 (seed 0)."""
    return itts.make_synthetic_weights(layers=24, seed=0)


def same_bits(a, b) -> bool:
    """Float32 arrays equal bit for bit (so -0.0 and +0.0 differ, unlike ==)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def rel_err(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
