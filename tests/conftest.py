import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a ROCm GPU")
    return torch.device("cuda", 0)


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def randn16(g: np.random.Generator, *shape, scale=1.0) -> np.ndarray:
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float16)


def rand_codebooks(g: np.random.Generator, M: int, C: int, d: int) -> np.ndarray:
    """quantization.py:108-115: N(0,1) * sqrt(2/d) in fp16."""
    return (g.standard_normal((M, C, d), dtype=np.float32) * np.float32((2.0 / d) ** 0.5)).astype(np.float16)
