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


def score_layout(pq, rvq, sidx, sval, t_base, cap):
    """The score-table K layout of one head, restated: token t = 32 tau + 16 u + r
    puts code byte j = 4g + b of its row (subspace 4g + (b ^ ((r >> 2) & 3)),
    odd tokens with the two stages swapped) at byte 512 tau + 32 r + 8 g + 4 u + b
    of each code array, and sparse entry e at 32 k tau + 2 k r + 2 e + u."""
    T = pq.shape[0]
    k = 0 if sidx is None else sidx.shape[1]
    out_p = np.zeros(cap * 16, np.uint8)
    out_r = np.zeros_like(out_p)
    out_i = np.zeros(cap * k, np.uint8)
    out_v = np.zeros(cap * k, np.float16)
    for i in range(T):
        t = t_base + i
        tau, u, r = t >> 5, (t >> 4) & 1, t & 15
        for j in range(16):
            m = (j & 12) | ((j & 3) ^ ((r >> 2) & 3))
            a, c = pq[i, m], rvq[i, m]
            pos = 512 * tau + 32 * r + 8 * (j >> 2) + 4 * u + (j & 3)
            out_p[pos], out_r[pos] = (c, a) if t & 1 else (a, c)
        for e in range(k):
            pos = 32 * k * tau + 2 * k * r + 2 * e + u
            out_i[pos], out_v[pos] = sidx[i, e], sval[i, e]
    return out_p, out_r, out_i, out_v
