"""Oracle k-means codebook fit: ``calibrate_quantizer``
(rfsn_v10_mlx_ane_complete.py:175-225), restated in numpy (test
infrastructure only).

Steps per subspace (rfsn:185-189): sample ``C`` rows with replacement and
store them as fp16.  Each iteration (rfsn:192-214): encode with the current
codebooks (canonical chain of ``numerics.pq_encode``); replace every centroid
that has members by the fp32 mean of its members (empty clusters keep the
old centroid) and store fp16; record the distortion of the *old* codes
against the *new* codebooks and the fraction of residual norms below the RVQ
threshold.

The member mean is accumulated in float64 and rounded to fp32 (numpy's own
f32 pairwise mean at rfsn:205 has no fixed order to restate); k-means output
is a fitted input, so the GPU fit is pinned by invariants (non-increasing
distortion, fixed point), not bit-for-bit.

The seeded sampling uses ``torch.Generator('cpu')`` (MLX's RNG stream at
rfsn:188 is not reproducible off Apple hardware).
"""

from __future__ import annotations

from typing import Dict, List, Tuple

import numpy as np

from . import numerics as nx


def init_codebooks(x16: np.ndarray, num_subspaces: int, codebook_size: int, seed: int) -> np.ndarray:
    """Seeded with-replacement row sampling per subspace (rfsn:185-189)."""
    import torch

    n, D = x16.shape
    d = D // num_subspaces
    g = torch.Generator(device="cpu").manual_seed(int(seed))
    cb = np.zeros((num_subspaces, codebook_size, d), dtype=np.float16)
    for m in range(num_subspaces):
        idx = torch.randint(0, n, (codebook_size,), generator=g).numpy()
        cb[m] = x16[idx, m * d:(m + 1) * d]
    return cb


def centroid_update(x16: np.ndarray, codes: np.ndarray, cb: np.ndarray) -> np.ndarray:
    """Per-centroid member mean; empty clusters keep the old row (rfsn:197-207)."""
    M, C, d = cb.shape
    new = cb.astype(np.float32).copy()
    x32 = x16.astype(np.float64)
    for m in range(M):
        sub = x32[:, m * d:(m + 1) * d]
        cnt = np.bincount(codes[:, m].astype(np.int64), minlength=C)
        sums = np.zeros((C, d))
        for j in range(d):
            sums[:, j] = np.bincount(codes[:, m].astype(np.int64), weights=sub[:, j], minlength=C)
        has = cnt > 0
        new[m][has] = (sums[has] / cnt[has, None]).astype(np.float32)
    return new.astype(np.float16)


def calibrate(x16: np.ndarray, num_subspaces: int, codebook_size: int, iterations: int,
              seed: int, rvq_threshold: float = 0.0) -> Tuple[np.ndarray, Dict[str, List[float]]]:
    """Returns (codebooks fp16 [M, C, d], metrics) like rfsn:175-225."""
    cb = init_codebooks(x16, num_subspaces, codebook_size, seed)
    metrics: Dict[str, List[float]] = {"avg_distortion": [], "sparsity_fraction": []}
    x32 = x16.astype(np.float32)
    for _ in range(iterations):
        codes, resid = nx.pq_encode(x16, cb)
        cb = centroid_update(x16, codes, cb)
        recon = nx.pq_decode(codes, cb).astype(np.float32)
        metrics["avg_distortion"].append(float(np.mean((x32 - recon) ** 2)))
        norms = nx.rvq_norms(resid)
        metrics["sparsity_fraction"].append(float(np.mean(norms < np.float32(rvq_threshold))))
    return cb, metrics
