"""PQ codebook calibration by k-means on the GPU -- ``calibrate_quantizer``
(rfsn_v10_mlx_ane_complete.py:175-225).

Initialisation samples ``C`` calibration rows with replacement per subspace
(rfsn:185-189) from a seeded torch generator; each iteration encodes with the
canonical nearest-centroid HIP kernel, replaces every centroid that has
members by the fp32 mean of its members (HIP segmented reduction; empty
clusters keep their row, rfsn:197-207), and records the distortion of the old
codes against the new codebooks and the fraction of residual norms below the
RVQ threshold (rfsn:209-214).
"""

from __future__ import annotations

import logging
from typing import Dict, List, Optional

import torch

from . import kernels as K
from .quantization import HybridQuantizerMLX

logger = logging.getLogger("RFSN_CALIBRATE")


def init_codebooks(x: torch.Tensor, num_subspaces: int, codebook_size: int,
                   generator: Optional[torch.Generator]) -> torch.Tensor:
    n, D = x.shape
    d = D // num_subspaces
    cb = torch.empty((num_subspaces, codebook_size, d), dtype=torch.float16, device=x.device)
    for m in range(num_subspaces):
        idx = torch.randint(0, n, (codebook_size,), generator=generator).to(x.device)
        cb[m] = x[idx, m * d:(m + 1) * d]
    return cb


def fit_codebooks(x: torch.Tensor, num_subspaces: int, codebook_size: int, iterations: int,
                  generator: Optional[torch.Generator] = None, threshold: float = 0.0
                  ) -> (torch.Tensor, Dict[str, List[float]]):
    """k-means fit of [M, C, D/M] fp16 codebooks on x [N, D] fp16 (device)."""
    x = x.to(torch.float16).contiguous()
    cb = init_codebooks(x, num_subspaces, codebook_size, generator).contiguous()
    metrics: Dict[str, List[float]] = {"avg_distortion": [], "sparsity_fraction": []}
    fmt = K.WarmFormat(x.shape[1], num_subspaces, codebook_size)
    x32 = x.float()
    for _ in range(iterations):
        codes, resid = K.pq_encode(x, cb)
        K.kmeans_update(x, codes, cb)
        recon = K.decode(fmt, codes, cb).float()
        metrics["avg_distortion"].append(float(((x32 - recon) ** 2).mean().item()))
        norms = torch.sqrt((resid.float() ** 2).sum(dim=1))
        metrics["sparsity_fraction"].append(float((norms < threshold).float().mean().item()))
    return cb, metrics


def calibrate_quantizer(quantizer: HybridQuantizerMLX, calibration_vectors: torch.Tensor,
                        num_iterations: int = 20, generator: Optional[torch.Generator] = None
                        ) -> Dict[str, List[float]]:
    """rfsn_v10_mlx_ane_complete.py:175-225: fits ``quantizer.pq.codebooks`` in place."""
    logger.info("Calibrating PQ codebooks with %d vectors", int(calibration_vectors.shape[0]))
    x = calibration_vectors.to(quantizer.device, torch.float16)
    cb, metrics = fit_codebooks(x, quantizer.config.num_subspaces, quantizer.pq.codebook_size, num_iterations,
                                generator, quantizer.config.rvq_sparsity_threshold)
    quantizer.pq.codebooks = cb
    return metrics
