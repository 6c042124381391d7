"""Synthetic decode workloads (shapes of the path's benchmark configurations)
and their seeded inputs.

Inputs are drawn on the host with ``torch.Generator('cpu')`` seeded
``17 + 1000*b`` for sequence ``b`` (the reference eval seed is 17,
rfsn_v10_eval_benchmark.py:385-387), in a fixed order: per-channel scales
U(0.5, 2) (when enabled), K, V, query; every draw is fp32 cast to fp16, as the
reference draws ``normal(..., float32).astype(float16)``
(rfsn_v10_eval_benchmark.py:319-321).  The same bits feed the GPU path and
the CPU checks.
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace
from typing import Dict, Optional, Tuple

import torch

from .storage import RFSNConfig


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    q_heads: int
    kv_heads: int
    head_dim: int
    context: int
    hot: int
    warm: int
    cold: int = 0
    cold_chunk: int = 512
    cold_attended: int = 0
    pq_subspaces: int = 16
    pq_centroids: int = 256
    rvq_subspaces: int = 16
    rvq_centroids: int = 256
    sparse_k: int = 4
    block: int = 256
    channel_scale: bool = True
    kmeans_iters: int = 10
    kmeans_sample: int = 65536

    def config(self) -> RFSNConfig:
        return RFSNConfig(
            hidden_dim=self.q_heads * self.head_dim, num_heads=self.q_heads, head_dim=self.head_dim,
            num_subspaces=self.pq_subspaces, subspace_dim=self.head_dim // self.pq_subspaces,
            pq_bits=(self.pq_centroids - 1).bit_length(), num_rvq_layers=1,
            rvq_codebook_size=self.rvq_centroids if self.rvq_subspaces else 256,
            rvq_sparsity_threshold=float("inf") if not self.rvq_subspaces else 0.0,
            hot_capacity=self.hot, warm_capacity=self.warm, cold_capacity=max(self.cold, 1),
            block_size_seq=self.block, num_kv_heads=self.kv_heads, rvq_subspaces=self.rvq_subspaces,
            sparse_topk=self.sparse_k, tier_policy="recency", cold_chunk_tokens=self.cold_chunk,
            cold_medium="pinned")

    def bytes_per_step(self) -> int:
        """Algorithmic HBM bytes of one decode step (all sequences): exact hot
        K/V, encoded K/V of the attended warm and cold tokens, per-sequence
        codebooks once, the queries read and the outputs written."""
        D, M, Mr, k = self.head_dim, self.pq_subspaces, self.rvq_subspaces, self.sparse_k
        d, dr = D // M, (D // Mr if Mr else 0)
        per_vec = M + Mr + 3 * k
        enc_tokens = self.warm + self.cold_attended * self.cold_chunk
        cb = 2 * (M * self.pq_centroids * d + Mr * self.rvq_centroids * dr) * 2
        per_seq = (self.hot * self.kv_heads * 2 * D * 2 + enc_tokens * self.kv_heads * 2 * per_vec + cb
                   + 2 * self.q_heads * D * 2)
        return self.batch * per_seq


WORKLOADS: Dict[str, Workload] = {
    # one attention layer, 8 heads, 1,024 context: 128 exact + 896 PQ-only (M=8, d=8)
    "smoke_1k": Workload("smoke_1k", batch=1, q_heads=8, kv_heads=8, head_dim=64, context=1024, hot=128,
                         warm=896, pq_subspaces=8, rvq_subspaces=0, sparse_k=0, block=128,
                         channel_scale=False, kmeans_sample=896 * 8),
    # Llama-3.2-1B layer shape, 8,192 context: 512 exact + 7,680 PQ+RVQ+top-4
    "llama1b_8k": Workload("llama1b_8k", batch=1, q_heads=32, kv_heads=8, head_dim=64, context=8192, hot=512,
                           warm=7680, block=256, kmeans_sample=7680 * 8),
    # warm-tier compression: 4,096-token chunks of 8 KV heads, PQ M=8 + RVQ M=8 + top-4
    "encode_4k": Workload("encode_4k", batch=1, q_heads=8, kv_heads=8, head_dim=64, context=4096, hot=0,
                          warm=4096, pq_subspaces=8, rvq_subspaces=8, block=256, kmeans_sample=4096 * 8),
    # batched decode: 32 sequences x 32,768 context, 1,024 exact + 31,744 PQ+RVQ+top-4
    "batched_32x32k": Workload("batched_32x32k", batch=32, q_heads=32, kv_heads=8, head_dim=64, context=32768,
                               hot=1024, warm=31744, block=256),
    # long context with cold tier: 1,024 exact + 15,360 warm + 114,688 cold in 512-token chunks, 16 attended
    "longctx_128k": Workload("longctx_128k", batch=1, q_heads=32, kv_heads=4, head_dim=64, context=131072,
                             hot=1024, warm=15360, cold=114688, cold_chunk=512, cold_attended=16, block=256),
}


def seq_generator(b: int, base_seed: int = 17) -> torch.Generator:
    return torch.Generator(device="cpu").manual_seed(base_seed + 1000 * b)


def make_sequence(w: Workload, b: int, tokens: Optional[int] = None
                  ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Generator]:
    """(keys [T, Hkv, D] fp16, values, query [Hq, D] fp16, generator) on the host."""
    g = seq_generator(b)
    T = w.context if tokens is None else tokens
    H, D = w.kv_heads, w.head_dim
    if w.channel_scale:
        scale = torch.rand((H, D), generator=g, dtype=torch.float32) * 1.5 + 0.5
    else:
        scale = torch.ones((H, D), dtype=torch.float32)
    k = (torch.randn((T, H, D), generator=g, dtype=torch.float32) * scale).to(torch.float16)
    v = (torch.randn((T, H, D), generator=g, dtype=torch.float32) * scale).to(torch.float16)
    q = torch.randn((w.q_heads, D), generator=g, dtype=torch.float32).to(torch.float16)
    return k, v, q, g


@dataclass(frozen=True)
class RefWorkload:
    """A decode step over reference-format tiers (arrival policy: hot then
    warm), attended by the decode-in-register kernel."""
    name: str
    heads: int
    head_dim: int
    context: int
    hot: int
    pq_subspaces: int
    pq_centroids: int
    rvq_layers: int
    rvq_centroids: int

    @property
    def warm(self) -> int:
        return self.context - self.hot

    def bytes_per_step(self) -> int:
        """Algorithmic HBM bytes: exact hot K/V; per warm vector its PQ codes,
        its L u16 RVQ codes and its 4-byte row index (every row active at the
        reference's 0.005 gate on N(0,1) data); K and V codebooks once; the
        query read and the output written."""
        D, H = self.head_dim, self.heads
        per_vec = self.pq_subspaces + 2 * self.rvq_layers + 4
        cb = 2 * (self.pq_centroids * D + self.rvq_layers * self.rvq_centroids * D) * 2
        return self.hot * H * 2 * D * 2 + self.warm * H * 2 * per_vec + cb + 2 * H * D * 2


REF_WORKLOADS: Dict[str, RefWorkload] = {
    # the reference's default RFSNConfig (storage.py:23-45): 32 heads, head_dim
    # 128, PQ 8 x 256 (d 16), 4 gated RVQ layers x 4,096, hot 8,192; 32,768
    # context, so 24,576 warm tokens
    "refdefault_32k": RefWorkload("refdefault_32k", heads=32, head_dim=128, context=32768, hot=8192,
                                  pq_subspaces=8, pq_centroids=256, rvq_layers=4, rvq_centroids=4096),
    # encode in the same format: one 4,096-token chunk of 32 heads through
    # HybridQuantizerMLX.encode (PQ, norm gate, 4 full-dimension stages of
    # 4,096 centroids), codebooks drawn as the reference initialises them
    "refencode_4k": RefWorkload("refencode_4k", heads=32, head_dim=128, context=4096, hot=0,
                                pq_subspaces=8, pq_centroids=256, rvq_layers=4, rvq_centroids=4096),
}
