"""Blockwise exact attention entry points on MI355X -- the counterpart of the
reference's ``attention.py`` (attention.py:16-171).

``_blockwise_exact_attention`` runs the HIP split-K kernel over fp16 K/V; the
``block_size`` argument is accepted for drop-in compatibility and, as in the
reference, only changes fp32 rounding (the kernel's tile is fixed).  Keys and
values may have fewer heads than the query (GQA): query head ``h`` reads KV
head ``h // (Hq // Hkv)`` (llama32_adapter.py:384-386).
``RFSNHybridAttentionMLX`` attends the two compressed stores in one launch
of the decode-in-register kernel (``kernels.ref_attention``), which rebuilds
each K/V vector in registers with the decode's rounding (attention.py:159-171
decodes both stores, then attends); stores outside that kernel's shapes are
decoded and attended as the reference does.  The tiled fused
dequant-attention kernel is driven by the cache (``cache.py``), which owns the
code layout that kernel streams.
"""

from __future__ import annotations

import logging
from typing import Optional, Sequence, Union

import torch

from . import kernels as K
from .quantization import HybridQuantizerMLX, _decode_compressed_tensor
from .storage import MASK_FILL_VALUE, CompressedTensorMLX, RFSNConfig

# query heads (queries x heads) up to which the fused path uses score tables
REF_TABLES_MAX_QUERY_HEADS = 256

logger = logging.getLogger("RFSN_ATTENTION")

Positions = Optional[Union[Sequence[int], torch.Tensor]]


def _normalize_query_positions(query_positions: Positions, batch_size: int, num_heads: int,
                               default_position: int, device=None) -> torch.Tensor:
    """int32 [B, H] positions (attention.py:16-36)."""
    if query_positions is None:
        return torch.full((batch_size, num_heads), default_position, dtype=torch.int32, device=device)
    if isinstance(query_positions, torch.Tensor):
        positions = query_positions.to(device=device)
    else:
        positions = torch.tensor(query_positions, dtype=torch.int32, device=device)
    if positions.dim() == 1:
        if int(positions.shape[0]) != batch_size:
            raise ValueError("query_positions length must equal batch size")
        return positions.reshape(batch_size, 1).to(torch.int32).expand(batch_size, num_heads).contiguous()
    if tuple(int(d) for d in positions.shape) == (batch_size, num_heads):
        return positions.to(torch.int32).contiguous()
    raise ValueError("query_positions must have shape [B] or [B, H]")


def _blockwise_exact_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, scale: float,
                               block_size: int, causal: bool = False,
                               query_positions: Positions = None) -> torch.Tensor:
    """attention.py:39-105 on the GPU.  q [B, Hq, D]; keys/values [T, Hkv, D]."""
    batch_size, num_heads, head_dim = q.shape
    seq_len = int(keys.shape[0])
    if seq_len == 0:
        return torch.zeros((batch_size, num_heads, head_dim), dtype=q.dtype, device=q.device)
    if int(block_size) <= 0:
        raise ValueError("block_size must be positive")
    pos = _normalize_query_positions(query_positions, batch_size, num_heads, seq_len - 1, q.device)
    qh = q.to(torch.float16)
    out = K.blockwise_attention(qh, keys.to(torch.float16), values.to(torch.float16), scale, causal,
                                pos if causal else None)
    return out.to(q.dtype)


class RFSNHybridAttentionMLX:
    """Attention over compressed key/value stores (attention.py:141-171)."""

    def __init__(self, config: RFSNConfig):
        self.config = config
        self.scale = config.head_dim ** -0.5
        self.block_size = config.block_size_seq

    def __call__(self, q: torch.Tensor, key_store: CompressedTensorMLX, value_store: CompressedTensorMLX,
                 quantizer: HybridQuantizerMLX, causal: bool = False,
                 query_positions: Positions = None) -> torch.Tensor:
        if key_store.num_tokens != value_store.num_tokens:
            raise ValueError("Key/value stores must have the same token count")
        if self._fused_ok(q, key_store, quantizer):
            return self._fused(q, key_store, value_store, quantizer, causal, query_positions)
        decoded_keys = _decode_compressed_tensor(key_store, quantizer)
        decoded_values = _decode_compressed_tensor(value_store, quantizer)
        return _blockwise_exact_attention(q=q, keys=decoded_keys, values=decoded_values, scale=self.scale,
                                          block_size=self.block_size, causal=causal,
                                          query_positions=query_positions)

    def _fused_ok(self, q: torch.Tensor, key_store: CompressedTensorMLX, quantizer: HybridQuantizerMLX) -> bool:
        if q.dim() != 3 or key_store.num_heads <= 0 or key_store.subspace != quantizer.subspace:
            return False
        M, C, _ = quantizer.pq.codebooks.shape
        f = quantizer.warm_format()
        sub = (f.rvq_subspaces, f.rvq_centroids, f.sparse_k) if quantizer.subspace else (0, 0, 0)
        return (q.shape[-1] == quantizer.config.head_dim and q.shape[1] % key_store.num_heads == 0
                and K.ref_attention_ok(int(q.shape[-1]), int(M), int(C), int(q.shape[1]), key_store.num_heads,
                                       True, *sub))

    def _fused(self, q, key_store, value_store, quantizer, causal, query_positions) -> torch.Tensor:
        """Decode-and-attend in one kernel: each K/V vector is rebuilt in
        registers with the reference's rounding (quantization.py:310-319) and
        never written to HBM (rfsn_ref_attention)."""
        B, Hq, _ = q.shape
        T = key_store.num_tokens
        if T == 0:
            return torch.zeros_like(q)
        dev = quantizer.device
        kst = _on(key_store, dev)
        vst = _on(value_store, dev)
        pos = _normalize_query_positions(query_positions, B, Hq, T - 1, dev) if causal else None
        cb, rcb = quantizer.pq.codebooks, quantizer.rvq_codebooks
        f = quantizer.warm_format()
        # score tables with their drift guard (config.score_table_tolerance)
        # for decode-sized calls of the reference format over enough coded
        # tokens for the tables to beat the exact decode
        tol = quantizer.config.score_table_tolerance
        tables = {}
        if (tol is not None and not quantizer.subspace and B * Hq <= REF_TABLES_MAX_QUERY_HEADS
                and T >= K.ref_tables_min_tokens(Hq // key_store.num_heads, B)):
            tables = dict(score_tables=float(tol), table_stats=self._table_stats(quantizer))
        # the tables read a head's codes in whole lines from a head-major
        # copy, kept per store (only for stores already on the device, which
        # outlive the call)
        hm = bool(tables) and kst is key_store and vst is value_store
        out = K.ref_attention(q.to(device=dev, dtype=torch.float16), kv_heads=key_store.num_heads,
                              scale=self.scale, causal=causal, qpos=pos,
                              segments=[K.ref_store_segment(kst, vst, 0, T, 0, head_major=hm)], k_pq_cb=cb, v_pq_cb=cb,
                              k_rvq_cb=rcb, v_rvq_cb=rcb, rvq_subspaces=f.rvq_subspaces if quantizer.subspace else 0,
                              sparse_k=f.sparse_k if quantizer.subspace else 0, **tables)
        return out.to(q.dtype)

    def _table_stats(self, quantizer: HybridQuantizerMLX) -> torch.Tensor:
        """The score tables' guard statistics of the quantizer's codebooks,
        rebuilt when the quantizer or a codebook changes."""
        cbs = (quantizer.pq.codebooks, quantizer.rvq_codebooks)
        key = (quantizer,) + cbs + tuple(None if t is None else t._version for t in cbs)
        memo = getattr(self, "_stats_memo", None)
        if memo is None or len(memo[0]) != len(key) or not all(
                (a is b) if not isinstance(a, int) else a == b for a, b in zip(memo[0], key)):
            memo = (key, K.ref_table_stats(cbs[0], cbs[0], cbs[1], cbs[1]))
            self._stats_memo = memo
        return memo[1]


def _on(store: CompressedTensorMLX, device) -> CompressedTensorMLX:
    if store.pq_codes.device == torch.device(device):
        return store
    d = lambda t: None if t is None else t.to(device)
    return CompressedTensorMLX(d(store.pq_codes), d(store.rvq_codes), d(store.rvq_mask), d(store.rvq_offsets),
                               store.num_heads, d(store.sparse_idx), d(store.sparse_val))
