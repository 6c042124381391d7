"""Configuration, compressed containers, cold-chunk storage and the chunk
router -- the MI355X counterpart of the reference's ``storage.py``.

Same names, fields, defaults and error behaviour as storage.py:19-237, with
torch tensors in place of MLX arrays.  Extension fields (no reference
counterpart) describe the warm-tier format of the long-context
configurations: ``num_kv_heads`` (GQA storage), ``rvq_subspaces`` (a
subspace RVQ stage instead of the gated full-dimension one), ``sparse_topk``,
``tier_policy`` ("arrival" as in cache.py:103-118, or "recency": hot holds the
newest tokens), ``cold_chunk_tokens`` and ``cold_medium`` ("npz" files as in
storage.py:113-140, or "pinned" host memory), and ``fused_score_tables``
(the fused kernel may score K codes through fp16 q . centroid tables; False
keeps the exact codebook path, whose scores are q . fp16(K^) as in the
reference).
"""

from __future__ import annotations

import asyncio
import bisect
import logging
from dataclasses import dataclass, field
from pathlib import Path
from typing import Dict, List, Optional

import numpy as np
import torch

logger = logging.getLogger("RFSN_STORAGE")

SUPPORTED_GROUP_SIZES = (128, 64, 32)
MASK_FILL_VALUE = -1e30


@dataclass
class RFSNConfig:
    """Hyperparameters (storage.py:19-59)."""

    hidden_dim: int = 4096
    num_heads: int = 32
    head_dim: int = 128
    num_layers: int = 32

    num_subspaces: int = 8
    pq_bits: int = 8
    subspace_dim: int = 16
    pq_codebook_dtype: str = "float16"

    num_rvq_layers: int = 4
    rvq_codebook_size: int = 4096
    rvq_sparsity_threshold: float = 0.005
    max_rvq_sparse: int = 64

    hot_capacity: int = 8192
    warm_capacity: int = 65536
    cold_capacity: int = 2_000_000

    block_size_seq: int = 128

    ane_quant_bits: int = 6
    ane_group_size: int = 128

    disk_cache_dir: str = "./rfsn_disk_cache"
    max_open_files: int = 8
    prefetch_throttle_s: float = 0.5

    cpu_threads: int = 4

    # ---- extensions (no reference counterpart) ----
    num_kv_heads: Optional[int] = None
    rvq_subspaces: int = 0
    sparse_topk: int = 0
    tier_policy: str = "arrival"
    cold_chunk_tokens: Optional[int] = None
    cold_medium: str = "npz"
    # score K through q . centroid tables where the format allows (16 + 16
    # subspaces, <= 4 query heads per KV head): faster, but each table entry
    # is rounded to fp16, so scores drift from q . fp16(K^) in proportion to
    # |q|; False keeps the exact codebook path
    fused_score_tables: bool = True
    # drift guard of the score tables: a block whose estimated output drift
    # (from |q|, the codebook magnitudes, sum p^2 and max |V|) exceeds this
    # tolerance recomputes its output on the exact codebook path; None: no
    # guard (the K sparse entries then carry no corrected-coordinate plane)
    score_table_tolerance: Optional[float] = 2e-3

    def __post_init__(self) -> None:
        expected = self.num_subspaces * self.subspace_dim
        if expected != self.head_dim:
            raise ValueError(
                "head_dim must equal num_subspaces * subspace_dim: "
                f"{self.head_dim} != {expected}"
            )
        if self.rvq_subspaces and self.head_dim % self.rvq_subspaces:
            raise ValueError("head_dim must be a multiple of rvq_subspaces")
        if self.tier_policy not in ("arrival", "recency"):
            raise ValueError("tier_policy must be 'arrival' or 'recency'")
        if self.cold_medium not in ("npz", "pinned"):
            raise ValueError("cold_medium must be 'npz' or 'pinned'")
        if self.score_table_tolerance is not None and not self.score_table_tolerance >= 0:
            raise ValueError("score_table_tolerance must be None or >= 0")

    @property
    def kv_heads(self) -> int:
        return self.num_heads if self.num_kv_heads is None else self.num_kv_heads

    @property
    def subspace_rvq(self) -> bool:
        return self.rvq_subspaces > 0

    @property
    def ext_format(self) -> bool:
        """Warm format of the long-context configurations (subspace RVQ stage
        and/or sparse residual) instead of the reference's gated RVQ."""
        return self.rvq_subspaces > 0 or self.sparse_topk > 0

    @property
    def chunk_tokens(self) -> int:
        return max(1, self.cold_chunk_tokens or self.block_size_seq)


@dataclass
class CompressedTensorMLX:
    """Compressed representation of a [T, H, D] tensor (storage.py:75-98).

    Reference format: ``pq_codes`` u8 [T, H, M], ``rvq_codes`` u16 [A, L],
    ``rvq_mask`` bool [T, H], ``rvq_offsets`` int32 [A] (flat t*H+h, ascending).
    Subspace format (extension): ``rvq_codes`` u8 [T, H, M_r] (every vector),
    ``rvq_mask`` all True, ``rvq_offsets`` empty, plus ``sparse_idx`` u8
    [T, H, k] and ``sparse_val`` fp16 [T, H, k].
    """

    pq_codes: torch.Tensor
    rvq_codes: torch.Tensor
    rvq_mask: torch.Tensor
    rvq_offsets: torch.Tensor
    num_heads: int
    sparse_idx: Optional[torch.Tensor] = None
    sparse_val: Optional[torch.Tensor] = None

    @property
    def num_tokens(self) -> int:
        return int(self.pq_codes.shape[0])

    @property
    def subspace(self) -> bool:
        return self.rvq_codes.dim() == 3

    @classmethod
    def empty(cls, config: RFSNConfig, num_heads: Optional[int] = None,
              device: Optional[torch.device] = None) -> "CompressedTensorMLX":
        heads = config.num_heads if num_heads is None else num_heads
        dev = device if device is not None else torch.device("cpu")
        if config.ext_format:
            return cls(
                pq_codes=torch.zeros((0, heads, config.num_subspaces), dtype=torch.uint8, device=dev),
                rvq_codes=torch.zeros((0, heads, config.rvq_subspaces), dtype=torch.uint8, device=dev),
                rvq_mask=torch.zeros((0, heads), dtype=torch.bool, device=dev),
                rvq_offsets=torch.zeros((0,), dtype=torch.int32, device=dev),
                num_heads=heads,
                sparse_idx=torch.zeros((0, heads, config.sparse_topk), dtype=torch.uint8, device=dev),
                sparse_val=torch.zeros((0, heads, config.sparse_topk), dtype=torch.float16, device=dev),
            )
        return cls(
            pq_codes=torch.zeros((0, heads, config.num_subspaces), dtype=torch.uint8, device=dev),
            rvq_codes=torch.zeros((0, config.num_rvq_layers), dtype=torch.uint16, device=dev),
            rvq_mask=torch.zeros((0, heads), dtype=torch.bool, device=dev),
            rvq_offsets=torch.zeros((0,), dtype=torch.int32, device=dev),
            num_heads=heads,
        )


def _as_i16(t: torch.Tensor) -> torch.Tensor:
    """uint16 tensors are indexed and concatenated through an int16 view (same
    bits): torch implements few uint16 kernels."""
    return t.view(torch.int16) if t.dtype == torch.uint16 else t


def _like(src: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint16) if src.dtype == torch.uint16 else t


def _concat0(lhs: torch.Tensor, rhs: torch.Tensor) -> torch.Tensor:
    """Concat on axis 0 skipping empty operands (storage.py:101-106)."""
    if lhs.shape[0] == 0:
        return rhs
    if rhs.shape[0] == 0:
        return lhs
    return _like(lhs, torch.cat([_as_i16(lhs), _as_i16(rhs)], dim=0))


def _index0(t: torch.Tensor, sel: torch.Tensor) -> torch.Tensor:
    """t[sel] along axis 0 for any dtype, uint16 included."""
    return _like(t, _as_i16(t)[sel])


def _numpy_ints(values: torch.Tensor) -> np.ndarray:
    """int64 host copy (storage.py:109-110)."""
    return values.detach().to("cpu").numpy().astype(np.int64)


def _host(t: Optional[torch.Tensor]) -> Optional[np.ndarray]:
    if t is None:
        return None
    t = t.detach().to("cpu")
    if t.dtype == torch.uint16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _from_host(a: np.ndarray, device) -> torch.Tensor:
    if a.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.uint16).to(device)
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def chunk_file_path(root: Path, layer_idx: int, chunk_id: int) -> Path:
    """storage.py:113-114."""
    return root / f"layer{layer_idx}_chunk{chunk_id}.npz"


def save_compressed_chunk(chunk_path: Path, keys: CompressedTensorMLX, values: CompressedTensorMLX) -> None:
    """NPZ chunk schema of storage.py:117-135 (plus sparse arrays when present)."""
    chunk_path.parent.mkdir(parents=True, exist_ok=True)
    arrays = dict(
        num_tokens=np.array([keys.num_tokens], dtype=np.int32),
        num_heads=np.array([keys.num_heads], dtype=np.int32),
    )
    for prefix, t in (("key", keys), ("value", values)):
        arrays[f"{prefix}_pq_codes"] = _host(t.pq_codes)
        arrays[f"{prefix}_rvq_codes"] = _host(t.rvq_codes)
        arrays[f"{prefix}_rvq_mask"] = _host(t.rvq_mask)
        arrays[f"{prefix}_rvq_offsets"] = _host(t.rvq_offsets)
        if t.sparse_idx is not None:
            arrays[f"{prefix}_sparse_idx"] = _host(t.sparse_idx)
            arrays[f"{prefix}_sparse_val"] = _host(t.sparse_val)
    np.savez_compressed(chunk_path, **arrays)


def load_compressed_chunk(chunk_path: Path, device=None) -> Dict[str, torch.Tensor]:
    """storage.py:138-140 (no pickle: ``allow_pickle`` stays False)."""
    data = np.load(chunk_path, allow_pickle=False)
    dev = device if device is not None else torch.device("cpu")
    return {key: _from_host(data[key], dev) for key in data.files}


def compressed_tensor_from_loaded(loaded: Dict[str, torch.Tensor], prefix: str) -> CompressedTensorMLX:
    """storage.py:143-151."""
    num_heads = int(loaded["num_heads"].reshape(-1)[0].item())
    return CompressedTensorMLX(
        pq_codes=loaded[f"{prefix}_pq_codes"],
        rvq_codes=loaded[f"{prefix}_rvq_codes"],
        rvq_mask=loaded[f"{prefix}_rvq_mask"],
        rvq_offsets=loaded[f"{prefix}_rvq_offsets"].to(torch.int32),
        num_heads=num_heads,
        sparse_idx=loaded.get(f"{prefix}_sparse_idx"),
        sparse_val=loaded.get(f"{prefix}_sparse_val"),
    )


class AsyncHierarchicalRouterMLX:
    """Cold-chunk prefetcher (storage.py:154-237).

    Ranking is the reference's: existing chunk ids in
    ``[(pos - w)//cs, (pos + w)//cs]`` ordered by ``|cid*cs - pos|``, top-k
    loaded, FIFO cache of 16.  For a cache whose cold tier lives in pinned
    host memory, ``bind(cache)`` makes the router rank that cache's chunk ids
    instead of probing files, and ``get_chunk`` reports chunks already
    resident in the cache's device slots.
    """

    def __init__(self, config: RFSNConfig, layer_idx: int = 0):
        self.config = config
        self.layer_idx = layer_idx
        self.disk_dir = Path(config.disk_cache_dir)
        self.throttle = config.prefetch_throttle_s
        self._cache: Dict[int, Dict[str, torch.Tensor]] = {}
        self._max_cache_size = 16
        self._pending_prefetch: set = set()
        self._bound = None
        self._rank_memo = None  # (key, last chunk start, order) of the bound cache's last ranking

    def bind(self, cache) -> "AsyncHierarchicalRouterMLX":
        self._bound = cache
        return self

    def _chunk_size(self) -> int:
        if self._bound is not None:
            return self._bound.config.chunk_tokens
        return max(self.config.block_size_seq, 1)

    def _exists(self, chunk_id: int) -> bool:
        if self._bound is not None:
            return self._bound.has_cold_chunk(chunk_id)
        return chunk_file_path(self.disk_dir, self.layer_idx, chunk_id).exists()

    def rank(self, current_position: int, context_window: int) -> List[int]:
        cs = self._chunk_size()
        start_chunk = max(0, (current_position - context_window) // cs)
        end_chunk = max(start_chunk, (current_position + context_window) // cs)
        if self._bound is not None:
            ids = self._bound.cold_chunk_ids()
            # a decode loop asks again every token: while the bound cache's id
            # list and the candidate range stay, and every candidate starts at
            # or before the position (distance = position - start, so the
            # order is descending id whatever the position), the last order holds
            key = (id(ids), len(ids), start_chunk, end_chunk)
            memo = self._rank_memo
            if memo is not None and memo[0] == key and current_position >= memo[1]:
                return list(memo[2])
            cands = ids[bisect.bisect_left(ids, start_chunk):bisect.bisect_right(ids, end_chunk)]
        else:
            cands = [cid for cid in range(start_chunk, end_chunk + 1) if self._exists(cid)]
        cands.sort(key=lambda cid: abs(cid * cs - current_position))
        if self._bound is not None:
            last = max(cands) * cs if cands else 0
            self._rank_memo = (key, last, tuple(cands)) if current_position >= last else None
        return cands

    async def predict_and_prefetch(self, current_position: int, context_window: int, top_k: int = 2) -> List[int]:
        candidates = self.rank(current_position, context_window)
        if self._bound is not None:
            # pinned medium: the chunks not yet held move in one batch of copies
            ids = candidates[:top_k]
            new = [cid for cid in ids if cid not in self._cache]
            if new:
                slots = self._bound.prefetch_cold_chunks(new)
                for cid in new:
                    self._cache[cid] = slots[cid]
            self._trim()
            return ids
        loaded: List[int] = []
        for chunk_id in candidates[:top_k]:
            if chunk_id in self._cache:
                loaded.append(chunk_id)
                continue
            if chunk_id in self._pending_prefetch:
                continue
            self._pending_prefetch.add(chunk_id)
            await self._load_chunk(chunk_id)
            self._pending_prefetch.discard(chunk_id)
            loaded.append(chunk_id)
            if self.throttle > 0:
                await asyncio.sleep(self.throttle)
        self._trim()
        return loaded

    def _trim(self) -> None:
        """FIFO of at most 16 chunks (storage.py:197-199)."""
        while len(self._cache) > self._max_cache_size:
            oldest_key = next(iter(self._cache))
            del self._cache[oldest_key]

    def prefetch_ahead(self, current_position: int, context_window: int, top_k: int = 2) -> List[int]:
        """For a router bound to a pinned-medium cache: rank the chunks for
        ``current_position`` and start their copies on the side stream
        without waiting, one decode step ahead; the next attention call
        orders itself after them.  Returns the ranked chunk ids."""
        if self._bound is None:
            raise RuntimeError("prefetch_ahead needs a router bound to a pinned-medium cache (bind)")
        ids = self.rank(current_position, context_window)[:top_k]
        slots = self._bound.prefetch_cold_chunks(ids, wait=False)
        for cid in ids:
            self._cache[cid] = slots[cid]
        self._trim()
        return ids

    def prefetch_sync(self, current_position: int, context_window: int, top_k: int = 2) -> List[int]:
        try:
            return asyncio.run(self.predict_and_prefetch(current_position, context_window, top_k))
        except RuntimeError:
            loop = asyncio.new_event_loop()
            try:
                return loop.run_until_complete(self.predict_and_prefetch(current_position, context_window, top_k))
            finally:
                loop.close()

    async def _load_chunk(self, chunk_id: int) -> None:
        loop = asyncio.get_running_loop()
        loaded = await loop.run_in_executor(None, self._load_chunk_sync, chunk_id)
        self._cache[chunk_id] = loaded

    def _load_chunk_sync(self, chunk_id: int) -> Dict[str, torch.Tensor]:
        path = chunk_file_path(self.disk_dir, self.layer_idx, chunk_id)
        if not path.exists():
            return {}
        return load_compressed_chunk(path)

    def get_chunk(self, chunk_id: int) -> Optional[Dict[str, torch.Tensor]]:
        if self._bound is not None and chunk_id in self._cache:
            # a chunk the router fetched counts while it is still in a device slot
            return self._bound.resident_cold_chunk(chunk_id)
        return self._cache.get(chunk_id)
