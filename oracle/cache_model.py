"""Oracle model of the tiered KV cache ``RFSNv10KVCacheMLX`` (cache.py:33-440)
and of the cold-chunk router ``AsyncHierarchicalRouterMLX``
(storage.py:154-237), in numpy (test infrastructure only).

Restated behaviour:

* tier fill by arrival: hot, then warm (encoded), then cold (cache.py:89-120);
* cold chunking by ``block_size_seq`` with ``chunk_id = global_start // chunk``
  and merge-on-append of a contiguous partial chunk (cache.py:134-191); the
  chunk payload is kept in memory instead of an NPZ file (same content);
* window bounds and adjusted query positions (cache.py:199-241);
* per-tier materialization with the access counters (cache.py:250-393);
* ``attention_forward`` = materialize + blockwise attention (cache.py:395-428);
* ``memory_usage_bytes`` (cache.py:430-440);
* router ranking ``|cid*cs - pos|`` over existing chunks, top-k prefetch,
  FIFO cache of 16 (storage.py:166-201).

Parity: pinned by the reference test suite's assertions replayed as known
answers (rfsn_v10_mlx_ane_complete.py:448-554) and by the byte columns of
benchmark_outputs/dense_vs_hot_warm.csv (see tests/test_oracle.py).
"""

from __future__ import annotations

from typing import Dict, List, Optional

import numpy as np

from . import numerics as nx


class OracleQuantizer:
    """Reference-mode hybrid quantizer: PQ [M,C,d] + gated full-D RVQ [L,C,D]."""

    def __init__(self, pq_cb: np.ndarray, rvq_cb: np.ndarray, threshold: float):
        self.pq_cb = pq_cb
        self.rvq_cb = rvq_cb
        self.threshold = threshold

    def compress(self, t16: np.ndarray) -> dict:
        return nx.compress_tensor_sequence(t16, self.pq_cb, self.rvq_cb, self.threshold)

    def decompress(self, store: dict) -> np.ndarray:
        return nx.decode_compressed(store, self.pq_cb, self.rvq_cb)


def empty_store(H: int, M: int, L: int) -> dict:
    return {"pq_codes": np.zeros((0, H, M), np.uint8), "rvq_codes": np.zeros((0, L), np.uint16),
            "rvq_mask": np.zeros((0, H), bool), "rvq_offsets": np.zeros((0,), np.int32), "num_heads": H}


def empty_stats() -> Dict[str, int]:
    """``_empty_access_stats`` (cache.py:59-76)."""
    return {"window_start": 0, "window_end": 0, "window_tokens": 0, "context_window": -1,
            "query_tokens": 0, "used_router": 0, "hot_tokens_materialized": 0,
            "warm_tokens_materialized": 0, "cold_tokens_materialized": 0, "reconstructed_tokens": 0,
            "warm_chunk_decodes": 0, "cold_chunk_decodes": 0, "cold_chunks_touched": 0,
            "cold_chunk_cache_hits": 0, "cold_chunk_cache_misses": 0}


class OracleRouter:
    """``AsyncHierarchicalRouterMLX`` ranking and FIFO cache (storage.py:154-237)."""

    def __init__(self, cache: "OracleCache", chunk_tokens: int):
        self.cache = cache
        self.cs = max(chunk_tokens, 1)
        self._cache: Dict[int, dict] = {}

    def prefetch(self, current_position: int, context_window: int, top_k: int = 2) -> List[int]:
        start = max(0, (current_position - context_window) // self.cs)
        end = max(start, (current_position + context_window) // self.cs)
        cands = [cid for cid in range(start, end + 1) if cid in self.cache.cold_chunks]
        cands.sort(key=lambda cid: abs(cid * self.cs - current_position))
        loaded = []
        for cid in cands[:top_k]:
            if cid not in self._cache:
                self._cache[cid] = self.cache.cold_chunks[cid]
            loaded.append(cid)
        while len(self._cache) > 16:
            del self._cache[next(iter(self._cache))]
        return loaded

    def get_chunk(self, cid: int) -> Optional[dict]:
        return self._cache.get(cid)


class OracleCache:
    def __init__(self, num_heads: int, head_dim: int, num_subspaces: int, num_rvq_layers: int,
                 hot_capacity: int, warm_capacity: int, block_size_seq: int):
        self.H, self.D, self.M, self.L = num_heads, head_dim, num_subspaces, num_rvq_layers
        self.hot_capacity, self.warm_capacity, self.block = hot_capacity, warm_capacity, block_size_seq
        self.hot_keys = np.zeros((0, num_heads, head_dim), np.float16)
        self.hot_values = np.zeros((0, num_heads, head_dim), np.float16)
        self.warm_keys = empty_store(num_heads, num_subspaces, num_rvq_layers)
        self.warm_values = empty_store(num_heads, num_subspaces, num_rvq_layers)
        self.cold_chunks: Dict[int, dict] = {}     # chunk_id -> {"key": store, "value": store}
        self.cold_meta: List[dict] = []
        self.num_hot = self.num_warm = self.num_cold = self.total_tokens = 0
        self.quantizer: Optional[OracleQuantizer] = None
        self.last_access_stats = empty_stats()

    # -- update (cache.py:89-191) ------------------------------------------------
    def update(self, keys: np.ndarray, values: np.ndarray, quantizer: OracleQuantizer) -> None:
        if keys.shape != values.shape:
            raise ValueError("new_keys and new_values must have identical shapes")
        self.quantizer = quantizer
        T = keys.shape[0]
        off = 0
        hot_space = max(self.hot_capacity - self.num_hot, 0)
        if hot_space > 0 and off < T:
            take = min(hot_space, T - off)
            self.hot_keys = np.concatenate([self.hot_keys, keys[off:off + take]])
            self.hot_values = np.concatenate([self.hot_values, values[off:off + take]])
            self.num_hot += take
            off += take
        warm_space = max(self.warm_capacity - self.num_warm, 0)
        if warm_space > 0 and off < T:
            take = min(warm_space, T - off)
            self.warm_keys = nx.append_compressed(self.warm_keys, quantizer.compress(keys[off:off + take]))
            self.warm_values = nx.append_compressed(self.warm_values, quantizer.compress(values[off:off + take]))
            self.num_warm += take
            off += take
        if off < T:
            self._add_to_cold(keys[off:], values[off:], quantizer)
        self.total_tokens += T

    def _add_to_cold(self, keys, values, quantizer):
        ct = max(1, self.block)
        start_token = self.num_hot + self.num_warm + self.num_cold
        for o in range(0, keys.shape[0], ct):
            e = min(o + ct, keys.shape[0])
            n = e - o
            cstart = start_token + o
            cid = cstart // ct
            ck, cv = quantizer.compress(keys[o:e]), quantizer.compress(values[o:e])
            meta = next((m for m in self.cold_meta if m["chunk_id"] == cid), None)
            if meta is not None and cid in self.cold_chunks:
                if cstart != meta["end_token"]:
                    raise ValueError("Cold chunk append must be contiguous with existing metadata")
                old = self.cold_chunks[cid]
                self.cold_chunks[cid] = {"key": nx.append_compressed(old["key"], ck),
                                         "value": nx.append_compressed(old["value"], cv)}
                meta["end_token"] += n
                meta["num_tokens"] += n
            else:
                self.cold_chunks[cid] = {"key": ck, "value": cv}
                self.cold_meta.append({"chunk_id": cid, "start_token": cstart,
                                       "end_token": cstart + n, "num_tokens": n})
        self.num_cold += keys.shape[0]

    # -- window (cache.py:199-248) ---------------------------------------------------
    def window_bounds(self, query_positions, context_window, current_position):
        if self.total_tokens == 0:
            return 0, 0, None if query_positions is None else np.asarray(query_positions, np.int32)
        if query_positions is not None:
            max_q = int(np.max(np.asarray(query_positions, dtype=np.int64)))
        elif current_position is not None:
            max_q = current_position
        else:
            max_q = max(self.total_tokens - 1, 0)
        end = min(max_q + 1, self.total_tokens)
        start = 0 if context_window is None else max(0, end - context_window)
        if query_positions is None:
            return start, end, None
        adj = np.maximum(np.asarray(query_positions, np.int32) - start, -1).astype(np.int32)
        return start, end, adj

    @staticmethod
    def _overlap(s, e, ss, se):
        a, b = max(s, ss), min(e, se)
        return None if a >= b else (a, b)

    # -- materialize (cache.py:250-393) ---------------------------------------------
    def materialize_window(self, query_positions=None, context_window=None, router=None,
                           current_position=None):
        if self.quantizer is None:
            raise RuntimeError("Cache cannot materialize values before update() provides a quantizer")
        start, end, adj = self.window_bounds(query_positions, context_window, current_position)
        st = empty_stats()
        st["window_start"], st["window_end"] = start, end
        st["window_tokens"] = max(0, end - start)
        st["context_window"] = -1 if context_window is None else context_window
        st["used_router"] = int(router is not None)
        ks, vs = [], []
        ov = self._overlap(start, end, 0, self.num_hot)
        if ov is not None:
            st["hot_tokens_materialized"] += ov[1] - ov[0]
            ks.append(self.hot_keys[ov[0]:ov[1]])
            vs.append(self.hot_values[ov[0]:ov[1]])
        ov = self._overlap(start, end, self.num_hot, self.num_hot + self.num_warm)
        if ov is not None:
            ls, le = ov[0] - self.num_hot, ov[1] - self.num_hot
            for cs in range(ls, le, max(1, self.block)):
                ce = min(cs + max(1, self.block), le)
                ks.append(self.quantizer.decompress(nx.slice_compressed(self.warm_keys, cs, ce)))
                vs.append(self.quantizer.decompress(nx.slice_compressed(self.warm_values, cs, ce)))
                st["warm_tokens_materialized"] += ce - cs
                st["reconstructed_tokens"] += ce - cs
                st["warm_chunk_decodes"] += 1
        if self.cold_meta:
            if router is not None and current_position is not None and context_window is not None:
                ct = max(1, self.block)
                router.prefetch(current_position, context_window, max(1, (context_window + ct - 1) // ct))
            for meta in self.cold_meta:
                ov = self._overlap(start, end, meta["start_token"], meta["end_token"])
                if ov is None:
                    continue
                cid = meta["chunk_id"]
                loaded = router.get_chunk(cid) if router is not None else None
                if loaded is None:
                    loaded = self.cold_chunks[cid]
                    if router is not None:
                        st["cold_chunk_cache_misses"] += 1
                else:
                    st["cold_chunk_cache_hits"] += 1
                ls, le = ov[0] - meta["start_token"], ov[1] - meta["start_token"]
                ks.append(self.quantizer.decompress(nx.slice_compressed(loaded["key"], ls, le)))
                vs.append(self.quantizer.decompress(nx.slice_compressed(loaded["value"], ls, le)))
                st["cold_tokens_materialized"] += le - ls
                st["reconstructed_tokens"] += le - ls
                st["cold_chunk_decodes"] += 1
                st["cold_chunks_touched"] += 1
        self.last_access_stats = dict(st)
        if not ks:
            empty = np.zeros((0, self.H, self.D), np.float16)
            return empty, empty, adj
        return np.concatenate(ks), np.concatenate(vs), adj

    def attention_forward(self, q, causal=True, query_positions=None, router=None,
                          current_position=None, context_window=None):
        if self.quantizer is None:
            raise RuntimeError("Cache cannot run attention before update() provides a quantizer")
        k, v, adj = self.materialize_window(query_positions, context_window, router, current_position)
        self.last_access_stats["query_tokens"] = int(q.shape[0])
        if k.shape[0] == 0:
            return np.zeros_like(q)
        return nx.blockwise_attention(q, k, v, self.D ** -0.5, self.block, causal, adj)

    def memory_usage_bytes(self) -> Dict[str, int]:
        """cache.py:430-440."""
        warm_rvq = int(self.warm_keys["rvq_codes"].shape[0] + self.warm_values["rvq_codes"].shape[0])
        return {"hot_bytes": self.num_hot * self.H * self.D * 2 * 2,
                "warm_pq_bytes": self.num_warm * self.H * self.M * 2,
                "warm_rvq_bytes": warm_rvq * self.L * 2,
                "cold_chunks": len(self.cold_meta), "cold_tokens": self.num_cold}
