"""The reference's error contracts and the host-forceable failure cases, on
the MI355X product path (the oracle's counterparts are in test_oracle.py):

* use before ``update`` -> RuntimeError (cache.py:351-352, 407-408);
* mismatched K/V shapes -> ValueError (cache.py:96-97), and K/V stores of
  different token counts -> ValueError (attention.py:159-160);
* a cold append that is not contiguous with its chunk's metadata ->
  ValueError (cache.py:159-163), for NPZ files and for the pinned medium;
* a chunk dropped from the pinned device pool -> a router miss
  (cache.py:323-326) and a synchronous copy, with the output unchanged;
* an error status from the C ABI -> RuntimeError (ValueError for a contract
  violation), raised by the product call that received it.
"""

import numpy as np
import pytest
import torch

from oracle import numerics as nx
from tests.conftest import rand_codebooks, randn16, rng
from tests.test_gpu_fused import TOL, _cold_cache, H, T

pytestmark = pytest.mark.gpu


def _ref_cfg(tmp_path, **kw):
    from apple_amd.storage import RFSNConfig

    base = dict(hidden_dim=256, num_heads=2, head_dim=64, num_layers=1, num_subspaces=8, subspace_dim=8,
                num_rvq_layers=2, rvq_codebook_size=256, rvq_sparsity_threshold=0.25, hot_capacity=8,
                warm_capacity=8, block_size_seq=8, disk_cache_dir=str(tmp_path), prefetch_throttle_s=0.0)
    base.update(kw)
    return RFSNConfig(**base)


def _ref_quantizer(cfg, device, seed=3):
    from apple_amd.quantization import HybridQuantizerMLX

    g = rng(seed)
    rv = rand_codebooks(g, 2, 256, 64)
    rv[:, 0] = 0
    return HybridQuantizerMLX(cfg, device=device, pq_codebooks=T(rand_codebooks(g, 8, 256, 8), device),
                              rvq_codebooks=T(rv, device))


def test_use_before_update_raises(device, tmp_path):
    from apple_amd.cache import RFSNv10KVCacheMLX

    c = RFSNv10KVCacheMLX(_ref_cfg(tmp_path), device=device)
    with pytest.raises(RuntimeError, match="before update"):
        c.materialize_window()
    with pytest.raises(RuntimeError, match="before update"):
        c.attention_forward(torch.zeros((1, 2, 64), dtype=torch.float16, device=device))


def test_mismatched_kv_raises(device, tmp_path):
    from apple_amd.attention import RFSNHybridAttentionMLX
    from apple_amd.cache import RFSNv10KVCacheMLX
    from apple_amd.quantization import _compress_tensor_sequence

    cfg = _ref_cfg(tmp_path)
    qz = _ref_quantizer(cfg, device)
    g = rng(4)
    c = RFSNv10KVCacheMLX(cfg, device=device)
    with pytest.raises(ValueError, match="identical shapes"):
        c.update(T(randn16(g, 5, 2, 64), device), T(randn16(g, 6, 2, 64), device), qz)
    assert c.total_tokens == 0 and c.quantizer is None  # nothing was taken in
    ks = _compress_tensor_sequence(T(randn16(g, 5, 2, 64), device), qz)
    vs = _compress_tensor_sequence(T(randn16(g, 6, 2, 64), device), qz)
    with pytest.raises(ValueError, match="same token count"):
        RFSNHybridAttentionMLX(cfg)(T(randn16(g, 1, 2, 64), device), ks, vs, qz)


def test_non_contiguous_cold_append_raises_npz(device, tmp_path):
    """The reference's guard on merge-on-append: a chunk whose metadata ends
    elsewhere than where the new tokens start is refused."""
    from apple_amd.cache import RFSNv10KVCacheMLX

    cfg = _ref_cfg(tmp_path)
    qz = _ref_quantizer(cfg, device)
    g = rng(5)
    c = RFSNv10KVCacheMLX(cfg, device=device)
    c.update(T(randn16(g, 20, 2, 64), device), T(randn16(g, 20, 2, 64), device), qz, disk_dir=tmp_path)
    meta = c.cold_chunk_metadata[-1]
    assert (meta["chunk_id"], meta["start_token"], meta["end_token"]) == (2, 16, 20)  # a partial chunk
    meta["end_token"] -= 1
    with pytest.raises(ValueError, match="contiguous"):
        c.update(T(randn16(g, 2, 2, 64), device), T(randn16(g, 2, 2, 64), device), qz, disk_dir=tmp_path)


def test_non_contiguous_cold_append_raises_pinned(device):
    from apple_amd.cache import RFSNv10KVCacheMLX
    from apple_amd.quantization import HybridQuantizerMLX
    from apple_amd.storage import RFSNConfig

    D, M = 64, 16
    cfg = RFSNConfig(num_heads=8, head_dim=D, num_subspaces=M, subspace_dim=D // M, num_rvq_layers=1,
                     rvq_codebook_size=256, hot_capacity=32, warm_capacity=64, block_size_seq=32, num_kv_heads=2,
                     rvq_subspaces=M, sparse_topk=4, cold_medium="pinned", cold_chunk_tokens=32)
    g = rng(6)
    qz = HybridQuantizerMLX(cfg, pq_codebooks=torch.from_numpy(rand_codebooks(g, M, 256, 4)),
                            rvq_codebooks=torch.from_numpy(rand_codebooks(g, M, 256, 4)))
    c = RFSNv10KVCacheMLX(cfg, device=device)
    c.update(T(randn16(g, 130, 2, D), device), T(randn16(g, 130, 2, D), device), qz)
    meta = c.cold_chunk_metadata[-1]
    assert (meta["chunk_id"], meta["start_token"], meta["end_token"]) == (4, 128, 130)  # a partial chunk
    meta["end_token"] += 3
    with pytest.raises(ValueError, match="contiguous"):
        c.update(T(randn16(g, 4, 2, D), device), T(randn16(g, 4, 2, D), device), qz)


def test_pinned_chunk_dropped_counts_a_miss(device):
    """A bound router's chunk evicted from the device pool: the next call
    counts it as a router miss, copies it in during the step and attends the
    same window as before."""
    from apple_amd.storage import AsyncHierarchicalRouterMLX

    total, nh, nw, chunk = 1664, 64, 600, 100
    ncold = total - nh - nw
    g, cfg, cache, keys, values, dec = _cold_cache(device, 91, total, nh, nw, chunk)
    router = AsyncHierarchicalRouterMLX(cfg).bind(cache)
    cw = 914  # window [750, 1664): chunks 7 (partly), 8 and 9
    q = randn16(g, 1, 32, 64)
    qd = T(q, device)
    pos = np.arange(total - cw, total)
    hot = (pos >= total - nh)[:, None, None]
    wk = np.where(hot, keys[pos], dec[0][pos])
    wv = np.where(hot, values[pos], dec[1][pos])
    ref = nx.blockwise_attention(q, wk, wv, 0.125, 256)
    cache.evict_cold_slots()
    kw = dict(causal=False, router=router, current_position=total - 1, context_window=cw)
    first = cache.attention_forward(qd, **kw)
    st = cache.get_last_access_stats()
    assert (st["cold_chunk_cache_hits"], st["cold_chunk_cache_misses"], st["cold_chunks_touched"]) == (3, 0, 3)
    assert np.abs(H(first).astype(np.float32) - ref.astype(np.float32)).max() <= TOL
    assert cache.resident_cold_chunk(8) is not None
    cache.evict_cold_slots([8])
    second = cache.attention_forward(qd, **kw)
    st = cache.get_last_access_stats()
    assert (st["cold_chunk_cache_hits"], st["cold_chunk_cache_misses"], st["cold_chunks_touched"]) == (2, 1, 3)
    assert np.abs(H(second).astype(np.float32) - ref.astype(np.float32)).max() <= TOL
    assert cache.resident_cold_chunk(8) is not None  # copied back in by the fallback


class _FailingLib:
    """The bound library with one entry point answering a fixed status."""

    def __init__(self, real, name, status):
        self._real, self._name, self._status = real, name, status

    def __getattr__(self, attr):
        if attr == self._name:
            return lambda *a: self._status
        return getattr(self._real, attr)


@pytest.mark.parametrize("status,exc", [(-3, RuntimeError), (-2, RuntimeError), (-4, RuntimeError),
                                        (-1, ValueError)])
def test_abi_error_status_reaches_the_caller(device, monkeypatch, status, exc):
    from apple_amd import _lib
    from apple_amd.quantization import ProductQuantizerMLX
    from apple_amd.storage import RFSNConfig

    cfg = RFSNConfig(num_heads=2, head_dim=64, num_subspaces=8, subspace_dim=8)
    pq = ProductQuantizerMLX(cfg, device=device, codebooks=T(rand_codebooks(rng(7), 8, 256, 8), device))
    x = T(randn16(rng(8), 16, 64), device)
    codes, _ = pq.quantize(x)  # the real library first
    assert np.array_equal(H(codes), nx.pq_encode(H(x), H(pq.codebooks))[0])
    monkeypatch.setattr(_lib, "_lib", _FailingLib(_lib.load(), "rfsn_pq_encode", status))
    with pytest.raises(exc, match="rfsn_pq_encode"):
        pq.quantize(x)
