"""Drop-in replay on the GPU: the reference's own test suite
(rfsn_v10_mlx_ane_complete.py:374-554) run against the MI355X cache in the
reference format (PQ + gated 3-stage full-D RVQ, NPZ cold chunks), checked
against the oracle cache model on the same inputs: tier counts, chunk ids,
access counters and byte accounting exactly, materialized windows
bit-exact, attention within 2e-3 (the reference suite asks 1e-4 between its
own two paths, which the same comparison here meets as well)."""

import numpy as np
import pytest
import torch

from oracle import cache_model as cm
from oracle import numerics as nx
from tests.conftest import rand_codebooks, randn16, rng

pytestmark = pytest.mark.gpu

TOL = 2e-3


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def H(t):
    return t.detach().cpu().numpy()


def _ref_config(tmp_path, **kw):
    from apple_amd.storage import RFSNConfig

    base = dict(hidden_dim=512, num_heads=4, head_dim=128, num_layers=2, num_subspaces=8, subspace_dim=16,
                num_rvq_layers=3, rvq_codebook_size=256, rvq_sparsity_threshold=0.25, hot_capacity=16,
                warm_capacity=24, cold_capacity=128, block_size_seq=16, disk_cache_dir=str(tmp_path),
                prefetch_throttle_s=0.0)
    base.update(kw)
    return RFSNConfig(**base)


def _quantizers(cfg, dev, seed, threshold=0.25):
    from apple_amd.quantization import HybridQuantizerMLX

    g = rng(seed)
    pq = rand_codebooks(g, 8, 256, 16)
    rv = rand_codebooks(g, 3, 256, 128)
    rv[:, 0] = 0
    q = HybridQuantizerMLX(cfg, device=dev, pq_codebooks=T(pq, dev), rvq_codebooks=T(rv, dev))
    return q, cm.OracleQuantizer(pq, rv, threshold)


def _pair(dev, tmp_path, seed, n, **kw):
    from apple_amd.cache import RFSNv10KVCacheMLX

    cfg = _ref_config(tmp_path, **kw)
    q, oq = _quantizers(cfg, dev, seed, cfg.rvq_sparsity_threshold)
    g = rng(seed + 1)
    k, v = randn16(g, n, 4, 128), randn16(g, n, 4, 128)
    c = RFSNv10KVCacheMLX(cfg, layer_idx=0, device=dev)
    c.update(T(k, dev), T(v, dev), q, disk_dir=tmp_path)
    o = cm.OracleCache(num_heads=4, head_dim=128, num_subspaces=8, num_rvq_layers=3, hot_capacity=cfg.hot_capacity,
                       warm_capacity=cfg.warm_capacity, block_size_seq=cfg.block_size_seq)
    o.update(k, v, oq)
    return cfg, c, o, g


def _same16(a, b):
    return np.array_equal(np.asarray(a).view(np.uint16), np.asarray(b).view(np.uint16))


def test_kv_cache_tiers_and_attention(device, tmp_path):
    """rfsn_v10_mlx_ane_complete.py:448-486."""
    cfg, c, o, g = _pair(device, tmp_path, 1, 60)
    assert (c.num_hot, c.num_warm, c.num_cold) == (16, 24, 20)
    assert len(c.cold_chunk_paths) == 2
    assert [m["chunk_id"] for m in c.cold_chunk_metadata] == [m["chunk_id"] for m in o.cold_meta]
    q = randn16(g, 1, 4, 128)
    qp = np.array([59], np.int32)
    out = H(c.attention_forward(T(q, device), causal=True, query_positions=T(qp, device)))
    st = c.get_last_access_stats()
    ref = o.attention_forward(q, causal=True, query_positions=qp)
    assert np.abs(out.astype(np.float32) - ref.astype(np.float32)).max() <= TOL
    assert {k: st[k] for k in o.last_access_stats} == o.last_access_stats
    kw, vw, adj = c.materialize_window(query_positions=T(qp, device))
    okw, ovw, oadj = o.materialize_window(query_positions=qp)
    assert _same16(H(kw), okw) and _same16(H(vw), ovw) and int(H(adj)[0]) == int(oadj[0])
    mem = c.memory_usage_bytes()
    assert mem == o.memory_usage_bytes() and mem["cold_chunks"] == 2


def test_warm_window_materialization(device, tmp_path):
    """rfsn_v10_mlx_ane_complete.py:488-521."""
    cfg, c, o, g = _pair(device, tmp_path, 2, 36)
    qp = np.array([35], np.int32)
    fk, fv, _ = c.materialize_window(query_positions=T(qp, device))
    wk, wv, adj = c.materialize_window(query_positions=T(qp, device), context_window=8)
    st = c.get_last_access_stats()
    assert tuple(wk.shape) == (8, 4, 128) and int(H(adj)[0]) == 7
    assert _same16(H(wk), H(fk)[-8:]) and _same16(H(wv), H(fv)[-8:])
    okw, _, _ = o.materialize_window(query_positions=qp, context_window=8)
    assert _same16(H(wk), okw)
    assert {k: st[k] for k in o.last_access_stats} == o.last_access_stats
    assert st["warm_chunk_decodes"] == 1 and st["reconstructed_tokens"] == 8


def test_async_router(device, tmp_path):
    """rfsn_v10_mlx_ane_complete.py:532-554 (NPZ cold chunks on disk)."""
    from apple_amd.storage import AsyncHierarchicalRouterMLX

    cfg, c, o, g = _pair(device, tmp_path, 3, 48)
    router = AsyncHierarchicalRouterMLX(cfg, layer_idx=0)
    ids = router.prefetch_sync(current_position=0, context_window=1024, top_k=1)
    assert ids == cm.OracleRouter(o, 16).prefetch(0, 1024, 1) and router.get_chunk(ids[0]) is not None
    q = randn16(g, 1, 4, 128)
    qp = np.array([47], np.int32)
    out = H(c.attention_forward(T(q, device), causal=True, query_positions=T(qp, device), router=router,
                                current_position=47, context_window=16))
    assert c.get_last_access_stats()["cold_chunk_cache_hits"] >= 1
    oref = o.attention_forward(q, causal=True, query_positions=qp, router=cm.OracleRouter(o, 16),
                               current_position=47, context_window=16)
    assert np.abs(out.astype(np.float32) - oref.astype(np.float32)).max() <= TOL


def test_hybrid_attention_matches_reference(device, tmp_path):
    """rfsn_v10_mlx_ane_complete.py:406-446: RFSNHybridAttentionMLX over two
    compressed stores equals blockwise attention over their decode."""
    from apple_amd.attention import RFSNHybridAttentionMLX, _blockwise_exact_attention
    from apple_amd.quantization import _compress_tensor_sequence, _decode_compressed_tensor

    cfg = _ref_config(tmp_path)
    q_, oq = _quantizers(cfg, device, 4)
    g = rng(5)
    q = randn16(g, 2, 4, 128)
    k, v = randn16(g, 24, 4, 128), randn16(g, 24, 4, 128)
    ks, vs = _compress_tensor_sequence(T(k, device), q_), _compress_tensor_sequence(T(v, device), q_)
    dk, dv = _decode_compressed_tensor(ks, q_), _decode_compressed_tensor(vs, q_)
    assert _same16(H(dk), oq.decompress(oq.compress(k)))
    qp = T(np.array([12, 18], np.int32), device)
    out = RFSNHybridAttentionMLX(cfg)(T(q, device), ks, vs, q_, causal=True, query_positions=qp)
    ref = _blockwise_exact_attention(T(q, device), dk, dv, 128 ** -0.5, 16, causal=True, query_positions=qp)
    assert float((out.float() - ref.float()).abs().max()) < 1e-4
    oref = nx.blockwise_attention(q, H(dk), H(dv), 128 ** -0.5, 16, True, np.array([12, 18]))
    assert np.abs(H(out).astype(np.float32) - oref.astype(np.float32)).max() <= TOL


@pytest.mark.parametrize("T_,mode,cache_bytes", [(64, "pq_only", 67584), (64, "pq_rvq", 69120),
                                                  (192, "pq_only", 75776), (192, "pq_rvq", 83456)])
def test_csv_byte_known_answers(device, tmp_path, T_, mode, cache_bytes):
    """benchmark_outputs/dense_vs_hot_warm.csv: cache_bytes of the hot_warm
    profile (rfsn_v10_eval_benchmark.py:43-45, 398-414)."""
    thr = float("inf") if mode == "pq_only" else 0.25
    cfg, c, o, g = _pair(device, tmp_path, 6, T_, hot_capacity=32, warm_capacity=max(1, T_ - 32),
                         cold_capacity=T_, rvq_sparsity_threshold=thr)
    mem = c.memory_usage_bytes()
    assert mem["hot_bytes"] + mem["warm_pq_bytes"] + mem["warm_rvq_bytes"] == cache_bytes
    assert mem == o.memory_usage_bytes()


def test_warm_append_pair_matches_per_store_appends(device):
    """rfsn_warm_append_pair (one launch for a K/V block) writes the same
    bytes as the per-store appends (sparse fold and delta, score-row and
    tiled packing): every array of both stores, K's corrected-coordinate
    plane included, bit for bit, for a block that starts inside a tile, with
    K as score-table rows and as tiled rows."""
    from types import SimpleNamespace

    from apple_amd import kernels as K

    fmt = K.WarmFormat(64, 16, 256, 16, 256, 4)
    g = rng(77)
    Hh = 4
    qz = [SimpleNamespace(pq=SimpleNamespace(codebooks=T(rand_codebooks(g, 16, 256, 4), device)),
                          rvq_codebooks=T(rand_codebooks(g, 16, 256, 4) * np.float16(0.35), device)) for _ in range(2)]

    def block(n):
        out = []
        for _ in range(2):
            pq = T(g.integers(0, 256, (Hh, n, 16), dtype=np.uint8), device)
            rvq = T(g.integers(0, 256, (Hh, n, 16), dtype=np.uint8), device)
            si = T(np.stack([np.stack([g.choice(64, 4, replace=False) for _ in range(n)]) for _ in range(Hh)])
                   .astype(np.uint8), device)
            sv = T(randn16(g, Hh, n, 4, scale=0.2), device)
            out.append((pq, rvq, si, sv))
        return out

    for score in (True, False):
        _pair_case(device, fmt, Hh, qz, block, score)


def _pair_case(device, fmt, Hh, qz, block, score):
    from apple_amd.cache import TiledCodes

    stores = []
    for _ in range(2):
        stores.append((TiledCodes(fmt, Hh, device, cap=128, score_rows=score, exact_plane=score),
                       TiledCodes(fmt, Hh, device, cap=128)))
    first, second = block(40), block(29)
    for kt, vt in stores:
        for t, c, q in ((kt, first[0], qz[0]), (vt, first[1], qz[1])):
            t.append(*c, q.pq.codebooks, q.rvq_codebooks)
    a, b = stores
    for t, c, q in ((a[0], second[0], qz[0]), (a[1], second[1], qz[1])):
        t.append(*c, q.pq.codebooks, q.rvq_codebooks)
    assert TiledCodes.append_pair(b[0], b[1], second[0], second[1], qz[0], qz[1])
    assert (a[0].len, a[1].len) == (b[0].len, b[1].len) == (69, 69)
    for x, y in zip(a, b):
        assert set(x.t) == set(y.t)
        for key in x.t:
            if x.t[key] is not None:
                assert torch.equal(x.t[key].view(torch.uint8), y.t[key].view(torch.uint8)), key
    # a block past the capacity is refused (the per-store append grows the stores)
    assert not TiledCodes.append_pair(b[0], b[1], *block(60)[:2], qz[0], qz[1])
