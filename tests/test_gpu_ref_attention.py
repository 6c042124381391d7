"""Fused attention over reference-format stores (rfsn_ref_attention): PQ codes
with the gated full-dimension RVQ correction (quantization.py:178-319)
decoded in registers, never written to HBM, checked against the oracle's
decode (oracle.numerics.decode_compressed) followed by its blockwise
attention (attention.py:39-105) within 2e-3 -- over segment tables mixing
exact rows and coded stores, GQA groups up to 8, head_dim 64 / 128 / 256,
ragged segments, per-head causal positions (including -1: no key, zeros)
and split-K merges; then through the cache (attention_forward over the
reference suite's tiers, rfsn_v10_mlx_ane_complete.py:448-486) and
RFSNHybridAttentionMLX (attention.py:150-171) with the decode paths made to
raise, so nothing is materialized."""

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


def _random_store(g, n_tok, heads, M, C, L, Cr, p_active):
    """Reference-format store dict with random codes (the kernel's job is the
    decode and the attention, not the choice of codes)."""
    mask = g.random((n_tok, heads)) < p_active if L else np.zeros((n_tok, heads), bool)
    offs = np.flatnonzero(mask.reshape(-1)).astype(np.int32)
    return {"pq_codes": g.integers(0, C, (n_tok, heads, M), dtype=np.uint8),
            "rvq_codes": g.integers(0, max(Cr, 1), (offs.size, L), dtype=np.uint16),
            "rvq_mask": mask, "rvq_offsets": offs, "num_heads": heads}


def _dev_store(st, dev):
    from apple_amd.storage import CompressedTensorMLX

    return CompressedTensorMLX(pq_codes=T(st["pq_codes"], dev), rvq_codes=T(st["rvq_codes"], dev),
                               rvq_mask=T(st["rvq_mask"], dev), rvq_offsets=T(st["rvq_offsets"], dev),
                               num_heads=st["num_heads"])


CASES = [
    # D, M, C, L, Cr, B, Hq, Hkv, causal, splits
    (128, 8, 256, 3, 256, 1, 4, 4, True, 0),      # the reference suite's quantizer
    (64, 4, 256, 2, 512, 2, 8, 2, True, 1),
    (256, 32, 64, 3, 1024, 3, 8, 1, False, 0),
    (128, 16, 256, 0, 0, 2, 4, 2, True, 3),       # pq-only stores (no RVQ stage)
    (128, 8, 256, 3, 256, 2, 16, 2, True, 7),     # 8 query heads per KV head
    (256, 16, 128, 1, 65536, 1, 2, 2, True, 0),   # 16-bit RVQ codes
    (64, 32, 64, 2, 128, 1, 4, 4, True, 0),       # 2-wide PQ subspaces: 2 coordinates per lane, 2 token groups
]


@pytest.mark.parametrize("D,M,C,L,Cr,B,Hq,Hkv,causal,splits", CASES)
def test_segments_match_oracle(device, D, M, C, L, Cr, B, Hq, Hkv, causal, splits):
    from apple_amd import kernels as K

    g = rng(1000 + D + M + Hq + splits)
    d = D // M
    pq_cb = rand_codebooks(g, M, C, d)
    rv_cb = rand_codebooks(g, max(L, 1), max(Cr, 1), D)
    rv_cb[:, 0] = 0
    # window: a store slice (tokens 5..41 of 50), an exact ring segment
    # ([Hkv][cap][D] with its first token at ring slot 3), one token of a
    # second store, the whole second store
    s1 = _random_store(g, 50, Hkv, M, C, L, Cr, 0.6)
    s1v = _random_store(g, 50, Hkv, M, C, L, Cr, 0.3)
    s2 = _random_store(g, 71, Hkv, M, C, L, Cr, 0.5)
    s2v = _random_store(g, 71, Hkv, M, C, L, Cr, 0.9)
    cap = 40
    ring_k, ring_v = randn16(g, Hkv, cap, D), randn16(g, Hkv, cap, D)
    dec = lambda st: nx.decode_compressed(st, pq_cb, rv_cb)
    keys = np.concatenate([dec(s1)[5:42], ring_k[:, 3:32].transpose(1, 0, 2), dec(s2)[17:18], dec(s2)])
    vals = np.concatenate([dec(s1v)[5:42], ring_v[:, 3:32].transpose(1, 0, 2), dec(s2v)[17:18], dec(s2v)])
    W = keys.shape[0]
    q = randn16(g, B, Hq, D)
    qp = g.integers(-1, W, (B, Hq)).astype(np.int32)
    flat = qp.reshape(-1)
    flat[0], flat[-1] = W - 1, -1
    if flat.size > 2:
        flat[1] = 36  # the last token of the first segment
    ds1, ds1v, ds2, ds2v = (_dev_store(s, device) for s in (s1, s1v, s2, s2v))
    rk, rv = T(ring_k, device), T(ring_v, device)
    segs = [K.ref_store_segment(ds1, ds1v, 5, 37, 0),
            K.ref_exact_segment(rk, rv, rk.stride(1), rk.stride(0), 3, 29, 37),
            K.ref_store_segment(ds2, ds2v, 17, 1, 66),
            K.ref_store_segment(ds2, ds2v, 0, 71, 67)]
    cbs = dict(k_pq_cb=T(pq_cb, device), v_pq_cb=T(pq_cb, device),
               k_rvq_cb=T(rv_cb, device) if L else None, v_rvq_cb=T(rv_cb, device) if L else None)
    out = K.ref_attention(T(q, device), kv_heads=Hkv, scale=D ** -0.5, causal=causal,
                          qpos=T(qp, device) if causal else None, segments=segs, splits=splits, **cbs)
    got = H(out).astype(np.float32)
    ref = nx.blockwise_attention(q, keys, vals, D ** -0.5, 16, causal, qp if causal else None)
    assert np.abs(got - ref.astype(np.float32)).max() <= TOL
    if causal:
        assert not got[-1, -1].any()  # position -1 sees no key: zeros (attention.py:104-105)
    # the same window over head-major copies of the stores' codes (code
    # strides 1 and T): the same tokens in the same order, bit-identical
    hm = [K.ref_store_segment(ds1, ds1v, 5, 37, 0, head_major=True), segs[1],
          K.ref_store_segment(ds2, ds2v, 17, 1, 66, head_major=True),
          K.ref_store_segment(ds2, ds2v, 0, 71, 67, head_major=True)]
    assert hm[0]["rows"] == (1, 50) and hm[3]["rows"] == (1, 71)
    out_hm = K.ref_attention(T(q, device), kv_heads=Hkv, scale=D ** -0.5, causal=causal,
                             qpos=T(qp, device) if causal else None, segments=hm, splits=splits, **cbs)
    assert torch.equal(out_hm, out)


def _ext_store(g, n_tok, heads, M, C, Mr, Cr, k, D):
    """Long-context-format store dict: PQ, subspace RVQ, k distinct sparse
    coordinates per row with fp16 residuals."""
    idx = np.argsort(g.random((n_tok * heads, D)), axis=1)[:, :k].astype(np.uint8).reshape(n_tok, heads, k)
    return {"pq_codes": g.integers(0, C, (n_tok, heads, M), dtype=np.uint8),
            "rvq_codes": g.integers(0, max(Cr, 1), (n_tok, heads, Mr), dtype=np.uint8),
            "sparse_idx": idx, "sparse_val": randn16(g, n_tok, heads, k, scale=0.3)}


def _ext_decode(st, pq_cb, rv_cb):
    T_, H_, M = st["pq_codes"].shape
    n = T_ * H_
    Mr, k = st["rvq_codes"].shape[-1], st["sparse_idx"].shape[-1]
    out = nx.ext_decode(st["pq_codes"].reshape(n, M), pq_cb, st["rvq_codes"].reshape(n, Mr) if Mr else None,
                        rv_cb if Mr else None, st["sparse_idx"].reshape(n, k), st["sparse_val"].reshape(n, k))
    return out.reshape(T_, H_, -1)


def _ext_dev_store(st, dev):
    from apple_amd.storage import CompressedTensorMLX

    T_, H_ = st["pq_codes"].shape[:2]
    return CompressedTensorMLX(pq_codes=T(st["pq_codes"], dev), rvq_codes=T(st["rvq_codes"], dev),
                               rvq_mask=torch.ones((T_, H_), dtype=torch.bool, device=dev),
                               rvq_offsets=torch.zeros((0,), dtype=torch.int32, device=dev), num_heads=H_,
                               sparse_idx=T(st["sparse_idx"], dev), sparse_val=T(st["sparse_val"], dev))


EXT_CASES = [
    # D, M, C, Mr, Cr, k, B, Hq, Hkv
    (128, 16, 256, 16, 256, 4, 1, 32, 4),   # head_dim 128 long-context format
    (64, 8, 256, 4, 64, 3, 2, 8, 8),        # stage shapes the tiled kernel does not take
    (256, 32, 256, 32, 256, 8, 1, 8, 2),
    (128, 8, 128, 0, 0, 2, 2, 4, 4),        # PQ + sparse, no RVQ stage
    (64, 16, 256, 32, 64, 4, 1, 4, 2),      # 2-wide RVQ subspaces: a lane's 4 coordinates span two
    (64, 32, 64, 16, 128, 4, 1, 4, 4),      # 2-wide PQ subspaces: 2 coordinates per lane, 2 token groups
]


@pytest.mark.parametrize("D,M,C,Mr,Cr,k,B,Hq,Hkv", EXT_CASES)
def test_long_context_format_matches_oracle(device, D, M, C, Mr, Cr, k, B, Hq, Hkv):
    from apple_amd import kernels as K

    g = rng(2000 + D + M + Mr + k)
    pq_cb = rand_codebooks(g, M, C, D // M)
    rv_cb = rand_codebooks(g, max(Mr, 1), max(Cr, 1), D // max(Mr, 1))
    sk, sv = _ext_store(g, 90, Hkv, M, C, Mr, Cr, k, D), _ext_store(g, 90, Hkv, M, C, Mr, Cr, k, D)
    cap = 24
    ring_k, ring_v = randn16(g, Hkv, cap, D), randn16(g, Hkv, cap, D)
    keys = np.concatenate([_ext_decode(sk, pq_cb, rv_cb)[3:80], ring_k[:, :20].transpose(1, 0, 2)])
    vals = np.concatenate([_ext_decode(sv, pq_cb, rv_cb)[3:80], ring_v[:, :20].transpose(1, 0, 2)])
    W = keys.shape[0]
    q = randn16(g, B, Hq, D, scale=2.0)
    qp = g.integers(0, W, (B, Hq)).astype(np.int32)
    qp.reshape(-1)[0] = W - 1
    rk, rv = T(ring_k, device), T(ring_v, device)
    segs = [K.ref_store_segment(_ext_dev_store(sk, device), _ext_dev_store(sv, device), 3, 77, 0),
            K.ref_exact_segment(rk, rv, rk.stride(1), rk.stride(0), 0, 20, 77)]
    rcb = T(rv_cb, device) if Mr else None
    cb = T(pq_cb, device)  # one table for K and V: 256 x 256 x 2 B = 128 KB of LDS at head_dim 256
    out = K.ref_attention(T(q, device), kv_heads=Hkv, scale=D ** -0.5, causal=True, qpos=T(qp, device),
                          segments=segs, k_pq_cb=cb, v_pq_cb=cb, k_rvq_cb=rcb, v_rvq_cb=rcb, rvq_subspaces=Mr,
                          sparse_k=k)
    ref = nx.blockwise_attention(q, keys, vals, D ** -0.5, 16, True, qp)
    assert np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max() <= TOL
    # head-major copies of the long-context arrays (rvq_sub, sparse_idx, sparse_val)
    dsk, dsv = _ext_dev_store(sk, device), _ext_dev_store(sv, device)
    hm = [K.ref_store_segment(dsk, dsv, 3, 77, 0, head_major=True), segs[1]]
    out_hm = K.ref_attention(T(q, device), kv_heads=Hkv, scale=D ** -0.5, causal=True, qpos=T(qp, device),
                             segments=hm, k_pq_cb=cb, v_pq_cb=cb, k_rvq_cb=rcb, v_rvq_cb=rcb, rvq_subspaces=Mr,
                             sparse_k=k)
    assert torch.equal(out_hm, out)


def test_long_window_split_merge(device):
    """5000 coded tokens: the automatic split count (> 1) and the partial merge."""
    from apple_amd import kernels as K

    g = rng(77)
    D, M, C, L, Cr, Hkv, Hq = 128, 8, 256, 3, 256, 4, 8
    pq_cb, rv_cb = rand_codebooks(g, M, C, D // M), rand_codebooks(g, L, Cr, D)
    rv_cb[:, 0] = 0
    sk, sv = _random_store(g, 5000, Hkv, M, C, L, Cr, 0.5), _random_store(g, 5000, Hkv, M, C, L, Cr, 0.5)
    q = randn16(g, 1, Hq, D, scale=2.0)
    qp = np.array([[4999, 4000, 2500, 64, 63, 0, 1, 4998]], np.int32)
    lib = K.L.load()
    p = K.L.RefParams()
    p.head_dim, p.batch, p.q_heads, p.kv_heads, p.total_tokens = D, 1, Hq, Hkv, 5000
    assert lib.rfsn_ref_attention_workspace_bytes(K.C.byref(p)) > 0
    out = K.ref_attention(T(q, device), kv_heads=Hkv, scale=D ** -0.5, causal=True, qpos=T(qp, device),
                          segments=[K.ref_store_segment(_dev_store(sk, device), _dev_store(sv, device), 0, 5000, 0)],
                          k_pq_cb=T(pq_cb, device), v_pq_cb=T(pq_cb, device), k_rvq_cb=T(rv_cb, device),
                          v_rvq_cb=T(rv_cb, device))
    keys = nx.decode_compressed(sk, pq_cb, rv_cb)
    vals = nx.decode_compressed(sv, pq_cb, rv_cb)
    ref = nx.blockwise_attention(q, keys, vals, D ** -0.5, 16, True, qp)
    assert np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max() <= TOL


# ------------------------------------------------------------------ through the cache

def _ref_config(tmp_path, **kw):
    from apple_amd.storage import RFSNConfig

    base = dict(hidden_dim=512, num_heads=4, head_dim=128, num_layers=2, num_subspaces=8, subspace_dim=16,
                num_rvq_layers=3, rvq_codebook_size=256, rvq_sparsity_threshold=0.25, hot_capacity=16,
                warm_capacity=24, cold_capacity=128, block_size_seq=16, disk_cache_dir=str(tmp_path),
                prefetch_throttle_s=0.0)
    base.update(kw)
    return RFSNConfig(**base)


def _no_decode(monkeypatch):
    """Make every path that writes a decoded window raise."""
    import apple_amd.attention as A
    import apple_amd.cache as CA

    def boom(*a, **k):
        raise AssertionError("a decoded window was materialized")

    monkeypatch.setattr(CA, "_decode_compressed_tensor", boom)
    monkeypatch.setattr(A, "_decode_compressed_tensor", boom)
    monkeypatch.setattr(CA.RFSNv10KVCacheMLX, "materialize_window", boom)


def _build(dev, tmp_path, seed, n, **kw):
    from apple_amd.cache import RFSNv10KVCacheMLX
    from apple_amd.quantization import HybridQuantizerMLX

    cfg = _ref_config(tmp_path, **kw)
    g = rng(seed)
    pq, rv = rand_codebooks(g, 8, 256, 16), rand_codebooks(g, 3, 256, 128)
    rv[:, 0] = 0
    qz = HybridQuantizerMLX(cfg, device=dev, pq_codebooks=T(pq, dev), rvq_codebooks=T(rv, dev))
    k, v = randn16(g, n, 4, 128), randn16(g, n, 4, 128)
    c = RFSNv10KVCacheMLX(cfg, layer_idx=0, device=dev)
    c.update(T(k, dev), T(v, dev), qz, disk_dir=tmp_path)
    return cfg, c, cm.OracleQuantizer(pq, rv, cfg.rvq_sparsity_threshold), k, v, g


def test_reference_suite_cache_attends_without_materializing(device, tmp_path, monkeypatch):
    """rfsn_v10_mlx_ane_complete.py:448-486: 60 tokens over hot 16 / warm 24 /
    NPZ cold (20 tokens, 2 chunks), causal query at position 59."""
    cfg, c, oq, k, v, g = _build(device, tmp_path, 1, 60)
    o = cm.OracleCache(num_heads=4, head_dim=128, num_subspaces=8, num_rvq_layers=3, hot_capacity=16,
                       warm_capacity=24, block_size_seq=16)
    o.update(k, v, oq)
    assert (c.num_hot, c.num_warm, c.num_cold) == (16, 24, 20)
    assert int(c.warm_keys.rvq_codes.shape[0]) > 0 and not c._fused_ok(4) and c._ref_ok(4)
    q = randn16(g, 1, 4, 128)
    qp = np.array([59], np.int32)
    kw_, vw_, adj = c.materialize_window(query_positions=T(qp, device))
    with monkeypatch.context() as mp:
        _no_decode(mp)
        out = H(c.attention_forward(T(q, device), causal=True, query_positions=T(qp, device)))
        st = c.get_last_access_stats()
    ref = o.attention_forward(q, causal=True, query_positions=qp)
    assert np.abs(out.astype(np.float32) - ref.astype(np.float32)).max() <= TOL
    assert {k_: st[k_] for k_ in o.last_access_stats} == o.last_access_stats
    # and the materialized path (decode + blockwise) agrees on the same window
    mat = nx.blockwise_attention(q, H(kw_), H(vw_), 128 ** -0.5, 16, True, H(adj))
    assert np.abs(out.astype(np.float32) - mat.astype(np.float32)).max() <= TOL
    # a causal position inside the window, a context window, several queries
    q3 = randn16(g, 3, 4, 128)
    qp3 = np.array([[59, 10, 30, 45], [40, 41, 42, 43], [0, 15, 16, 39]], np.int32)
    for cw in (None, 24):
        with monkeypatch.context() as mp:
            _no_decode(mp)
            out3 = H(c.attention_forward(T(q3, device), causal=True, query_positions=T(qp3, device),
                                         context_window=cw))
        ref3 = o.attention_forward(q3, causal=True, query_positions=qp3, context_window=cw)
        assert np.abs(out3.astype(np.float32) - ref3.astype(np.float32)).max() <= TOL


def test_recency_pinned_cache(device, tmp_path, monkeypatch):
    """Recency tiers with pinned cold chunks: the fused window equals the
    materialized window's attention."""
    cfg, c, oq, k, v, g = _build(device, tmp_path, 5, 150, tier_policy="recency", cold_medium="pinned")
    assert c.num_cold > 0 and c.num_warm > 0 and c.num_hot > 0
    q = randn16(g, 2, 8, 128)
    qp = np.array([149, 100], np.int32)
    kw_, vw_, adj = c.materialize_window(query_positions=T(qp, device), context_window=120)
    with monkeypatch.context() as mp:
        _no_decode(mp)
        out = H(c.attention_forward(T(q, device), causal=True, query_positions=T(qp, device), context_window=120))
    mat = nx.blockwise_attention(q, H(kw_), H(vw_), 128 ** -0.5, 16, True, H(adj))
    assert np.abs(out.astype(np.float32) - mat.astype(np.float32)).max() <= TOL


def test_hybrid_attention_fused(device, tmp_path, monkeypatch):
    """rfsn_v10_mlx_ane_complete.py:406-446: RFSNHybridAttentionMLX over two
    compressed stores, now one fused launch, against the oracle's decode +
    blockwise attention."""
    from apple_amd.attention import RFSNHybridAttentionMLX
    from apple_amd.quantization import HybridQuantizerMLX, _compress_tensor_sequence

    cfg = _ref_config(tmp_path)
    g = rng(4)
    pq, rv = rand_codebooks(g, 8, 256, 16), rand_codebooks(g, 3, 256, 128)
    rv[:, 0] = 0
    qz = HybridQuantizerMLX(cfg, device=device, pq_codebooks=T(pq, device), rvq_codebooks=T(rv, device))
    q = randn16(g, 2, 4, 128)
    k, v = randn16(g, 24, 4, 128), randn16(g, 24, 4, 128)
    ks, vs = _compress_tensor_sequence(T(k, device), qz), _compress_tensor_sequence(T(v, device), qz)
    qp = np.array([12, 18], np.int32)
    with monkeypatch.context() as mp:
        _no_decode(mp)
        out = RFSNHybridAttentionMLX(cfg)(T(q, device), ks, vs, qz, causal=True, query_positions=T(qp, device))
    oq = cm.OracleQuantizer(pq, rv, 0.25)
    dk, dv = oq.decompress(oq.compress(k)), oq.decompress(oq.compress(v))
    ref = nx.blockwise_attention(q, dk, dv, 128 ** -0.5, 16, True, qp)
    assert np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max() <= TOL


def test_head_dim_128_long_context_cache(device, tmp_path, monkeypatch):
    """A head_dim-128 cache in the long-context format (PQ M16 + RVQ M16 +
    top-4, recency tiers, pinned cold chunks): the tiled kernel does not
    take it, and attention_forward attends it fused, within 2e-3 of the
    oracle's blockwise attention over the materialized window."""
    from apple_amd.cache import RFSNv10KVCacheMLX
    from apple_amd.quantization import HybridQuantizerMLX
    from apple_amd.storage import RFSNConfig

    cfg = RFSNConfig(hidden_dim=1024, num_heads=8, head_dim=128, num_subspaces=16, subspace_dim=8,
                     num_rvq_layers=1, rvq_codebook_size=256, rvq_sparsity_threshold=0.0, hot_capacity=64,
                     warm_capacity=96, cold_capacity=512, block_size_seq=32, num_kv_heads=2, rvq_subspaces=16,
                     sparse_topk=4, tier_policy="recency", cold_chunk_tokens=32, cold_medium="pinned",
                     disk_cache_dir=str(tmp_path))
    g = rng(31)
    qz = HybridQuantizerMLX(cfg, device=device, pq_codebooks=T(rand_codebooks(g, 16, 256, 8), device),
                            rvq_codebooks=T(rand_codebooks(g, 16, 256, 8), device))
    c = RFSNv10KVCacheMLX(cfg, layer_idx=0, device=device)
    k, v = randn16(g, 300, 2, 128), randn16(g, 300, 2, 128)
    c.update(T(k[:250], device), T(v[:250], device), qz)
    c.update(T(k[250:], device), T(v[250:], device), qz)
    assert c.num_cold > 0 and c.num_warm > 0 and c.num_hot > 0
    assert not c._fused_ok(8) and c._ref_ok(8)
    q = randn16(g, 2, 8, 128)
    qp = np.array([299, 180], np.int32)
    for cw in (None, 200):
        kw_, vw_, adj = c.materialize_window(query_positions=T(qp, device), context_window=cw)
        with monkeypatch.context() as mp:
            _no_decode(mp)
            out = H(c.attention_forward(T(q, device), causal=True, query_positions=T(qp, device), context_window=cw))
        mat = nx.blockwise_attention(q, H(kw_), H(vw_), 128 ** -0.5, 16, True, H(adj))
        assert np.abs(out.astype(np.float32) - mat.astype(np.float32)).max() <= TOL
    # the materialized window itself is the oracle's decode of the cache's codes
    ks = c.warm_keys
    n = ks.num_tokens * 2
    dec = nx.ext_decode(H(ks.pq_codes).reshape(n, 16), H(qz.pq.codebooks), H(ks.rvq_codes).reshape(n, 16),
                        H(qz.rvq.codebooks), H(ks.sparse_idx).reshape(n, 4), H(ks.sparse_val).reshape(n, 4))
    kw_, _, _ = c.materialize_window(query_positions=T(np.array([299, 299], np.int32), device))
    w0 = c.num_cold
    assert np.array_equal(H(kw_)[w0:w0 + ks.num_tokens].view(np.uint16), dec.reshape(-1, 2, 128).view(np.uint16))


def test_decode_session_head_dim_128(device, tmp_path):
    """A decode session over a head_dim-128 long-context cache: each step is
    update + the decode-in-register attention, equal to attention_forward at
    the newest position."""
    from apple_amd.cache import RFSNv10KVCacheMLX
    from apple_amd.quantization import HybridQuantizerMLX
    from apple_amd.storage import RFSNConfig

    cfg = RFSNConfig(hidden_dim=1024, num_heads=8, head_dim=128, num_subspaces=16, subspace_dim=8,
                     num_rvq_layers=1, rvq_codebook_size=256, rvq_sparsity_threshold=0.0, hot_capacity=64,
                     warm_capacity=96, cold_capacity=512, block_size_seq=32, num_kv_heads=2, rvq_subspaces=16,
                     sparse_topk=4, tier_policy="recency", cold_chunk_tokens=32, cold_medium="pinned",
                     disk_cache_dir=str(tmp_path))
    g = rng(41)
    qz = HybridQuantizerMLX(cfg, device=device, pq_codebooks=T(rand_codebooks(g, 16, 256, 8), device),
                            rvq_codebooks=T(rand_codebooks(g, 16, 256, 8), device))
    c = RFSNv10KVCacheMLX(cfg, layer_idx=0, device=device)
    k, v = randn16(g, 260, 2, 128), randn16(g, 260, 2, 128)
    c.update(T(k[:200], device), T(v[:200], device), qz)
    q = T(randn16(g, 1, 8, 128), device)
    sess = c.decode_session(q, qz)
    for t in range(200, 260):
        out = sess.step(T(k[t:t + 1], device), T(v[t:t + 1], device))
    ref = c.attention_forward(q, causal=True)
    assert sess.rebuilds == 60 and c.total_tokens == 260
    assert float((out.float() - ref.float()).abs().max()) == 0.0
    kw_, vw_, _ = c.materialize_window()
    mat = nx.blockwise_attention(H(q), H(kw_), H(vw_), 128 ** -0.5, 16, False, None)
    assert np.abs(H(out).astype(np.float32) - mat.astype(np.float32)).max() <= TOL
