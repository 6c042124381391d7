"""Score tables of rfsn_ref_attention (score_tables = 1): the coded segments
of a reference-format window attended through q . codeword tables and
per-codeword sums of the softmax weights, under the drift guard that sends a
(query, KV head) group back to the exact decode (quantization.py:310-319,
attention.py:39-105 through rfsn_ref_attention's exact pass).

Checked: against the oracle's decode + blockwise attention over windows
mixing coded stores and exact rows, every supported PQ width, 0 to 8 gated
layers, ragged codebook sizes, GQA groups up to 8, head_dim 64 / 128 / 256
and per-head causal positions; bit-identity with the exact path when the
guard sends every group back (tolerance 0); the guard's estimate against a
numpy restatement of its formula; its codebook statistics against numpy;
the envelope over query scales 1 to 8 at the reference's default format; the
cache and the attention module taking the tables for decode steps."""

import numpy as np
import pytest
import torch

from oracle import numerics as nx
from tests.conftest import rand_codebooks, randn16, rng

pytestmark = pytest.mark.gpu

TOL = 2e-3


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def H(t):
    return t.detach().cpu().numpy()


def _store(g, n_tok, heads, M, C, L, Cr, p_active):
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


def _excess(out: np.ndarray, ref: np.ndarray) -> tuple:
    """(max |out - ref|, max of |out - ref| - max(TOL, ulp(ref))): fp16
    outputs at |x| >= 4 are a rounding step of 3.9e-3 apart."""
    o, r = out.astype(np.float32), ref.astype(np.float32)
    d = np.abs(o - r)
    ulp = np.spacing(np.abs(ref.astype(np.float16))).astype(np.float32)
    return float(d.max()), float((d - np.maximum(TOL, ulp)).max())


def _window(g, dev, D, M, C, L, Cr, Hkv, n1, n2, hot):
    """Coded store slice (tokens 3 .. n1 + 3), an exact ring segment of
    ``hot`` tokens, a second whole store: segments, oracle K/V, codebooks."""
    from apple_amd import kernels as K

    d = D // M
    pq_cb = rand_codebooks(g, M, C, d)
    rv_cb = rand_codebooks(g, max(L, 1), max(Cr, 1), D)
    rv_cb[:, 0] = 0
    s1, s1v = _store(g, n1 + 7, Hkv, M, C, L, Cr, 0.7), _store(g, n1 + 7, Hkv, M, C, L, Cr, 0.4)
    s2, s2v = _store(g, n2, Hkv, M, C, L, Cr, 0.5), _store(g, n2, Hkv, M, C, L, Cr, 0.9)
    ring_k, ring_v = randn16(g, Hkv, hot + 5, D), randn16(g, Hkv, hot + 5, D)
    dec = lambda st: nx.decode_compressed(st, pq_cb, rv_cb)
    keys = np.concatenate([dec(s1)[3:3 + n1], ring_k[:, 2:2 + hot].transpose(1, 0, 2), dec(s2)])
    vals = np.concatenate([dec(s1v)[3:3 + n1], ring_v[:, 2:2 + hot].transpose(1, 0, 2), dec(s2v)])
    ds1, ds1v, ds2, ds2v = (_dev_store(s, dev) for s in (s1, s1v, s2, s2v))
    rk, rv = T(ring_k, dev), T(ring_v, dev)
    segs = [K.ref_store_segment(ds1, ds1v, 3, n1, 0),
            K.ref_exact_segment(rk, rv, rk.stride(1), rk.stride(0), 2, hot, n1),
            K.ref_store_segment(ds2, ds2v, 0, n2, n1 + hot)]
    cbs = dict(k_pq_cb=T(pq_cb, dev), v_pq_cb=T(pq_cb, dev),
               k_rvq_cb=T(rv_cb, dev) if L else None, v_rvq_cb=T(rv_cb, dev) if L else None)
    keep = (ds1, ds1v, ds2, ds2v, rk, rv)
    return segs, keys, vals, cbs, keep, (pq_cb, rv_cb if L else None)


CASES = [
    # D, M, C, L, Cr, B, Hq, Hkv, causal
    (128, 8, 256, 4, 4096, 1, 8, 8, False),     # the reference's default format
    (128, 8, 256, 3, 256, 2, 8, 2, True),
    (64, 4, 256, 2, 512, 1, 8, 2, True),
    (256, 32, 64, 3, 1024, 1, 8, 1, False),     # 8 query heads per KV head
    (128, 16, 256, 0, 0, 2, 4, 2, True),        # PQ only
    (256, 16, 128, 1, 16384, 1, 2, 2, True),    # 16-bit codes, E = 18,432
    (64, 32, 64, 2, 128, 1, 4, 4, True),        # 2-wide PQ subspaces
    (128, 8, 100, 5, 300, 1, 4, 4, False),      # ragged sections, 5 layers
]


@pytest.mark.parametrize("D,M,C,L,Cr,B,Hq,Hkv,causal", CASES)
def test_tables_match_oracle(device, monkeypatch, D, M, C, L, Cr, B, Hq, Hkv, causal):
    from apple_amd import kernels as K

    monkeypatch.setattr(K, "REF_TABLES_MIN_TOKENS", 0)
    g = rng(3000 + D + M + L + Hq)
    segs, keys, vals, cbs, keep, _ = _window(g, device, D, M, C, L, Cr, Hkv, 700, 1300, 96)
    W = keys.shape[0]
    q = randn16(g, B, Hq, D)
    qp = g.integers(-1, W, (B, Hq)).astype(np.int32)
    flat = qp.reshape(-1)
    flat[0], flat[-1] = W - 1, -1
    if flat.size > 2:
        flat[1] = 699  # the last token of the first coded segment
    if flat.size > 3:
        flat[2] = 750  # inside the exact segment: the second store is masked
    info, drift = {}, torch.empty((B, Hq), dtype=torch.float32, device=device)
    out = K.ref_attention(T(q, device), kv_heads=Hkv, scale=D ** -0.5, causal=causal,
                          qpos=T(qp, device) if causal else None, segments=segs, score_tables=TOL, drift=drift,
                          info=info, **cbs)
    assert info["score_tables"]
    got = H(out)
    ref = nx.blockwise_attention(q, keys, vals, D ** -0.5, 16, causal, qp if causal else None)
    err, excess = _excess(got, ref)
    assert excess <= 0, (err, float(H(drift).max()))
    dr = H(drift)
    assert np.isfinite(dr).all() and (dr >= 0).all()
    if causal:
        assert not got[-1, -1].any()  # position -1 sees no key: zeros (attention.py:104-105)


def test_group_moves_the_break_even(device):
    """The same window of 6,000 coded tokens over 2 KV heads: one query of 2
    heads (one per KV head, at least 4,096 coded tokens) goes through the
    score tables, one of 8 heads (groups of 4, below 8,192) through the exact
    decode, and 4 queries of 8 heads (at least 5,120) through the tables
    again; all agree with the oracle."""
    from apple_amd import kernels as K

    assert K.ref_tables_min_tokens(1) == K.REF_TABLES_MIN_TOKENS <= 6000 < K.ref_tables_min_tokens(4)
    assert K.ref_tables_min_tokens(4, 4) <= 6000
    g = rng(3050)
    D = 128
    segs, keys, vals, cbs, keep, _ = _window(g, device, D, 8, 256, 4, 4096, 2, 3000, 3000, 64)
    for B, Hq, tables in ((1, 2, True), (1, 8, False), (4, 8, True)):
        q = randn16(g, B, Hq, D)
        info = {}
        out = K.ref_attention(T(q, device), kv_heads=2, scale=D ** -0.5, causal=False, qpos=None,
                              segments=segs, score_tables=TOL, info=info, **cbs)
        assert info["score_tables"] == tables, (B, Hq)
        ref = nx.blockwise_attention(q, keys, vals, D ** -0.5, 16, False, None)
        assert _excess(H(out), ref)[1] <= 0, (B, Hq)


@pytest.mark.parametrize("splits", [0, 1, 3])
def test_tolerance_zero_is_the_exact_path(device, monkeypatch, splits):
    """With tolerance 0 every group's estimate exceeds it, the exact pass
    decodes every coded token and the tables' slot is empty: bit-identical to
    the exact path with the same splits."""
    from apple_amd import kernels as K

    monkeypatch.setattr(K, "REF_TABLES_MIN_TOKENS", 0)
    g = rng(3100 + splits)
    D, M, C, L, Cr, B, Hq, Hkv = 128, 8, 256, 4, 4096, 2, 8, 4
    segs, keys, vals, cbs, keep, _ = _window(g, device, D, M, C, L, Cr, Hkv, 500, 900, 64)
    q = T(randn16(g, B, Hq, D), device)
    info = {}
    tab = K.ref_attention(q, kv_heads=Hkv, scale=D ** -0.5, causal=False, qpos=None, segments=segs,
                          splits=splits, score_tables=0.0, info=info, **cbs)
    assert info["score_tables"]
    exact = K.ref_attention(q, kv_heads=Hkv, scale=D ** -0.5, causal=False, qpos=None, segments=segs,
                            splits=splits, **cbs)
    assert torch.equal(tab, exact)


HM_CASES = CASES[:2] + [CASES[7], (128, 8, 256, 4, 1024, 1, 32, 8, True)]  # + 8 KV units of 4 query heads


@pytest.mark.parametrize("case", range(len(HM_CASES)))
@pytest.mark.parametrize("tables", [False, True])
def test_head_major_codes_match(device, monkeypatch, case, tables):
    """The window over head-major copies of its stores' codes (code strides 1
    and T; the stores keep 40-90 % of their rows active, so the gated codes go
    through active maps) attends bit-identically to the stores' own order, on
    the exact path and with score tables, for 4, 3 and 5 gated layers (3 and
    5: the tables' per-token loads) and for 8 (query, KV head) units of 4
    query heads (the histogram blocks grouped per unit on an XCD)."""
    from apple_amd import kernels as K

    monkeypatch.setattr(K, "REF_TABLES_MIN_TOKENS", 0)
    D, M, C, L, Cr, B, Hq, Hkv, causal = HM_CASES[case]
    g = rng(3600 + 2 * case + int(tables))
    n1, n2, hot = 900, 1500, 64
    segs, keys, vals, cbs, keep, _ = _window(g, device, D, M, C, L, Cr, Hkv, n1, n2, hot)
    ds1, ds1v, ds2, ds2v = keep[:4]
    hm = [K.ref_store_segment(ds1, ds1v, 3, n1, 0, head_major=True), segs[1],
          K.ref_store_segment(ds2, ds2v, 0, n2, n1 + hot, head_major=True)]
    q = T(randn16(g, B, Hq, D), device)
    W = n1 + hot + n2
    qp = T(g.integers(W // 2, W, (B, Hq)).astype(np.int32), device) if causal else None
    kw = dict(kv_heads=Hkv, scale=D ** -0.5, causal=causal, qpos=qp, score_tables=TOL if tables else None, **cbs)
    info = {}
    a = K.ref_attention(q, segments=segs, info=info, **kw)
    assert info["score_tables"] == tables
    b = K.ref_attention(q, segments=hm, **kw)
    assert torch.equal(a, b)


def _estimate(q, s, stats, scale, blocks):
    """The guard's estimate restated for one query head over its coded
    tokens' scores s (base 2): p = 2^(s - max), L = sum p, Q = sum p^2, and
    per histogram block b (its own maximum m_b) QE_b = sum (p~ - p)^2 with p~
    = p rounded to 2^-19, weighted by 2^(2 (m_b - max))."""
    s = s.astype(np.float64)
    M = s.max()
    p = np.exp2(s - M)
    Lsum, Q = p.sum(), (p * p).sum()
    QE = 0.0
    for sb in blocks:
        mb = float(sb.max())
        pb = np.exp2(sb.astype(np.float32) - np.float32(mb)).astype(np.float64)
        qb = np.rint(pb * 2.0 ** 19) / 2.0 ** 19
        QE += np.exp2(2 * (mb - M)) * ((qb - pb) ** 2).sum()
    var = 1.0 / (12.0 * 1048576.0)
    q64 = q.astype(np.float64)
    s2 = (q64 * q64 * stats[0]).sum()
    sq = np.sqrt(Q) / Lsum
    vm = stats[2].max()
    return scale * np.sqrt(var * s2) * sq * 2 * vm + sq * np.sqrt(var * stats[1].max()) + np.sqrt(QE) / Lsum * vm


def test_guard_estimate_matches_restatement(device, monkeypatch):
    """The drift written per query head equals the formula over the coded
    tokens' table scores (numpy, float64), within 3% (the fixed-point term and
    fp32 sums); the statistics equal numpy's."""
    from apple_amd import kernels as K

    monkeypatch.setattr(K, "REF_TABLES_MIN_TOKENS", 0)
    g = rng(3200)
    D, M, C, L, Cr, B, Hq, Hkv = 128, 8, 256, 4, 4096, 1, 8, 4
    segs, keys, vals, cbs, keep, (pq_cb, rv_cb) = _window(g, device, D, M, C, L, Cr, Hkv, 1500, 2500, 64)
    stats = H(K.ref_table_stats(cbs["k_pq_cb"], cbs["v_pq_cb"], cbs["k_rvq_cb"], cbs["v_rvq_cb"]))
    p32, r32 = pq_cb.astype(np.float64), rv_cb.astype(np.float64)
    d = D // M
    w_pq = (p32 ** 2).mean(1).reshape(D)                      # [M, d] -> coordinate m d + i
    w_rv = 2 * (r32 ** 2).mean(1).sum(0)                      # [D]
    vmax = np.abs(p32).max(1).reshape(D) + np.abs(r32).max(1).sum(0)
    np.testing.assert_allclose(stats[0], w_pq + w_rv, rtol=1e-5)
    np.testing.assert_allclose(stats[1], w_pq + w_rv, rtol=1e-5)  # K and V share the codebooks here
    np.testing.assert_allclose(stats[2], vmax, rtol=1e-5)
    q = randn16(g, B, Hq, D, scale=2.0)
    drift = torch.empty((B, Hq), dtype=torch.float32, device=device)
    K.ref_attention(T(q, device), kv_heads=Hkv, scale=D ** -0.5, causal=False, qpos=None, segments=segs,
                    score_tables=1e9, drift=drift, **cbs)
    # scores of the coded tokens (the decoded K: the tables skip its fp16
    # roundings, which moves the estimate far less than the tolerance)
    coded = np.concatenate([keys[:1500], keys[1564:]])  # the exact ring is not the tables'
    # histogram blocks: 32 splits of the coded tokens (256 blocks over 8 query heads)
    S = 32
    tps = -(-coded.shape[0] // S)
    log2e = 1.4426950408889634
    for hq in range(Hq):
        h = hq // (Hq // Hkv)
        s = (coded[:, h].astype(np.float32) @ q[0, hq].astype(np.float32)) * np.float32(D ** -0.5 * log2e)
        est = _estimate(q[0, hq], s, stats, D ** -0.5, blocks=[s[i:i + tps] for i in range(0, s.size, tps)])
        np.testing.assert_allclose(float(H(drift)[0, hq]), est, rtol=0.03)
    del d


ENVELOPE_SCALES = tuple(1.0 + 0.5 * i for i in range(15))  # 1, 1.5, ..., 8


@pytest.mark.parametrize("seed,family", [(41, "outlier"), (42, "plain")])
def test_tables_envelope(device, seed, family):
    """At the reference's default format (PQ 8 x 256, 4 gated layers of
    4096) over 8,192 coded and 512 exact tokens, the default path holds 2e-3
    (or one fp16 ulp of outputs at |x| >= 4) at every query scale from 1 to 8:
    where the guard stays quiet that is the tables' own error, where it fires
    the exact pass's.  "outlier": channels scaled by U(0.5, 4) per head."""
    from apple_amd import kernels as K

    g = rng(seed)
    D, M, C, L, Cr, B, Hq, Hkv = 128, 8, 256, 4, 4096, 1, 16, 8
    segs, keys, vals, cbs, keep, _ = _window(g, device, D, M, C, L, Cr, Hkv, 4096, 4096, 512)
    chan = (g.random((1, Hq, D), dtype=np.float32) * 3.5 + 0.5) if family == "outlier" else np.float32(1.0)
    q0 = g.standard_normal((B, Hq, D), dtype=np.float32) * chan
    rows = []
    for scale in ENVELOPE_SCALES:
        q = (q0 * np.float32(scale)).astype(np.float16)
        ref = nx.blockwise_attention(q, keys, vals, D ** -0.5, 256, False, None)
        info, drift = {}, torch.empty((B, Hq), dtype=torch.float32, device=device)
        out = K.ref_attention(T(q, device), kv_heads=Hkv, scale=D ** -0.5, causal=False, qpos=None,
                              segments=segs, score_tables=TOL, drift=drift, info=info, **cbs)
        assert info["score_tables"]
        e, x = _excess(H(out), ref)
        dr = H(drift)
        rows.append((scale, e, x, float(dr.max()), float((dr > TOL).mean())))
    print("\nscale  err        excess      max estimate  fired")
    for r in rows:
        print("%5.1f  %.3e  %+.3e  %.3e     %.2f" % r)
    bad = [r for r in rows if not r[2] <= 0]
    assert not bad, bad
    if family == "plain":
        assert rows[0][4] == 0.0  # the tables serve every head of plain queries at scale 1


def test_cache_decode_takes_the_tables(device, tmp_path):
    """attention_forward over a reference-format cache whose window holds
    more than REF_TABLES_MIN_TOKENS coded tokens: the decode step uses the
    tables (last_ref_tables) and writes its drift estimates, within 2e-3 of
    the same cache with score_table_tolerance None (the exact decode)."""
    import dataclasses

    from apple_amd.cache import RFSNv10KVCacheMLX
    from apple_amd.quantization import HybridQuantizerMLX
    from apple_amd.storage import RFSNConfig

    g = rng(3300)
    cfg = RFSNConfig(hidden_dim=512, num_heads=4, head_dim=128, num_layers=2, num_subspaces=8, subspace_dim=16,
                     num_rvq_layers=3, rvq_codebook_size=256, rvq_sparsity_threshold=0.25, hot_capacity=64,
                     warm_capacity=8192, cold_capacity=128, block_size_seq=64, disk_cache_dir=str(tmp_path),
                     prefetch_throttle_s=0.0)
    pq, rv = rand_codebooks(g, 8, 256, 16), rand_codebooks(g, 3, 256, 128)
    rv[:, 0] = 0
    qz = HybridQuantizerMLX(cfg, device=device, pq_codebooks=T(pq, device), rvq_codebooks=T(rv, device))
    n = 6000
    k, v = randn16(g, n, 4, 128), randn16(g, n, 4, 128)
    q = randn16(g, 1, 4, 128)
    outs = {}
    for tol in (cfg.score_table_tolerance, None):
        c = RFSNv10KVCacheMLX(dataclasses.replace(cfg, score_table_tolerance=tol), layer_idx=0, device=device)
        c.update(T(k, device), T(v, device), qz, disk_dir=tmp_path)
        assert c.num_warm >= 4096 and not c._fused_ok(4) and c._ref_ok(4)
        outs[tol] = H(c.attention_forward(T(q, device), causal=True))
        assert c.last_ref_tables == (tol is not None)
        if tol is not None:
            dr = H(c.last_ref_drift)
            assert dr.shape == (1, 4) and np.isfinite(dr).all()
    err, excess = _excess(outs[cfg.score_table_tolerance], outs[None])
    assert excess <= 0, err


def test_cache_tables_follow_the_warm_tier(device, tmp_path):
    """A decode loop over a reference-format cache with score tables: every
    update demotes blocks into warm (new warm stores), and each step's
    attention reads a head-major copy of the current stores, remade when they
    change and reused while they stay; every step within 2e-3 of the same
    cache decoded exactly (tolerance None)."""
    import dataclasses

    from apple_amd import kernels as K
    from apple_amd.cache import RFSNv10KVCacheMLX
    from apple_amd.quantization import HybridQuantizerMLX
    from apple_amd.storage import RFSNConfig

    g = rng(3310)
    cfg = RFSNConfig(hidden_dim=512, num_heads=4, head_dim=128, num_layers=2, num_subspaces=8, subspace_dim=16,
                     num_rvq_layers=4, rvq_codebook_size=512, rvq_sparsity_threshold=0.25, hot_capacity=64,
                     warm_capacity=8192, cold_capacity=128, block_size_seq=64, disk_cache_dir=str(tmp_path),
                     prefetch_throttle_s=0.0)
    pq, rv = rand_codebooks(g, 8, 256, 16), rand_codebooks(g, 4, 512, 128)
    rv[:, 0] = 0
    qz = HybridQuantizerMLX(cfg, device=device, pq_codebooks=T(pq, device), rvq_codebooks=T(rv, device))
    caches = {tol: RFSNv10KVCacheMLX(dataclasses.replace(cfg, score_table_tolerance=tol), layer_idx=0, device=device)
              for tol in (cfg.score_table_tolerance, None)}
    k0, v0 = randn16(g, 4500, 4, 128), randn16(g, 4500, 4, 128)
    for c in caches.values():
        c.update(T(k0, device), T(v0, device), qz, disk_dir=tmp_path)
    tab = caches[cfg.score_table_tolerance]
    copies, stores = [], []
    for step in range(5):
        q = T(randn16(g, 1, 4, 128), device)
        outs = {tol: H(c.attention_forward(q, causal=True)) for tol, c in caches.items()}
        assert tab.last_ref_tables
        hm = K._HEAD_MAJOR.get(id(tab.warm_keys.pq_codes))
        assert hm is not None and hm[0]() is tab.warm_keys.pq_codes
        copies.append(hm[2][0])
        stores.append(tab.warm_keys.pq_codes)
        err, excess = _excess(outs[cfg.score_table_tolerance], outs[None])
        assert excess <= 0, (step, err)
        if step == 2:  # a second call over unchanged stores reuses the copy
            tab.attention_forward(q, causal=True)
            assert K._HEAD_MAJOR[id(tab.warm_keys.pq_codes)][2][0] is hm[2][0]
        k1, v1 = randn16(g, 96, 4, 128), randn16(g, 96, 4, 128)  # 96 tokens: at least one block demoted
        for c in caches.values():
            c.update(T(k1, device), T(v1, device), qz, disk_dir=tmp_path)
    # every update replaced the warm stores, and each version got its own copy
    assert all(a is not b for a, b in zip(stores, stores[1:]))
    assert all(a is not b for a, b in zip(copies, copies[1:]))


def test_cache_tables_wait_for_the_group_break_even(device, tmp_path):
    """A cache of 8 query heads over 2 KV heads (groups of 4: the tables pay
    off from 8,192 coded tokens): with about 6,000 warm tokens the decode step
    is the exact one and makes no head-major copy; after 3,000 more it takes
    the tables over a copy.  Both within 2e-3 of the same cache decoded
    exactly (tolerance None)."""
    import dataclasses

    from apple_amd import kernels as K
    from apple_amd.cache import RFSNv10KVCacheMLX
    from apple_amd.quantization import HybridQuantizerMLX
    from apple_amd.storage import RFSNConfig

    g = rng(3320)
    cfg = RFSNConfig(hidden_dim=1024, num_heads=8, num_kv_heads=2, head_dim=128, num_layers=2, num_subspaces=8,
                     subspace_dim=16, num_rvq_layers=4, rvq_codebook_size=512, rvq_sparsity_threshold=0.25,
                     hot_capacity=64, warm_capacity=16384, cold_capacity=128, block_size_seq=64,
                     disk_cache_dir=str(tmp_path), prefetch_throttle_s=0.0)
    assert K.ref_tables_min_tokens(4) == 8192
    pq, rv = rand_codebooks(g, 8, 256, 16), rand_codebooks(g, 4, 512, 128)
    rv[:, 0] = 0
    qz = HybridQuantizerMLX(cfg, device=device, pq_codebooks=T(pq, device), rvq_codebooks=T(rv, device))
    caches = {tol: RFSNv10KVCacheMLX(dataclasses.replace(cfg, score_table_tolerance=tol), layer_idx=0, device=device)
              for tol in (cfg.score_table_tolerance, None)}
    tab = caches[cfg.score_table_tolerance]
    for n, tables in ((6000, False), (3000, True)):
        k, v = randn16(g, n, 2, 128), randn16(g, n, 2, 128)
        for c in caches.values():
            c.update(T(k, device), T(v, device), qz, disk_dir=tmp_path)
        q = T(randn16(g, 1, 8, 128), device)
        outs = {tol: H(c.attention_forward(q, causal=True)) for tol, c in caches.items()}
        assert tab.last_ref_tables == tables, n
        assert (id(tab.warm_keys.pq_codes) in K._HEAD_MAJOR) == tables, n
        err, excess = _excess(outs[cfg.score_table_tolerance], outs[None])
        assert excess <= 0, (n, err)


@pytest.mark.parametrize("tables", [False, True])
def test_dense_rows_match_the_active_map(device, monkeypatch, tables):
    """A store whose rows are all active is attended without its active map
    (the gated codes of row r are row r): bit-identical to the same segment
    given the identity map, on the exact path and with score tables."""
    from apple_amd import kernels as K

    monkeypatch.setattr(K, "REF_TABLES_MIN_TOKENS", 0)
    g = rng(3400 + int(tables))
    D, M, C, L, Cr, B, Hq, Hkv = 128, 8, 256, 4, 4096, 1, 8, 4
    d = D // M
    pq_cb = rand_codebooks(g, M, C, d)
    rv_cb = rand_codebooks(g, L, Cr, D)
    sk, sv = _store(g, 3000, Hkv, M, C, L, Cr, 1.0), _store(g, 3000, Hkv, M, C, L, Cr, 1.0)
    assert sk["rvq_offsets"].size == 3000 * Hkv
    dk, dv = _dev_store(sk, device), _dev_store(sv, device)
    dense = K.ref_store_segment(dk, dv, 0, 3000, 0)
    assert dense["k"][2] is None and dense["v"][2] is None and dense["k"][1] is not None
    mapped = dict(dense)
    for name, st in (("k", dk), ("v", dv)):
        pq, rvq, _, rsub, sidx, sval = dense[name]
        mapped[name] = (pq, rvq, K.active_map(st.rvq_offsets, 3000 * Hkv), rsub, sidx, sval)
    q = T(randn16(g, B, Hq, D), device)
    kw = dict(kv_heads=Hkv, scale=D ** -0.5, causal=False, qpos=None, k_pq_cb=T(pq_cb, device),
              v_pq_cb=T(pq_cb, device), k_rvq_cb=T(rv_cb, device), v_rvq_cb=T(rv_cb, device),
              score_tables=TOL if tables else None)
    a = K.ref_attention(q, segments=[dense], **kw)
    b = K.ref_attention(q, segments=[mapped], **kw)
    assert torch.equal(a, b)
    # dense rows over the head-major copy ([heads][T][L] gated codes)
    hm = K.ref_store_segment(dk, dv, 0, 3000, 0, head_major=True)
    assert hm["k"][2] is None and hm["rows"] == (1, 3000)
    assert torch.equal(K.ref_attention(q, segments=[hm], **kw), a)
    ref = nx.blockwise_attention(H(q), nx.decode_compressed(sk, pq_cb, rv_cb), nx.decode_compressed(sv, pq_cb, rv_cb),
                                 D ** -0.5, 16, False, None)
    assert _excess(H(a), ref)[1] <= 0


@pytest.mark.parametrize("k_active,v_active", [(1.0, 0.6), (0.6, 1.0)])
def test_mixed_gated_kinds(device, monkeypatch, k_active, v_active):
    """K codes with every row active (no map) beside V codes through an active
    map, and the reverse: the histogram blocks' loads specialized on each
    side's kind agree with the oracle on the tables path, and the head-major
    copies attend bit-identically to the stores' own order."""
    from apple_amd import kernels as K

    monkeypatch.setattr(K, "REF_TABLES_MIN_TOKENS", 0)
    g = rng(3700 + int(10 * k_active))
    D, M, C, L, Cr, B, Hq, Hkv = 128, 8, 256, 4, 1024, 1, 8, 8
    pq_cb = rand_codebooks(g, M, C, D // M)
    rv_cb = rand_codebooks(g, L, Cr, D)
    rv_cb[:, 0] = 0
    n = 2600
    sk, sv = _store(g, n, Hkv, M, C, L, Cr, k_active), _store(g, n, Hkv, M, C, L, Cr, v_active)
    dk, dv = _dev_store(sk, device), _dev_store(sv, device)
    own = K.ref_store_segment(dk, dv, 0, n, 0)
    hm = K.ref_store_segment(dk, dv, 0, n, 0, head_major=True)
    assert (own["k"][2] is None) == (k_active == 1.0) and (own["v"][2] is None) == (v_active == 1.0)
    q = T(randn16(g, B, Hq, D), device)
    kw = dict(kv_heads=Hkv, scale=D ** -0.5, causal=False, qpos=None, k_pq_cb=T(pq_cb, device),
              v_pq_cb=T(pq_cb, device), k_rvq_cb=T(rv_cb, device), v_rvq_cb=T(rv_cb, device), score_tables=TOL)
    info = {}
    a = K.ref_attention(q, segments=[own], info=info, **kw)
    assert info["score_tables"]
    assert torch.equal(K.ref_attention(q, segments=[hm], **kw), a)
    ref = nx.blockwise_attention(H(q), nx.decode_compressed(sk, pq_cb, rv_cb), nx.decode_compressed(sv, pq_cb, rv_cb),
                                 D ** -0.5, 16, False, None)
    assert _excess(H(a), ref)[1] <= 0


def test_hybrid_attention_takes_the_tables(device, tmp_path):
    """RFSNHybridAttentionMLX over two stores of 5,000 tokens (more than
    REF_TABLES_MIN_TOKENS): the decode step goes through the score tables
    (once per codebook set the guard's statistics, kept between calls) and
    agrees with the same call at score_table_tolerance None; with the
    codebooks written in place the statistics are rebuilt."""
    import dataclasses

    from apple_amd import kernels as K
    from apple_amd.attention import RFSNHybridAttentionMLX
    from apple_amd.quantization import HybridQuantizerMLX, _compress_tensor_sequence
    from apple_amd.storage import RFSNConfig

    g = rng(3500)
    cfg = RFSNConfig(hidden_dim=512, num_heads=4, head_dim=128, num_layers=2, num_subspaces=8, subspace_dim=16,
                     num_rvq_layers=3, rvq_codebook_size=256, rvq_sparsity_threshold=0.25, hot_capacity=16,
                     warm_capacity=24, cold_capacity=128, block_size_seq=16, disk_cache_dir=str(tmp_path))
    pq, rv = rand_codebooks(g, 8, 256, 16), rand_codebooks(g, 3, 256, 128)
    rv[:, 0] = 0
    qz = HybridQuantizerMLX(cfg, device=device, pq_codebooks=T(pq, device), rvq_codebooks=T(rv, device))
    k, v = randn16(g, 5000, 4, 128), randn16(g, 5000, 4, 128)
    ks, vs = _compress_tensor_sequence(T(k, device), qz), _compress_tensor_sequence(T(v, device), qz)
    q = T(randn16(g, 1, 4, 128), device)
    calls = []
    orig = K.ref_table_stats

    def counted(*a, **kw):
        calls.append(1)
        return orig(*a, **kw)

    K.ref_table_stats = counted
    try:
        att = RFSNHybridAttentionMLX(cfg)
        a = H(att(q, ks, vs, qz, causal=False))
        b = H(att(q, ks, vs, qz, causal=False))
        assert len(calls) == 1 and np.array_equal(a, b)
        qz.pq.codebooks.mul_(1.0)  # an in-place write bumps the version
        att(q, ks, vs, qz, causal=False)
        assert len(calls) == 2
    finally:
        K.ref_table_stats = orig
    qz.config = dataclasses.replace(cfg, score_table_tolerance=None)
    exact = H(RFSNHybridAttentionMLX(qz.config)(q, ks, vs, qz, causal=False))
    assert _excess(a, exact)[1] <= 0
