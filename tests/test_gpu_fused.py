"""GPU parity of the fused warm-tier dequant + decode attention against the
oracle (decode the window, then blockwise attention), within 2e-3 max-abs."""

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


def _kv(g, n, Hkv, D):
    s = (g.random((Hkv, D), dtype=np.float32) * 1.5 + 0.5).astype(np.float32)
    k = (g.standard_normal((n, Hkv, D), dtype=np.float32) * s).astype(np.float16)
    v = (g.standard_normal((n, Hkv, D), dtype=np.float32) * s).astype(np.float16)
    return k, v


def _setup(seed, Hq, Hkv, M, Mr, k, nw, nh, D=64):
    from apple_amd.quantization import HybridQuantizerMLX
    from apple_amd.storage import RFSNConfig

    g = rng(seed)
    keys, values = _kv(g, nw + nh, Hkv, D)
    cbs = {n: rand_codebooks(g, M, 256, D // M) for n in ("kp", "vp")}
    if Mr:
        cbs.update({n: rand_codebooks(g, Mr, 256, D // Mr) * np.float16(0.35) for n in ("kr", "vr")})
    # Mr = k = 0 is the reference format in its pq_only mode (threshold = inf)
    cfg = RFSNConfig(num_heads=Hq, head_dim=D, num_subspaces=M, subspace_dim=D // M, num_rvq_layers=1,
                     rvq_codebook_size=256, rvq_sparsity_threshold=float("inf") if not (Mr or k) else 0.005,
                     hot_capacity=nh, warm_capacity=nw + 4096, block_size_seq=128,
                     num_kv_heads=Hkv, rvq_subspaces=Mr, sparse_topk=k, tier_policy="recency", cold_medium="pinned")
    kq = HybridQuantizerMLX(cfg, pq_codebooks=torch.from_numpy(cbs["kp"]),
                            rvq_codebooks=torch.from_numpy(cbs["kr"]) if Mr else None)
    vq = HybridQuantizerMLX(cfg, pq_codebooks=torch.from_numpy(cbs["vp"]),
                            rvq_codebooks=torch.from_numpy(cbs["vr"]) if Mr else None)
    return g, cfg, keys, values, cbs, kq, vq


def _oracle_window(keys, values, cbs, Mr, k, nw):
    Hkv, D = keys.shape[1], keys.shape[2]
    outs = []
    for x, p, r in ((keys, cbs["kp"], cbs.get("kr")), (values, cbs["vp"], cbs.get("vr"))):
        flat = x[:nw].reshape(-1, D)
        enc = nx.ext_encode(flat, p, r if Mr else None, k)
        dec = nx.ext_decode(enc["pq_codes"], p, enc.get("rvq_codes"), r, enc.get("sparse_idx"),
                            enc.get("sparse_val"))
        if not (Mr or k):  # reference pq_only mode: fp16(base + 0) (quantization.py:319)
            dec = nx.hybrid_add(dec, np.zeros_like(dec))
        dec = dec.reshape(nw, Hkv, D)
        outs.append(np.concatenate([dec, x[nw:]], 0))
    return outs


CASES = [
    # seed, Hq, Hkv, M, Mr, k, nw, nh
    (1, 8, 8, 8, 0, 0, 896, 128),       # 1,024-token smoke shape, PQ-only
    (2, 32, 8, 16, 16, 4, 7680, 512),   # Llama-3.2-1B layer shape, PQ+RVQ+top-4
    (3, 32, 4, 16, 16, 4, 1000, 100),   # GQA 8:1, ragged tiles
    (4, 16, 8, 8, 8, 4, 333, 33),       # M=8 with RVQ and sparse, ragged
    (5, 8, 8, 16, 0, 4, 64, 0),         # no hot tier
    (6, 8, 4, 16, 16, 0, 0, 77),        # hot tier only
    (7, 16, 4, 16, 16, 0, 333, 20),     # score tables without a sparse stage, ragged
    (8, 8, 8, 16, 16, 4, 200, 16),      # score tables for one query head per KV head (3 padded columns)
]


@pytest.mark.parametrize("case", CASES)
def test_fused_cache_attention(device, case):
    from apple_amd.cache import RFSNv10KVCacheMLX

    seed, Hq, Hkv, M, Mr, k, nw, nh = case
    g, cfg, keys, values, cbs, kq, vq = _setup(seed, Hq, Hkv, M, Mr, k, nw, nh)
    cache = RFSNv10KVCacheMLX(cfg, device=device)
    cache.update(T(keys, device), T(values, device), (kq, vq))
    assert cache._fused_ok()
    wk, wv = _oracle_window(keys, values, cbs, Mr, k, nw)
    # the cache materializes exactly the oracle's window
    mk, mv, _ = cache.materialize_window()
    assert np.array_equal(H(mk).view(np.uint16), wk.view(np.uint16))
    assert np.array_equal(H(mv).view(np.uint16), wv.view(np.uint16))
    B = 3
    q = randn16(g, B, Hq, 64)
    Ttot = nw + nh
    # per-head positions: in one wave some heads have nothing allowed in the
    # first tiles (the hot tier holds the latest positions) while others do
    for causal, qp in ((True, None), (False, None), (True, g.integers(-1, Ttot, (B,)).astype(np.int32)),
                       (True, g.integers(-1, Ttot, (B, Hq)).astype(np.int32))):
        out = cache.attention_forward(T(q, device), causal=causal, query_positions=None if qp is None else T(qp, device))
        ref = nx.blockwise_attention(q, wk, wv, 64 ** -0.5, 256, causal, qp)
        err = np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max()
        assert err <= TOL, (causal, qp, err)


def test_fused_split_counts(device):
    """One window of 8,064 tokens for 8 query heads on one KV head, attended
    with 1, 3, 64 and 200 splits per (sequence, KV head) (at 200, splits
    past the last tile hold no tokens): every split count gives the oracle's
    result, repeated calls of one prepared launch give bit-identical outputs,
    and so does a second launch prepared with the same split count."""
    from apple_amd.cache import RFSNv10KVCacheMLX

    seed, Hq, Hkv, M, Mr, k, nw, nh = 11, 8, 1, 16, 16, 4, 8000, 64
    g, cfg, keys, values, cbs, kq, vq = _setup(seed, Hq, Hkv, M, Mr, k, nw, nh)
    cache = RFSNv10KVCacheMLX(cfg, device=device)
    cache.update(T(keys, device), T(values, device), (kq, vq))
    assert cache._fused_ok()
    wk, wv = _oracle_window(keys, values, cbs, Mr, k, nw)
    q = randn16(g, 2, Hq, 64)
    qd = T(q, device)
    ref = nx.blockwise_attention(q, wk, wv, 64 ** -0.5, 256, False, None)
    first = {}
    for splits in (1, 3, 64, 200, 64):
        out = torch.empty_like(qd)
        launch = cache.prepare(qd, causal=False, splits=splits, out=out)
        runs = [H(launch()).copy() for _ in range(3)]
        torch.cuda.synchronize()
        for r in runs[1:]:
            assert np.array_equal(r.view(np.uint16), runs[0].view(np.uint16)), splits
        err = np.abs(runs[0].astype(np.float32) - ref.astype(np.float32)).max()
        assert err <= TOL, (splits, err)
        if splits in first:  # a second prepared launch repeats the same bits
            assert np.array_equal(runs[0].view(np.uint16), first[splits].view(np.uint16))
        first[splits] = runs[0]
    assert np.abs(first[200].astype(np.float32) - first[1].astype(np.float32)).max() <= 2e-3


def test_fused_codebook_k_path(device):
    """With ``fused_score_tables=False`` the kernel rebuilds K^ from the
    codebooks for a format the score tables would serve: the same parity."""
    from apple_amd.cache import RFSNv10KVCacheMLX

    seed, Hq, Hkv, M, Mr, k, nw, nh = 2, 32, 8, 16, 16, 4, 2000, 96
    g, cfg, keys, values, cbs, kq, vq = _setup(seed, Hq, Hkv, M, Mr, k, nw, nh)
    cfg.fused_score_tables = False
    cache = RFSNv10KVCacheMLX(cfg, device=device)
    cache.update(T(keys, device), T(values, device), (kq, vq))
    assert cache._fused_ok() and cache._k_layout == 0 and not cache._warm_tiled[0].score_rows
    wk, wv = _oracle_window(keys, values, cbs, Mr, k, nw)
    q = randn16(g, 2, Hq, 64)
    for causal in (True, False):
        out = cache.attention_forward(T(q, device), causal=causal)
        ref = nx.blockwise_attention(q, wk, wv, 64 ** -0.5, 256, causal, None)
        assert np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max() <= TOL


def _guard_estimate(q, cbs, vmax, wk, wv, scale=64 ** -0.5):
    """The drift guard's estimate per (query, head), restated in numpy over
    the oracle's softmax: scale * sqrt(2^-20/12 * sum_i q_i^2 W_i) *
    sqrt(sum_t p_t^2) / sum_t p_t * 2 * vmax, W_i the second moments of K^_i
    and of its subspace's centroids over the K codebooks."""
    p, r = cbs["kp"].astype(np.float64), cbs["kr"].astype(np.float64)
    W = ((p * p).mean(1) + (r * r).mean(1)).reshape(64) + np.repeat((p * p).sum(2).mean(1) + (r * r).sum(2).mean(1), 4)
    B, Hq, _ = q.shape
    G = Hq // wk.shape[1]
    est = np.zeros((B, Hq))
    for b in range(B):
        for h in range(Hq):
            qv = q[b, h].astype(np.float64)
            lg = wk[:, h // G].astype(np.float64) @ qv * scale
            w = np.exp(lg - lg.max())
            est[b, h] = scale * np.sqrt((qv * qv * W).sum() / 12 / 2 ** 20) * np.sqrt((w * w).sum()) / w.sum() * 2 * vmax
    return est


def test_fused_error_envelope_peaked_queries(device):
    """Sharper attention (queries scaled up to 8x, 2,064-token window): both
    K paths stay within 2e-3 of the oracle at every scale.  The codebook path
    scores q . fp16(K^) as the reference does.  The score tables sum q .
    centroid per subspace without K^'s fp16 rounding, which moves their
    output by up to 1.3e-2 at 8x (measured on one MI355X without the guard);
    their drift guard estimates that per block and recomputes the blocks
    over the tolerance exactly: it stays quiet at 1x, where the tables hold
    2e-3 by themselves, and fires at 4x and 8x (one split per query and KV
    head; with several, each split estimates over its own tokens, an upper
    bound on its share of the window's estimate, so it fires at least as
    often).  The kernel's estimates match the numpy restatement of the
    formula over the oracle's softmax."""
    from apple_amd.cache import RFSNv10KVCacheMLX

    fired = {}
    for tables in (False, True):
        g, cfg, keys, values, cbs, kq, vq = _setup(11, 32, 8, 16, 16, 4, 2000, 64)
        cfg.fused_score_tables = tables
        cache = RFSNv10KVCacheMLX(cfg, device=device)
        cache.update(T(keys, device), T(values, device), (kq, vq))
        assert cache._k_layout == int(tables) and cache._guarded == tables
        wk, wv = _oracle_window(keys, values, cbs, 16, 4, 2000)
        vmax = max(float(np.abs(values.astype(np.float32)).max()),
                   float((np.abs(cbs["vp"].astype(np.float32)).max(1) + np.abs(cbs["vr"].astype(np.float32)).max(1)).max()))
        q0 = randn16(g, 4, 32, 64).astype(np.float32)
        for scale in (1, 2, 4, 8):
            q = (q0 * scale).astype(np.float16)
            out = cache.attention_forward(T(q, device), causal=False)
            ref = nx.blockwise_attention(q, wk, wv, 64 ** -0.5, 256, False, None)
            err = np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max()
            assert err <= TOL, (tables, scale, err)
            if tables:
                # one split per (query, KV head): the block's estimate is the whole window's
                one = torch.empty_like(T(q, device))
                cache.prepare(T(q, device), causal=False, splits=1, out=one)()
                assert np.abs(H(one).astype(np.float32) - ref.astype(np.float32)).max() <= TOL
                drift = H(cache.last_drift)[:, :, 0]
                est = _guard_estimate(q, cbs, vmax, wk, wv)
                np.testing.assert_allclose(drift, est, rtol=0.05, atol=1e-7)
                fired[scale] = bool((drift > cfg.score_table_tolerance).any())
    assert not fired[1] and fired[4] and fired[8], fired


ENVELOPE_SCALES = tuple(1.0 + 0.5 * i for i in range(15))  # 1, 1.5, ..., 8


def _excess(out: np.ndarray, ref: np.ndarray) -> tuple:
    """(max |out - ref|, max of |out - ref| - max(TOL, ulp(ref))): outputs are
    fp16, and from |ref| = 4 up one rounding step (3.9e-3 at [4, 8)) exceeds
    2e-3 whatever the arithmetic before it, so the envelope allows the larger
    of 2e-3 and one fp16 ulp of the reference output."""
    o, r = out.astype(np.float32), ref.astype(np.float32)
    d = np.abs(o - r)
    ulp = np.spacing(np.abs(ref.astype(np.float16))).astype(np.float32)
    return float(d.max()), float((d - np.maximum(TOL, ulp)).max())


@pytest.mark.parametrize("seed,family", [(21, "outlier"), (22, "outlier"), (23, "plain")])
def test_guard_envelope(device, seed, family):
    """The default path (score tables with the drift guard) holds 2e-3 (or
    one fp16 ulp of outputs at |x| >= 4) at every query scale from 1 to 8 in
    steps of 0.5, with the guard's own split count and with one split per
    (query, KV head).  "outlier": queries whose channels carry per-head
    scales drawn from U(0.5, 4) (the shape RoPE'd decoder queries have: some
    channels several times the rest); the guard fires on nearly every block
    from scale 1.  "plain": N(0, 1) queries, where it is quiet at 1 and fires
    on a growing share of blocks above.  Points where the guard stays quiet
    are the tables' own error; points where it fires are the exact pass."""
    from apple_amd.cache import RFSNv10KVCacheMLX

    g, cfg, keys, values, cbs, kq, vq = _setup(seed, 32, 8, 16, 16, 4, 2000, 64)
    cache = RFSNv10KVCacheMLX(cfg, device=device)
    cache.update(T(keys, device), T(values, device), (kq, vq))
    assert cache._k_layout == 1 and cache._guarded
    wk, wv = _oracle_window(keys, values, cbs, 16, 4, 2000)
    chan = (g.random((1, 32, 64), dtype=np.float32) * 3.5 + 0.5).astype(np.float32) if family == "outlier" else 1.0
    q0 = g.standard_normal((4, 32, 64), dtype=np.float32) * chan
    rows = []
    for scale in ENVELOPE_SCALES:
        q = (q0 * np.float32(scale)).astype(np.float16)
        ref = nx.blockwise_attention(q, wk, wv, 64 ** -0.5, 256, False, None)
        out = H(cache.attention_forward(T(q, device), causal=False))
        one = torch.empty_like(T(q, device))
        cache.prepare(T(q, device), causal=False, splits=1, out=one)()
        drift = H(cache.last_drift)[:, :, 0]
        e, x = _excess(out, ref)
        e1, x1 = _excess(H(one), ref)
        rows.append((scale, e, x, e1, x1, float(drift.max()), float((drift > cfg.score_table_tolerance).mean())))
    print("\nscale  err        excess      err(1 split)  excess      max estimate  fired")
    for r in rows:
        print("%5.1f  %.3e  %+.3e  %.3e     %+.3e  %.3e     %.2f" % r)
    bad = [r for r in rows if not (r[2] <= 0 and r[4] <= 0)]
    assert not bad, bad


def test_guard_follows_recalibrated_codebooks(device):
    """The drift guard's weights and the entry tables follow the K codebooks:
    after calibrate_quantizer replaces them, and after an in-place write, the
    next call's guard row is the new codebooks' weights."""
    from apple_amd import kernels as K
    from apple_amd.cache import RFSNv10KVCacheMLX
    from apple_amd.calibrate import calibrate_quantizer

    g, cfg, keys, values, cbs, kq, vq = _setup(12, 32, 8, 16, 16, 4, 600, 64)
    cache = RFSNv10KVCacheMLX(cfg, device=device)
    cache.update(T(keys, device), T(values, device), (kq, vq))
    assert cache._guarded
    q = T(randn16(g, 1, 32, 64), device)

    def row():
        return H(cache._guard[0, :64]).copy()

    def want():
        return H(K.score_guard(kq.pq.codebooks, kq.rvq.codebooks, 0.0)[:64])

    cache.attention_forward(q, causal=False)
    first = row()
    np.testing.assert_array_equal(first, want())
    calibrate_quantizer(kq, T(keys.reshape(-1, 64), device), num_iterations=2,
                        generator=torch.Generator().manual_seed(3))
    cache.attention_forward(q, causal=False)
    second = row()
    assert not np.array_equal(first, second)
    np.testing.assert_array_equal(second, want())
    kq.rvq.codebooks.mul_(2.0)  # written in place: same tensor, new version
    cache.attention_forward(q, causal=False)
    np.testing.assert_array_equal(row(), want())
    assert not np.array_equal(row(), second)


def test_fused_exact_pass_matches_codebook_path(device):
    """With the guard's tolerance at 0 every block of the score-table kernel
    recomputes its output on the exact pass, which rebuilds K^ from the
    codebooks while reading the score-table rows and the corrected-coordinate
    plane: the outputs are bit-identical to the codebook path's over the
    codebook layout, for one split and for several (split partials merged),
    per-sequence cache and batched cache alike.  A guarded launch of several
    splits with fewer than 256 tiles per block runs the exact pass alone
    (3,080 tokens in 5 splits; its drift entries are 0); 2 splits of 16,580
    tokens hold 260 tiles each and run the table pass first."""
    from apple_amd.batched import RFSNBatchedKVCache
    from apple_amd.cache import RFSNv10KVCacheMLX

    outs = {}
    for mode in ("exact", "codebook"):
        for nw, split_counts in ((3000, (1, 5)), (16500, (2,))):
            g, cfg, keys, values, cbs, kq, vq = _setup(21, 32, 8, 16, 16, 4, nw, 80)
            cfg.fused_score_tables = mode == "exact"
            cfg.score_table_tolerance = 0.0
            cache = RFSNv10KVCacheMLX(cfg, device=device)
            cache.update(T(keys, device), T(values, device), (kq, vq))
            q = T(randn16(g, 2, 32, 64), device)
            for splits in split_counts:
                out = torch.empty_like(q)
                cache.prepare(q, causal=True, splits=splits, out=out)()
                outs[(mode, nw, splits)] = H(out).copy()
                if mode == "exact":
                    drift = H(cache.last_drift)
                    assert drift.shape[-1] == splits
                    if splits == 5:
                        assert (drift == 0).all()  # exact pass alone
                    else:
                        assert (drift > 0).all()   # table pass, every block recomputed
            if nw == 3000:
                bc = RFSNBatchedKVCache(cfg, 2, device=device)
                for b in range(2):
                    bc.prefill(b, T(keys, device), T(values, device), kq, vq)
                assert bc.k_layout == int(mode == "exact")
                outs[(mode, "batched")] = H(bc.attention_forward(q)).copy()
    for key in ((3000, 1), (3000, 5), (16500, 2), "batched"):
        assert np.array_equal(outs[("exact",) + (key if isinstance(key, tuple) else (key,))].view(np.uint16),
                              outs[("codebook",) + (key if isinstance(key, tuple) else (key,))].view(np.uint16)), key


def test_fused_score_tables_in_use(device):
    """The Llama-3.2-1B layer format (16 + 16 subspaces, 4 query heads per
    KV head) streams its K codes as score-table rows."""
    from apple_amd.cache import RFSNv10KVCacheMLX

    g, cfg, keys, values, cbs, kq, vq = _setup(2, 32, 8, 16, 16, 4, 300, 40)
    cache = RFSNv10KVCacheMLX(cfg, device=device)
    cache.update(T(keys, device), T(values, device), (kq, vq))
    assert cache._k_layout == 1 and cache._warm_tiled[0].score_rows and not cache._warm_tiled[1].score_rows
    # 8 query heads per KV head: no score tables, the materialized path serves it
    q = randn16(g, 1, 64, 64)
    assert not cache._fused_ok(64)
    wk, wv = _oracle_window(keys, values, cbs, 16, 4, 300)
    out = cache.attention_forward(T(q, device), causal=False)
    ref = nx.blockwise_attention(q, wk, wv, 64 ** -0.5, 256, False, None)
    assert np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max() <= TOL


@pytest.mark.parametrize("cw", [1, 31, 100, 1500])
def test_fused_context_window(device, cw):
    from apple_amd.cache import RFSNv10KVCacheMLX

    g, cfg, keys, values, cbs, kq, vq = _setup(40 + cw, 32, 8, 16, 16, 4, 1200, 96)
    cache = RFSNv10KVCacheMLX(cfg, device=device)
    cache.update(T(keys, device), T(values, device), (kq, vq))
    wk, wv = _oracle_window(keys, values, cbs, 16, 4, 1200)
    q = randn16(g, 1, 32, 64)
    qpos = np.array([1250], np.int32)
    out = cache.attention_forward(T(q, device), causal=True, query_positions=T(qpos, device), context_window=cw)
    st = cache.get_last_access_stats()
    start = max(0, 1251 - cw)
    ref = nx.blockwise_attention(q, wk[start:1251], wv[start:1251], 0.125, 256, True, qpos - start)
    err = np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max()
    assert err <= TOL
    assert st["window_start"] == start and st["window_tokens"] == 1251 - start
    mk, _, adj = cache.materialize_window(query_positions=T(qpos, device), context_window=cw)
    assert np.array_equal(H(mk).view(np.uint16), wk[start:1251].view(np.uint16))
    assert int(H(adj)[0]) == 1250 - start


def test_batched_matches_per_sequence(device):
    from apple_amd.batched import RFSNBatchedKVCache
    from apple_amd.quantization import HybridQuantizerMLX

    B, Hq, Hkv, nw, nh = 4, 32, 8, 2048, 256
    seqs = [_setup(70 + b, Hq, Hkv, 16, 16, 4, nw, nh) for b in range(B)]
    cfg = seqs[0][1]
    bc = RFSNBatchedKVCache(cfg, B, device=device)
    refs = []
    for b, (g, _, keys, values, cbs, kq, vq) in enumerate(seqs):
        bc.prefill(b, T(keys, device), T(values, device), kq, vq)
        refs.append(_oracle_window(keys, values, cbs, 16, 4, nw))
    q = randn16(rng(99), B, Hq, 64)
    out = H(bc.attention_forward(T(q, device)))
    for b in range(B):
        mk, mv = bc.sequence_window(b)
        assert np.array_equal(H(mk).view(np.uint16), refs[b][0].view(np.uint16))
        assert np.array_equal(H(mv).view(np.uint16), refs[b][1].view(np.uint16))
        ref = nx.blockwise_attention(q[b:b + 1], refs[b][0], refs[b][1], 0.125, 256, False, None)
        assert np.abs(out[b:b + 1].astype(np.float32) - ref.astype(np.float32)).max() <= TOL


def _cold_cache(device, seed, total, nh, nw, chunk, Hq=32, Hkv=4, cold_slots=32):
    """A recency cache (PQ M16 + RVQ M16 + top-4) whose oldest tokens sit in
    pinned cold chunks of ``chunk`` tokens, filled by two appends, with the
    oracle's decode of every token."""
    from apple_amd.cache import RFSNv10KVCacheMLX
    from apple_amd.quantization import HybridQuantizerMLX
    from apple_amd.storage import RFSNConfig

    g = rng(seed)
    D, M = 64, 16
    keys, values = _kv(g, total, Hkv, D)
    cbs = {n: rand_codebooks(g, M, 256, D // M) for n in ("kp", "vp")}
    cbs.update({n: rand_codebooks(g, M, 256, D // M) * np.float16(0.35) for n in ("kr", "vr")})
    cfg = RFSNConfig(num_heads=Hq, head_dim=D, num_subspaces=M, subspace_dim=D // M, num_rvq_layers=1,
                     rvq_codebook_size=256, rvq_sparsity_threshold=0.005, hot_capacity=nh, warm_capacity=nw,
                     block_size_seq=128, num_kv_heads=Hkv, rvq_subspaces=M, sparse_topk=4, tier_policy="recency",
                     cold_medium="pinned", cold_chunk_tokens=chunk)
    kq = HybridQuantizerMLX(cfg, pq_codebooks=torch.from_numpy(cbs["kp"]), rvq_codebooks=torch.from_numpy(cbs["kr"]))
    vq = HybridQuantizerMLX(cfg, pq_codebooks=torch.from_numpy(cbs["vp"]), rvq_codebooks=torch.from_numpy(cbs["vr"]))
    cache = RFSNv10KVCacheMLX(cfg, device=device, cold_slots=cold_slots)
    cut = total - 300
    cache.update(T(keys[:cut], device), T(values[:cut], device), (kq, vq))
    cache.update(T(keys[cut:], device), T(values[cut:], device), (kq, vq))
    dec = []
    for x, p, r in ((keys, cbs["kp"], cbs["kr"]), (values, cbs["vp"], cbs["vr"])):
        enc = nx.ext_encode(x.reshape(-1, D), p, r, 4)
        dec.append(nx.ext_decode(enc["pq_codes"], p, enc["rvq_codes"], r, enc["sparse_idx"],
                                 enc["sparse_val"]).reshape(total, Hkv, D))
    return g, cfg, cache, keys, values, dec


def _cold_window(ids, chunk, ncold, total, nh, keys, values, dec):
    """Positions and oracle K/V of [chosen cold chunks | warm | hot], in position order."""
    pos = np.concatenate([np.arange(c * chunk, min((c + 1) * chunk, ncold)) for c in sorted(ids)]
                         + [np.arange(ncold, total)])
    hot = (pos >= total - nh)[:, None, None]
    return pos, np.where(hot, keys[pos], dec[0][pos]), np.where(hot, values[pos], dec[1][pos])


def test_fused_cold_pinned_prefetch(device):
    """Pinned cold chunks chosen by the router's ranking (and an arbitrary
    set): the fused path with every chunk copied in during the step (resident
    part attended while the copies run, partials merged), with every chunk
    resident (one launch), and with half of them resident; prepared steps of
    both kinds; materialized windows bit-exact."""
    from apple_amd import kernels as K
    from apple_amd.storage import AsyncHierarchicalRouterMLX

    total, nh, nw, chunk = 1664, 64, 600, 100
    ncold = total - nh - nw
    g, cfg, cache, keys, values, dec = _cold_cache(device, 90, total, nh, nw, chunk)
    assert (cache.num_hot, cache.num_warm, cache.num_cold) == (nh, nw, ncold)
    assert [m["chunk_id"] for m in cache.cold_chunk_metadata] == list(range(10))
    router = AsyncHierarchicalRouterMLX(cfg).bind(cache)
    near = router.rank(total - 1, total)[:4]
    assert near == [9, 8, 7, 6]
    B, Hq = 2, 32
    q = randn16(g, B, Hq, 64)
    qd = T(q, device)
    qp = g.integers(-1, total, (B, Hq)).astype(np.int32)
    qp[0, 0] = total - 1  # the window ends at the newest token
    for ids in (near, [0, 3, 7]):
        pos, wk, wv = _cold_window(ids, chunk, ncold, total, nh, keys, values, dec)
        mk, mv, _ = cache.materialize_window(cold_chunks=ids)
        assert np.array_equal(H(mk).view(np.uint16), wk.view(np.uint16))
        assert np.array_equal(H(mv).view(np.uint16), wv.view(np.uint16))
        qidx = (np.searchsorted(pos, qp, side="right") - 1).astype(np.int32)
        for mode in ("copied", "resident", "half"):
            for causal, qpa, rqp in ((False, None, None), (True, None, None), (True, qp, qidx)):
                if mode == "copied":
                    cache.evict_cold_slots()
                elif mode == "half":
                    cache.evict_cold_slots()
                    cache.prefetch_cold_chunks(ids[::2])
                out = cache.attention_forward(qd, causal=causal, cold_chunks=ids,
                                              query_positions=None if qpa is None else T(qpa, device))
                st = cache.get_last_access_stats()
                assert st["cold_chunks_touched"] == len(ids)
                ref = nx.blockwise_attention(q, wk, wv, 0.125, 256, causal, rqp)
                err = np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max()
                assert err <= TOL, (ids, mode, causal, qpa is None, err)
        # prepared steps: copies re-issued by every call, then all resident
        ref = nx.blockwise_attention(q, wk, wv, 0.125, 256, True, None)
        cache.evict_cold_slots()
        step = cache.prepare(qd, causal=True, cold_chunks=ids)
        assert isinstance(step, K.PrefetchedStep) and step.copy_bytes == len(ids) * cache._chunk_bytes()
        assert step.ncopies == (1 if ids == near else len(ids))  # consecutive chunks move in one copy
        for _ in range(2):
            err = np.abs(H(step()).astype(np.float32) - ref.astype(np.float32)).max()
            assert err <= TOL
        one = cache.prepare(qd, causal=True, cold_chunks=ids)
        assert isinstance(one, K.FusedLaunch)
        for _ in range(2):
            assert np.abs(H(one()).astype(np.float32) - ref.astype(np.float32)).max() <= TOL


def test_fused_cold_slot_limit_and_partial_contract(device):
    """More chunks than device slots is a ValueError; partial-mode calls whose
    slots do not fit are rejected before any launch."""
    from apple_amd import kernels as K

    total, nh, nw, chunk = 900, 32, 200, 64
    g, cfg, cache, keys, values, dec = _cold_cache(device, 91, total, nh, nw, chunk, Hq=8, Hkv=4, cold_slots=3)
    q = T(randn16(g, 1, 8, 64), device)
    with pytest.raises(ValueError):
        cache.attention_forward(q, cold_chunks=[0, 1, 2, 3])
    out = cache.attention_forward(q, cold_chunks=[0, 1, 2])
    assert out.shape == (1, 8, 64)
    fmt = cache._fmt()
    kt, vt = cache._warm_tiled
    nw = cache.num_warm  # whole-chunk migrations leave fewer than the capacity
    assert nw > 64
    with pytest.raises(ValueError):  # a segment longer than its code rows is refused on the host
        K.SegmentTable(1).add(0, kt.codes(0), vt.codes(0), kt.cap, kt.cap + 1, 0)
    table = K.SegmentTable(1)
    table.add(0, kt.codes(0), vt.codes(0), kt.cap, nw, 0)
    ws = torch.empty(1 << 16, dtype=torch.uint8, device=device)
    common = dict(kv_heads=4, scale=0.125, causal=False, qpos=None, hot_k=None, hot_v=None, hot_len=0,
                  hot_pos0=0, hot_seq_stride=0, segments=table, k_pq_cb=cache._kq.pq.codebooks,
                  v_pq_cb=cache._vq.pq.codebooks, k_rvq_cb=cache._kq.rvq.codebooks,
                  v_rvq_cb=cache._vq.rvq.codebooks, cb_batch_stride=False, max_tokens=nw, workspace=ws)
    with pytest.raises(ValueError):
        K.fused_attention(q, fmt, splits=4, part=(2, 5, False), **common)   # 2 + 4 > 5 slots
    with pytest.raises(ValueError):
        K.fused_attention(q, fmt, splits=2, part=(0, 4, True), **common)    # merging call not last
    # two partial calls over two halves of the warm tier equal one call
    half = K.round_up(nw // 2, K.TILE)
    t1, t2 = K.SegmentTable(1), K.SegmentTable(1)
    t1.add(0, kt.codes(0), vt.codes(0), kt.cap, half, 0)
    t2.add(0, kt.codes(half // K.TILE), vt.codes(half // K.TILE), kt.cap, nw - half, half)
    whole = K.fused_attention(q, fmt, splits=0, **{**common, "workspace": None})
    out = torch.empty_like(q)
    K.fused_attention(q, fmt, splits=3, part=(0, 5, False), out=out, **{**common, "segments": t1, "max_tokens": half})
    K.fused_attention(q, fmt, splits=2, part=(3, 5, True), out=out,
                      **{**common, "segments": t2, "max_tokens": nw - half})
    assert float((out.float() - whole.float()).abs().max()) <= 1e-3


def _policy_counts(appends, hc, wc, chunk, block=32):
    """Tier sizes under the recency policy, restated in plain arithmetic:
    hot overflow demoted in multiples of ``block``, warm overflow moved to
    cold up to the next chunk boundary."""
    hot = warm = cold = 0
    for T in appends:
        keep = min(T, hc)
        direct = T - keep
        ov = max(hot + keep - hc, 0)
        if ov and hc >= block:
            ov = -(-ov // block) * block
        pop = min(ov, hot)
        hot -= pop
        n = pop + direct
        if n:
            excess = warm + n - wc
            if excess > 0:
                cut = min(-(-(cold + excess) // chunk) * chunk - cold, warm + n)
                moved = min(warm, cut)
                warm, cold = warm - moved, cold + moved
                cold += cut - moved
                n -= cut - moved
            warm += n
        hot += keep
    return hot, warm, cold


@pytest.mark.parametrize("chunk,wc", [(64, 256), (100, 256), (64, 40)])
def test_streaming_appends(device, chunk, wc):
    """Token-by-token and ragged appends into a recency cache with a pinned
    cold tier: tier sizes follow the policy, every cold chunk but the last is
    whole, the materialized window is bit-exact against the oracle's decode
    of every token (exact where hot), and the fused attention over the whole
    context (every cold chunk) is within 2e-3.  With 64-token chunks the
    tiled warm store migrates by moving its head (no rebuild); with 100 it
    takes the rebuild path whenever a move is not whole tiles; a warm tier
    smaller than a chunk leaves partial chunks that later moves complete
    (merge-on-append into pinned chunks)."""
    total, hc = 1500, 64
    g, cfg, bulk, keys, values, dec = _cold_cache(device, 92 + chunk, total, hc, wc, chunk, Hq=8, Hkv=4)
    # _cold_cache filled ``bulk`` with two appends; start again from empty with ragged ones
    from apple_amd.cache import RFSNv10KVCacheMLX

    cache = RFSNv10KVCacheMLX(cfg, device=device, cold_slots=32)
    kq, vq = bulk._kq, bulk._vq
    sizes, done = [], 0
    pick = [1, 1, 1, 3, 17, 64, 100, 1, 5]
    while done < total:
        s = min(pick[len(sizes) % len(pick)], total - done)
        sizes.append(s)
        done += s
    o = 0
    heads_moved = False
    for s in sizes:
        cache.update(T(keys[o:o + s], device), T(values[o:o + s], device), (kq, vq))
        o += s
        heads_moved |= cache._warm_tiled is not None and cache._warm_tiled[0].head > 0
    assert (cache.num_hot, cache.num_warm, cache.num_cold) == _policy_counts(sizes, hc, wc, chunk)
    if chunk % 32 == 0 and wc >= chunk:
        assert heads_moved
    lens = [m["num_tokens"] for m in cache.cold_chunk_metadata]
    assert all(n == chunk for n in lens[:-1]) and sum(lens) == cache.num_cold
    ids = [m["chunk_id"] for m in cache.cold_chunk_metadata]
    enc = cache.num_cold + cache.num_warm
    wk = np.concatenate([dec[0][:enc], keys[enc:]], 0)
    wv = np.concatenate([dec[1][:enc], values[enc:]], 0)
    mk, mv, _ = cache.materialize_window(cold_chunks=ids)
    assert np.array_equal(H(mk).view(np.uint16), wk.view(np.uint16))
    assert np.array_equal(H(mv).view(np.uint16), wv.view(np.uint16))
    q = randn16(g, 2, 8, 64)
    for causal in (False, True):
        out = cache.attention_forward(T(q, device), causal=causal, cold_chunks=ids)
        ref = nx.blockwise_attention(q, wk, wv, 0.125, 256, causal, None)
        assert np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max() <= TOL


def test_prefetch_ahead_decode_loop(device):
    """Decode steps whose cold chunk sets alternate, each set's copies
    started one step ahead without the launch stream waiting
    (``prefetch_cold_chunks(wait=False)``, then the router's
    ``prefetch_ahead``): every step equals the oracle over its window, and
    the copies land in the half of the slot pool the running step does not
    read."""
    from apple_amd.storage import AsyncHierarchicalRouterMLX

    total, nh, nw, chunk = 2600, 64, 256, 64
    g, cfg, cache, keys, values, dec = _cold_cache(device, 93, total, nh, nw, chunk, Hq=8, Hkv=4, cold_slots=16)
    ncold, hot = cache.num_cold, cache.num_hot
    ids_all = [m["chunk_id"] for m in cache.cold_chunk_metadata]
    sets = [ids_all[-8:], ids_all[-16:-8]]
    q = randn16(g, 1, 8, 64)
    qd = T(q, device)
    cache.prefetch_cold_chunks(sets[0])
    for i in range(6):
        cur, nxt = sets[i % 2], sets[(i + 1) % 2]
        out = cache.attention_forward(qd, causal=False, cold_chunks=cur)
        cur_slots = {cache.resident_cold_chunk(c)["slot"] for c in cur}
        cache.prefetch_cold_chunks(nxt, wait=False)
        assert not cur_slots & {cache.resident_cold_chunk(c)["slot"] for c in nxt}
        assert all(cache.resident_cold_chunk(c) is not None for c in cur)  # the running set kept its slots
        pos, wk, wv = _cold_window(cur, chunk, ncold, total, hot, keys, values, dec)
        ref = nx.blockwise_attention(q, wk, wv, 0.125, 256, False, None)
        assert np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max() <= TOL, i
    router = AsyncHierarchicalRouterMLX(cfg).bind(cache)
    cache.evict_cold_slots()
    for step in range(3):
        p = total - 1 - 700 * step
        ids = router.prefetch_ahead(p, total, top_k=8)
        assert ids == router.rank(p, total)[:8] and all(router.get_chunk(c) is not None for c in ids)
        out = cache.attention_forward(qd, causal=False, cold_chunks=ids)
        pos, wk, wv = _cold_window(ids, chunk, ncold, total, hot, keys, values, dec)
        ref = nx.blockwise_attention(q, wk, wv, 0.125, 256, False, None)
        assert np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max() <= TOL, step


@pytest.mark.parametrize("M, Mr, k", [(16, 16, 4), (8, 8, 0), (16, 0, 4), (8, 0, 0)])
def test_paired_head_major_encode_matches_per_tensor(device, M, Mr, k):
    """A demotion's K + V encode (one launch, head-major codes) gives the
    per-tensor encode's codes bit for bit, from token-major inputs and from
    head-major ones (the popped hot tokens); None where it does not apply."""
    from apple_amd.quantization import _compress_tensor_sequence, _encode_pair_head_major, _head_major_store

    g, cfg, keys, values, cbs, kq, vq = _setup(11, 8, 4, M, Mr, k, 37, 16)
    kd, vd = T(keys, device), T(values, device)
    if not (Mr or k):  # the reference format keeps its own encode
        assert _encode_pair_head_major(kd, vd, kq, vq) is None
        return
    head_major = lambda x: x.permute(1, 0, 2).contiguous().permute(1, 0, 2)
    for kin, vin in ((kd, vd), (head_major(kd), head_major(vd))):
        hm = _encode_pair_head_major(kin, vin, kq, vq)
        assert hm is not None
        for codes, x, qz in zip(hm, (kin, vin), (kq, vq)):
            ref = _compress_tensor_sequence(x, qz)
            for plain in (False, True):
                got = _head_major_store(codes, plain)
                for f in ("pq_codes", "rvq_codes", "rvq_mask", "sparse_idx", "sparse_val"):
                    a, b = getattr(got, f), getattr(ref, f)
                    assert a.shape == b.shape and a.dtype == b.dtype and torch.equal(a.contiguous(), b), f
                    assert not plain or a.is_contiguous(), f
    assert _encode_pair_head_major(kd[:0], vd[:0], kq, vq) is None


def test_decode_session_streaming(device):
    """A decode loop through ``DecodeSession``: 90 one-token steps on a cache
    with pinned cold chunks (64 hot tokens, so a 32-token block is demoted
    every 32 steps, and warm overflow migrates whole 64-token chunks), the
    router's 4 nearest chunks attended.  Every step is within 2e-3 of the
    oracle over the step's window; the hot tier holds the newest tokens bit
    for bit; the launch is rebuilt only when a step migrates chunks or
    changes the chunk set, and a demotion that leaves the segments in place
    (warm grows at its tail) patches the prepared launch instead."""
    from apple_amd.quantization import HybridQuantizerMLX
    from apple_amd.storage import AsyncHierarchicalRouterMLX, RFSNConfig
    from apple_amd.cache import RFSNv10KVCacheMLX

    total0, steps, nh, nw, chunk, Hq, Hkv, D, M = 1500, 90, 64, 256, 64, 8, 4, 64, 16
    g = rng(97)
    keys, values = _kv(g, total0 + steps, Hkv, D)
    cbs = {n: rand_codebooks(g, M, 256, D // M) for n in ("kp", "vp")}
    cbs.update({n: rand_codebooks(g, M, 256, D // M) * np.float16(0.35) for n in ("kr", "vr")})
    cfg = RFSNConfig(num_heads=Hq, head_dim=D, num_subspaces=M, subspace_dim=D // M, num_rvq_layers=1,
                     rvq_codebook_size=256, hot_capacity=nh, warm_capacity=nw, block_size_seq=128,
                     num_kv_heads=Hkv, rvq_subspaces=M, sparse_topk=4, tier_policy="recency",
                     cold_medium="pinned", cold_chunk_tokens=chunk)
    kq = HybridQuantizerMLX(cfg, pq_codebooks=torch.from_numpy(cbs["kp"]), rvq_codebooks=torch.from_numpy(cbs["kr"]))
    vq = HybridQuantizerMLX(cfg, pq_codebooks=torch.from_numpy(cbs["vp"]), rvq_codebooks=torch.from_numpy(cbs["vr"]))
    cache = RFSNv10KVCacheMLX(cfg, device=device, cold_slots=16)
    cache.update(T(keys[:total0], device), T(values[:total0], device), (kq, vq))
    dec = []
    for x, p, r in ((keys, cbs["kp"], cbs["kr"]), (values, cbs["vp"], cbs["vr"])):
        enc = nx.ext_encode(x.reshape(-1, D), p, r, 4)
        dec.append(nx.ext_decode(enc["pq_codes"], p, enc["rvq_codes"], r, enc["sparse_idx"],
                                 enc["sparse_val"]).reshape(-1, Hkv, D))
    router = AsyncHierarchicalRouterMLX(cfg).bind(cache)
    q = randn16(g, 1, Hq, D)
    qd = T(q, device)
    sess = cache.decode_session(qd, (kq, vq), router=router, cold_attended=4)
    changes = 0
    prev = None
    for i in range(steps):
        t = total0 + i
        before = (cache.num_warm, cache.num_cold)
        out = sess.step(T(keys[t:t + 1], device), T(values[t:t + 1], device))
        ids = router.rank(t, t + 1)[:4]
        changes += (cache.num_warm, cache.num_cold) != before or ids != prev
        prev = ids
        pos, wk, wv = _cold_window(ids, chunk, cache.num_cold, t + 1, cache.num_hot, keys, values, dec)
        ref = nx.blockwise_attention(q, wk, wv, 0.125, 256, False, None)
        err = np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max()
        assert err <= TOL, (i, err)
        # a launch prepared afresh over the cache after the step, with the
        # session's split count, gives the same bits: the launch that appended
        # the token itself, or was patched after a demotion, attended the same
        # window as one built from the cache's state
        if sess._launch is not None:
            fresh = torch.empty_like(qd)
            cache.prepare(qd, causal=False, cold_chunks=ids, splits=int(sess._launch.params.splits), out=fresh)()
            assert torch.equal(fresh, out), (i, sess.rebuilds, sess.regrows)
    total = total0 + steps
    assert cache.total_tokens == total and cache.num_hot + cache.num_warm + cache.num_cold == total
    for tier, src in ((cache.hot_keys, keys), (cache.hot_values, values)):  # [T_hot, H, D], oldest first
        assert np.array_equal(H(tier.contiguous()).view(np.uint16), src[total - cache.num_hot:total].view(np.uint16))
    assert sess.rebuilds <= changes + 1 and sess.rebuilds < steps // 4, (sess.rebuilds, changes)
    assert sess.regrows >= 1, (sess.rebuilds, sess.regrows, changes)


def test_cold_chunks_npz_roundtrip(device, tmp_path):
    """The pinned cold tier written as the reference's chunk files
    (layer{L}_chunk{id}.npz, its key names) and read back into an empty cache:
    after the remaining tokens are appended the new cache materializes the
    same window bit for bit and attends identically; gaps in the chunk ids
    are refused."""
    from apple_amd.cache import RFSNv10KVCacheMLX

    total, nh, nw, chunk = 1500, 64, 256, 64
    g, cfg, cache, keys, values, dec = _cold_cache(device, 94, total, nh, nw, chunk, Hq=8, Hkv=4)
    paths = cache.export_cold_chunks(tmp_path)
    assert [p.name for p in paths] == [f"layer0_chunk{m['chunk_id']}.npz" for m in cache.cold_chunk_metadata]
    with np.load(paths[0], allow_pickle=False) as z:
        for key in ("num_tokens", "num_heads", "key_pq_codes", "key_rvq_codes", "key_rvq_mask", "key_rvq_offsets",
                    "value_pq_codes", "value_rvq_codes", "value_rvq_mask", "value_rvq_offsets"):
            assert key in z.files
        assert int(z["num_tokens"][0]) == chunk and int(z["num_heads"][0]) == 4
    again = RFSNv10KVCacheMLX(cfg, device=device)
    assert again.import_cold_chunks(tmp_path, (cache._kq, cache._vq)) == cache.num_cold
    rest = cache.num_cold
    again.update(T(keys[rest:], device), T(values[rest:], device), (cache._kq, cache._vq))
    assert (again.num_hot, again.num_warm, again.num_cold) == (cache.num_hot, cache.num_warm, cache.num_cold)
    ids = [m["chunk_id"] for m in cache.cold_chunk_metadata]
    a, b = cache.materialize_window(cold_chunks=ids), again.materialize_window(cold_chunks=ids)
    assert np.array_equal(H(a[0]).view(np.uint16), H(b[0]).view(np.uint16))
    assert np.array_equal(H(a[1]).view(np.uint16), H(b[1]).view(np.uint16))
    q = T(randn16(g, 1, 8, 64), device)
    assert torch.equal(cache.attention_forward(q, cold_chunks=ids), again.attention_forward(q, cold_chunks=ids))
    paths[1].unlink()
    with pytest.raises(ValueError):
        RFSNv10KVCacheMLX(cfg, device=device).import_cold_chunks(tmp_path, (cache._kq, cache._vq))
