"""Pins of the CPU oracle (no GPU).

Every oracle function is checked against something other than its own
formula: float64 brute force, textbook attention, closed-form known answers,
the reference test suite's assertions (rfsn_v10_mlx_ane_complete.py:374-554)
replayed on the oracle cache model, and the byte columns of the reference's
checked-in benchmark CSV (benchmark_outputs/dense_vs_hot_warm.csv).
``test_planted_mistakes`` shows that each pin fails on a plausible mistake
planted in the oracle.
"""

import math

import numpy as np
import pytest

from oracle import cache_model as cm
from oracle import kmeans as km
from oracle import numerics as nx
from tests.conftest import rand_codebooks, randn16, rng

F32 = np.float32


# ---------------------------------------------------------------- pin helpers

def exact_sqdist(x, c):
    """Float64 squared distance of fp16 rows (exact up to float64 rounding)."""
    x = np.asarray(x, np.float64)
    c = np.asarray(c, np.float64)
    return ((x[:, None, :] - c[None, :, :]) ** 2).sum(-1)


def check_sqdist(fn, g):
    """fp32 distances agree with the exact float64 distance to the fp32
    rounding bound of ``L - 2X + R``."""
    x = randn16(g, 64, 8)
    c = rand_codebooks(g, 1, 256, 8)[0]
    got = fn(x, c).astype(np.float64)
    ex = exact_sqdist(x, c)
    x64, c64 = x.astype(np.float64), c.astype(np.float64)
    mag = (x64 ** 2).sum(1)[:, None] + 2 * np.abs(x64 @ c64.T) + (c64 ** 2).sum(1)[None, :]
    return bool(np.all(np.abs(got - ex) <= 4 * np.finfo(F32).eps * mag + 1e-30))


def brute_topk(r2, k):
    """Top-k of |r2| by exhaustive sort on (-|r|, index)."""
    out = []
    for row in r2:
        order = sorted(range(len(row)), key=lambda i: (-abs(float(row[i])), i))
        out.append(order[:k])
    return np.array(out, dtype=np.int64)


def check_sparse(fn, g):
    x = randn16(g, 40, 16)
    recon = randn16(g, 40, 16)
    # planted ties: equal magnitudes of both signs in row 0 and row 1
    x[0, :] = np.float16(0)
    recon[0, :] = np.float16(0)
    x[0, [3, 9, 12]] = np.float16([1.5, -1.5, 1.5])
    x[1, :] = recon[1, :]
    x[1, [2, 5]] = recon[1, [2, 5]] + np.float16(0.25)
    idx, val = fn(x, recon, 4)
    r2 = x.astype(np.float64) - recon.astype(np.float64)
    want = brute_topk(r2, 4)
    if not np.array_equal(idx.astype(np.int64), want):
        return False
    wantv = np.take_along_axis(r2, want, 1).astype(np.float16)
    return bool(np.array_equal(val.view(np.uint16), wantv.view(np.uint16)))


def check_attention(fn, g):
    """Blockwise attention against textbook float64 softmax attention with
    the key/value heads expanded by plain repetition (llama32_adapter.py:384-386),
    causal masks with -1 (nothing allowed) and ragged blocks."""
    B, Hq, Hkv, T, D = 3, 8, 2, 45, 16
    q = randn16(g, B, Hq, D)
    k = randn16(g, T, Hkv, D)
    v = randn16(g, T, Hkv, D)
    qp = np.array([44, 7, -1], np.int32)
    out = fn(q, k, v, D ** -0.5, 16, True, qp).astype(np.float64)
    kx = np.repeat(k, Hq // Hkv, axis=1).astype(np.float64)
    vx = np.repeat(v, Hq // Hkv, axis=1).astype(np.float64)
    ref = np.zeros((B, Hq, D))
    for b in range(B):
        n = qp[b] + 1
        if n <= 0:
            continue
        for h in range(Hq):
            s = kx[:n, h] @ q[b, h].astype(np.float64) * D ** -0.5
            w = np.exp(s - s.max())
            ref[b, h] = (w[:, None] * vx[:n, h]).sum(0) / w.sum()
    return bool(np.abs(out - ref).max() <= 2e-3)


def check_score_delta(fn, g):
    """Score deltas put the decoded coordinate back on top of the unrounded
    base + rvq sum: dec[idx] = base[idx] + rvq[idx] + delta up to the fp16
    rounding of delta (and fp32 rounding of the sum), for every sparse entry."""
    pq = rand_codebooks(g, 16, 256, 4)
    rv = (rand_codebooks(g, 16, 256, 4).astype(F32) * 0.35).astype(np.float16)
    x = randn16(g, 300, 64)
    e = nx.ext_encode(x, pq, rv, 4)
    delta = fn(e["pq_codes"], pq, e["rvq_codes"], rv, e["sparse_idx"], e["sparse_val"]).astype(np.float64)
    dec = nx.ext_decode(e["pq_codes"], pq, e["rvq_codes"], rv, e["sparse_idx"], e["sparse_val"])
    ix = e["sparse_idx"].astype(np.int64)
    take = lambda a: np.take_along_axis(a.astype(np.float64), ix, axis=1)
    b, r, c = take(nx.pq_decode(e["pq_codes"], pq)), take(nx.pq_decode(e["rvq_codes"], rv)), take(dec)
    bound = np.abs(delta) * 2 ** -11 + (np.abs(b) + np.abs(r) + np.abs(c)) * 2 ** -23 + 2 ** -40
    return bool(np.all(np.abs(c - (b + r + delta)) <= bound))


# ---------------------------------------------------------------- distances, PQ

def test_sqdist_float64_bound():
    assert check_sqdist(nx.canonical_sqdist, rng(1))


def test_nearest_is_first_min_of_exact_distance():
    g = rng(2)
    x = randn16(g, 300, 4)
    c = rand_codebooks(g, 1, 64, 4)[0]
    code = nx.nearest(x, c)
    ex = exact_sqdist(x, c)
    best = ex.min(1)
    x64 = x.astype(np.float64)
    tol = 4 * np.finfo(F32).eps * ((x64 ** 2).sum(1) + 2 * np.abs(x64 @ c.astype(np.float64).T).max(1) + 8)
    assert np.all(ex[np.arange(300), code] <= best + tol)


def test_nearest_known_answers():
    g = rng(3)
    c = rand_codebooks(g, 1, 32, 8)[0]
    # inputs equal to codebook rows return those rows (distinct rows)
    assert np.array_equal(nx.nearest(c, c), np.arange(32))
    # duplicated rows: the lowest index wins (first-min argmin, quantization.py:139)
    c2 = c.copy()
    c2[7] = c2[3]
    c2[20] = c2[3]
    assert nx.nearest(c2[[3, 7, 20]], c2).tolist() == [3, 3, 3]
    # equidistant point between two rows: the lower index wins
    c3 = np.zeros((4, 2), np.float16)
    c3[1] = [1, 0]
    c3[2] = [-1, 0]
    c3[3] = [0, 5]
    assert nx.nearest(np.zeros((1, 2), np.float16) + np.float16([0, 2.5]), c3).tolist() == [0]
    assert nx.nearest(np.array([[0, 0]], np.float16), c3[1:]).tolist() == [0]


def test_pq_encode_residual_and_decode():
    g = rng(4)
    cb = rand_codebooks(g, 8, 256, 8)
    x = randn16(g, 200, 64)
    codes, resid = nx.pq_encode(x, cb)
    assert codes.dtype == np.uint8 and codes.shape == (200, 8)
    for m in range(8):
        sl = slice(8 * m, 8 * m + 8)
        ex = exact_sqdist(x[:, sl], cb[m])
        chosen = ex[np.arange(200), codes[:, m]]
        assert np.all(chosen <= ex.min(1) + 1e-4 * (1 + ex.min(1)))
    rec = nx.pq_decode(codes, cb)
    for m in range(8):
        assert np.array_equal(rec[:, 8 * m:8 * m + 8], cb[m][codes[:, m]])
    want = (x.astype(np.float64) - rec.astype(np.float64)).astype(np.float16)
    assert np.array_equal(resid.view(np.uint16), want.view(np.uint16))
    # codebook rows encode to themselves with a zero residual
    rows = np.concatenate([cb[m][[5]] for m in range(8)], 1)
    c5, r5 = nx.pq_encode(rows, cb)
    assert c5.tolist() == [[5] * 8] and not np.any(r5.astype(np.float32))
    with pytest.raises(ValueError):
        nx.pq_encode(x[:, :60], cb)


# ---------------------------------------------------------------- gated RVQ

def _rvq_codebooks(g, L, C, D):
    cb = rand_codebooks(g, L, C, D)
    cb[:, 0] = 0  # quantization.py:196-197
    return cb


def test_rvq_known_answers():
    g = rng(5)
    cb = _rvq_codebooks(g, 3, 64, 32)
    r = randn16(g, 50, 32)
    codes, mask, offs = nx.rvq_encode_full(r, cb, float("inf"))
    assert codes.shape == (0, 3) and not mask.any() and offs.size == 0
    z = np.zeros((4, 32), np.float16)
    codes, mask, offs = nx.rvq_encode_full(z, cb, -1.0)
    assert mask.all() and np.array_equal(codes, np.zeros((4, 3), np.uint16))
    # strict gate on the fp32 norm: a row whose norm equals the threshold is inactive
    e = np.zeros((2, 32), np.float16)
    e[0, 0] = 0.5
    e[1, 0] = 0.75
    _, mask, offs = nx.rvq_encode_full(e, cb, 0.5)
    assert mask.tolist() == [False, True] and offs.tolist() == [1]


def test_rvq_greedy_stages_match_brute_force():
    g = rng(6)
    L, C, D = 3, 48, 16
    cb = _rvq_codebooks(g, L, C, D)
    r = randn16(g, 80, 16, scale=0.5)
    r[::7] = (r[::7].astype(np.float32) * 0.01).astype(np.float16)
    thr = 0.3
    codes, mask, offs = nx.rvq_encode_full(r, cb, thr)
    norm64 = np.sqrt((r.astype(np.float64) ** 2).sum(1))
    assert np.array_equal(mask, norm64 > thr)
    assert np.array_equal(offs, np.flatnonzero(norm64 > thr))
    assert np.all(np.diff(offs) > 0)
    run = r[offs].astype(np.float64)
    for layer in range(L):
        ex = exact_sqdist(run, cb[layer])
        ch = ex[np.arange(len(offs)), codes[:, layer]]
        assert np.all(ch <= ex.min(1) + 1e-5 * (1 + ex.min(1)))
        run = run - cb[layer][codes[:, layer]].astype(np.float64)
    corr = nx.rvq_decode_correction(codes, mask, offs, cb)
    want = sum(cb[layer][codes[:, layer]].astype(np.float64) for layer in range(L)).astype(np.float16)
    assert np.array_equal(corr[offs].view(np.uint16), want.view(np.uint16))
    assert not np.any(corr[~mask].astype(np.float32))


def test_hybrid_roundtrip_not_worse_than_pq():
    """rfsn_v10_mlx_ane_complete.py:397-404: hybrid MSE <= PQ MSE + 1e-5."""
    g = rng(7)
    pq = rand_codebooks(g, 8, 256, 16)
    rv = _rvq_codebooks(g, 3, 256, 128)
    x = randn16(g, 96, 128)
    codes, _ = nx.pq_encode(x, pq)
    pq_mse = np.mean((x.astype(F32) - nx.pq_decode(codes, pq).astype(F32)) ** 2)
    hy = nx.hybrid_decode(*nx.hybrid_encode(x, pq, rv, 0.25), pq, rv)
    hy_mse = np.mean((x.astype(F32) - hy.astype(F32)) ** 2)
    assert hy_mse <= pq_mse + 1e-5


def test_rvq_sparsity_fraction():
    """rfsn_v10_mlx_ane_complete.py:384-392: small residuals stay inactive."""
    g = rng(8)
    rv = _rvq_codebooks(g, 3, 256, 128)
    res = np.concatenate([(randn16(g, 32, 128).astype(F32) * 0.01).astype(np.float16), randn16(g, 32, 128)])
    codes, mask, offs = nx.rvq_encode_full(res, rv, 0.25)
    assert 1.0 - mask.mean() > 0.2 and offs.shape[0] == codes.shape[0]


# ---------------------------------------------------------------- subspace RVQ + sparse

def test_sparse_topk_brute_force_and_ties():
    assert check_sparse(nx.sparse_topk, rng(9))


def test_apply_sparse_elementwise():
    g = rng(10)
    rec = randn16(g, 30, 64)
    idx = np.stack([g.permutation(64)[:4] for _ in range(30)]).astype(np.uint8)
    val = randn16(g, 30, 4, scale=0.1)
    out = nx.apply_sparse(rec, idx, val)
    want = rec.copy()
    for i in range(30):
        for j in range(4):
            want[i, idx[i, j]] = np.float16(float(rec[i, idx[i, j]]) + float(val[i, j]))
    assert np.array_equal(out.view(np.uint16), want.view(np.uint16))


def test_score_delta_restores_decoded_coordinates():
    assert check_score_delta(nx.score_delta, rng(12))
    # the deltas of a token without an RVQ stage are the same identity on base alone
    g = rng(14)
    pq = rand_codebooks(g, 16, 256, 4)
    x = randn16(g, 50, 64)
    e = nx.ext_encode(x, pq, None, 4)
    d = nx.score_delta(e["pq_codes"], pq, None, None, e["sparse_idx"], e["sparse_val"])
    ix = e["sparse_idx"].astype(np.int64)
    dec = nx.ext_decode(e["pq_codes"], pq, None, None, e["sparse_idx"], e["sparse_val"])
    want = (np.take_along_axis(dec, ix, 1).astype(F32)
            - np.take_along_axis(nx.pq_decode(e["pq_codes"], pq), ix, 1).astype(F32)).astype(np.float16)
    assert np.array_equal(d.view(np.uint16), want.view(np.uint16))


def test_ext_format_roundtrip():
    g = rng(11)
    pq = rand_codebooks(g, 16, 256, 4)
    rv = (rand_codebooks(g, 16, 256, 4).astype(F32) * 0.35).astype(np.float16)
    rv[:, 0] = 0  # a zero entry: the RVQ stage can never make a subspace worse
    x = randn16(g, 256, 64)
    e0 = nx.ext_encode(x, pq, None, 0)
    e1 = nx.ext_encode(x, pq, rv, 0)
    e2 = nx.ext_encode(x, pq, rv, 4)
    assert np.array_equal(e0["pq_codes"], e1["pq_codes"])
    d0 = nx.ext_decode(e0["pq_codes"], pq)
    d1 = nx.ext_decode(e1["pq_codes"], pq, e1["rvq_codes"], rv)
    d2 = nx.ext_decode(e2["pq_codes"], pq, e2["rvq_codes"], rv, e2["sparse_idx"], e2["sparse_val"])
    mse = [np.mean((x.astype(F32) - d.astype(F32)) ** 2) for d in (d0, d1, d2)]
    assert mse[2] <= mse[1] <= mse[0] + 1e-6
    # the stage-2 codes are the PQ codes of the fp16 stage-1 residual
    _, r1 = nx.pq_encode(x, pq)
    assert np.array_equal(e1["rvq_codes"], nx.pq_encode(r1, rv)[0])
    # after the sparse stage the kept coordinates are exact up to two fp16
    # roundings: of the stored value and of the final sum
    rows = np.arange(256)[:, None]
    kept = e2["sparse_idx"].astype(np.int64)
    xk = x[rows, kept].astype(np.float64)
    err = np.abs(xk - d2[rows, kept].astype(np.float64))
    bound = (np.abs(xk) + np.abs(e2["sparse_val"].astype(np.float64))) * 2 ** -11 + 2 ** -23
    assert np.all(err <= bound)


# ---------------------------------------------------------------- compressed helpers

def test_compressed_helpers_append_slice_decode():
    g = rng(12)
    pq = rand_codebooks(g, 4, 64, 8)
    rv = _rvq_codebooks(g, 2, 64, 32)
    a_t = randn16(g, 10, 3, 32)
    b_t = randn16(g, 7, 3, 32)
    b_t[2] = (b_t[2].astype(F32) * 0.001).astype(np.float16)
    a = nx.compress_tensor_sequence(a_t, pq, rv, 0.5)
    b = nx.compress_tensor_sequence(b_t, pq, rv, 0.5)
    ab = nx.append_compressed(a, b)
    assert ab["pq_codes"].shape == (17, 3, 4)
    assert np.all(np.diff(ab["rvq_offsets"]) > 0)
    full = nx.decode_compressed(ab, pq, rv)
    both = np.concatenate([nx.decode_compressed(a, pq, rv), nx.decode_compressed(b, pq, rv)])
    assert np.array_equal(full.view(np.uint16), both.view(np.uint16))
    for s, e in ((0, 17), (3, 12), (10, 11), (5, 5)):
        sl = nx.slice_compressed(ab, s, e)
        assert np.all((sl["rvq_offsets"] >= 0) & (sl["rvq_offsets"] < (e - s) * 3))
        assert np.array_equal(nx.decode_compressed(sl, pq, rv).view(np.uint16), full[s:e].view(np.uint16))
    with pytest.raises(ValueError):
        nx.slice_compressed(ab, 4, 18)
    with pytest.raises(ValueError):
        nx.append_compressed(a, nx.compress_tensor_sequence(randn16(g, 2, 2, 32), pq, rv, 0.5))


# ---------------------------------------------------------------- attention

def test_normalize_query_positions():
    assert nx.normalize_query_positions(None, 2, 3, 9).tolist() == [[9] * 3] * 2
    assert nx.normalize_query_positions(np.array([4, 5]), 2, 3, 9).tolist() == [[4] * 3, [5] * 3]
    p = np.arange(6).reshape(2, 3)
    assert np.array_equal(nx.normalize_query_positions(p, 2, 3, 9), p)
    for bad in (np.arange(3), np.zeros((3, 2))):
        with pytest.raises(ValueError):
            nx.normalize_query_positions(bad, 2, 3, 9)


def test_blockwise_vs_textbook_attention():
    assert check_attention(nx.blockwise_attention, rng(13))


def test_blockwise_block_size_invariance_and_edges():
    g = rng(14)
    q = randn16(g, 2, 4, 32)
    k = randn16(g, 100, 4, 32)
    v = randn16(g, 100, 4, 32)
    outs = [nx.blockwise_attention(q, k, v, 32 ** -0.5, bs).astype(np.float32) for bs in (1, 7, 16, 100, 512)]
    for o in outs[1:]:
        assert np.abs(o - outs[0]).max() <= 1e-3
    dense = nx.dense_attention_f64(q, k, v, 32 ** -0.5)
    assert np.abs(outs[0] - dense).max() <= 2e-3
    # empty key set -> zeros in q's dtype
    z = nx.blockwise_attention(q, k[:0], v[:0], 1.0, 16)
    assert z.dtype == np.float16 and not z.any()
    # a query that sees only token 0 returns v[0]
    o = nx.blockwise_attention(q, k, v, 1.0, 16, True, np.array([0, 0]))
    assert np.abs(o.astype(np.float32) - v[0][None].astype(np.float32)).max() <= 1e-3


def test_blockwise_vs_torch_sdpa():
    import torch

    g = rng(15)
    q = randn16(g, 1, 8, 64)
    k = randn16(g, 300, 8, 64)
    v = randn16(g, 300, 8, 64)
    out = nx.blockwise_attention(q, k, v, 0.125, 64).astype(np.float32)
    tq = torch.from_numpy(q.astype(np.float32)).permute(1, 0, 2)[None]
    tk = torch.from_numpy(k.astype(np.float32)).permute(1, 0, 2)[None]
    tv = torch.from_numpy(v.astype(np.float32)).permute(1, 0, 2)[None]
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, scale=0.125)[0].permute(1, 0, 2).numpy()
    assert np.abs(out - ref).max() <= 2e-3


def test_gqa_map():
    assert nx.kv_head_map(32, 8).tolist() == [i // 4 for i in range(32)]
    with pytest.raises(ValueError):
        nx.kv_head_map(6, 4)


# ---------------------------------------------------------------- k-means

def test_kmeans_invariants():
    g = rng(16)
    x = randn16(g, 512, 32)
    cb, met = km.calibrate(x, 4, 16, 6, seed=7, rvq_threshold=0.25)
    d = met["avg_distortion"]
    assert d[-1] <= d[0]
    assert all(b <= a + 1e-6 for a, b in zip(d, d[1:]))
    # a converged codebook is a fixed point of the Lloyd step
    for _ in range(30):
        codes, _ = nx.pq_encode(x, cb)
        nxt = km.centroid_update(x, codes, cb)
        if np.array_equal(nxt, cb):
            break
        cb = nxt
    codes, _ = nx.pq_encode(x, cb)
    assert np.array_equal(km.centroid_update(x, codes, cb), cb)
    # the centroid update is the member mean (empty clusters keep their row)
    codes = np.zeros((512, 4), np.uint8)
    codes[:256, 0] = 1
    up = km.centroid_update(x, codes, cb)
    assert np.allclose(up[0, 1].astype(np.float64), x[:256, :8].astype(np.float64).mean(0), atol=1e-3)
    assert np.array_equal(up[0, 5], cb[0, 5])


# ---------------------------------------------------------------- cache model

REF_SUITE = dict(num_heads=4, head_dim=128, num_subspaces=8, num_rvq_layers=3, hot_capacity=16,
                 warm_capacity=24, block_size_seq=16)


def _ref_quantizer(g, threshold=0.25):
    return cm.OracleQuantizer(rand_codebooks(g, 8, 256, 16), _rvq_codebooks(g, 3, 256, 128), threshold)


def test_reference_suite_cache_tiers():
    """rfsn_v10_mlx_ane_complete.py:448-486 on the oracle cache model."""
    g = rng(17)
    qz = _ref_quantizer(g)
    c = cm.OracleCache(**REF_SUITE)
    k, v = randn16(g, 60, 4, 128), randn16(g, 60, 4, 128)
    c.update(k, v, qz)
    assert (c.num_hot, c.num_warm, c.num_cold) == (16, 24, 20)
    assert len(c.cold_meta) == 2
    assert [m["chunk_id"] for m in c.cold_meta] == [2, 3]  # 40 // 16, 56 // 16
    q = randn16(g, 1, 4, 128)
    out = c.attention_forward(q, causal=True, query_positions=np.array([59]))
    st = dict(c.last_access_stats)
    kw, vw, adj = c.materialize_window(query_positions=np.array([59]))
    ref = nx.blockwise_attention(q, kw, vw, 128 ** -0.5, 16, True, adj)
    assert np.abs(out.astype(np.float32) - ref.astype(np.float32)).max() < 1e-4
    assert c.memory_usage_bytes()["cold_chunks"] == 2
    assert st["window_tokens"] == 60 and st["hot_tokens_materialized"] == 16
    assert st["warm_tokens_materialized"] == 24 and st["cold_tokens_materialized"] == 20
    assert st["reconstructed_tokens"] == 44
    assert st["warm_chunk_decodes"] == 2 and st["cold_chunk_decodes"] == 2
    # the window is hot, then warm, then cold in position order
    assert np.array_equal(kw[:16].view(np.uint16), k[:16].view(np.uint16))
    warm = qz.decompress(qz.compress(k[16:40]))
    assert np.array_equal(kw[16:40].view(np.uint16), warm.view(np.uint16))


def test_reference_suite_warm_window():
    """rfsn_v10_mlx_ane_complete.py:488-521."""
    g = rng(18)
    qz = _ref_quantizer(g)
    c = cm.OracleCache(**REF_SUITE)
    k, v = randn16(g, 36, 4, 128), randn16(g, 36, 4, 128)
    c.update(k, v, qz)
    fk, fv, _ = c.materialize_window(query_positions=np.array([35]))
    wk, wv, adj = c.materialize_window(query_positions=np.array([35]), context_window=8)
    st = c.last_access_stats
    assert wk.shape == (8, 4, 128) and int(adj[0]) == 7
    assert np.array_equal(wk.view(np.uint16), fk[-8:].view(np.uint16))
    assert np.array_equal(wv.view(np.uint16), fv[-8:].view(np.uint16))
    assert (st["window_tokens"], st["hot_tokens_materialized"], st["warm_tokens_materialized"]) == (8, 0, 8)
    assert st["cold_tokens_materialized"] == 0 and st["reconstructed_tokens"] == 8
    assert st["warm_chunk_decodes"] == 1


def test_reference_suite_router():
    """rfsn_v10_mlx_ane_complete.py:532-554."""
    g = rng(19)
    qz = _ref_quantizer(g)
    c = cm.OracleCache(**REF_SUITE)
    c.update(randn16(g, 48, 4, 128), randn16(g, 48, 4, 128), qz)
    r = cm.OracleRouter(c, 16)
    ids = r.prefetch(0, 1024, top_k=1)
    assert ids == [2] and r.get_chunk(2) is not None
    c.attention_forward(randn16(g, 1, 4, 128), causal=True, query_positions=np.array([47]), router=r,
                        current_position=47, context_window=16)
    assert c.last_access_stats["cold_chunk_cache_hits"] >= 1
    # ranking |cid*cs - pos| ascending over existing chunks (storage.py:182)
    c2 = cm.OracleCache(**REF_SUITE)
    c2.update(randn16(g, 120, 4, 128), randn16(g, 120, 4, 128), qz)
    r2 = cm.OracleRouter(c2, 16)
    assert r2.prefetch(70, 40, top_k=3) == [4, 5, 3]


def test_reference_suite_empty_and_errors():
    c = cm.OracleCache(**REF_SUITE)
    with pytest.raises(RuntimeError):
        c.materialize_window()
    g = rng(20)
    with pytest.raises(ValueError):
        c.update(randn16(g, 3, 4, 128), randn16(g, 4, 4, 128), _ref_quantizer(g))


@pytest.mark.parametrize("T,mode,cache_bytes", [(64, "pq_only", 67584), (64, "pq_rvq", 69120),
                                                 (192, "pq_only", 75776), (192, "pq_rvq", 83456)])
def test_csv_byte_known_answers(T, mode, cache_bytes):
    """benchmark_outputs/dense_vs_hot_warm.csv rows 20-21 and 56-57: the
    hot_warm profile of the eval harness (rfsn_v10_eval_benchmark.py:398-414,
    hot 32, warm T-32; pq_only = threshold +inf, :119)."""
    g = rng(21)
    pq = rand_codebooks(g, 8, 256, 16)
    rv = _rvq_codebooks(g, 3, 256, 128)
    qz = cm.OracleQuantizer(pq, rv, float("inf") if mode == "pq_only" else 0.25)
    c = cm.OracleCache(num_heads=4, head_dim=128, num_subspaces=8, num_rvq_layers=3, hot_capacity=32,
                       warm_capacity=max(1, T - 32), block_size_seq=16)
    c.update(randn16(g, T, 4, 128), randn16(g, T, 4, 128), qz)
    mem = c.memory_usage_bytes()
    assert mem["hot_bytes"] + mem["warm_pq_bytes"] + mem["warm_rvq_bytes"] == cache_bytes
    assert T * 4 * 128 * 2 * 2 == {64: 131072, 192: 393216}[T]  # dense_bytes column


# ---------------------------------------------------------------- planted mistakes

def test_planted_mistakes():
    """Each pin above rejects a plausible mistake planted in the oracle."""
    g = rng(22)

    def sq_no_R(x, c):  # dropped the ||c||^2 term
        L = nx.seq_sum_products(x, x).astype(F32)
        X = nx.seq_sum_products(x[:, None, :], c[None, :, :]).astype(F32)
        return L[:, None] - F32(2) * X

    def sq_sign(x, c):  # wrong sign of the cross term
        L = nx.seq_sum_products(x, x).astype(F32)
        R = nx.seq_sum_products(c, c).astype(F32)
        X = nx.seq_sum_products(x[:, None, :], c[None, :, :]).astype(F32)
        return (L[:, None] + F32(2) * X) + R[None, :]

    assert not check_sqdist(sq_no_R, g) and not check_sqdist(sq_sign, g)

    def topk_hi_ties(x, recon, k):  # ties to the higher index
        r2 = x.astype(F32) - recon.astype(F32)
        order = np.argsort(-np.abs(r2)[:, ::-1], axis=1, kind="stable")[:, :k]
        order = r2.shape[1] - 1 - order
        return order.astype(np.uint8), np.take_along_axis(r2, order, 1).astype(np.float16)

    def topk_signed(x, recon, k):  # ranks by signed value instead of magnitude
        r2 = x.astype(F32) - recon.astype(F32)
        order = np.argsort(-r2, axis=1, kind="stable")[:, :k]
        return order.astype(np.uint8), np.take_along_axis(r2, order, 1).astype(np.float16)

    assert not check_sparse(topk_hi_ties, rng(9)) and not check_sparse(topk_signed, rng(9))

    real_map = nx.kv_head_map

    def interleaved_map(hq, hkv):  # h % Hkv instead of h // (Hq/Hkv)
        return np.arange(hq) % hkv

    try:
        nx.kv_head_map = interleaved_map
        assert not check_attention(nx.blockwise_attention, rng(13))
    finally:
        nx.kv_head_map = real_map

    def attn_causal_off_by_one(q, k, v, s, bs, causal, qp):
        return nx.blockwise_attention(q, k, v, s, bs, causal, None if qp is None else np.asarray(qp) + 1)

    assert not check_attention(attn_causal_off_by_one, rng(13))
    assert check_attention(nx.blockwise_attention, rng(13))

    def delta_sign(*a):  # (base + rvq) - c
        return (-nx.score_delta(*a).astype(F32)).astype(np.float16)

    def delta_no_rvq(pq_codes, pq_cb, rvq_codes, rvq_cb, sidx, sval):  # the RVQ term dropped
        ix = sidx.astype(np.int64)
        c = np.take_along_axis(nx.ext_decode(pq_codes, pq_cb, rvq_codes, rvq_cb, sidx, sval), ix, 1)
        return (c.astype(F32) - np.take_along_axis(nx.pq_decode(pq_codes, pq_cb), ix, 1).astype(F32)).astype(np.float16)

    def delta_residual(pq_codes, pq_cb, rvq_codes, rvq_cb, sidx, sval):  # the stored residual itself
        return sval

    for bad in (delta_sign, delta_no_rvq, delta_residual):
        assert not check_score_delta(bad, rng(12)), bad.__name__


def test_cpu_baseline_matches_oracle():
    """The torch-CPU baseline computes the same decode (bit-exact) and the
    same attention (fp32 rounding) as the numpy oracle."""
    import torch

    from oracle import cpu_baseline as cb

    g = rng(23)
    pq = rand_codebooks(g, 16, 256, 4)
    rv = (rand_codebooks(g, 16, 256, 4).astype(F32) * 0.35).astype(np.float16)
    x = randn16(g, 96, 64)
    e = nx.ext_encode(x, pq, rv, 4)
    want = nx.ext_decode(e["pq_codes"], pq, e["rvq_codes"], rv, e["sparse_idx"], e["sparse_val"])
    got = cb.warm_decode(*(torch.from_numpy(a) for a in (e["pq_codes"], pq, e["rvq_codes"], rv, e["sparse_idx"],
                                                          e["sparse_val"]))).numpy()
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    q = randn16(g, 1, 8, 64)
    k, v = randn16(g, 90, 2, 64), randn16(g, 90, 2, 64)
    a = cb.blockwise_attention(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), 0.125, 32).numpy()
    b = nx.blockwise_attention(q, k, v, 0.125, 32)
    assert np.abs(a.astype(np.float32) - b.astype(np.float32)).max() <= 1e-3
    assert math.isfinite(float(a.astype(np.float32).sum()))


def test_cpu_baseline_encode_matches_oracle():
    """The timed torch-CPU encode (cdist^2 + argmin per subspace, both stages,
    top-4) gives the oracle's codes and sparse entries on data without
    near-ties (its fp32 distances carry no canonical rounding chain)."""
    import torch

    from oracle import cpu_baseline as cb

    g = np.random.default_rng(5)
    x = (g.standard_normal((512, 64)) * np.linspace(0.5, 2.0, 64)).astype(np.float16)
    p = (g.standard_normal((8, 256, 8)) * 0.5).astype(np.float16)
    r = (g.standard_normal((8, 256, 8)) * 0.2).astype(np.float16)
    out = cb.warm_encode(torch.from_numpy(x), torch.from_numpy(p), torch.from_numpy(r), 4)
    ref = nx.ext_encode(x, p, r, 4)
    assert np.array_equal(out["pq"].numpy(), ref["pq_codes"])
    assert np.array_equal(out["rvq"].numpy(), ref["rvq_codes"])
    assert np.array_equal(out["sparse_idx"].numpy(), ref["sparse_idx"])
    assert np.array_equal(out["sparse_val"].numpy().view(np.uint16), ref["sparse_val"].view(np.uint16))


# ---------------------------------------------------------------- timed CPU baselines, decode steps

def _ref_store(g, T, H, pq, rv, thr):
    """A reference-format warm store [T, H] encoded by the pinned oracle."""
    x = randn16(g, T * H, pq.shape[0] * pq.shape[2])
    pq_codes, rvq_codes, mask, offs = nx.hybrid_encode(x, pq, rv, thr)
    return x, {"pq": pq_codes.reshape(T, H, -1), "rvq": rvq_codes, "mask": mask, "offsets": offs}


def check_ref_decode(fn, g) -> bool:
    """``fn`` (cpu_baseline.ref_decode's signature) equals the pinned
    ``numerics.hybrid_decode`` bit for bit, active and inactive rows."""
    import torch

    pq = rand_codebooks(g, 8, 256, 16)
    rv = _rvq_codebooks(g, 4, 512, 128)
    ok = True
    for thr in (0.25, 1.6, float("inf")):  # every row, about half the rows, no row gated
        _, st = _ref_store(g, 24, 4, pq, rv, thr)
        n = 24 * 4
        want = nx.hybrid_decode(st["pq"].reshape(n, -1), st["rvq"], st["mask"], st["offsets"], pq, rv)
        got = fn(torch.from_numpy(st["pq"].reshape(n, -1)), torch.from_numpy(pq),
                 torch.from_numpy(st["rvq"].astype(np.int64)), torch.from_numpy(st["offsets"]),
                 torch.from_numpy(rv)).numpy()
        ok &= bool(np.array_equal(got.view(np.uint16), want.view(np.uint16)))
    return ok


def check_ref_decode_step(fn, g) -> bool:
    """``fn`` (cpu_baseline.ref_decode_step's signature) is the textbook
    float64 softmax attention over [hot | warm] decoded by the pinned oracle,
    within 1e-3 on the fp16 output (fp32 blockwise recurrence), GQA 4:1."""
    import torch

    H, Hq, D, T, Th = 2, 8, 128, 40, 9
    pq = rand_codebooks(g, 8, 256, 16)
    rv = _rvq_codebooks(g, 4, 256, 128)
    _, wk = _ref_store(g, T, H, pq, rv, 1.6)
    _, wv = _ref_store(g, T, H, pq, rv, 1.6)
    hot_k, hot_v = randn16(g, Th, H, D), randn16(g, Th, H, D)
    q = randn16(g, 1, Hq, D, scale=2.0)
    dec = [nx.hybrid_decode(w["pq"].reshape(T * H, -1), w["rvq"], w["mask"], w["offsets"], pq, rv).reshape(T, H, D)
           for w in (wk, wv)]
    want = nx.dense_attention_f64(q, np.concatenate([hot_k, dec[0]]), np.concatenate([hot_v, dec[1]]), D ** -0.5)
    tw = {k: torch.from_numpy(v if k != "rvq" else v.astype(np.int64)) for k, v in wk.items()}
    tv = {k: torch.from_numpy(v if k != "rvq" else v.astype(np.int64)) for k, v in wv.items()}
    got = fn(torch.from_numpy(q), torch.from_numpy(hot_k), torch.from_numpy(hot_v), tw, tv,
             {"pq": torch.from_numpy(pq), "rvq": torch.from_numpy(rv)}, D ** -0.5, 16).numpy()
    return float(np.abs(got.astype(np.float64) - want).max()) <= 1e-3


def check_decode_step(fn, g) -> bool:
    """``fn`` (cpu_baseline.decode_step's signature) is the textbook float64
    attention over [warm | hot] with the warm tier decoded by the pinned
    ``numerics.ext_decode`` (separate K and V codebooks, PQ + RVQ + top-4),
    within 1e-3 on the fp16 output, GQA 4:1."""
    import torch

    Hkv, Hq, D, T, Th = 2, 8, 64, 70, 11
    cbs = {n: rand_codebooks(g, 16, 256, 4) for n in ("k_pq", "k_rvq", "v_pq", "v_rvq")}
    for n in ("k_rvq", "v_rvq"):
        cbs[n] = (cbs[n].astype(F32) * 0.35).astype(np.float16)
    warm, dec = {}, {}
    for s in ("k", "v"):
        x = randn16(g, Hkv * T, D)
        e = nx.ext_encode(x, cbs[s + "_pq"], cbs[s + "_rvq"], 4)
        dec[s] = nx.ext_decode(e["pq_codes"], cbs[s + "_pq"], e["rvq_codes"], cbs[s + "_rvq"], e["sparse_idx"],
                               e["sparse_val"]).reshape(Hkv, T, D).transpose(1, 0, 2)
        warm[s] = {"pq": e["pq_codes"].reshape(Hkv, T, -1), "rvq": e["rvq_codes"].reshape(Hkv, T, -1),
                   "sparse_idx": e["sparse_idx"].reshape(Hkv, T, -1), "sparse_val": e["sparse_val"].reshape(Hkv, T, -1)}
    hot_k, hot_v = randn16(g, Hkv, Th, D), randn16(g, Hkv, Th, D)  # [Hkv, T_hot, D] as the bench holds them
    q = randn16(g, 1, Hq, D, scale=2.0)
    want = nx.dense_attention_f64(q, np.concatenate([dec["k"], hot_k.transpose(1, 0, 2)]),
                                  np.concatenate([dec["v"], hot_v.transpose(1, 0, 2)]), 0.125)
    tw = {s: {k: torch.from_numpy(v) for k, v in warm[s].items()} for s in ("k", "v")}
    got = fn(torch.from_numpy(q), torch.from_numpy(hot_k), torch.from_numpy(hot_v), tw["k"], tw["v"],
             {k: torch.from_numpy(v) for k, v in cbs.items()}, 0.125, 32).numpy()
    return float(np.abs(got.astype(np.float64) - want).max()) <= 1e-3


def test_cpu_baseline_decode_steps_pinned():
    """The three timed decode baselines against the pinned oracle: the
    reference-format decode bit for bit, both decode steps within fp32
    rounding of textbook attention over the oracle-decoded window."""
    from oracle import cpu_baseline as cb

    assert check_ref_decode(cb.ref_decode, rng(31))
    assert check_ref_decode_step(cb.ref_decode_step, rng(32))
    assert check_decode_step(cb.decode_step, rng(33))


def test_cpu_baseline_planted_mistakes():
    """Each baseline pin rejects a plausible mistake planted in the baseline."""
    import torch
    import torch.nn.functional as F

    from oracle import cpu_baseline as cb

    def ref_decode_shuffled(pq, pq_cb, rvq, offsets, rvq_cb):  # corrections scattered to the wrong rows
        return cb.ref_decode(pq, pq_cb, rvq, torch.roll(offsets, 1), rvq_cb)

    def ref_decode_f16_sum(pq, pq_cb, rvq, offsets, rvq_cb):  # stage sum rounded to fp16 at every stage
        base = cb.decode_codes(pq, pq_cb)
        corr = torch.zeros_like(base)
        if rvq.shape[0]:
            tot = torch.zeros((rvq.shape[0], base.shape[1]), dtype=torch.float16)
            for layer in range(rvq.shape[1]):
                tot = (tot.float() + F.embedding(rvq[:, layer].long(), rvq_cb[layer]).float()).half()
            corr[offsets.long()] = tot
        return (base.float() + corr.float()).half()

    def ref_decode_no_base(pq, pq_cb, rvq, offsets, rvq_cb):  # the correction alone on active rows
        out = cb.ref_decode(pq, pq_cb, rvq, offsets, rvq_cb)
        out[offsets.long()] = (out[offsets.long()].float() - cb.decode_codes(pq, pq_cb)[offsets.long()].float()).half()
        return out

    for bad in (ref_decode_shuffled, ref_decode_f16_sum, ref_decode_no_base):
        assert not check_ref_decode(bad, rng(31)), bad.__name__

    def swapped_kv(q, hot_k, hot_v, warm_k, warm_v, cbs, scale, block):  # V decoded with K's codebooks
        return cb.decode_step(q, hot_k, hot_v, warm_k, warm_v,
                              dict(cbs, v_pq=cbs["k_pq"], v_rvq=cbs["k_rvq"], k_pq=cbs["v_pq"], k_rvq=cbs["v_rvq"]),
                              scale, block)

    def no_sparse(q, hot_k, hot_v, warm_k, warm_v, cbs, scale, block):  # sparse stage dropped
        strip = lambda w: {k: v for k, v in w.items() if not k.startswith("sparse")}
        return cb.decode_step(q, hot_k, hot_v, strip(warm_k), strip(warm_v), cbs, scale, block)

    for bad in (swapped_kv, no_sparse):
        assert not check_decode_step(bad, rng(33)), bad.__name__

    def ref_step_values_as_keys(q, hot_k, hot_v, warm_k, warm_v, cbs, scale, block):
        return cb.ref_decode_step(q, hot_k, hot_v, warm_k, warm_k, cbs, scale, block)

    real_attn = cb.blockwise_attention

    def interleaved_gqa(q, keys, values, scale, block):  # kv head h % Hkv instead of h // rep
        rep = q.shape[1] // keys.shape[1]
        return real_attn(q, keys.repeat(1, rep, 1), values.repeat(1, rep, 1), scale, block)

    assert not check_ref_decode_step(ref_step_values_as_keys, rng(32))
    try:
        cb.blockwise_attention = interleaved_gqa
        assert not check_ref_decode_step(cb.ref_decode_step, rng(32))
        assert not check_decode_step(cb.decode_step, rng(33))
    finally:
        cb.blockwise_attention = real_attn


def _ref_encode_le(x, pq_cb, rvq_cb, threshold):
    """cpu_baseline.ref_encode with a planted mistake: the chunk merge written
    with <= (a tie moves to the later chunk) instead of the reference's <."""
    import torch

    from oracle import cpu_baseline as cb

    pqc, r1 = cb.pq_encode_cdist(x, pq_cb)
    rr = r1.float()
    m = torch.sqrt((rr * rr).sum(dim=1)) > threshold
    o = torch.nonzero(m).flatten().to(torch.int32)
    run = rr[o.long()]
    Ln, Cn, _ = rvq_cb.shape
    out = torch.zeros((run.shape[0], Ln), dtype=torch.int64)
    for layer in range(Ln):
        c_all = rvq_cb[layer].float()
        x2 = (run * run).sum(dim=1, keepdim=True)
        best = torch.full((run.shape[0],), float("inf"))
        idx = torch.zeros((run.shape[0],), dtype=torch.int64)
        for s0 in range(0, Cn, 512):
            c = c_all[s0:s0 + 512]
            d = (x2 - 2.0 * run @ c.T) + (c * c).sum(dim=1)[None, :]
            lb, li = d.min(dim=1)
            upd = lb <= best
            best = torch.where(upd, lb, best)
            idx = torch.where(upd, li + s0, idx)
        out[:, layer] = idx
        run = run - c_all[idx]
    return pqc, out, m, o


def test_cpu_baseline_ref_encode_matches_oracle():
    """The timed torch-CPU reference-format encode (cdist^2 PQ, norm gate,
    chunked (|x|^2 - 2xc) + |c|^2 stages) gives the oracle's PQ codes, mask,
    offsets and every stage's code on data without near-ties, across three
    512-centroid chunks; with a planted mistake (the chunk merge keeping the
    later index on ties) it differs on a row that ties two chunks."""
    import torch

    from oracle import cpu_baseline as cb

    g = np.random.default_rng(8)
    x = (g.standard_normal((160, 64)) * np.linspace(0.5, 2.0, 64)).astype(np.float16)
    p = (g.standard_normal((4, 256, 16)) * 0.5).astype(np.float16)
    for i in range(20):  # rows that are PQ centroids exactly: zero residual, gated off
        x[i] = p[np.arange(4), g.integers(0, 256, 4)].reshape(-1)
    r = (g.standard_normal((3, 1536, 64)) * 0.25).astype(np.float16)
    r[:, 0] = 0
    r[:, 1100] = r[:, 77]  # a duplicate in a later chunk: the first index must win
    # a row whose PQ residual is exactly centroid 77 of stage 0
    x[20] = (p[np.arange(4), [3, 4, 5, 6]].reshape(-1).astype(np.float32)
             + r[0, 77].astype(np.float32)).astype(np.float16)
    args = (torch.from_numpy(x), torch.from_numpy(p), torch.from_numpy(r), 0.005)
    pq, codes, mask, offs = cb.ref_encode(*args)
    rp, rc, rm, ro = nx.hybrid_encode(x, p, r, 0.005)
    assert np.array_equal(pq.numpy(), rp)
    assert np.array_equal(mask.numpy(), rm) and not rm[:20].any()
    assert np.array_equal(offs.numpy(), ro)
    assert np.array_equal(codes.numpy(), rc.astype(np.int64))
    assert 77 in rc[:, 0] and 1100 not in rc[:, 0]
    _, bad, _, _ = _ref_encode_le(*args)
    assert not np.array_equal(bad.numpy(), rc.astype(np.int64))
