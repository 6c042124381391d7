"""GPU parity of every HIP kernel against the CPU oracle (bit-exact codes and
reconstructions; attention within 2e-3 max-abs on fp16 outputs)."""

import numpy as np
import pytest
import torch

from oracle import numerics as nx
from tests.conftest import rand_codebooks, randn16, rng

pytestmark = pytest.mark.gpu

TOL = 2e-3


def T(a, dev):
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).view(torch.uint16).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def H(t):
    t = t.detach().cpu()
    if t.dtype == torch.uint16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


@pytest.mark.parametrize("M,d,C,n", [(8, 8, 256, 1000), (16, 4, 256, 777), (8, 16, 256, 300), (4, 16, 100, 129)])
def test_pq_encode_bit_exact(device, M, d, C, n):
    from apple_amd import kernels as K

    g = rng(11 + M + d)
    x = randn16(g, n, M * d)
    cb = rand_codebooks(g, M, C, d)
    codes, resid = K.pq_encode(T(x, device), T(cb, device))
    rc, rr = nx.pq_encode(x, cb)
    assert np.array_equal(H(codes), rc)
    assert np.array_equal(H(resid).view(np.uint16), rr.view(np.uint16))


def test_pq_encode_known_answers(device):
    """Rows equal to centroids return those centroids; duplicated rows return
    the lowest index; a zero vector against a zero row 0 returns 0."""
    from apple_amd import kernels as K

    g = rng(5)
    cb = rand_codebooks(g, 4, 64, 4)
    cb[:, 10] = cb[:, 3]  # duplicate centroid 3 at index 10
    pick = np.array([3, 10, 0, 63, 17, 10])
    x = np.concatenate([cb[m][pick] for m in range(4)], axis=1)
    codes, resid = K.pq_encode(T(x, device), T(cb, device))
    want = np.where(pick == 10, 3, pick)
    assert np.array_equal(H(codes), np.repeat(want[:, None], 4, axis=1))
    assert not H(resid).any()
    cb0 = cb.copy()
    cb0[:, 0] = 0
    zc, _ = K.pq_encode(T(np.zeros((5, 16), np.float16), device), T(cb0, device))
    assert not H(zc).any()


@pytest.mark.parametrize("d", [4, 8])
@pytest.mark.parametrize("C", [1, 16, 100, 256])
def test_pq_encode_screening_paths(device, d, C):
    """The MFMA search (d = 4, 8) through each of its decisions: a unique
    screened minimum, duplicated centroids (two exact ties), a triplicated
    centroid and exactly equidistant centroid pairs (wider near-ties), vectors
    whose |x|^2 / 2 overflows fp16, and codebooks with |c|^2 / 2 beyond fp16;
    codes and residuals bit-exact against the oracle."""
    from apple_amd import kernels as K

    g = rng(300 + 7 * d + C)
    M = 4
    cb = rand_codebooks(g, M, C, d)
    rows = [randn16(g, 64, M * d)]
    if C >= 16:
        cb[:, 5] = cb[:, 2]                      # a pair
        cb[:, 9] = cb[:, 2]                      # ... a triple
        cb[:, C - 1] = cb[:, 7]                  # a pair across chunks
        rows.append(np.concatenate([cb[m][[2, 7, 9, 5, 0, C - 1]] for m in range(M)], axis=1))
        # centroids 11, 12 at exactly +-delta from a vector along coordinate 0
        base = randn16(g, 1, d)[0]
        delta = np.float16(0.25)
        for m in range(M):
            cb[m, 11] = base
            cb[m, 12] = base
            cb[m, 11, 0] = base[0] + delta
            cb[m, 12, 0] = base[0] - delta
        rows.append(np.tile(base, (3, M)))
        # near the pair, perturbed in the last fp16 bit
        near = np.tile(base, (8, M)).view(np.uint16)
        near[np.arange(8), np.arange(8) % (M * d)] ^= 1
        rows.append(near.view(np.float16))
    rows.append((randn16(g, 16, M * d).astype(np.float32) * 300.0).astype(np.float16))  # L / 2 > 65504
    x = np.concatenate(rows, 0)
    codes, resid = K.pq_encode(T(x, device), T(cb, device))
    rc, rr = nx.pq_encode(x, cb)
    assert np.array_equal(H(codes), rc)
    assert np.array_equal(H(resid).view(np.uint16), rr.view(np.uint16))
    big = cb.copy()
    big[:, 0] = (big[:, 0].astype(np.float32) * 200.0).astype(np.float16)  # R / 2 > 60000 for centroid 0
    codes, resid = K.pq_encode(T(x, device), T(big, device))
    rc, rr = nx.pq_encode(x, big)
    assert np.array_equal(H(codes), rc)
    assert np.array_equal(H(resid).view(np.uint16), rr.view(np.uint16))


@pytest.mark.parametrize("M,Mr,k", [(16, 16, 4), (8, 8, 4), (8, 0, 0), (16, 16, 0), (16, 0, 4)])
def test_warm_encode_bit_exact(device, M, Mr, k):
    from apple_amd import kernels as K

    g = rng(100 + M + Mr + k)
    n, D = 901, 64
    x = (randn16(g, n, D).astype(np.float32) * np.linspace(0.5, 2.0, D, dtype=np.float32)).astype(np.float16)
    pq_cb = rand_codebooks(g, M, 256, D // M)
    rvq_cb = rand_codebooks(g, Mr, 256, D // Mr) * np.float16(0.3) if Mr else None
    fmt = K.WarmFormat(D, M, 256, Mr, 256 if Mr else 0, k)
    out = K.warm_encode(T(x, device), fmt, T(pq_cb, device), None if rvq_cb is None else T(rvq_cb, device))
    ref = nx.ext_encode(x, pq_cb, rvq_cb, k)
    assert np.array_equal(H(out["pq"]), ref["pq_codes"])
    if Mr:
        assert np.array_equal(H(out["rvq"]), ref["rvq_codes"])
    if k:
        assert np.array_equal(H(out["sparse_idx"]), ref["sparse_idx"])
        assert np.array_equal(H(out["sparse_val"]).view(np.uint16), ref["sparse_val"].view(np.uint16))
    # decode round trip, bit-exact
    dec = K.decode(fmt, out["pq"], T(pq_cb, device), out.get("rvq"), None if rvq_cb is None else T(rvq_cb, device),
                   out.get("sparse_idx"), out.get("sparse_val"))
    rdec = nx.ext_decode(ref["pq_codes"], pq_cb, ref.get("rvq_codes"), rvq_cb, ref.get("sparse_idx"),
                         ref.get("sparse_val"))
    assert np.array_equal(H(dec).view(np.uint16), rdec.view(np.uint16))


@pytest.mark.parametrize("d", [4, 8])
@pytest.mark.parametrize("C", [1, 16, 100, 256])
def test_warm_encode_screening_paths(device, d, C):
    """The one-launch warm encode (PQ, RVQ on the register-resident residual,
    top-4) through each decision of its search, in both stages: duplicated,
    triplicated and exactly equidistant centroids, vectors near them, |x|^2/2
    beyond fp16, codebooks shorter than 256 and |c|^2/2 beyond fp16; codes
    and sparse entries bit-exact against the oracle."""
    from apple_amd import kernels as K

    g = rng(700 + 7 * d + C)
    D = 64
    M = D // d
    cb = rand_codebooks(g, M, C, d)
    rcb = rand_codebooks(g, M, C, d) * np.float16(0.3)
    rows = [randn16(g, 200, D)]
    if C >= 16:
        for c in (cb, rcb):
            c[:, 5] = c[:, 2]
            c[:, 9] = c[:, 2]
            c[:, C - 1] = c[:, 7]
        rows.append(np.concatenate([cb[m][[2, 7, 9, 5, 0, C - 1]] for m in range(M)], axis=1))
        base = randn16(g, 1, d)[0]
        for m in range(M):
            cb[m, 11] = base
            cb[m, 12] = base
            cb[m, 11, 0] = base[0] + np.float16(0.25)
            cb[m, 12, 0] = base[0] - np.float16(0.25)
        rows.append(np.tile(base, (3, M)))
        near = np.tile(base, (8, M)).view(np.uint16)
        near[np.arange(8), np.arange(8) % D] ^= 1
        rows.append(near.view(np.float16))
    rows.append((randn16(g, 16, D).astype(np.float32) * 300.0).astype(np.float16))  # L / 2 > 65504
    x = np.concatenate(rows, 0)
    for pq_cb in (cb, None):
        if pq_cb is None:  # R / 2 beyond fp16 for centroid 0 of every subspace
            pq_cb = cb.copy()
            pq_cb[:, 0] = (pq_cb[:, 0].astype(np.float32) * 200.0).astype(np.float16)
        fmt = K.WarmFormat(D, M, C, M, C, 4)
        out = K.warm_encode(T(x, device), fmt, T(pq_cb, device), T(rcb, device))
        ref = nx.ext_encode(x, pq_cb, rcb, 4)
        assert np.array_equal(H(out["pq"]), ref["pq_codes"])
        assert np.array_equal(H(out["rvq"]), ref["rvq_codes"])
        assert np.array_equal(H(out["sparse_idx"]), ref["sparse_idx"])
        assert np.array_equal(H(out["sparse_val"]).view(np.uint16), ref["sparse_val"].view(np.uint16))


def test_warm_encode_batch_one_launch(device):
    """A chunk's K and V (and a third set, and an empty one) in one launch:
    the same codes, bit for bit, as separate warm_encode calls and the oracle;
    a format the one-launch encode does not serve is refused."""
    from apple_amd import kernels as K

    g = rng(811)
    fmt = K.WarmFormat(64, 16, 256, 16, 256, 4)
    sets = []
    for n in (1000, 777, 33, 0):
        x = (randn16(g, n, 64).astype(np.float32) * np.linspace(0.5, 2.0, 64, dtype=np.float32)).astype(np.float16)
        sets.append((x, rand_codebooks(g, 16, 256, 4), rand_codebooks(g, 16, 256, 4) * np.float16(0.3)))
    outs = K.warm_encode_batch([(T(x, device), T(p, device), T(r, device)) for x, p, r in sets], fmt)
    for (x, p, r), out in zip(sets, outs):
        one = K.warm_encode(T(x, device), fmt, T(p, device), T(r, device))
        for key in ("pq", "rvq", "sparse_idx", "sparse_val"):
            assert np.array_equal(H(out[key]).view(np.uint8), H(one[key]).view(np.uint8)), key
        if len(x):
            ref = nx.ext_encode(x, p, r, 4)
            assert np.array_equal(H(out["pq"]), ref["pq_codes"]) and np.array_equal(H(out["rvq"]), ref["rvq_codes"])
            assert np.array_equal(H(out["sparse_val"]).view(np.uint16), ref["sparse_val"].view(np.uint16))
    with pytest.raises(RuntimeError, match="one-launch encode"):
        K.warm_encode_batch([(T(sets[0][0], device), T(rand_codebooks(g, 4, 256, 16), device), None)],
                            K.WarmFormat(64, 4, 256, 0, 0, 0))


@pytest.mark.parametrize("M,Mr", [(16, 16), (8, 8), (16, 0)])
def test_sparse_fold_bit_exact(device, M, Mr):
    """Corrected coordinates fp16(K[idx] + val) equal the warm decode's value
    at each sparse index."""
    from apple_amd import kernels as K

    g = rng(200 + M + Mr)
    n, D, k = 517, 64, 4
    x = randn16(g, n, D)
    pq_cb = rand_codebooks(g, M, 256, D // M)
    rvq_cb = rand_codebooks(g, Mr, 256, D // Mr) * np.float16(0.3) if Mr else None
    fmt = K.WarmFormat(D, M, 256, Mr, 256 if Mr else 0, k)
    ref = nx.ext_encode(x, pq_cb, rvq_cb, k)
    dec = nx.ext_decode(ref["pq_codes"], pq_cb, ref.get("rvq_codes"), rvq_cb, ref["sparse_idx"], ref["sparse_val"])
    want = np.take_along_axis(dec, ref["sparse_idx"].astype(np.int64), axis=1)
    got = K.sparse_fold(fmt, T(ref["pq_codes"], device), T(pq_cb, device),
                        T(ref["rvq_codes"], device) if Mr else None, T(rvq_cb, device) if Mr else None,
                        T(ref["sparse_idx"], device), T(ref["sparse_val"], device))
    assert np.array_equal(H(got).view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("Mr", [16, 0])
def test_sparse_delta_bit_exact(device, Mr):
    """Score deltas fp16(c - (base[idx] + rvq[idx])) equal the oracle's."""
    from apple_amd import kernels as K

    g = rng(230 + Mr)
    n, D, k, M = 611, 64, 4, 16
    x = randn16(g, n, D)
    pq_cb = rand_codebooks(g, M, 256, D // M)
    rvq_cb = rand_codebooks(g, Mr, 256, D // Mr) * np.float16(0.3) if Mr else None
    fmt = K.WarmFormat(D, M, 256, Mr, 256 if Mr else 0, k)
    ref = nx.ext_encode(x, pq_cb, rvq_cb, k)
    want = nx.score_delta(ref["pq_codes"], pq_cb, ref.get("rvq_codes"), rvq_cb, ref["sparse_idx"],
                          ref["sparse_val"])
    got = K.sparse_fold(fmt, T(ref["pq_codes"], device), T(pq_cb, device),
                        T(ref["rvq_codes"], device) if Mr else None, T(rvq_cb, device) if Mr else None,
                        T(ref["sparse_idx"], device), T(ref["sparse_val"], device), delta=True)
    assert np.array_equal(H(got).view(np.uint16), want.view(np.uint16))


def test_pack_score_codes_bit_exact(device):
    """pack_score_codes writes the score-table K layout (appends at any token
    base) and unpack_score_codes inverts it."""
    from apple_amd import kernels as K
    from tests.conftest import score_layout

    g = rng(19)
    Hh, Tt, k = 3, 133, 4
    pq = g.integers(0, 256, (Hh, Tt, 16)).astype(np.uint8)
    rv = g.integers(0, 256, (Hh, Tt, 16)).astype(np.uint8)
    si = g.integers(0, 64, (Hh, Tt, k)).astype(np.uint8)
    sv = randn16(g, Hh, Tt, k)
    cap = K.round_up(Tt + 40, 32)
    dst = {"pq": torch.zeros((Hh, cap * 16), dtype=torch.uint8, device=device),
           "sparse_idx": torch.zeros((Hh, cap, k), dtype=torch.uint8, device=device),
           "sparse_val": torch.zeros((Hh, cap, k), dtype=torch.float16, device=device)}
    dst["rvq"] = torch.zeros_like(dst["pq"])
    for a, b in ((0, 50), (50, Tt)):
        K.pack_score_codes(T(pq[:, a:b], device), T(rv[:, a:b], device), T(si[:, a:b], device), T(sv[:, a:b], device),
                           dst, a)
    for h in range(Hh):
        wp, wr, wi, wv = score_layout(pq[h], rv[h], si[h], sv[h], 0, cap)
        assert np.array_equal(H(dst["pq"][h]), wp) and np.array_equal(H(dst["rvq"][h]), wr)
        assert np.array_equal(H(dst["sparse_idx"][h]).reshape(-1), wi)
        assert np.array_equal(H(dst["sparse_val"][h]).reshape(-1).view(np.uint16), wv.view(np.uint16))
    up, ur, ui, uv = K.unpack_score_codes(dst, Tt)
    assert np.array_equal(H(up), pq) and np.array_equal(H(ur), rv) and np.array_equal(H(ui), si)


@pytest.mark.parametrize("n,M,d", [(40_000, 16, 4), (3_000, 8, 8), (5, 16, 4)])
def test_kmeans_update_matches_oracle(device, n, M, d):
    """One Lloyd update on the GPU equals the oracle's member mean (float64
    sums, fp32 mean, fp16 row) up to one fp16 ulp, with nearly every row
    bit-exact; empty clusters keep their rows."""
    from apple_amd import kernels as K
    from oracle import kmeans as km

    g = rng(40 + n)
    D, C = M * d, 256
    x = randn16(g, n, D)
    cb = rand_codebooks(g, M, C, d)
    codes, _ = nx.pq_encode(x, cb)
    want = km.centroid_update(x, codes, cb)
    got = T(cb, device)
    K.kmeans_update(T(x, device), T(codes, device), got)
    got = H(got)
    diff = np.abs(got.view(np.uint16).astype(np.int32) - want.view(np.uint16).astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() >= 0.999, (diff.max(), (diff == 0).mean())
    empty = np.ones((M, C), bool)
    for m in range(M):
        empty[m, np.unique(codes[:, m])] = False
    assert np.array_equal(got[empty].view(np.uint16), cb[empty].view(np.uint16))


def test_fit_codebooks_distortion_non_increasing(device):
    """The GPU k-means fit (calibrate_quantizer's loop): distortion of the
    old codes under the new centroids never rises."""
    from apple_amd.calibrate import fit_codebooks

    g = rng(44)
    x = torch.from_numpy(randn16(g, 20_000, 64)).to(device)
    _, met = fit_codebooks(x, 16, 256, 6, torch.Generator().manual_seed(3))
    d = met["avg_distortion"]
    assert all(b <= a + 1e-6 for a, b in zip(d, d[1:])), d


@pytest.mark.parametrize("thr", [0.25, 5.0, float("inf"), 0.0])
def test_rvq_full_bit_exact(device, thr):
    from apple_amd import kernels as K

    g = rng(7)
    n, D, L, C = 300, 128, 3, 256
    resid = np.concatenate([randn16(g, n // 2, D, scale=0.01), randn16(g, n - n // 2, D)], 0)
    cb = rand_codebooks(g, L, C, D)
    cb[:, 0] = 0
    codes, mask, offs = K.rvq_encode_full(T(resid, device), T(cb, device), thr)
    rc, rm, ro = nx.rvq_encode_full(resid, cb, thr)
    assert np.array_equal(H(mask), rm)
    assert np.array_equal(H(offs), ro)
    assert np.array_equal(H(codes), rc)
    # reference hybrid decode
    pq_cb = rand_codebooks(g, 8, 256, 16)
    pq = g.integers(0, 256, (n, 8)).astype(np.uint8)
    dec = K.decode_ref(T(pq, device), T(pq_cb, device), T(rc, device), T(ro, device), T(cb, device))
    rdec = nx.hybrid_decode(pq, rc, rm, ro, pq_cb, cb)
    assert np.array_equal(H(dec).view(np.uint16), rdec.view(np.uint16))


def _planted_rvq_case(g, n, D, L, C):
    """Reference-default RVQ codebooks (row 0 zeroed) with ties planted
    across the 512-centroid chunks that ResidualVQMLX.encode merges with a
    strict < (quantization.py:233-246): exact duplicates at j and j + 512 m,
    and sign-flipped copies whose distance to a vector equals the original's
    (placed above and below it); the vectors hit those ties in stage 0, plus
    random residuals at two scales."""
    cb = rand_codebooks(g, L, C, D)
    cb[:, 0] = 0
    x = np.concatenate([randn16(g, (n - 48) // 2, D, scale=0.015), randn16(g, n - 48 - (n - 48) // 2, D)], 0)
    picks = []
    for layer in range(L):
        for i, j in enumerate(range(3, 3 + 24)):
            m = 1 + (i % ((C - 1 - j) // 512))
            dup = j + 512 * m
            cb[layer, dup] = cb[layer, j]                        # exact duplicate in a later chunk
            flip = j + 512 * ((m + 1) % (C // 512)) + 100        # sign-flipped copy, later or earlier chunk
            cb[layer, flip] = cb[layer, j]
            cb[layer, flip, :8] = -cb[layer, j, :8]
            if layer == 0:
                picks.append(j)
    rows = []
    for j in picks:
        rows.append(cb[0, j].copy())                            # ties with its duplicate: distance 0
        r = cb[0, j].copy()
        r[:8] = 0                                               # equidistant from c_j and its flipped copy
        rows.append(r)
    x = np.concatenate([x, np.stack(rows)], 0)
    assert x.shape[0] == n
    return x.astype(np.float16), cb


@pytest.mark.parametrize("thr", [0.005, 0.25])
def test_rvq_full_reference_default_shape(device, thr):
    """ResidualVQMLX.encode at the reference's default shape (C = 4,096,
    L = 4, D = 128; storage.py:25, 33-34) with ties planted across the
    512-centroid chunks: mask, offsets and every stage's code bit-exact
    against the oracle's global first-min, which equals the reference's
    chunked strict-< merge."""
    from apple_amd import kernels as K

    g = rng(70 + int(thr * 1000))
    n, D, L, C = 512, 128, 4, 4096
    resid, cb = _planted_rvq_case(g, n, D, L, C)
    codes, mask, offs = K.rvq_encode_full(T(resid, device), T(cb, device), thr)
    rc, rm, ro = nx.rvq_encode_full(resid, cb, thr)
    assert rm.sum() > n // 2
    assert np.array_equal(H(mask), rm)
    assert np.array_equal(H(offs), ro)
    got = H(codes)
    assert np.array_equal(got, rc), np.argwhere(got != rc)[:8]
    # the planted tie rows took the lower index in stage 0
    tied = [i for i in range(n - 48, n) if rm[i]]
    pos = np.searchsorted(ro, tied)
    assert (rc[pos, 0] < 512).all()


def _qpos_cases(B, Hq, T_):
    g = rng(3)
    return [None, g.integers(-1, T_, (B, Hq)).astype(np.int32)]


@pytest.mark.parametrize("Hq,Hkv,D,T_", [(8, 8, 64, 1024), (32, 8, 64, 3000), (4, 4, 128, 60), (32, 4, 64, 777),
                                         (16, 8, 128, 1)])
def test_blockwise_attention(device, Hq, Hkv, D, T_):
    from apple_amd import kernels as K

    g = rng(Hq + Hkv + D + T_)
    B = 2
    q = randn16(g, B, Hq, D)
    k = randn16(g, T_, Hkv, D)
    v = randn16(g, T_, Hkv, D)
    for causal in (False, True):
        for qp in _qpos_cases(B, Hq, T_):
            out = K.blockwise_attention(T(q, device), T(k, device), T(v, device), D ** -0.5, causal,
                                        None if qp is None else T(qp, device))
            ref = nx.blockwise_attention(q, k, v, D ** -0.5, 128, causal, qp)
            err = np.abs(H(out).astype(np.float32) - ref.astype(np.float32)).max()
            assert err <= TOL, (causal, qp is None, err)


def test_pack_untile_roundtrip(device):
    from apple_amd import kernels as K
    from apple_amd.batched import untile

    g = rng(9)
    for M in (8, 16):
        Hh, Tt = 3, 133
        src = g.integers(0, 256, (Hh, Tt, M)).astype(np.uint8)
        cap = K.round_up(Tt + 40, 32)
        dst = torch.zeros((Hh, cap * M), dtype=torch.uint8, device=device)
        K.pack_codes(T(src[:, :50], device), dst, 0)
        K.pack_codes(T(src[:, 50:], device), dst, 50)
        assert np.array_equal(H(untile(dst, M, Tt)), src)
