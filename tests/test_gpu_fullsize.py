"""Parity at the benchmark workloads' full sizes, against the oracle.

* encode_4k: one 4,096-token x 8-head chunk of K and of V (65,536 vectors)
  through the MFMA encode, every code and sparse entry bit-exact.
* batched_32x32k: 32 sequences x 32,768 tokens (1,024 exact + 31,744
  PQ+RVQ+top-4), GPU-fitted per-sequence codebooks as in the benchmark;
  codes bit-exact on a seeded sample of 4,096 rows per sequence (K and V),
  and the fused attention of all 32 sequences at the benchmark's launch
  shape (256 blocks, one split) within 2e-3 of the oracle's blockwise
  attention over the oracle's decode of the cache's codes.
* longctx_128k: one 131,072-token sequence (1,024 exact, 15,360 warm,
  224 pinned 512-token cold chunks), the router's 16 nearest chunks; codes
  bit-exact on a seeded sample, and the attention over the 24,576-token
  window within 2e-3 of the oracle with the chunks resident, copied in
  during the step, and prefetched one step ahead.

The oracle runs in a thread pool (numpy releases the GIL in its array work).
"""

import concurrent.futures as cf

import numpy as np
import pytest
import torch

from oracle import numerics as nx

pytestmark = pytest.mark.gpu

TOL = 2e-3
THREADS = 8


def _pool():
    return cf.ThreadPoolExecutor(THREADS)


def _np(t):
    return None if t is None else t.detach().cpu().numpy()


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float16:
        a, b = a.view(np.uint16), b.view(np.uint16)
    return a.shape == b.shape and np.array_equal(a, b)


def _check_codes(got: dict, ref: dict, what: str) -> None:
    pairs = (("pq", "pq_codes"), ("rvq", "rvq_codes"), ("sparse_idx", "sparse_idx"), ("sparse_val", "sparse_val"))
    for g, r in pairs:
        if ref.get(r) is None:
            continue
        bad = np.nonzero(~(np.asarray(got[g]).view(np.uint8) == np.asarray(ref[r]).view(np.uint8)).all(axis=-1))[0]
        assert bad.size == 0, f"{what} {g}: {bad.size} rows differ (first {bad[:5]})"


def _err(out, ref):
    return float(np.abs(np.asarray(out, np.float32) - np.asarray(ref, np.float32)).max())


# --------------------------------------------------------------------------- encode_4k

def test_encode_4k_chunk_bit_exact(device):
    import bench
    from apple_amd import kernels as K
    from apple_amd.workloads import WORKLOADS, make_sequence

    w = WORKLOADS["encode_4k"]
    cfg = w.config()
    k, v, _, g = make_sequence(w, 0)
    kd, vd = k.to(device), v.to(device)
    kq = bench.fit_quantizer(cfg, kd, g, w, device)
    vq = bench.fit_quantizer(cfg, vd, g, w, device)
    fmt = kq.warm_format()
    assert (fmt.pq_subspaces, fmt.rvq_subspaces, fmt.sparse_k) == (8, 8, 4)
    with _pool() as ex:
        for name, x, qz in (("K", kd, kq), ("V", vd, vq)):
            flat = x.reshape(-1, w.head_dim).contiguous()
            assert flat.shape[0] == 4096 * 8
            got = {n: _np(t) for n, t in K.warm_encode(flat, fmt, qz.pq.codebooks, qz.rvq.codebooks).items()}
            xs = _np(flat)
            pcb, rcb = _np(qz.pq.codebooks), _np(qz.rvq.codebooks)
            parts = list(ex.map(lambda a: nx.ext_encode(xs[a:a + 4096], pcb, rcb, 4), range(0, xs.shape[0], 4096)))
            ref = {n: np.concatenate([p[n] for p in parts], 0) for n in parts[0]}
            _check_codes(got, ref, f"encode_4k {name}")


# --------------------------------------------------------------------------- batched_32x32k

@pytest.fixture(scope="module")
def batched(device):
    import bench
    from apple_amd.workloads import WORKLOADS

    w = WORKLOADS["batched_32x32k"]
    cache, q = bench.setup_decode(w, device)
    yield w, cache, q
    del cache
    torch.cuda.empty_cache()


def test_batched_32x32k_codes_bit_exact(batched):
    """Sequence 0: every warm row of K and V (2 x 253,952 vectors); the
    other 31 sequences: 4,096 sampled rows each of K and V."""
    from apple_amd.workloads import make_sequence

    w, cache, _ = batched
    sample = 4096
    jobs = []
    for b in range(w.batch):
        k, v, _, _ = make_sequence(w, b)
        nw = cache.num_warm[b]
        assert nw == w.warm and cache.num_hot[b] == w.hot
        if b == 0:
            pick = np.arange(nw * w.kv_heads)
        else:
            pick = np.random.default_rng(1000 + b).choice(nw * w.kv_heads, sample, replace=False)
        h, t = pick // nw, pick % nw  # head-major rows of the warm tier
        for kv, x in (("k", k), ("v", v)):
            codes = {n: _np(c) for n, c in cache.plain_codes(kv, b).items()}
            got = {n: c[h, t] for n, c in codes.items()}
            rows = x.numpy()[t, h]
            cbs = (_np(cache.cb[f"{kv}_pq"][b]), _np(cache.cb[f"{kv}_rvq"][b]))
            for a in range(0, len(pick), sample):  # oracle work in pieces of 4,096 rows
                jobs.append((f"seq {b} {kv} rows {a}..", rows[a:a + sample], cbs,
                             {n: c[a:a + sample] for n, c in got.items()}))
    with _pool() as ex:
        refs = list(ex.map(lambda j: nx.ext_encode(j[1], j[2][0], j[2][1], w.sparse_k), jobs))
    for (what, _, _, got), ref in zip(jobs, refs):
        _check_codes(got, ref, what)


def test_batched_32x32k_fused_attention(batched):
    import ctypes

    from apple_amd import _lib as L

    w, cache, q = batched
    out = torch.empty_like(q)
    launch = cache.prepare(q, out=out)
    assert L.load().rfsn_fused_splits(ctypes.byref(launch.params)) == 1  # the benchmark's launch shape
    assert w.batch * w.kv_heads == 256
    launch()
    got = _np(out)
    qn = _np(q)

    def ref(b):
        dec = []
        for kv in ("k", "v"):
            c = {n: _np(t) for n, t in cache.plain_codes(kv, b).items()}
            H, nw, M = c["pq"].shape
            flat = lambda a: a.reshape(H * nw, -1)
            d = nx.ext_decode(flat(c["pq"]), _np(cache.cb[f"{kv}_pq"][b]), flat(c["rvq"]),
                              _np(cache.cb[f"{kv}_rvq"][b]), flat(c["sparse_idx"]), flat(c["sparse_val"]))
            hot = _np((cache.hot_k if kv == "k" else cache.hot_v)[b, :, :cache.num_hot[b]])
            dec.append(np.concatenate([d.reshape(H, nw, -1), hot], 1).transpose(1, 0, 2))
        return nx.blockwise_attention(qn[b:b + 1], dec[0], dec[1], w.head_dim ** -0.5, w.block)

    with _pool() as ex:
        refs = list(ex.map(ref, range(w.batch)))
    errs = [_err(got[b:b + 1], r) for b, r in enumerate(refs)]
    print(f"batched_32x32k max abs err per sequence: max {max(errs):.3g}", flush=True)
    assert max(errs) <= TOL, errs


# --------------------------------------------------------------------------- longctx_128k

@pytest.fixture(scope="module")
def longctx(device):
    import bench
    from apple_amd.cache import RFSNv10KVCacheMLX
    from apple_amd.storage import AsyncHierarchicalRouterMLX
    from apple_amd.workloads import WORKLOADS, make_sequence

    w = WORKLOADS["longctx_128k"]
    cfg = w.config()
    k, v, q, g = make_sequence(w, 0)
    kd, vd = k.to(device), v.to(device)
    kq = bench.fit_quantizer(cfg, kd[w.cold:w.cold + w.warm], g, w, device)
    vq = bench.fit_quantizer(cfg, vd[w.cold:w.cold + w.warm], g, w, device)
    cache = RFSNv10KVCacheMLX(cfg, device=device, cold_slots=max(32, w.cold_attended))
    cache.update(kd, vd, (kq, vq))
    torch.cuda.synchronize()
    del kd, vd
    router = AsyncHierarchicalRouterMLX(cfg).bind(cache)
    yield w, cache, router, k.numpy(), v.numpy(), q.numpy()[None]
    del cache
    torch.cuda.empty_cache()


def _store_codes(store):
    """Reference-layout store -> plain (pq, rvq, sparse_idx, sparse_val) [T, H, .] numpy."""
    return [_np(getattr(store, n)) for n in ("pq_codes", "rvq_codes", "sparse_idx", "sparse_val")]


def _longctx_window(w, cache, ids, k, v):
    """The oracle's window: chunks (ascending), warm, hot; encoded tokens
    decoded by the oracle from the cache's stored codes."""
    dec = {}
    for kv, qz in (("key", cache._kq), ("value", cache._vq)):
        stores = [cache.load_cold_chunk(c)[kv] for c in sorted(ids)]
        stores.append(cache.warm_keys if kv == "key" else cache.warm_values)
        parts = []
        for s in stores:
            pq, rvq, si, sv = _store_codes(s)
            T, Hh, _ = pq.shape
            flat = lambda a: a.reshape(T * Hh, -1)
            d = nx.ext_decode(flat(pq), _np(qz.pq.codebooks), flat(rvq), _np(qz.rvq.codebooks), flat(si), flat(sv))
            parts.append(d.reshape(T, Hh, -1))
        hot0 = w.context - cache.num_hot
        parts.append((k if kv == "key" else v)[hot0:])
        dec[kv] = np.concatenate(parts, 0)
    return dec["key"], dec["value"]


def test_longctx_128k_tiers_and_codes(longctx):
    w, cache, router, k, v, _ = longctx
    assert (cache.num_hot, cache.num_warm, cache.num_cold) == (w.hot, w.warm, w.cold)
    assert [m["chunk_id"] for m in cache.cold_chunk_metadata] == list(range(w.cold // w.cold_chunk))
    assert all(m["num_tokens"] == w.cold_chunk for m in cache.cold_chunk_metadata)
    assert len(cache.cold_chunk_metadata) == 224
    rng = np.random.default_rng(128)
    jobs = []
    # warm rows, and rows of 24 chunks spread over the cold tier
    for kind, cid in [("warm", None)] + [("cold", int(c)) for c in rng.choice(224, 24, replace=False)]:
        for kv, x, qz in (("key", k, cache._kq), ("value", v, cache._vq)):
            if kind == "warm":
                store, t0 = (cache.warm_keys if kv == "key" else cache.warm_values), w.cold
            else:
                store, t0 = cache.load_cold_chunk(cid)[kv], cid * w.cold_chunk
            pq, rvq, si, sv = _store_codes(store)
            T, Hh, _ = pq.shape
            n = min(2048 if kind == "warm" else 256, T * Hh)
            pick = rng.choice(T * Hh, n, replace=False)
            t, h = pick // Hh, pick % Hh
            got = {"pq": pq[t, h], "rvq": rvq[t, h], "sparse_idx": si[t, h], "sparse_val": sv[t, h]}
            jobs.append((f"{kind} {cid} {kv}", x[t0 + t, h], (_np(qz.pq.codebooks), _np(qz.rvq.codebooks)), got))
    with _pool() as ex:
        refs = list(ex.map(lambda j: nx.ext_encode(j[1], j[2][0], j[2][1], w.sparse_k), jobs))
    for (what, _, _, got), ref in zip(jobs, refs):
        _check_codes(got, ref, what)


def test_longctx_128k_window_modes(longctx):
    w, cache, router, k, v, q = longctx
    dev = cache.device
    ranked = router.rank(w.context - 1, w.context)
    sets = [ranked[:w.cold_attended], ranked[w.cold_attended:2 * w.cold_attended]]
    assert sets[0] == list(range(223, 207, -1))  # the 16 chunks nearest the newest token
    qd = torch.from_numpy(q).to(dev)
    scale = w.head_dim ** -0.5
    with _pool() as ex:
        refs = list(ex.map(lambda ids: nx.blockwise_attention(q, *_longctx_window(w, cache, ids, k, v), scale,
                                                              w.block), sets))
    window = cache.num_hot + cache.num_warm + w.cold_attended * w.cold_chunk
    assert window == 24576
    # chunks resident in device slots (one launch)
    cache.prefetch_cold_chunks(sets[0])
    out = cache.attention_forward(qd, causal=True, cold_chunks=sets[0])
    st = cache.get_last_access_stats()
    assert st["cold_chunks_touched"] == w.cold_attended
    e_res = _err(_np(out), refs[0])
    # every chunk copied in during the step (resident part || copies, then the copied part + merge)
    cache.evict_cold_slots()
    out = cache.attention_forward(qd, causal=True, cold_chunks=sets[0])
    e_copy = _err(_np(out), refs[0])
    # the next step's chunks prefetched during the current step, sets alternating
    cache.evict_cold_slots()
    outs = [torch.empty_like(qd), torch.empty_like(qd)]
    launches = []
    for i in range(2):
        cache.prefetch_cold_chunks(sets[i])
        launches.append(cache.prepare(qd, causal=True, cold_chunks=sets[i], out=outs[i]))
        cache.note_reads(sets[i])
    e_ahead = []
    for i in range(6):
        cache.wait_for_prefetch()
        launches[i % 2]()
        cache.note_reads(sets[i % 2])
        nxt = sets[(i + 1) % 2]
        cache.evict_cold_slots(nxt)
        cache.prefetch_cold_chunks(nxt, wait=False)
        torch.cuda.synchronize()
        e_ahead.append(_err(_np(outs[i % 2]), refs[i % 2]))
    cache.wait_for_prefetch()
    print(f"longctx_128k max abs err: resident {e_res:.3g} copied {e_copy:.3g} ahead {max(e_ahead):.3g}", flush=True)
    assert e_res <= TOL and e_copy <= TOL and max(e_ahead) <= TOL, (e_res, e_copy, e_ahead)
