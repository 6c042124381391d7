"""Host-side logic that needs no GPU: configuration checks, the NPZ chunk
schema (storage.py:113-151), the router's ranking over chunk files
(storage.py:166-201), query-position normalization (attention.py:16-36),
the tiled code layout, workload byte accounting and the bench contract."""

import json
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from apple_amd.storage import (AsyncHierarchicalRouterMLX, CompressedTensorMLX, RFSNConfig, _concat0, _index0,
                               chunk_file_path, compressed_tensor_from_loaded, load_compressed_chunk,
                               save_compressed_chunk)

ROOT = Path(__file__).resolve().parent.parent


def test_config_validation():
    with pytest.raises(ValueError):
        RFSNConfig(head_dim=64, num_subspaces=8, subspace_dim=4)
    c = RFSNConfig(num_heads=32, head_dim=64, num_subspaces=16, subspace_dim=4, num_kv_heads=8,
                   rvq_subspaces=16, sparse_topk=4)
    assert c.kv_heads == 8 and c.ext_format and c.subspace_rvq
    r = RFSNConfig(num_heads=4, head_dim=128, num_subspaces=8, subspace_dim=16)
    assert r.kv_heads == 4 and not r.ext_format
    assert r.chunk_tokens == r.block_size_seq
    with pytest.raises(ValueError):
        RFSNConfig(head_dim=64, num_subspaces=16, subspace_dim=4, cold_medium="tape")


def test_compressed_empty_and_uint16_helpers():
    cfg = RFSNConfig(num_heads=4, head_dim=128, num_subspaces=8, subspace_dim=16, num_rvq_layers=3)
    e = CompressedTensorMLX.empty(cfg)
    assert e.num_tokens == 0 and e.rvq_codes.dtype == torch.uint16 and e.rvq_codes.shape == (0, 3)
    a = torch.tensor([1, 65535, 7], dtype=torch.int32).to(torch.uint16)
    b = torch.tensor([40000], dtype=torch.int32).to(torch.uint16)
    ab = _concat0(a, b)
    assert ab.dtype == torch.uint16 and ab.to(torch.int32).tolist() == [1, 65535, 7, 40000]
    assert _concat0(a[:0], b) is b
    assert _index0(ab, torch.tensor([3, 1])).to(torch.int32).tolist() == [40000, 65535]


def test_npz_chunk_schema_roundtrip(tmp_path):
    g = torch.Generator().manual_seed(0)
    T, H, M, L = 5, 3, 8, 2

    def store():
        mask = torch.rand((T, H), generator=g) > 0.5
        A = int(mask.sum())
        return CompressedTensorMLX(
            pq_codes=torch.randint(0, 256, (T, H, M), generator=g, dtype=torch.uint8),
            rvq_codes=torch.randint(0, 65536, (A, L), generator=g, dtype=torch.int32).to(torch.uint16),
            rvq_mask=mask, rvq_offsets=torch.nonzero(mask.reshape(-1)).reshape(-1).to(torch.int32), num_heads=H)

    k, v = store(), store()
    p = chunk_file_path(tmp_path, 2, 7)
    assert p.name == "layer2_chunk7.npz"
    save_compressed_chunk(p, k, v)
    with np.load(p, allow_pickle=False) as z:
        assert sorted(z.files) == sorted(["num_tokens", "num_heads"] + [
            f"{s}_{f}" for s in ("key", "value") for f in ("pq_codes", "rvq_codes", "rvq_mask", "rvq_offsets")])
        assert z["key_rvq_codes"].dtype == np.uint16 and z["num_tokens"].tolist() == [T]
    loaded = load_compressed_chunk(p)
    for prefix, ref in (("key", k), ("value", v)):
        t = compressed_tensor_from_loaded(loaded, prefix)
        assert t.num_heads == H and t.num_tokens == T
        assert torch.equal(t.pq_codes, ref.pq_codes) and torch.equal(t.rvq_mask, ref.rvq_mask)
        assert torch.equal(t.rvq_codes.view(torch.int16), ref.rvq_codes.view(torch.int16))
        assert torch.equal(t.rvq_offsets, ref.rvq_offsets)


def test_router_ranking_over_chunk_files(tmp_path):
    cfg = RFSNConfig(num_heads=4, head_dim=128, num_subspaces=8, subspace_dim=16, block_size_seq=16,
                     disk_cache_dir=str(tmp_path), prefetch_throttle_s=0.0)
    cfg_e = RFSNConfig(num_heads=4, head_dim=128, num_subspaces=8, subspace_dim=16, num_rvq_layers=3)
    e = CompressedTensorMLX.empty(cfg_e)
    for cid in (2, 3, 4, 5, 9):
        save_compressed_chunk(chunk_file_path(tmp_path, 0, cid), e, e)
    r = AsyncHierarchicalRouterMLX(cfg, 0)
    # candidates in [(70-40)//16, (70+40)//16] = [1, 6] that exist, by |cid*16 - 70|
    assert r.rank(70, 40) == [4, 5, 3, 2]
    assert r.prefetch_sync(70, 40, top_k=3) == [4, 5, 3]
    assert r.get_chunk(4) is not None and r.get_chunk(2) is None
    assert r.prefetch_sync(0, 1024, top_k=1) == [2]


def test_normalize_query_positions_host():
    from apple_amd.attention import _normalize_query_positions as nqp

    assert nqp(None, 2, 3, 9).tolist() == [[9] * 3] * 2
    assert nqp([4, 5], 2, 3, 9).tolist() == [[4] * 3, [5] * 3]
    assert nqp(torch.arange(6).reshape(2, 3), 2, 3, 9).tolist() == [[0, 1, 2], [3, 4, 5]]
    for bad in ([1, 2, 3], torch.zeros(3, 2)):
        with pytest.raises(ValueError):
            nqp(bad, 2, 3, 9)


@pytest.mark.parametrize("M", [8, 16])
def test_tiled_layout_is_a_bijection(M):
    """untile() inverts the tiled code layout: every (token, subspace) of a
    tile owns one byte, and a tile's bytes are contiguous."""
    from apple_amd.batched import untile

    T = 96
    tiled = torch.arange(T * M, dtype=torch.int64).reshape(1, -1)
    plain = untile(tiled, M, T)[0]
    assert sorted(plain.reshape(-1).tolist()) == list(range(T * M))
    for t in range(0, T, 32):
        assert plain[t:t + 32].min() == t * M and plain[t:t + 32].max() == (t + 32) * M - 1
    # one lane's IPT bytes hold one subspace m for TPI-strided tokens of its tile
    tpi, ipt = 64 // M, 32 // (64 // M)
    lane = 5
    j, m = lane // M, lane % M
    for i in range(ipt):
        assert plain[tpi * i + j, m] == lane * ipt + i


def test_score_layout_roundtrip():
    """unpack_score_codes inverts the score-table K layout at any token base."""
    from apple_amd import kernels as K
    from tests.conftest import score_layout

    g = np.random.default_rng(3)
    for t_base in (0, 5, 32):
        T, k = 70, 4
        cap = (t_base + T + 31) // 32 * 32
        pq = g.integers(0, 256, (T, 16)).astype(np.uint8)
        rv = g.integers(0, 256, (T, 16)).astype(np.uint8)
        si = g.integers(0, 64, (T, k)).astype(np.uint8)
        sv = g.standard_normal((T, k)).astype(np.float16)
        p, r, i, v = score_layout(pq, rv, si, sv, t_base, cap)
        dst = {"pq": torch.from_numpy(p[None]), "rvq": torch.from_numpy(r[None]),
               "sparse_idx": torch.from_numpy(i.reshape(1, cap, k)), "sparse_val": torch.from_numpy(v.reshape(1, cap, k))}
        up, ur, ui, uv = K.unpack_score_codes(dst, T, t0=t_base)
        assert np.array_equal(up[0].numpy(), pq) and np.array_equal(ur[0].numpy(), rv)
        assert np.array_equal(ui[0].numpy(), si) and np.array_equal(uv[0].numpy().view(np.uint16), sv.view(np.uint16))


def test_score_table_lanes_cover_slots_without_bank_conflicts():
    """The fused kernel's score-table reads, restated from its lane
    constants: lane (n, g) = (lane & 15, lane >> 4) handles token row
    tokr = 4(n & 3) + (n >> 2) of both halves and code block beta; it loads 8
    bytes at 32 tokr + 8 beta of each code array (u = 0 in the low word),
    gather k reads byte k of half u's word at the slot offsets lca / lcb, and
    it loads sparse entry g of both tokens at entry 8 tokr + 2 g.  Every
    (token, slot) is read exactly once, each slot offset is the slot that
    byte holds, every sparse entry is read once, and in every 32-lane LDS
    pass of a gather the lanes read 32 distinct slots (the 256-byte table
    entry spans all 64 banks)."""
    from tests.conftest import score_layout

    g0 = np.random.default_rng(4)
    pq = g0.integers(0, 256, (32, 16)).astype(np.uint8)
    rv = g0.integers(0, 256, (32, 16)).astype(np.uint8)
    si = np.arange(128, dtype=np.uint8).reshape(32, 4)
    sv = np.zeros((32, 4), np.float16)
    p, r, sidx, _ = score_layout(pq, rv, si, sv, 0, 32)
    seen, seen_sparse = set(), set()
    for u in range(2):
        for k in range(4):
            for arr_i, arr in enumerate((p, r)):
                slots = []
                for lane in range(64):
                    n, gg = lane & 15, lane >> 4
                    tokr = 4 * (n & 3) + (n >> 2)
                    beta = (gg + 2 * (n >> 3)) & 3
                    todd = (n >> 2) & 1
                    off = 32 * beta + 8 * (k ^ (n & 3)) + (128 if todd ^ arr_i else 0)
                    slot = off // 8  # 0..15 PQ subspace, 16..31 RVQ subspace
                    t = 16 * u + tokr
                    code = arr[32 * tokr + 8 * beta + 4 * u + k]
                    assert code == (pq if slot < 16 else rv)[t, slot % 16], (u, k, lane)
                    assert (t, slot) not in seen
                    seen.add((t, slot))
                    slots.append(slot)
                for p0 in (0, 32):
                    assert len(set(slots[p0:p0 + 32])) == 32, (u, k, arr_i, p0)
        for lane in range(64):
            n, gg = lane & 15, lane >> 4
            tokr = 4 * (n & 3) + (n >> 2)
            e = int(sidx[8 * tokr + 2 * gg + u])
            assert e == si[16 * u + tokr, gg]
            seen_sparse.add(e)
    assert len(seen) == 32 * 32 and len(seen_sparse) == 128


def test_workload_bytes_known_answers():
    from apple_amd.workloads import WORKLOADS

    want = {"smoke_1k": 444_416, "llama1b_8k": 6_594_560, "batched_32x32k": 786_694_144,
            "longctx_128k": 9_478_144}
    for name, b in want.items():
        assert WORKLOADS[name].bytes_per_step() == b, name
    w = WORKLOADS["batched_32x32k"]
    assert (w.batch, w.context, w.q_heads, w.kv_heads, w.hot, w.warm) == (32, 32768, 32, 8, 1024, 31744)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]


def test_kernel_query_positions_shape():
    """The kernels index query positions as int32 [B, Hq]; [B] is broadcast
    and any other shape is rejected before a launch."""
    from apple_amd.kernels import _qpos

    assert _qpos(torch.tensor([3, 4]), 2, 3, "cpu").tolist() == [[3] * 3, [4] * 3]
    assert _qpos(torch.arange(6).reshape(2, 3), 2, 3, "cpu").dtype == torch.int32
    for bad in (torch.arange(3), torch.zeros(2, 2), torch.zeros(2, 3, 1)):
        with pytest.raises(ValueError):
            _qpos(bad, 2, 3, "cpu")


def test_product_path_refuses_cpu_tensors():
    from apple_amd import kernels as K

    x = torch.zeros((4, 64), dtype=torch.float16)
    cb = torch.zeros((16, 256, 4), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU only"):
        K.pq_encode(x, cb)


def _check_windows(slot_cid, wanted, missing, arena, windows):
    used = set()
    got = []
    for j, part in windows:
        assert part and all(b == a + 1 for a, b in zip(part, part[1:]))          # consecutive ids
        assert len({c // arena for c in part}) == 1                               # one pinned arena
        slots = range(j, j + len(part))
        assert 0 <= j and j + len(part) <= len(slot_cid)
        assert not used.intersection(slots)
        used.update(slots)
        assert all(slot_cid[s] < 0 or slot_cid[s] not in wanted for s in slots)  # no wanted chunk evicted
        got += part
    assert sorted(got) == sorted(missing)


def test_cold_slot_windows():
    """Placement of missing cold chunks in the device slot pool: the router's
    16 consecutive chunks in an empty pool are one copy; a run that crosses a
    pinned arena is two; wanted resident chunks split a run around them; the
    least recently used occupants are evicted first; random pool states keep
    every invariant."""
    from apple_amd.cache import plan_slot_windows

    free = [-1] * 32
    ids = list(range(208, 224))
    assert plan_slot_windows(free, [], set(ids), ids, 64) == [(0, ids)]
    w = plan_slot_windows(free, [], {62, 63, 64, 65}, [62, 63, 64, 65], 64)
    assert w == [(0, [62, 63]), (2, [64, 65])]
    pool = [-1] * 16
    pool[4], pool[10] = 100, 101                       # wanted and resident
    w = plan_slot_windows(pool, [4, 10], {100, 101, *range(6)}, list(range(6)), 64)
    _check_windows(pool, {100, 101, *range(6)}, list(range(6)), 64, w)
    assert [len(p) for _, p in w] == [5, 1]
    full = list(range(50, 58))                         # 8 slots, all unwanted occupants
    lru = [6, 7, 0, 1, 2, 3, 4, 5]                     # slots 6 and 7 hold the oldest chunks
    assert plan_slot_windows(full, lru, {0, 1}, [0, 1], 64) == [(6, [0, 1])]
    g = np.random.default_rng(5)
    for _ in range(300):
        S = int(g.integers(1, 40))
        slot_cid = [-1] * S
        occ = g.choice(1000, size=int(g.integers(0, S + 1)), replace=False)
        for s, c in zip(g.permutation(S)[:len(occ)], occ):
            slot_cid[s] = int(c)
        resident = [c for c in slot_cid if c >= 0]
        keep = [c for c in resident if g.random() < 0.4]
        room = S - len(keep)
        missing = sorted({int(x) for x in g.integers(1000, 1100, int(g.integers(0, room + 1)))})
        wanted = set(keep) | set(missing)
        lru = [s for s in g.permutation(S) if slot_cid[s] >= 0]
        arena = int(g.integers(1, 70))
        _check_windows(slot_cid, wanted, missing, arena, plan_slot_windows(slot_cid, lru, wanted, missing, arena))
        busy = frozenset(int(s) for s in g.permutation(S)[:int(g.integers(0, S + 1))])
        w = plan_slot_windows(slot_cid, lru, wanted, missing, arena, busy)
        _check_windows(slot_cid, wanted, missing, arena, w)
        used = [j for s0, part in w for j in range(s0, s0 + len(part))]
        free_idle = [j for j in range(S) if j not in busy and slot_cid[j] < 0]
        if len(free_idle) >= len(missing):  # enough free idle slots: no eviction, no wait
            assert all(j not in busy and slot_cid[j] < 0 for j in used)


def test_cold_slot_windows_avoid_busy_slots():
    """A prefetch one step ahead: the slots the running step reads are busy,
    so the next window's chunks go to the other half of the pool; free slots
    come before evicting a resident chunk, even when they are still busy."""
    from apple_amd.cache import plan_slot_windows

    pool = list(range(100, 116)) + [-1] * 16       # slots 0-15 hold the current window
    busy = frozenset(range(16))
    nxt = list(range(200, 216))
    assert plan_slot_windows(pool, list(range(16)), set(nxt), nxt, 64, busy) == [(16, nxt)]
    # without the busy set the least recently used (free) slots are the same here
    pool2 = list(range(100, 132))                  # full pool of stale chunks, 0-15 busy
    w = plan_slot_windows(pool2, list(range(32)), set(nxt), nxt, 64, busy)
    assert w == [(16, nxt)]
    pool3 = list(range(100, 116)) + [-1] * 16      # the other half is free but its last reader still runs
    assert plan_slot_windows(pool3, list(range(16)), set(nxt), nxt, 64, frozenset(range(32))) == [(16, nxt)]


def test_llama3_rope_frequencies_closed_form():
    """Rotary inverse frequencies of the Llama-3.2 layer against closed forms
    (head_dim 64, theta 500000, llama3 scaling factor 32, low / high
    frequency factors 1 / 4, original context 8192):
    * without scaling f_i = theta^(-2i/64) exactly;
    * components with wavelength 2 pi / f below 8192 / 4 = 2048 tokens keep
      f_i, those above 8192 tokens become f_i / 32 (for head_dim 64 and
      theta 500000 the band edges fall between i = 14 | 15 and 17 | 18);
    * between, the value lies strictly inside (f_i / 32, f_i) and the
      interpolation weight is affine in 1 / wavelength: it reaches 0 and 1
      where the bands begin;
    * factor 1 is the identity; the tables are cos / sin of p * f."""
    import math

    from apple_amd.layer import LLAMA3_ROPE_SCALING, rope_cos_sin, rope_inv_freq

    base = rope_inv_freq(64, 500000.0).numpy()
    exact = np.array([500000.0 ** (-(2 * i) / 64) for i in range(32)])
    assert np.array_equal(base, exact)
    f = rope_inv_freq(64, 500000.0, LLAMA3_ROPE_SCALING).numpy()
    wl = 2 * math.pi / base
    high, low = wl < 2048, wl > 8192
    assert list(np.nonzero(high)[0]) == list(range(15)) and list(np.nonzero(low)[0]) == list(range(18, 32))
    assert np.array_equal(f[high], base[high])
    assert np.allclose(f[low], base[low] / 32, rtol=1e-15, atol=0)
    mid = ~(high | low)
    assert mid.sum() == 3
    assert np.all(f[mid] > base[mid] / 32) and np.all(f[mid] < base[mid])
    w = (f[mid] - base[mid] / 32) / (base[mid] - base[mid] / 32)      # interpolation weight
    x = 8192 / wl[mid]                                                  # periods in the original context
    slope = np.diff(w) / np.diff(x)
    assert np.allclose(slope, 1 / 3, rtol=1e-9) and np.isclose(w[0] - (x[0] - 1) / 3, 0, atol=1e-12)
    ident = dict(LLAMA3_ROPE_SCALING, factor=1.0)
    assert np.allclose(rope_inv_freq(64, 500000.0, ident).numpy(), base, rtol=1e-15, atol=0)
    pos = torch.tensor([0, 1, 400, 131071])
    cos, sin = rope_cos_sin(pos, 64, 500000.0, LLAMA3_ROPE_SCALING)
    ang = pos.numpy()[:, None].astype(np.float64) * np.concatenate([f, f])[None, :]
    assert np.allclose(cos.numpy(), np.cos(ang), atol=1e-6) and np.allclose(sin.numpy(), np.sin(ang), atol=1e-6)
    assert np.all(cos.numpy()[0] == 1) and np.all(sin.numpy()[0] == 0)
    with pytest.raises(ValueError):
        rope_inv_freq(64, 500000.0, {"rope_type": "yarn", "factor": 4.0})


def test_score_guard_weights():
    """The drift guard's per-sequence row: W_i = mean_c PQ_c,i^2 + mean_c
    RVQ_c,i^2 + mean_c |PQ_c(s)|^2 + mean_c |RVQ_c(s)|^2 (s = i // 4), then
    the V bound; closed form on constant codebooks, and per-sequence rows of
    stacked codebooks equal the rows of each."""
    from apple_amd import kernels as K

    p = torch.full((16, 256, 4), 0.5, dtype=torch.float16)
    r = torch.full((16, 256, 4), -0.25, dtype=torch.float16)
    g = K.score_guard(p, r, 3.0)
    # 0.25 + 0.0625 per coordinate, 4 * that per subspace norm
    assert torch.allclose(g[:64], torch.full((64,), 0.3125 * 5))
    assert float(g[64]) == 3.0
    gen = torch.Generator().manual_seed(3)
    ps = torch.randn((3, 16, 256, 4), generator=gen).half()
    rs = (torch.randn((3, 16, 256, 4), generator=gen) * 0.3).half()
    rows = K.score_guard(ps, rs, torch.tensor([1.0, 2.0, 4.0]))
    assert rows.shape == (3, 65)
    for b in range(3):
        one = K.score_guard(ps[b], rs[b], float(2 ** b))
        assert torch.allclose(rows[b], one)
        pf, rf = ps[b].double().numpy(), rs[b].double().numpy()
        W = ((pf * pf).mean(1) + (rf * rf).mean(1)).reshape(64) \
            + np.repeat((pf * pf).sum(2).mean(1) + (rf * rf).sum(2).mean(1), 4)
        np.testing.assert_allclose(one[:64].numpy(), W, rtol=1e-5)


def test_router_rank_memo_matches_fresh_ranking():
    """The bound router's memoized ranking (reused while the cache's chunk
    ids and the candidate range stay, and every candidate starts at or before
    the position) equals a fresh ranking at every position, including when
    the position falls back before the last chunk and when chunks are added."""
    from apple_amd.storage import AsyncHierarchicalRouterMLX, RFSNConfig

    cfg = RFSNConfig(num_heads=4, head_dim=64, num_subspaces=16, subspace_dim=4, cold_chunk_tokens=64,
                     tier_policy="recency", cold_medium="pinned")

    class Ids:  # the bound cache's side of the ranking: its config and sorted chunk ids
        config = cfg

        def __init__(self):
            self.ids = list(range(0, 40, 2))

        def cold_chunk_ids(self):
            return self.ids

    src = Ids()
    memo = AsyncHierarchicalRouterMLX(cfg).bind(src)
    for pos in [2600, 2601, 2700, 1000, 2601, 5000, 5001]:
        for window in (pos + 1, 700):
            fresh = AsyncHierarchicalRouterMLX(cfg).bind(src).rank(pos, window)
            assert memo.rank(pos, window) == fresh, (pos, window)
        src.ids = src.ids + [src.ids[-1] + 1]  # a new list object: chunks added


def test_tile_map_walks_segments_in_order():
    """The fused kernel's tile map: for every encoded tile past segment 0, in
    window order, (segment << 16) | tile within the segment -- checked
    against a plain walk over the segment lengths, with empty and one-token
    segments, and memoized rows identical to fresh ones."""
    from apple_amd import _lib as L
    from apple_amd import kernels as K

    t = K.SegmentTable(3)
    lens = [[100, 33, 0, 1, 64, 700], [15360] + [512] * 16, [5]]
    for b, row in enumerate(lens):
        for n in row:
            t.add_codes(b, L.Codes(), L.Codes(), [], 0, n, 0, 1 << 24)
    maps, stride = t.tile_map()
    for b, row in enumerate(lens):
        want = [(s << 16) | j for s in range(1, len(row)) for j in range((row[s] + 31) // 32)]
        assert maps[b].tolist() == want
    assert stride == max(len(m) for m in maps) == 256
    again, _ = t.tile_map()  # memo hits give the same rows
    assert all(np.array_equal(a, m) for a, m in zip(again, maps))
    big = K.SegmentTable(1)
    big.add_codes(0, L.Codes(), L.Codes(), [], 0, 32, 0, 1 << 24)
    big.add_codes(0, L.Codes(), L.Codes(), [], 0, 32 * 0x10001, 0, 1 << 26)
    with pytest.raises(ValueError):
        big.tile_map()


def test_entry_tables_layout():
    """kernels.entry_tables: entry e = [PQ entries e of the subspaces | RVQ
    entries e], zeros past a short codebook, the PQ half repeated without an
    RVQ stage, per-sequence leading dimensions kept."""
    from apple_amd import kernels as K

    g = torch.Generator().manual_seed(5)
    pq = torch.randn(16, 256, 4, generator=g).half()
    rv = torch.randn(16, 200, 4, generator=g).half()
    t = K.entry_tables(pq, rv)
    assert t.shape == (256, 128) and t.dtype == torch.float16
    for e in (0, 77, 199, 255):
        assert torch.equal(t[e, :64].view(16, 4), pq[:, e])
    for e in (0, 199):
        assert torch.equal(t[e, 64:].view(16, 4), rv[:, e])
    assert not t[200:, 64:].any()
    pq8 = torch.randn(3, 8, 256, 8, generator=g).half()
    t8 = K.entry_tables(pq8, None)
    assert t8.shape == (3, 256, 128)
    assert torch.equal(t8[2, 9, :64].view(8, 8), pq8[2, :, 9]) and torch.equal(t8[..., 64:], t8[..., :64])
    with pytest.raises(ValueError):
        K.entry_tables(torch.zeros(8, 256, 16).half(), None)  # head_dim 128: not a fused-kernel table


def test_reference_active_map_and_segments():
    """Row -> RVQ code row map of reference-format stores (the scatter of
    quantization.py:273-274), its memo, and the segment bounds checks."""
    from apple_amd import kernels as K

    offs = torch.tensor([1, 4, 5, 9], dtype=torch.int32)
    m = K.active_map(offs, 12)
    assert m.tolist() == [-1, 0, -1, -1, 1, 2, -1, -1, -1, 3, -1, -1]
    assert K.active_map(offs, 12) is m  # memoized per offsets tensor
    offs2 = offs.clone()
    m2 = K.active_map(offs2, 12)
    offs2[3] = 11  # an in-place write: the map is made again
    assert K.active_map(offs2, 12) is not m2 and int(K.active_map(offs2, 12)[11]) == 3
    assert K.active_map(offs, 16).shape == (16,)
    T, H, M, L = 6, 2, 8, 3
    st = CompressedTensorMLX(pq_codes=torch.zeros((T, H, M), dtype=torch.uint8),
                             rvq_codes=torch.zeros((4, L), dtype=torch.uint16),
                             rvq_mask=torch.zeros((T, H), dtype=torch.bool), rvq_offsets=offs, num_heads=H)
    seg = K.ref_store_segment(st, st, 2, 4, 10)
    assert seg["len"] == 4 and seg["token0"] == 2 and seg["pos0"] == 10 and seg["k"][2].tolist() == m.tolist()
    with pytest.raises(ValueError):
        K.ref_store_segment(st, st, 3, 4, 0)  # past the store
    ring = torch.zeros((H, 8, 64), dtype=torch.float16)
    K.ref_exact_segment(ring, ring, ring.stride(1), ring.stride(0), 2, 6, 0)
    with pytest.raises(ValueError):
        K.ref_exact_segment(ring, ring, ring.stride(1), ring.stride(0), 3, 6, 0)
    hm = K.ref_store_segment(st, st, 2, 4, 10, head_major=True)
    assert hm["rows"] == (1, T) and hm["k"][1] is not None and hm["k"][2] is not None
    assert K.ref_attention_ok(128, 8, 256, 4, 4, True) and not K.ref_attention_ok(96, 8, 256, 4, 4, True)
    assert not K.ref_attention_ok(256, 16, 256, 8, 1, False)  # 2 x 128 KB of tables
    assert K.ref_attention_ok(256, 16, 256, 8, 1, True, 16, 256, 4)


def test_guard_refuses_k_segments_without_exact_plane():
    """Under the drift guard the exact pass reads K's corrected coordinates
    kv_heads * head_stride * k values past each K sparse-value pointer: the
    host refuses a segment table in which some K segment lacks that plane
    (codes built without TiledCodes(exact_plane=True) or a direct caller),
    and accepts the plane both from precomputed addresses and from tensors."""
    from apple_amd import _lib as L
    from apple_amd import kernels as K
    from apple_amd.cache import TiledCodes

    H, cap, k = 2, 64, 4
    plane = H * cap * k * 2
    ok = K.SegmentTable(2)
    for b in range(2):
        ok.add_codes(b, L.Codes(), L.Codes(), [], cap, 40, 0, cap, k_plane=plane)
    ok.check_exact_planes(H, k)
    for bad_plane in (None, plane - 2, 2 * plane):
        t = K.SegmentTable(2)
        t.add_codes(0, L.Codes(), L.Codes(), [], cap, 40, 0, cap, k_plane=plane)
        t.add_codes(1, L.Codes(), L.Codes(), [], cap, 40, 0, cap, k_plane=bad_plane)
        with pytest.raises(ValueError, match="plane"):
            t.check_exact_planes(H, k)
    empty = K.SegmentTable(1)  # a zero-length segment reads nothing
    empty.add_codes(0, L.Codes(), L.Codes(), [], cap, 0, 0, cap)
    empty.check_exact_planes(H, k)

    fmt = K.WarmFormat(64, 16, 256, 16, 256, k)
    for exact in (True, False):
        tc = TiledCodes(fmt, H, torch.device("cpu"), cap=cap, score_rows=True, exact_plane=exact)
        assert tc.plane_bytes() == (plane if exact else None)
        t = K.SegmentTable(1)
        t.add(0, tc.codes(1), tc.codes(1), tc.cap, 20, 0)
        if exact:
            t.check_exact_planes(H, k)
        else:
            with pytest.raises(ValueError, match="plane"):
                t.check_exact_planes(H, k)


def test_ref_store_segment_head_major():
    """head_major segments carry [heads][T] copies of every per-row code array
    (row h * T + t; active entries still index the store's RVQ codes) for
    mapped, dense and long-context stores; a copy is reused while its store is
    unchanged and remade after an in-place write; stores of unequal lengths
    keep their own order."""
    from apple_amd import kernels as K
    from apple_amd.storage import CompressedTensorMLX

    g = torch.Generator().manual_seed(5)
    T, H, M, L, Mr, k = 6, 3, 8, 3, 4, 2
    rows = T * H
    pq = torch.randint(0, 256, (T, H, M), generator=g).to(torch.uint8)
    offs = torch.tensor([1, 4, 5, 9, 16], dtype=torch.int32)
    rvq = torch.randint(0, 500, (5, L), generator=g).to(torch.uint16)
    st = CompressedTensorMLX(pq_codes=pq, rvq_codes=rvq, rvq_mask=torch.zeros((T, H), dtype=torch.bool),
                             rvq_offsets=offs, num_heads=H)
    amap = K.active_map(offs, rows)
    seg = K.ref_store_segment(st, st, 1, 5, 0, head_major=True)
    assert seg["rows"] == (1, T)
    hpq, hrvq, hact = seg["k"][:3]
    assert torch.equal(hrvq, rvq)  # mapped: the codes stay, the map moves
    for t in range(T):
        for h in range(H):
            assert torch.equal(hpq.view(-1, M)[h * T + t], pq[t, h]) and int(hact[h * T + t]) == int(amap[t * H + h])
    assert K.ref_store_segment(st, st, 0, T, 0, head_major=True)["k"][0] is hpq  # reused
    pq[2, 1, 3] ^= 7
    again = K.ref_store_segment(st, st, 0, T, 0, head_major=True)["k"][0]
    assert again is not hpq and int(again.view(-1, M)[1 * T + 2, 3]) == int(pq[2, 1, 3])
    # every row active: dense gated codes, [heads][T][L]
    rv_d = torch.randint(0, 500, (rows, L), generator=g).to(torch.uint16)
    sd = CompressedTensorMLX(pq_codes=pq, rvq_codes=rv_d, rvq_mask=torch.ones((T, H), dtype=torch.bool),
                             rvq_offsets=torch.arange(rows, dtype=torch.int32), num_heads=H)
    dseg = K.ref_store_segment(sd, sd, 0, T, 0, head_major=True)
    assert dseg["k"][2] is None
    for t in range(T):
        for h in range(H):
            assert torch.equal(dseg["k"][1].view(-1, L)[h * T + t], rv_d[t * H + h])
    # long-context arrays
    rsub = torch.randint(0, 64, (T, H, Mr), generator=g).to(torch.uint8)
    sidx = torch.randint(0, 64, (T, H, k), generator=g).to(torch.uint8)
    sval = torch.randn((T, H, k), generator=g).half()
    se = CompressedTensorMLX(pq_codes=pq, rvq_codes=rsub, rvq_mask=torch.ones((T, H), dtype=torch.bool),
                             rvq_offsets=torch.zeros((0,), dtype=torch.int32), num_heads=H, sparse_idx=sidx,
                             sparse_val=sval)
    eseg = K.ref_store_segment(se, se, 0, T, 0, head_major=True)
    for arr, src in ((eseg["k"][3], rsub), (eseg["k"][4], sidx), (eseg["k"][5], sval)):
        assert torch.equal(arr, src.transpose(0, 1).contiguous())
    # unequal lengths: the stores' own order
    short = CompressedTensorMLX(pq_codes=pq[:5].contiguous(), rvq_codes=rvq, rvq_mask=torch.zeros((5, H), dtype=torch.bool),
                                rvq_offsets=offs[:4], num_heads=H)
    assert "rows" not in K.ref_store_segment(st, short, 0, 5, 0, head_major=True)
