"""Tiered KV cache on MI355X -- the counterpart of the reference's ``cache.py``
(``RFSNv10KVCacheMLX``, cache.py:33-440).

Reference behaviour kept: tier fill by arrival (hot, then warm, then cold;
cache.py:89-120), cold chunking by ``block_size_seq`` with merge-on-append
(cache.py:134-191), window bounds and adjusted positions (cache.py:199-241),
materialization order and access counters (cache.py:250-393),
``attention_forward`` semantics (cache.py:395-428) and ``memory_usage_bytes``
(cache.py:430-440).  ``append`` is an alias of ``update``.

MI355X design:
* the hot tier is a head-major device buffer ``[Hkv, cap, D]`` fp16 whose
  live range moves: appends write at the tail, demotions advance the head;
* warm codes are kept in the reference layout (``CompressedTensorMLX``; for
  the subspace format in token rings) and, for the subspace format, also in
  the tiled layout streamed by the fused dequant-attention kernel (one pass
  over hot + warm + attended cold chunks, no window written to HBM); under
  the recency policy whole cold chunks leave warm by moving ring heads;
* cold chunks go either to NPZ files (reference schema, storage.py:113-151)
  or to pinned host memory; attended pinned chunks are copied into device
  slots with hipMemcpyAsync on a side stream, ordered by events.

Extensions: ``num_kv_heads`` (GQA: the cache stores Hkv heads and attention
accepts Hq query heads), separate K/V quantizers (``update(..., (kq, vq))``),
``tier_policy="recency"`` (hot = newest tokens, window order cold|warm|hot),
explicit cold chunk sets (``attention_forward(..., cold_chunks=[...])``).
"""

from __future__ import annotations

import ctypes as C
import logging
import math
from collections import OrderedDict
from pathlib import Path
from typing import Any, Dict, List, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from . import _lib as L
from . import kernels as K
from .attention import _blockwise_exact_attention, _normalize_query_positions
from .quantization import (
    HybridQuantizerMLX,
    _append_compressed_tensor,
    _compress_tensor_sequence,
    _decode_compressed_tensor,
    _encode_pair_head_major,
    _head_major_store,
    _slice_compressed_tensor,
)
from .storage import (
    AsyncHierarchicalRouterMLX,
    CompressedTensorMLX,
    RFSNConfig,
    chunk_file_path,
    compressed_tensor_from_loaded,
    load_compressed_chunk,
    save_compressed_chunk,
)

logger = logging.getLogger("RFSN_CACHE")

QuantizerArg = Union[HybridQuantizerMLX, Tuple[HybridQuantizerMLX, HybridQuantizerMLX]]


def _pair(q: QuantizerArg) -> Tuple[HybridQuantizerMLX, HybridQuantizerMLX]:
    if isinstance(q, (tuple, list)):
        if len(q) != 2:
            raise ValueError("quantizer pair must be (key_quantizer, value_quantizer)")
        return q[0], q[1]
    return q, q


class TiledCodes:
    """Device codes of the subspace format in the fused kernel's tiled layout.
    Its ``sparse_val`` holds the corrected coordinates fp16(K[idx] + val)
    (``kernels.sparse_fold``), which the kernel stores over the reconstructed
    coordinate; the reference-layout stores keep the residuals.  With
    ``score_rows`` (K codes the kernel scores through q . centroid tables)
    codes and sparse entries are in the ``kernels.pack_score_codes`` layout
    and ``sparse_val`` holds the score deltas."""

    def __init__(self, fmt: K.WarmFormat, heads: int, device, pinned: bool = False, cap: int = 0,
                 backing: Optional[torch.Tensor] = None, score_rows: bool = False, exact_plane: bool = False):
        """``backing``: a uint8 buffer of at least ``nbytes(fmt, heads, cap)``
        that holds every array (fixed capacity), so that one copy moves the
        whole set; otherwise each array is its own growable allocation.
        ``exact_plane`` (with ``score_rows``): the sparse values are two
        planes [2, H, cap, k], the score deltas (``sparse_val``) and then the
        corrected coordinates (``sparse_cc``) in the same positions, which the
        fused kernel's exact pass reads when its drift guard fires."""
        self.fmt, self.heads, self.device, self.pinned = fmt, heads, device, pinned
        self.score_rows = score_rows
        self.exact_plane = bool(exact_plane and score_rows and fmt.sparse_k)
        self.cap = 0
        self.len = 0
        self.head = 0  # tiles before the oldest live token (pop_front_tiles)
        self.t: Dict[str, Optional[torch.Tensor]] = {}
        self._backing = backing
        self._carved = 0
        self._segs: Dict[Tuple[int, int], tuple] = {}  # (head, tile_skip) -> seg() result
        self._alloc(cap)

    @staticmethod
    def _arrays(fmt: K.WarmFormat, heads: int, cap: int, plane: bool = False):
        f, H = fmt, heads
        sv = (2, H, cap, f.sparse_k) if plane else (H, cap, f.sparse_k)
        return {"pq": ((H, cap * f.pq_subspaces), torch.uint8),
                "rvq": ((H, cap * f.rvq_subspaces), torch.uint8) if f.rvq_subspaces else None,
                "sparse_idx": ((H, cap, f.sparse_k), torch.uint8) if f.sparse_k else None,
                "sparse_val": (sv, torch.float16) if f.sparse_k else None}

    @staticmethod
    def nbytes(fmt: K.WarmFormat, heads: int, cap: int, plane: bool = False) -> int:
        """Bytes of one backing buffer: every array, each at a 256-byte boundary."""
        total = 0
        for spec in TiledCodes._arrays(fmt, heads, K.round_up(max(cap, 0), K.TILE), plane).values():
            if spec is not None:
                shape, dtype = spec
                n = math.prod(shape) * (2 if dtype == torch.float16 else 1)
                total += K.round_up(n, 256)
        return total

    def _new(self, shape, dtype):
        if self._backing is not None:
            n = 1
            for s in shape:
                n *= s
            nb = n * (2 if dtype == torch.float16 else 1)
            view = self._backing[self._carved:self._carved + nb]
            self._carved += K.round_up(nb, 256)
            return view.view(dtype).view(shape)
        if self.pinned:
            return torch.zeros(shape, dtype=dtype, pin_memory=True)
        return torch.zeros(shape, dtype=dtype, device=self.device)

    def _alloc(self, cap: int) -> None:
        cap = K.round_up(max(cap, 0), K.TILE)
        if cap <= self.cap and self.t:
            return
        if self._backing is not None:
            if self.t:
                raise ValueError("a TiledCodes set in one backing buffer has a fixed capacity")
            if self._backing.numel() < TiledCodes.nbytes(self.fmt, self.heads, cap, self.exact_plane):
                raise ValueError("backing buffer too small for the tiled arrays")
        new = {key: (None if spec is None else self._new(*spec))
               for key, spec in TiledCodes._arrays(self.fmt, self.heads, cap, self.exact_plane).items()}
        if self.exact_plane:
            planes = new["sparse_val"]
            new["sparse_val"], new["sparse_cc"] = planes[0], planes[1]
        if self.t and self.cap:
            self._move_live(self.t, new)
        self.t, self.cap, self.head = new, cap, 0
        self._segs = {}

    def _live_tiles(self) -> int:
        return (self.len + K.TILE - 1) // K.TILE

    def _move_live(self, src: Dict[str, Optional[torch.Tensor]], dst: Dict[str, Optional[torch.Tensor]]) -> None:
        """Copy the live tiles (from tile ``head``) of ``src`` to tile 0 of ``dst``."""
        f = self.fmt
        t0, nt = self.head * K.TILE, self._live_tiles() * K.TILE
        for key, old in src.items():
            if old is None:
                continue
            if key in ("pq", "rvq"):
                m = f.pq_subspaces if key == "pq" else f.rvq_subspaces
                live = old[:, t0 * m:(t0 + nt) * m]
                dst[key][:, :nt * m] = live.clone() if dst[key] is old else live
            else:
                live = old[:, t0:t0 + nt]
                dst[key][:, :nt] = live.clone() if dst[key] is old else live

    def pop_front_tiles(self, n: int) -> None:
        """Drop the n oldest whole tiles (32 n tokens)."""
        if n < 0 or n * K.TILE > self.len:
            raise ValueError("pop_front_tiles: more tiles than held")
        self.head += n
        self.len -= n * K.TILE
        self._segs = {}  # addresses of the old head are no longer asked for

    def append(self, pq: torch.Tensor, rvq: Optional[torch.Tensor], sidx: Optional[torch.Tensor],
               sval: Optional[torch.Tensor], pq_cb: Optional[torch.Tensor] = None,
               rvq_cb: Optional[torch.Tensor] = None) -> None:
        """Append plain codes [H, T, *] (device) at token ``len``; the sparse
        residuals ``sval`` are folded into corrected coordinates with the
        stream's codebooks."""
        H, T, _ = pq.shape
        cc = None
        if self.fmt.sparse_k and T:
            f = self.fmt
            flat = lambda t: None if t is None else t.reshape(H * T, -1)
            if self.exact_plane:
                cc = K.sparse_fold(f, flat(pq), pq_cb, flat(rvq), rvq_cb, flat(sidx), flat(sval)).view(H, T, -1)
            sval = K.sparse_fold(f, flat(pq), pq_cb, flat(rvq), rvq_cb, flat(sidx), flat(sval),
                                 delta=self.score_rows).view(H, T, -1)
        need = self.len + T
        if self.head * K.TILE + need > self.cap:
            if self._backing is None and self.head and 2 * K.round_up(need, K.TILE) <= self.cap:
                self._move_live(self.t, self.t)  # the live tiles move to the front
                self.head = 0
                self._segs = {}
            else:
                self._alloc(max(need, 2 * self.cap))
        t_base = self.head * K.TILE + self.len
        if self.score_rows:
            K.pack_score_codes(pq, rvq, sidx, sval, self.t, t_base)
            if cc is not None:
                K.pack_score_codes(pq, rvq, sidx, cc, dict(self.t, sparse_val=self.t["sparse_cc"]), t_base)
        else:
            K.pack_codes(pq, self.t["pq"], t_base)
            if self.fmt.rvq_subspaces:
                K.pack_codes(rvq, self.t["rvq"], t_base)
        if self.fmt.sparse_k and not self.score_rows:
            self.t["sparse_idx"][:, t_base:t_base + T] = sidx
            self.t["sparse_val"][:, t_base:t_base + T] = sval
        self.len = need

    @staticmethod
    def append_pair(kt: "TiledCodes", vt: "TiledCodes", kc: tuple, vc: tuple, kq, vq,
                    rings: Optional[tuple] = None) -> bool:
        """``append`` of a K/V block to a (K, V) pair of stores in one launch
        (``rfsn_warm_append_pair``) for the 16 + 16 subspace formats of
        head_dim 64 with a sparse stage, when both stores take the block in
        place at the same token; False, with nothing written, otherwise.
        kc / vc: plain head-major (pq, rvq, sparse_idx, sparse_val) [H, T, *]
        with residual sparse values.  ``rings`` (K, V ``_RingStore``): the same
        launch also appends the codes to them, which must then take the block
        in place as well."""
        f = kt.fmt
        if not (not vt.score_rows and vt.fmt == f and f.head_dim == 64 and f.pq_subspaces == 16
                and f.rvq_subspaces == 16 and 0 < f.sparse_k <= 16):
            return False
        if (kt.cap, kt.head, kt.len) != (vt.cap, vt.head, vt.len) or kt.heads != vt.heads:
            return False
        H, T = kt.heads, int(kc[0].shape[1])
        t_base = kt.head * K.TILE + kt.len
        if t_base + T > kt.cap:
            return False  # the stores grow or move: the per-store append handles it
        for c in (kc, vc):
            for t, last in zip(c, (16, 16, f.sparse_k, f.sparse_k)):
                if t is None or tuple(t.shape) != (H, T, last) or not t.is_contiguous():
                    return False
        ring_args = [None, None, None, None, 0]
        if rings is not None:
            kr, vr = rings
            if (kr.head, kr.n, kr._cap()) != (vr.head, vr.n, vr._cap()) or kr.head + kr.n + T > kr._cap():
                return False
            want = {"pq_codes": (16, torch.uint8), "rvq_codes": (16, torch.uint8), "rvq_mask": (None, torch.bool),
                    "sparse_idx": (f.sparse_k, torch.uint8), "sparse_val": (f.sparse_k, torch.float16)}
            for r in rings:
                for key, (w, dt) in want.items():
                    t = r.buf.get(key)
                    shape = (r._cap(), H) if w is None else (r._cap(), H, w)
                    if t is None or t.dtype != dt or tuple(t.shape) != shape or not t.is_contiguous():
                        return False
            rc = lambda r: L.Codes(*(r.buf[key].data_ptr() for key in ("pq_codes", "rvq_codes", "sparse_idx",
                                                                        "sparse_val")))
            ring_args = [C.byref(rc(kr)), kr.buf["rvq_mask"].data_ptr(), C.byref(rc(vr)), vr.buf["rvq_mask"].data_ptr(),
                         kr.head + kr.n]
        codes = lambda c: L.Codes(c[0].data_ptr(), c[1].data_ptr(), c[2].data_ptr(), c[3].data_ptr())
        ks, vs = codes(kc), codes(vc)
        kd = L.Codes(kt.t["pq"].data_ptr(), kt.t["rvq"].data_ptr(), kt.t["sparse_idx"].data_ptr(),
                     kt.t["sparse_val"].data_ptr())
        vd = L.Codes(vt.t["pq"].data_ptr(), vt.t["rvq"].data_ptr(), vt.t["sparse_idx"].data_ptr(),
                     vt.t["sparse_val"].data_ptr())
        cbs = [K._contig(x) for x in (kq.pq.codebooks, kq.rvq_codebooks, vq.pq.codebooks, vq.rvq_codebooks)]
        fc = f.c()
        L.call("rfsn_warm_append_pair", C.byref(fc), C.byref(ks), C.byref(vs), T, H, *(x.data_ptr() for x in cbs),
               C.byref(kd), int(kt.score_rows), kt.t["sparse_cc"].data_ptr() if kt.exact_plane else None, C.byref(vd),
               kt.cap, t_base, *ring_args, K._stream(kc[0]))
        kt.len += T
        vt.len += T
        if rings is not None:
            for r in rings:
                r.n += T
        return True

    def seg(self, tile_skip: int = 0):
        """(rfsn_codes addresses from live tile ``tile_skip``, the arrays to
        keep alive, tokens available from there): a segment without building
        tensor views.  The result depends only on the arrays, ``head`` and
        ``tile_skip``, so it is kept until the arrays are reallocated."""
        hit = self._segs.get((self.head, tile_skip))  # cleared whenever the arrays or head move
        if hit is not None:
            return hit
        f = self.fmt
        o = (self.head + tile_skip) * K.TILE
        t = self.t
        ptr = lambda key, scale: None if t[key] is None else t[key].data_ptr() + o * scale
        codes = L.Codes(ptr("pq", f.pq_subspaces), ptr("rvq", f.rvq_subspaces),
                          ptr("sparse_idx", f.sparse_k), ptr("sparse_val", 2 * f.sparse_k))
        hit = (codes, [x for x in t.values() if x is not None], self.cap - o)
        self._segs[(self.head, tile_skip)] = hit
        return hit

    def plane_bytes(self) -> Optional[int]:
        """Bytes from ``sparse_val`` to ``sparse_cc`` (the exact pass's plane), or None."""
        if not self.exact_plane:
            return None
        return self.t["sparse_cc"].data_ptr() - self.t["sparse_val"].data_ptr()

    def codes(self, tile_skip: int = 0) -> Dict[str, Optional[torch.Tensor]]:
        """Per-array views starting at live tile ``tile_skip`` (head stride unchanged)."""
        f = self.fmt
        o = (self.head + tile_skip) * K.TILE
        out = {"pq": self.t["pq"][:, o * f.pq_subspaces:]}
        out["rvq"] = self.t["rvq"][:, o * f.rvq_subspaces:] if f.rvq_subspaces else None
        out["sparse_idx"] = self.t["sparse_idx"][:, o:] if f.sparse_k else None
        out["sparse_val"] = self.t["sparse_val"][:, o:] if f.sparse_k else None
        if self.exact_plane:
            out["sparse_cc"] = self.t["sparse_cc"][:, o:]
        return out


class _RingStore:
    """Subspace-format codes in token-major device buffers with a live range
    [head, head + n).  Appends write at the tail (when the tail reaches the
    end the live range moves to the front, or the buffers double) and pops
    advance the head, so an append or a migration to the cold tier costs its
    own tokens, not the tier's length (the reference concatenates,
    quantization.py:346-361)."""

    FIELDS = ("pq_codes", "rvq_codes", "rvq_mask", "sparse_idx", "sparse_val")

    def __init__(self, empty: CompressedTensorMLX):
        self.heads = empty.num_heads
        self.offsets = empty.rvq_offsets
        self.buf = {f: getattr(empty, f) for f in self.FIELDS}
        self.head = 0
        self.n = 0

    def _cap(self) -> int:
        return int(self.buf["pq_codes"].shape[0])

    def view(self, a: int = 0, b: Optional[int] = None) -> CompressedTensorMLX:
        b = self.n if b is None else b
        lo, hi = self.head + a, self.head + b
        sl = {f: (None if t is None else t[lo:hi]) for f, t in self.buf.items()}
        return CompressedTensorMLX(pq_codes=sl["pq_codes"], rvq_codes=sl["rvq_codes"], rvq_mask=sl["rvq_mask"],
                                   rvq_offsets=self.offsets, num_heads=self.heads, sparse_idx=sl["sparse_idx"],
                                   sparse_val=sl["sparse_val"])

    def append(self, st: CompressedTensorMLX) -> None:
        T = st.num_tokens
        if T == 0:
            return
        need = self.n + T
        if self.head + need > self._cap():
            live = {f: (None if t is None else t[self.head:self.head + self.n]) for f, t in self.buf.items()}
            if 2 * need <= self._cap():
                for f, t in live.items():
                    if t is not None:
                        self.buf[f][:self.n] = t.clone()
            else:
                cap = max(need, 2 * self._cap(), 64)
                for f, t in live.items():
                    if t is not None:
                        nb = torch.empty((cap, *t.shape[1:]), dtype=t.dtype, device=t.device)
                        nb[:self.n] = t
                        self.buf[f] = nb
            self.head = 0
        o = self.head + self.n
        for f in self.FIELDS:
            if self.buf[f] is not None:
                self.buf[f][o:o + T] = getattr(st, f)
        self.n = need

    def pop_front(self, m: int) -> CompressedTensorMLX:
        """Remove the m oldest tokens and return them (copies)."""
        if m < 0 or m > self.n:
            raise ValueError("pop_front: more tokens than held")
        out = self.view(0, m)
        out = CompressedTensorMLX(
            pq_codes=out.pq_codes.clone(), rvq_codes=out.rvq_codes.clone(), rvq_mask=out.rvq_mask.clone(),
            rvq_offsets=self.offsets, num_heads=self.heads,
            sparse_idx=None if out.sparse_idx is None else out.sparse_idx.clone(),
            sparse_val=None if out.sparse_val is None else out.sparse_val.clone())
        self.head += m
        self.n -= m
        return out


def plan_slot_windows(slot_cid: Sequence[int], lru: Sequence[int], wanted: set, missing: Sequence[int],
                      arena: int, busy: frozenset = frozenset()) -> List[Tuple[int, List[int]]]:
    """Where missing cold chunks go in a pool of ``len(slot_cid)`` device slots.

    slot_cid[j]: the chunk in slot j (-1 free); lru: occupied slots, least
    recently used first; wanted: every chunk of the window (their slots are
    never taken); missing: the chunks to copy in; busy: slots that queued
    launches may still read (a copy into one first waits for them).  Usable
    slots rank free and idle, free and busy, holding an unwanted chunk and
    idle, holding one and busy.  Missing ids form runs of consecutive ids
    inside one pinned arena of ``arena`` ids; each run takes the longest
    window of consecutive slots of the best rank that has any (older
    occupants first among equals), and the rest of the run continues the
    same way.  Returns (first slot, chunk ids) per window, one copy each."""
    S = len(slot_cid)
    rank = {s: r for r, s in enumerate(lru)}
    taken = set()

    def klass(j: int) -> int:
        if j in taken or (slot_cid[j] >= 0 and slot_cid[j] in wanted):
            return 4  # unusable
        return (0 if slot_cid[j] < 0 else 2) + (1 if j in busy else 0)

    runs: List[List[int]] = []
    for cid in sorted(missing):
        if runs and cid == runs[-1][-1] + 1 and cid // arena == runs[-1][0] // arena:
            runs[-1].append(cid)
        else:
            runs.append([cid])
    out = []
    for run in runs:
        while run:
            cls = [klass(j) for j in range(S)]
            best = None
            for limit in range(4):
                j = 0
                while j < S:  # each maximal stretch of slots of rank <= limit
                    if cls[j] > limit:
                        j += 1
                        continue
                    a = j
                    while j < S and cls[j] <= limit:
                        j += 1
                    n = min(len(run), j - a)
                    for off in range(a, j - n + 1):
                        newest = max((rank.get(x, -1) for x in range(off, off + n)), default=-1)
                        cost = (-n, newest)
                        if best is None or cost < best[0]:
                            best = (cost, off, n)
                        if newest < 0:
                            break  # free slots: the first window of the stretch is as good as any
                if best is not None:
                    break
            if best is None:
                raise ValueError("more wanted cold chunks than device slots")
            _, j, n = best
            taken.update(range(j, j + n))
            out.append((j, run[:n]))
            run = run[n:]
    return out


def _plain_head_major(store: CompressedTensorMLX):
    """Reference-layout subspace codes [T, H, *] -> head-major [H, T, *]."""
    pm = lambda t: None if t is None else t.permute(1, 0, 2).contiguous()
    return pm(store.pq_codes), pm(store.rvq_codes), pm(store.sparse_idx), pm(store.sparse_val)


# query heads (queries x heads) up to which the reference-format path uses
# score tables: each query head builds its own table and histograms
REF_TABLES_MAX_QUERY_HEADS = 256


class _CodebookKey:
    """Memo key of tables built from a quantizer pair's codebooks.  It holds
    the objects themselves (compared by identity, so a freed tensor's address
    or id reused by a new one cannot match) and the tensors' versions."""

    __slots__ = ("objs", "versions")

    def __init__(self, objs: tuple, versions: tuple):
        self.objs, self.versions = objs, versions

    def __eq__(self, other) -> bool:
        return (isinstance(other, _CodebookKey) and self.versions == other.versions
                and len(self.objs) == len(other.objs) and all(a is b for a, b in zip(self.objs, other.objs)))

    def __ne__(self, other) -> bool:
        return not self.__eq__(other)

    __hash__ = None


class RFSNv10KVCacheMLX:
    """Tiered KV cache with exact hot storage and compressed warm/cold storage."""

    def __init__(self, config: RFSNConfig, layer_idx: int = 0, device=None, cold_slots: int = 32):
        self.config = config
        self.layer_idx = layer_idx
        self.hot_capacity = config.hot_capacity
        self.warm_capacity = config.warm_capacity
        if device is None:
            if not torch.cuda.is_available():
                raise RuntimeError("the RFSN MI355X cache needs a ROCm GPU; none is visible")
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = torch.device(device)
        self.H = config.kv_heads
        self.D = config.head_dim
        # hot tier: [H, cap, D] buffers, live tokens [_hot_head, _hot_head + num_hot)
        self._hot_k = torch.zeros((self.H, 0, self.D), dtype=torch.float16, device=self.device)
        self._hot_v = torch.zeros_like(self._hot_k)
        self._hot_head = 0

        # warm tier: the subspace format keeps its codes in rings (appends and
        # migrations cost their own tokens); the reference format concatenates
        if config.ext_format:
            self._wk = _RingStore(CompressedTensorMLX.empty(config, self.H, self.device))
            self._wv = _RingStore(CompressedTensorMLX.empty(config, self.H, self.device))
        else:
            self._wk = CompressedTensorMLX.empty(config, self.H, self.device)
            self._wv = CompressedTensorMLX.empty(config, self.H, self.device)
        self._warm_tiled: Optional[Tuple[TiledCodes, TiledCodes]] = None
        self._fmt_memo: Optional[Tuple[object, K.WarmFormat]] = None

        self.cold_chunk_paths: List[Path] = []
        self.cold_chunk_paths_by_id: Dict[int, Path] = {}
        self.cold_chunk_metadata: List[dict] = []
        self._cold_pinned: Dict[int, dict] = {}
        self._cold_ids: Tuple[int, int, List[int]] = (0, 0, [])  # (id of the source dict, its size, sorted ids)
        self._cold_slots: "OrderedDict[int, dict]" = OrderedDict()  # chunk id -> device slot, LRU first
        self._cold_arena: Dict[int, torch.Tensor] = {}
        self._slot_buf: Optional[torch.Tensor] = None
        self._slot_cid: List[int] = []
        self._slot_views: Dict[int, Tuple[TiledCodes, TiledCodes]] = {}
        # per slot: event recorded after the last launches that read it (None:
        # no reader; PREPARED: read by prepared steps, whose calls are not tracked)
        self._slot_reader: List[Any] = []
        self._read_events: List[int] = []
        self._read_next = 0
        self._copies_pending = False  # copies queued without the launch stream waiting on them
        self._cold_slot_limit = cold_slots
        self._side: Optional[K.SideStream] = None

        self.num_hot = 0
        self.num_warm = 0
        self.num_cold = 0
        self.total_tokens = 0
        self.quantizer: Optional[QuantizerArg] = None
        self._kq: Optional[HybridQuantizerMLX] = None
        self._vq: Optional[HybridQuantizerMLX] = None
        # drift guard of the score tables: running max |V| of the appended
        # values, the guard's input row and the last call's estimates
        self._guard = torch.zeros((1, 65), dtype=torch.float32, device=self.device)
        self._vabs = self._guard[0, 64:]  # the row's V bound, updated by every append
        self._guard_key: Optional[_CodebookKey] = None
        self._tables_key: Optional[_CodebookKey] = None
        self._tables: Optional[Tuple[torch.Tensor, torch.Tensor]] = None
        self.last_drift: Optional[torch.Tensor] = None
        # score tables of the reference-format path: codebook statistics of
        # their drift guard, whether the last call used them, its estimates
        self._ref_stats_key: Optional[_CodebookKey] = None
        self._ref_stats: Optional[torch.Tensor] = None
        self.last_ref_tables = False
        self.last_ref_drift: Optional[torch.Tensor] = None
        self.last_access_stats = self._empty_access_stats()

    # ------------------------------------------------------------------ stats
    def _empty_access_stats(self) -> Dict[str, int]:
        """cache.py:59-76."""
        return {
            "window_start": 0, "window_end": 0, "window_tokens": 0, "context_window": -1, "query_tokens": 0,
            "used_router": 0, "hot_tokens_materialized": 0, "warm_tokens_materialized": 0,
            "cold_tokens_materialized": 0, "reconstructed_tokens": 0, "warm_chunk_decodes": 0,
            "cold_chunk_decodes": 0, "cold_chunks_touched": 0, "cold_chunk_cache_hits": 0,
            "cold_chunk_cache_misses": 0,
        }

    def get_last_access_stats(self) -> Dict[str, int]:
        return dict(self.last_access_stats)

    @property
    def current_tier(self) -> str:
        if self.total_tokens < self.hot_capacity:
            return "hot"
        if self.total_tokens < self.hot_capacity + self.warm_capacity:
            return "warm"
        return "cold"

    @property
    def hot_keys(self) -> torch.Tensor:
        """[T_hot, H, D] view of the hot tier (oldest first)."""
        h = self._hot_head
        return self._hot_k[:, h:h + self.num_hot].permute(1, 0, 2)

    @property
    def hot_values(self) -> torch.Tensor:
        h = self._hot_head
        return self._hot_v[:, h:h + self.num_hot].permute(1, 0, 2)

    @property
    def warm_keys(self) -> CompressedTensorMLX:
        """The warm tier's key codes (cache.py:45-46), oldest first."""
        return self._wk.view() if isinstance(self._wk, _RingStore) else self._wk

    @warm_keys.setter
    def warm_keys(self, store: CompressedTensorMLX) -> None:
        self._wk = store

    @property
    def warm_values(self) -> CompressedTensorMLX:
        return self._wv.view() if isinstance(self._wv, _RingStore) else self._wv

    @warm_values.setter
    def warm_values(self, store: CompressedTensorMLX) -> None:
        self._wv = store

    # ------------------------------------------------------------------ helpers
    @property
    def _recency(self) -> bool:
        return self.config.tier_policy == "recency"

    @property
    def _subspace(self) -> bool:
        return self.config.ext_format

    def _fmt(self) -> K.WarmFormat:
        """The K quantizer's warm format, kept per quantizer object (its
        codebooks fix the format's shapes when it is built)."""
        memo = self._fmt_memo
        if memo is None or memo[0] is not self._kq:
            memo = self._fmt_memo = (self._kq, self._kq.warm_format())
        return memo[1]

    @property
    def _k_layout(self) -> int:
        """1 when K codes are score-table rows (``config.fused_score_tables``,
        subspace format, 16 + 16 subspaces, at most 4 query heads of the
        config per KV head)."""
        return int(self._subspace and self.config.fused_score_tables
                   and K.score_layout_ok(self._fmt(), self.config.num_heads, self.H))

    @property
    def _guarded(self) -> bool:
        """Score tables with the drift guard (``config.score_table_tolerance``):
        K's sparse values then carry the corrected-coordinate plane."""
        return bool(self._k_layout) and self.config.score_table_tolerance is not None

    def _tiled_pair(self, **kw) -> Tuple["TiledCodes", "TiledCodes"]:
        """Empty (K, V) tiled code sets; K as score-table rows when the kernel scores K that way."""
        fmt = self._fmt()
        return (TiledCodes(fmt, self.H, self.device, score_rows=bool(self._k_layout), exact_plane=self._guarded,
                           **kw),
                TiledCodes(fmt, self.H, self.device, **kw))

    def _codebook_key(self, rvq: bool = True) -> "_CodebookKey":
        """The quantizer pair and each codebook tensor with its version:
        differs when a quantizer is swapped or its codebooks are replaced
        (``calibrate_quantizer``) or written in place."""
        cbs = (self._kq.pq.codebooks, self._kq.rvq.codebooks if rvq else None,
               self._vq.pq.codebooks, self._vq.rvq.codebooks if rvq else None)
        return _CodebookKey((self._kq, self._vq) + cbs, tuple(None if t is None else t._version for t in cbs))

    def _guard_tensor(self) -> torch.Tensor:
        """The drift guard's [1, 65] input: the K codebooks' weights (rebuilt
        whenever a codebook changes) and the running bound on |V^| kept by the
        appends and the V codebooks."""
        key = self._codebook_key()
        if self._guard_key != key:
            self._guard[0, :64] = K.score_guard(self._kq.pq.codebooks, self._kq.rvq.codebooks, 0.0)[:64]
            vp, vr = self._vq.pq.codebooks.float(), self._vq.rvq.codebooks.float()
            vcb = (vp.abs().amax(-2) + vr.abs().amax(-2)).amax()
            torch.maximum(self._vabs, vcb.view(1), out=self._vabs)
            self._guard_key = key
        return self._guard

    def _ref_table_stats(self) -> torch.Tensor:
        """The reference-format score tables' guard statistics
        (``kernels.ref_table_stats``), rebuilt when a codebook changes."""
        kq, vq = self._kq, self._vq
        cbs = (kq.pq.codebooks, vq.pq.codebooks, kq.rvq_codebooks, vq.rvq_codebooks)
        key = _CodebookKey((kq, vq) + cbs, tuple(None if t is None else t._version for t in cbs))
        if self._ref_stats_key != key:
            self._ref_stats = K.ref_table_stats(*cbs)
            self._ref_stats_key = key
        return self._ref_stats

    def _entry_tables(self, rvq: bool) -> Tuple[torch.Tensor, torch.Tensor]:
        """The fused kernel's entry-major K and V tables (``kernels.entry_tables``),
        built once per codebook set (keyed like the guard, by the quantizers
        and their codebook tensors)."""
        cbs = [self._kq.pq.codebooks, self._kq.rvq.codebooks if rvq else None,
               self._vq.pq.codebooks, self._vq.rvq.codebooks if rvq else None]
        key = self._codebook_key(rvq)
        if self._tables_key != key:
            self._tables = (K.entry_tables(cbs[0], cbs[1]), K.entry_tables(cbs[2], cbs[3]))
            self._tables_key = key
        return self._tables

    def _dev16(self, t: torch.Tensor) -> torch.Tensor:
        """``t`` as fp16 on the cache's device (itself when it already is)."""
        if t.dtype is torch.float16 and t.device == self.device:
            return t
        return t.to(self.device, torch.float16)

    def _hot_append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append [T, H, D] tokens to the hot tier.  The buffers hold up to
        twice the hot capacity under the recency policy, so the live range
        moves to the front only once per hot_capacity appended tokens."""
        T = int(k.shape[0])
        need = self.num_hot + T
        h = self._hot_head
        cap = int(self._hot_k.shape[1])
        if h + need > cap:
            target = 2 * self.hot_capacity if self._recency else self.hot_capacity
            if need <= cap and 2 * need <= cap:
                self._hot_k[:, :self.num_hot] = self._hot_k[:, h:h + self.num_hot].clone()
                self._hot_v[:, :self.num_hot] = self._hot_v[:, h:h + self.num_hot].clone()
            else:
                cap = max(need, min(max(target, need), max(2 * cap, 32)))
                nk = torch.zeros((self.H, cap, self.D), dtype=torch.float16, device=self.device)
                nv = torch.zeros_like(nk)
                nk[:, : self.num_hot] = self._hot_k[:, h:h + self.num_hot]
                nv[:, : self.num_hot] = self._hot_v[:, h:h + self.num_hot]
                self._hot_k, self._hot_v = nk, nv
            self._hot_head = h = 0
        k, v = self._dev16(k), self._dev16(v)
        if T and k.is_contiguous() and v.is_contiguous() and not (k.data_ptr() % 16 or v.data_ptr() % 16) \
                and self.D % 8 == 0:
            # one launch for K and V, which also folds |v| into the drift guard's V bound
            L.call("rfsn_hot_append", k.data_ptr(), v.data_ptr(), self.H * self.D, T, self.H, self.D,
                   self._hot_k.data_ptr(), self._hot_v.data_ptr(), cap, h + self.num_hot,
                   self._vabs.data_ptr() if self._guarded else None, K._stream(k))
        else:
            self._hot_k[:, h + self.num_hot:h + need] = k.permute(1, 0, 2)
            self._hot_v[:, h + self.num_hot:h + need] = v.permute(1, 0, 2)
            if T and self._guarded:
                torch.maximum(self._vabs, v.abs().amax().float().view(1), out=self._vabs)
        self.num_hot = need

    def _hot_append_args(self, stream: Optional[int] = None) -> Tuple[Optional[int], int]:
        """(drift guard's V bound address or None, stream) of ``_try_hot_append``:
        fixed while the quantizers stay, so a decode session computes them once
        per rebuild."""
        return (self._vabs.data_ptr() if self._guarded else None,
                L.stream_handle(self.device) if stream is None else stream)

    def _session_layout(self) -> Optional[tuple]:
        """What a prepared fused launch's segments depend on, then the warm
        length: the warm tiled arrays (addresses, head tile, capacity), the
        cold tier's extent, the hot buffers and the codebooks.  Two layouts
        equal but for the last entry describe launches that differ only in
        the hot range and the length of the warm segment.  None when the
        warm tier has no tiled store."""
        if self._warm_tiled is None:
            return None
        warm = tuple((tuple(t.data_ptr() for t in w.t.values() if t is not None), w.head, w.cap)
                     for w in self._warm_tiled)
        return (warm, self.num_cold, len(self.cold_chunk_metadata), self._hot_k.data_ptr(),
                self._hot_v.data_ptr(), int(self._hot_k.shape[1]), self._codebook_key(bool(self._fmt().rvq_subspaces)),
                self.num_warm)

    def _hot_rows(self, k: torch.Tensor, v: torch.Tensor) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
        """New tokens [T, H, D] as device fp16 rows that a fused launch can
        append itself (``rfsn_fused_params.app_*``): the hot tier holds them
        without demoting (recency, num_hot + T <= hot_capacity, T <= 32), its
        buffers hold them at the current head, and the rows are 16-byte
        aligned.  None otherwise (the tokens then go through ``update``)."""
        T = k.shape[0]
        if not self._recency or not 0 < T <= K.TILE or self.num_hot + T > self.hot_capacity:
            return None
        if self._hot_head + self.num_hot + T > self._hot_k.shape[1]:
            return None
        f16 = torch.float16
        if not (k.dtype is f16 and k.is_contiguous() and k.device == self.device):
            k = k.to(self.device, f16).contiguous()
        if not (v.dtype is f16 and v.is_contiguous() and v.device == self.device):
            v = v.to(self.device, f16).contiguous()
        if k.shape != (T, self.H, self.D) or v.shape != (T, self.H, self.D):
            raise ValueError(f"new_keys and new_values must be [T, {self.H}, {self.D}]")
        if k.data_ptr() % 16 or v.data_ptr() % 16:
            return None
        return k, v

    def _try_hot_append(self, k: torch.Tensor, v: torch.Tensor,
                        args: Optional[Tuple[Optional[int], int]] = None) -> bool:
        """The decode loop's common append (recency tiers): new tokens [T, H, D]
        that the hot tier holds without demoting any (num_hot + T <=
        hot_capacity) and its buffers hold at the current head.  One
        ``rfsn_hot_append`` launch, which also folds |v| into the drift
        guard's V bound, on the current stream (``args``: the
        ``_hot_append_args`` to use instead).  Returns False, with the cache
        untouched, otherwise."""
        T = int(k.shape[0])
        if not self._recency or not T or self.num_hot + T > self.hot_capacity:
            return False
        t0 = self._hot_head + self.num_hot
        cap = int(self._hot_k.shape[1])
        if t0 + T > cap:
            return False
        if k.device != self.device or k.dtype != torch.float16 or not k.is_contiguous():
            k = k.to(self.device, torch.float16).contiguous()
        if v.device != self.device or v.dtype != torch.float16 or not v.is_contiguous():
            v = v.to(self.device, torch.float16).contiguous()
        if tuple(k.shape) != (T, self.H, self.D) or tuple(v.shape) != (T, self.H, self.D):
            raise ValueError(f"new_keys and new_values must be [T, {self.H}, {self.D}]")
        vabs, stream = self._hot_append_args(K._stream(k)) if args is None else args
        L.call("rfsn_hot_append", k.data_ptr(), v.data_ptr(), self.H * self.D, T, self.H, self.D,
               self._hot_k.data_ptr(), self._hot_v.data_ptr(), cap, t0, vabs, stream)
        self.num_hot += T
        self.total_tokens += T
        return True

    def decode_session(self, q: torch.Tensor, quantizer: QuantizerArg,
                       router: Optional[AsyncHierarchicalRouterMLX] = None, cold_attended: int = 0,
                       out: Optional[torch.Tensor] = None) -> "DecodeSession":
        """A prepared decode loop over this cache (``DecodeSession``)."""
        return DecodeSession(self, q, quantizer, router, cold_attended, out)

    def _hot_pop_oldest(self, n: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """Remove and return the n oldest hot tokens as [n, H, D] (copies,
        head-major in memory, as the warm encode reads them)."""
        h = self._hot_head
        k = self._hot_k[:, h:h + n].clone().permute(1, 0, 2)
        v = self._hot_v[:, h:h + n].clone().permute(1, 0, 2)
        self._hot_head += n
        self.num_hot -= n
        return k, v

    def _warm_tiled_append(self, ck: CompressedTensorMLX, cv: CompressedTensorMLX) -> None:
        """Mirror appended warm codes into the tiled layout of the fused kernel
        (for the reference format only the PQ codes, used while no RVQ row is
        active)."""
        fmt = self._fmt()
        if not fmt.fused_ok:
            return
        if self._warm_tiled is None:
            self._warm_tiled = self._tiled_pair()
        for tiled, store, qz in zip(self._warm_tiled, (ck, cv), (self._kq, self._vq)):
            if self._subspace:
                tiled.append(*_plain_head_major(store), qz.pq.codebooks, qz.rvq_codebooks)
            else:
                tiled.append(store.pq_codes.permute(1, 0, 2).contiguous(), None, None, None)

    # ------------------------------------------------------------------ update
    def update(self, new_keys: torch.Tensor, new_values: torch.Tensor, quantizer: QuantizerArg,
               disk_dir: Optional[Path] = None) -> None:
        """cache.py:89-120 (arrival policy) / newest-in-hot (recency policy)."""
        if tuple(new_keys.shape) != tuple(new_values.shape):
            raise ValueError("new_keys and new_values must have identical shapes")
        if new_keys.dim() != 3 or new_keys.shape[1] != self.H or new_keys.shape[2] != self.D:
            raise ValueError(f"new_keys must be [T, {self.H}, {self.D}]")
        self.quantizer = quantizer
        self._kq, self._vq = _pair(quantizer)
        keys, values = self._dev16(new_keys), self._dev16(new_values)
        num_tokens = int(keys.shape[0])
        if num_tokens and self._guarded and not (self._recency and num_tokens <= self.hot_capacity):
            # tokens that skip the hot tier (whose append folds its own |v|)
            torch.maximum(self._vabs, values.abs().amax().float().view(1), out=self._vabs)
        if self._recency:
            self._update_recency(keys, values, disk_dir)
        else:
            offset = 0
            hot_space = max(self.hot_capacity - self.num_hot, 0)
            if hot_space > 0 and offset < num_tokens:
                take = min(hot_space, num_tokens - offset)
                self._hot_append(keys[offset:offset + take], values[offset:offset + take])
                offset += take
            warm_space = max(self.warm_capacity - self.num_warm, 0)
            if warm_space > 0 and offset < num_tokens:
                take = min(warm_space, num_tokens - offset)
                self._add_to_warm(keys[offset:offset + take], values[offset:offset + take])
                offset += take
            if offset < num_tokens:
                self._add_to_cold(keys[offset:], values[offset:], disk_dir)
        self.total_tokens += num_tokens

    append = update

    HOT_BLOCK = 32  # hot tokens are demoted in multiples of one tile

    def _update_recency(self, keys, values, disk_dir) -> None:
        """Hot keeps the newest tokens, at most ``hot_capacity``; when an
        append overflows it, the oldest hot tokens are demoted to warm in
        multiples of HOT_BLOCK (a block of new tokens is demoted as it is).
        When warm overflows, its oldest tokens move to cold up to the next
        cold chunk boundary, so migrations move whole chunks.  A bulk fill of
        T >= hot_capacity tokens leaves exactly hot_capacity hot."""
        T = int(keys.shape[0])
        # tokens that never stay hot go straight to warm/cold, in order
        keep_new = min(T, self.hot_capacity)
        direct = T - keep_new
        overflow_hot = max(self.num_hot + keep_new - self.hot_capacity, 0)
        if overflow_hot and self.hot_capacity >= self.HOT_BLOCK:
            overflow_hot = -(-overflow_hot // self.HOT_BLOCK) * self.HOT_BLOCK
        demoted_k, demoted_v = [], []
        if overflow_hot:
            k_old, v_old = self._hot_pop_oldest(min(overflow_hot, self.num_hot))
            demoted_k.append(k_old)
            demoted_v.append(v_old)
        if direct:
            demoted_k.append(keys[:direct])
            demoted_v.append(values[:direct])
        if demoted_k:
            dk = demoted_k[0] if len(demoted_k) == 1 else torch.cat(demoted_k, 0)
            dv = demoted_v[0] if len(demoted_v) == 1 else torch.cat(demoted_v, 0)
            n = int(dk.shape[0])
            excess = self.num_warm + n - self.warm_capacity
            if excess > 0:
                # the oldest tokens (warm first, then demoted) move to cold up
                # to the next chunk boundary of their absolute positions
                chunk = self.config.chunk_tokens
                cut = -(-(self.num_cold + excess) // chunk) * chunk - self.num_cold
                cut = min(cut, self.num_warm + n)
                spill_warm = min(self.num_warm, cut)
                if spill_warm:
                    self._warm_to_cold(spill_warm, disk_dir)
                to_cold = cut - spill_warm
                if to_cold:
                    self._add_to_cold(dk[:to_cold], dv[:to_cold], disk_dir)
                    dk, dv = dk[to_cold:], dv[to_cold:]
            if dk.shape[0]:
                self._add_to_warm(dk, dv)
        self._hot_append(keys[direct:], values[direct:])

    def _add_to_warm(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """cache.py:122-132.  Under a subspace format that the one-launch
        encode serves, K and V share one launch whose head-major codes feed
        the tiled store as they are."""
        hm = _encode_pair_head_major(keys, values, self._kq, self._vq) if self._subspace else None
        if hm is not None and isinstance(self._wk, _RingStore) and self._warm_tiled is not None \
                and self._fmt().fused_ok:
            # one launch: the tiled stores and the reference-layout rings
            if TiledCodes.append_pair(*self._warm_tiled, hm[0], hm[1], self._kq, self._vq,
                                      rings=(self._wk, self._wv)):
                self.num_warm += int(keys.shape[0])
                return
        if hm is None:
            ck = _compress_tensor_sequence(keys, self._kq)
            cv = _compress_tensor_sequence(values, self._vq)
        else:
            plain = not isinstance(self._wk, _RingStore)  # a plain store keeps contiguous codes
            ck, cv = _head_major_store(hm[0], plain), _head_major_store(hm[1], plain)
        if isinstance(self._wk, _RingStore):
            self._wk.append(ck)
            self._wv.append(cv)
        else:
            self.warm_keys = _append_compressed_tensor(self.warm_keys, ck)
            self.warm_values = _append_compressed_tensor(self.warm_values, cv)
        if hm is None:
            self._warm_tiled_append(ck, cv)
        elif self._fmt().fused_ok:
            if self._warm_tiled is None:
                self._warm_tiled = self._tiled_pair()
            if not TiledCodes.append_pair(*self._warm_tiled, hm[0], hm[1], self._kq, self._vq):
                for tiled, codes, qz in zip(self._warm_tiled, hm, (self._kq, self._vq)):
                    tiled.append(*codes, qz.pq.codebooks, qz.rvq_codebooks)
        self.num_warm += int(keys.shape[0])

    def _warm_to_cold(self, n: int, disk_dir) -> None:
        """Move the n oldest warm tokens (already encoded) to the cold tier.
        Whole tiles leave the tiled store by moving its head; otherwise the
        tiled store is rebuilt from the remaining codes."""
        if isinstance(self._wk, _RingStore):
            ck, cv = self._wk.pop_front(n), self._wv.pop_front(n)
        else:
            ck = _slice_compressed_tensor(self.warm_keys, 0, n)
            cv = _slice_compressed_tensor(self.warm_values, 0, n)
            self.warm_keys = _slice_compressed_tensor(self.warm_keys, n, self.num_warm)
            self.warm_values = _slice_compressed_tensor(self.warm_values, n, self.num_warm)
        self._store_cold(ck, cv, disk_dir)
        self.num_warm -= n
        if self._warm_tiled is not None:
            if n % K.TILE == 0:
                for t in self._warm_tiled:
                    t.pop_front_tiles(n // K.TILE)
            else:
                self._warm_tiled = self._tiled_pair()
                if self.num_warm:
                    self._warm_tiled_append(self.warm_keys, self.warm_values)

    # ------------------------------------------------------------------ cold tier
    def _cold_start_token(self) -> int:
        if self._recency:
            return self.num_cold
        return self.num_hot + self.num_warm + self.num_cold

    def _add_to_cold(self, keys, values, disk_dir) -> None:
        """cache.py:134-191: encode per chunk and store."""
        chunk = self.config.chunk_tokens
        start_token = self._cold_start_token()
        for offset in range(0, int(keys.shape[0]), chunk):
            end = min(offset + chunk, int(keys.shape[0]))
            # align pieces to chunk boundaries of the absolute position
            ck = _compress_tensor_sequence(keys[offset:end], self._kq)
            cv = _compress_tensor_sequence(values[offset:end], self._vq)
            self._store_cold(ck, cv, disk_dir, start=start_token + offset)

    def _store_cold(self, ck: CompressedTensorMLX, cv: CompressedTensorMLX, disk_dir, start: Optional[int] = None
                    ) -> None:
        """Store encoded tokens starting at absolute token ``start`` as cold chunks."""
        chunk = self.config.chunk_tokens
        s0 = self._cold_start_token() if start is None else start
        n = ck.num_tokens
        o = 0
        while o < n:
            cstart = s0 + o
            cid = cstart // chunk
            take = min(n - o, (cid + 1) * chunk - cstart) if self._recency else min(n - o, chunk)
            k_part = _slice_compressed_tensor(ck, o, o + take)
            v_part = _slice_compressed_tensor(cv, o, o + take)
            self._store_cold_piece(cid, cstart, k_part, v_part, disk_dir)
            self.num_cold += take
            o += take

    def _store_cold_piece(self, cid, cstart, ck, cv, disk_dir) -> None:
        n = ck.num_tokens
        meta = next((m for m in self.cold_chunk_metadata if m["chunk_id"] == cid), None)
        if self.config.cold_medium == "npz":
            disk_root = Path(self.config.disk_cache_dir) if disk_dir is None else Path(disk_dir)
            disk_root.mkdir(parents=True, exist_ok=True)
            path = chunk_file_path(disk_root, self.layer_idx, cid)
            if meta is not None and cid in self.cold_chunk_paths_by_id:
                if cstart != meta["end_token"]:
                    raise ValueError(
                        "Cold chunk append must be contiguous with existing metadata: "
                        f"chunk_id={cid} start={cstart} expected={meta['end_token']}")
                loaded = load_compressed_chunk(self.cold_chunk_paths_by_id[cid], self.device)
                ck = _append_compressed_tensor(compressed_tensor_from_loaded(loaded, "key"), ck)
                cv = _append_compressed_tensor(compressed_tensor_from_loaded(loaded, "value"), cv)
                save_compressed_chunk(path, ck, cv)
                meta["end_token"] += n
                meta["num_tokens"] += n
                meta["path"] = str(path)
            else:
                save_compressed_chunk(path, ck, cv)
                self.cold_chunk_paths.append(path)
                self.cold_chunk_paths_by_id[cid] = path
                self.cold_chunk_metadata.append({"chunk_id": cid, "start_token": cstart, "end_token": cstart + n,
                                                 "num_tokens": n, "path": str(path)})
            return
        # pinned host memory
        if meta is not None:
            if cstart != meta["end_token"]:
                raise ValueError(
                    "Cold chunk append must be contiguous with existing metadata: "
                    f"chunk_id={cid} start={cstart} expected={meta['end_token']}")
            old = self._cold_pinned[cid]
            ck = _append_compressed_tensor(_to_device_store(old["key"], self.device), ck)
            cv = _append_compressed_tensor(_to_device_store(old["value"], self.device), cv)
            meta["end_token"] += n
            meta["num_tokens"] += n
            stale = self._cold_slots.pop(cid, None)
            if stale is not None:
                self._slot_cid[stale["slot"]] = -1
            if self._side is not None:
                self._side.synchronize()  # a queued copy may still read the pinned bytes rewritten below
        else:
            meta = {"chunk_id": cid, "start_token": cstart, "end_token": cstart + n, "num_tokens": n,
                    "path": f"pinned:{cid}"}
            self.cold_chunk_metadata.append(meta)
            self.cold_chunk_metadata.sort(key=lambda m: m["start_token"])
        self._cold_pinned[cid] = self._pin_chunk(cid, ck, cv)

    # Pinned chunks live in arenas of ARENA_CHUNKS consecutive chunk ids and
    # device slots in one buffer of cold_slots slots, so that a run of
    # consecutive chunks copied into consecutive slots is one hipMemcpyAsync.
    ARENA_CHUNKS = 64

    def _chunk_split(self) -> Tuple[int, int]:
        """Bytes of one chunk's tiled K codes and of its V codes (K first in
        the chunk's pinned buffer and device slot)."""
        chunk = K.round_up(self.config.chunk_tokens, K.TILE)
        return (TiledCodes.nbytes(self._fmt(), self.H, chunk, self._guarded and self._fmt().sparse_k > 0),
                TiledCodes.nbytes(self._fmt(), self.H, chunk))

    def _chunk_bytes(self) -> int:
        """Bytes of one chunk's tiled K and V codes (its pinned buffer and device slot)."""
        return sum(self._chunk_split())

    def _arena_view(self, cid: int) -> torch.Tensor:
        nb = self._chunk_bytes()
        blk = cid // self.ARENA_CHUNKS
        arena = self._cold_arena.get(blk)
        if arena is None:
            arena = torch.zeros(self.ARENA_CHUNKS * nb, dtype=torch.uint8, pin_memory=True)
            self._cold_arena[blk] = arena
        o = (cid % self.ARENA_CHUNKS) * nb
        return arena[o:o + nb]

    def _pin_chunk(self, cid: int, ck: CompressedTensorMLX, cv: CompressedTensorMLX) -> dict:
        """Keep a chunk in pinned host memory: the reference layout (for decode
        and NPZ export) and, for the subspace format, the tiled layout that
        prefetch copies into device slots (K then V in one buffer)."""
        entry = {"key": _to_host_store(ck), "value": _to_host_store(cv)}
        if self._subspace and self._fmt().fused_ok:
            fmt = self._fmt()
            chunk = K.round_up(self.config.chunk_tokens, K.TILE)
            kb, vb = self._chunk_split()
            dev_buf = torch.zeros(kb + vb, dtype=torch.uint8, device=self.device)
            host_buf = self._arena_view(cid)
            for i, (name, store, qz) in enumerate((("key", ck, self._kq), ("value", cv, self._vq))):
                o, n = (0, kb) if i == 0 else (kb, vb)
                dev_t = TiledCodes(fmt, self.H, self.device, cap=chunk, backing=dev_buf[o:o + n],
                                   score_rows=i == 0 and bool(self._k_layout), exact_plane=i == 0 and self._guarded)
                dev_t.append(*_plain_head_major(store), qz.pq.codebooks, qz.rvq_codebooks)
                host_t = TiledCodes(fmt, self.H, None, pinned=True, cap=chunk, backing=host_buf[o:o + n],
                                    score_rows=i == 0 and bool(self._k_layout), exact_plane=i == 0 and self._guarded)
                host_t.len = dev_t.len
                entry[f"{name}_tiled"] = host_t
            host_buf.copy_(dev_buf)
            entry["tiled_buf"] = host_buf
        return entry

    def cold_chunk_ids(self) -> List[int]:
        """Ids of the cold chunks this cache holds, ascending (chunks are only
        ever added or replaced in place, so the list is rebuilt when the
        count changes)."""
        src = self._cold_pinned if self.config.cold_medium == "pinned" else self.cold_chunk_paths_by_id
        if self._cold_ids[0] != id(src) or self._cold_ids[1] != len(src):
            self._cold_ids = (id(src), len(src), sorted(src))
        return self._cold_ids[2]

    def has_cold_chunk(self, chunk_id: int) -> bool:
        if self.config.cold_medium == "pinned":
            return chunk_id in self._cold_pinned
        return chunk_id in self.cold_chunk_paths_by_id

    def load_cold_chunk(self, chunk_id: int) -> Dict[str, torch.Tensor]:
        """cache.py:193-194 (NPZ) / the pinned chunk's arrays (pinned)."""
        if self.config.cold_medium == "pinned":
            e = self._cold_pinned[chunk_id]
            return {"key": e["key"], "value": e["value"]}
        return load_compressed_chunk(self.cold_chunk_paths_by_id[chunk_id], self.device)

    # ------------------------------------------------------------------ NPZ interop
    def export_cold_chunks(self, directory: Union[str, Path]) -> List[Path]:
        """Write every pinned cold chunk as ``layer{L}_chunk{id}.npz`` in the
        reference's chunk schema (storage.py:113-135), which the reference's
        ``load_compressed_chunk`` reads (the subspace format adds its sparse
        arrays and keeps its own code shapes)."""
        if self.config.cold_medium != "pinned":
            raise RuntimeError("export_cold_chunks needs cold_medium='pinned' (NPZ caches already hold files)")
        root = Path(directory)
        paths = []
        for m in self.cold_chunk_metadata:
            e = self._cold_pinned[m["chunk_id"]]
            path = chunk_file_path(root, self.layer_idx, m["chunk_id"])
            save_compressed_chunk(path, e["key"], e["value"])
            paths.append(path)
        return paths

    def import_cold_chunks(self, directory: Union[str, Path], quantizer: QuantizerArg) -> int:
        """Load ``layer{L}_chunk{id}.npz`` files (the reference's chunk schema,
        storage.py:113-151) into the pinned cold tier of an empty cache under
        the recency policy: chunk ``id`` holds the tokens from
        ``id * cold_chunk_tokens``, so the ids must run 0, 1, ... and every
        chunk but the last must be full.  Later appends continue after them.
        Returns the number of tokens loaded."""
        if self.config.cold_medium != "pinned" or not self._recency:
            raise RuntimeError("import_cold_chunks needs cold_medium='pinned' and tier_policy='recency'")
        if self.total_tokens:
            raise RuntimeError("import_cold_chunks loads into an empty cache")
        chunk = self.config.chunk_tokens
        prefix = f"layer{self.layer_idx}_chunk"
        found = {}
        for path in Path(directory).glob(f"{prefix}*.npz"):
            tail = path.stem[len(prefix):]
            if tail.isdigit():
                found[int(tail)] = path
        ids = sorted(found)
        if ids != list(range(len(ids))):
            raise ValueError(f"chunk files must be layer{self.layer_idx}_chunk0.npz, chunk1, ... without gaps")
        self.quantizer = quantizer
        self._kq, self._vq = _pair(quantizer)
        for cid in ids:
            loaded = load_compressed_chunk(found[cid], self.device)
            ck = compressed_tensor_from_loaded(loaded, "key")
            cv = compressed_tensor_from_loaded(loaded, "value")
            if ck.num_heads != self.H or (ck.subspace != self._subspace):
                raise ValueError(f"{found[cid].name}: heads or code format differ from this cache's")
            n = ck.num_tokens
            if n > chunk or (n < chunk and cid != ids[-1]) or cv.num_tokens != n:
                raise ValueError(f"{found[cid].name}: every chunk but the last must hold {chunk} tokens")
            self._store_cold_piece(cid, cid * chunk, ck, cv, None)
            self.num_cold += n
        self.total_tokens = self.num_cold
        return self.num_cold

    def _chunk_store(self, loaded, prefix: str) -> CompressedTensorMLX:
        if self.config.cold_medium == "pinned":
            return _to_device_store(loaded[prefix], self.device)
        return compressed_tensor_from_loaded(loaded, prefix)

    def _slot_pool(self) -> torch.Tensor:
        if self._slot_buf is None:
            self._slot_buf = torch.empty(self._cold_slot_limit * self._chunk_bytes(), dtype=torch.uint8,
                                         device=self.device)
            self._slot_cid = [-1] * self._cold_slot_limit
            self._slot_reader = [None] * self._cold_slot_limit
        return self._slot_buf

    PREPARED = "prepared"
    READ_EVENTS = 8

    def _reader_done(self, ev, cache: Dict[Any, bool]) -> bool:
        if ev is None:
            return True
        if ev == self.PREPARED:
            return False
        if ev not in cache:
            st = L.load().rfsn_event_query(ev)
            if st < 0:
                L.check(st, "rfsn_event_query")
            cache[ev] = st == 1
        return cache[ev]

    def _busy_slots(self) -> set:
        """Slots whose last readers may still be running.  Slots read by
        prepared steps count as idle once the launch stream has drained
        (queried, without waiting)."""
        if self.PREPARED in self._slot_reader:
            st = L.load().rfsn_stream_query(L.stream_handle(self.device))
            if st < 0:
                L.check(st, "rfsn_stream_query")
            if st == 1:
                self._slot_reader = [None if ev == self.PREPARED else ev for ev in self._slot_reader]
        seen: Dict[Any, bool] = {}
        return {j for j, ev in enumerate(self._slot_reader) if not self._reader_done(ev, seen)}

    def _wait_readers(self, slots: Sequence[int], stream: Optional[int] = None) -> None:
        """Block the host until the launches that read ``slots`` are done
        (the copies that overwrite them are then queued with no device wait,
        see ``SideStream.drain``)."""
        seen: Dict[Any, bool] = {}
        evs = {self._slot_reader[j] for j in slots}
        if self.PREPARED in evs:
            self._side_stream().drain(L.stream_handle(self.device) if stream is None else stream)
            return
        for ev in evs:
            if not self._reader_done(ev, seen):
                L.call("rfsn_event_synchronize", ev)

    def _record_reads(self, slots: Sequence[int], prepared: bool = False) -> None:
        """Mark ``slots`` as read by the launches just queued on the current stream."""
        if not slots:
            return
        if prepared:
            for j in slots:
                self._slot_reader[j] = self.PREPARED
            return
        if len(self._read_events) < self.READ_EVENTS:
            e = C.c_void_p()
            L.call("rfsn_event_create", C.byref(e))
            self._read_events.append(e.value)
            ev = e.value
        else:
            # re-recording an event only moves it later: its slots wait longer, never less
            ev = self._read_events[self._read_next]
            self._read_next = (self._read_next + 1) % self.READ_EVENTS
        L.call("rfsn_event_record", ev, L.stream_handle(self.device))
        for j in slots:
            self._slot_reader[j] = ev

    def _slot_entry(self, cid: int, slot: int) -> dict:
        """The slot's K and V views (built once per slot) holding chunk ``cid``."""
        if slot not in self._slot_views:
            kb, vb = self._chunk_split()
            nb = kb + vb
            pool = self._slot_pool()
            cap = K.round_up(self.config.chunk_tokens, K.TILE)
            self._slot_views[slot] = tuple(
                TiledCodes(self._fmt(), self.H, self.device, cap=cap, backing=pool[o:o + n],
                           score_rows=i == 0 and bool(self._k_layout), exact_plane=i == 0 and self._guarded)
                for i, (o, n) in enumerate(((slot * nb, kb), (slot * nb + kb, vb))))
        e = self._cold_pinned[cid]
        kt, vt = self._slot_views[slot]
        kt.len, vt.len = e["key_tiled"].len, e["value_tiled"].len
        return {"slot": slot, "key": kt, "value": vt}

    def _stage_cold(self, chunk_ids: Sequence[int]) -> Tuple[Dict[int, dict], List[int], list, List[int]]:
        """Device slots for ``chunk_ids``: (slots by id, ids still to copy,
        their (dst, src, bytes) copies, the slots those copies overwrite).
        Resident chunks keep their slot and become the most recently used.
        The missing ones, in runs of consecutive ids inside one pinned arena,
        take the longest windows of consecutive slots that hold no chunk of
        ``chunk_ids``, avoiding slots whose readers may still run, then
        preferring free slots and the least recently used; each window is
        one copy."""
        if self.config.cold_medium != "pinned":
            raise RuntimeError("cold-chunk prefetch needs cold_medium='pinned'")
        ids = list(dict.fromkeys(int(c) for c in chunk_ids))
        S = self._cold_slot_limit
        if len(ids) > S:
            raise ValueError(f"{len(ids)} cold chunks requested; the device slot pool holds "
                             f"{S} (raise cold_slots)")
        out: Dict[int, dict] = {}
        for cid in ids:
            if cid in self._cold_slots:
                self._cold_slots.move_to_end(cid)
                out[cid] = self._cold_slots[cid]
        missing = sorted(cid for cid in ids if cid not in out)
        if not missing:
            return out, [], [], []
        pool = self._slot_pool()
        nb = self._chunk_bytes()
        lru = [d["slot"] for d in self._cold_slots.values()]
        fetched, copies, targets = [], [], []
        busy = self._busy_slots()
        for j, part in plan_slot_windows(self._slot_cid, lru, set(ids), missing, self.ARENA_CHUNKS, busy):
            targets.extend(range(j, j + len(part)))
            for t, cid in enumerate(part):
                old = self._slot_cid[j + t]
                if old >= 0:
                    del self._cold_slots[old]
                self._slot_cid[j + t] = cid
                dev = self._slot_entry(cid, j + t)
                self._cold_slots[cid] = dev
                out[cid] = dev
                fetched.append(cid)
            src = self._cold_pinned[part[0]]["tiled_buf"]
            copies.append((pool.data_ptr() + j * nb, src.data_ptr(), len(part) * nb))
        return out, fetched, copies, targets

    def _side_stream(self) -> K.SideStream:
        if self._side is None:
            self._side = K.SideStream()
        return self._side

    def prefetch_cold_chunks(self, chunk_ids: Sequence[int], wait: bool = True) -> Dict[int, dict]:
        """Make pinned chunks resident in device slots.  The copies are
        issued with hipMemcpyAsync on a side stream once the launches that
        last read the slots they overwrite are done (slots no queued launch
        reads are preferred).  With ``wait`` the current stream waits on
        them now; otherwise the next attention call does (a prefetch one
        decode step ahead, overlapped with the current step)."""
        out, _, copies, targets = self._stage_cold(chunk_ids)
        if copies:
            side = self._side_stream()
            self._wait_readers(targets)
            side.prefetch(copies)
            if wait:
                side.make_current_wait(self.device)
            else:
                self._copies_pending = True
        return out

    def _order_after_copies(self) -> None:
        """The current stream waits for every copy queued so far (cheap)."""
        if self._copies_pending:
            self._side_stream().make_current_wait(self.device)
            self._copies_pending = False

    def resident_cold_chunk(self, chunk_id: int) -> Optional[dict]:
        """The device slot holding a pinned chunk, or None."""
        return self._cold_slots.get(int(chunk_id))

    def evict_cold_slots(self, chunk_ids: Optional[Sequence[int]] = None) -> None:
        """Drop chunks (every chunk by default) from the device slots; the
        slot buffer is kept and its last readers are still tracked."""
        if chunk_ids is None:
            self._cold_slots.clear()
            self._slot_cid = [-1] * len(self._slot_cid)
            return
        for cid in chunk_ids:
            dev = self._cold_slots.pop(int(cid), None)
            if dev is not None:
                self._slot_cid[dev["slot"]] = -1

    def note_reads(self, chunk_ids: Sequence[int]) -> None:
        """Record that the launches just queued on the current stream (a
        prepared step, which does not record it itself) read these chunks'
        slots, so that later copies wait only for those launches."""
        self._record_reads([self._cold_slots[int(c)]["slot"] for c in chunk_ids if int(c) in self._cold_slots])

    def wait_for_prefetch(self) -> None:
        """Order the current stream after the copies of ``prefetch_cold_chunks(wait=False)``
        (attention calls do this themselves; prepared launches need it)."""
        self._order_after_copies()

    # ------------------------------------------------------------------ windows
    def _max_query_position(self, query_positions, current_position) -> int:
        if query_positions is not None:
            if isinstance(query_positions, torch.Tensor):
                return int(query_positions.max().item())
            return int(np.max(np.asarray(query_positions, dtype=np.int64)))
        if current_position is not None:
            return current_position
        return max(self.total_tokens - 1, 0)

    def _window_bounds(self, query_positions, context_window, current_position):
        """cache.py:210-241."""
        def to_query_array(value):
            if value is None:
                return None
            if isinstance(value, torch.Tensor):
                return value.to(device=self.device, dtype=torch.int32)
            return torch.tensor(np.asarray(value), dtype=torch.int32, device=self.device)

        if self.total_tokens == 0:
            return 0, 0, to_query_array(query_positions)
        max_query = self._max_query_position(query_positions, current_position)
        window_end = min(max_query + 1, self.total_tokens)
        window_start = 0 if context_window is None else max(0, window_end - context_window)
        if query_positions is None:
            return window_start, window_end, None
        adjusted = to_query_array(query_positions) - window_start
        adjusted = torch.clamp(adjusted, min=-1).to(torch.int32)
        return window_start, window_end, adjusted

    @staticmethod
    def _overlap(start, end, span_start, span_end):
        a, b = max(start, span_start), min(end, span_end)
        return None if a >= b else (a, b)

    def _tier_spans(self) -> Dict[str, Tuple[int, int]]:
        """Absolute position span of the hot and warm tiers."""
        if self._recency:
            return {"warm": (self.num_cold, self.num_cold + self.num_warm),
                    "hot": (self.num_cold + self.num_warm, self.total_tokens)}
        return {"hot": (0, self.num_hot), "warm": (self.num_hot, self.num_hot + self.num_warm)}

    def _warm_chunks(self, ov) -> int:
        chunk = max(1, self.config.block_size_seq)
        return (ov[1] - ov[0] + chunk - 1) // chunk

    def _plan(self, start, end, stats, router, current_position, context_window, cold_chunks):
        """Which tier spans the window touches, in position order, with the
        reference's access counters (cache.py:250-342)."""
        spans = self._tier_spans()
        parts = []
        hov = self._overlap(start, end, *spans["hot"])
        wov = self._overlap(start, end, *spans["warm"])
        if hov is not None:
            stats["hot_tokens_materialized"] += hov[1] - hov[0]
        if wov is not None and self.quantizer is not None:
            n = wov[1] - wov[0]
            stats["warm_tokens_materialized"] += n
            stats["reconstructed_tokens"] += n
            stats["warm_chunk_decodes"] += self._warm_chunks(wov)
        cold = []
        if self.quantizer is not None and self.cold_chunk_metadata:
            loaded_by_router = {}
            if cold_chunks is not None:
                wanted = set(int(c) for c in cold_chunks)
                metas = [m for m in self.cold_chunk_metadata if m["chunk_id"] in wanted]
            else:
                if router is not None and current_position is not None and context_window is not None:
                    ct = self.config.chunk_tokens
                    top_k = max(1, (context_window + ct - 1) // ct)
                    router.prefetch_sync(current_position=current_position, context_window=context_window,
                                         top_k=top_k)
                metas = [m for m in self.cold_chunk_metadata
                         if self._overlap(start, end, m["start_token"], m["end_token"]) is not None]
            for m in metas:
                cid = m["chunk_id"]
                got = router.get_chunk(cid) if router is not None else None
                if got is None:
                    if router is not None:
                        stats["cold_chunk_cache_misses"] += 1
                else:
                    stats["cold_chunk_cache_hits"] += 1
                if cold_chunks is not None:
                    ov = (m["start_token"], m["end_token"])
                else:
                    ov = self._overlap(start, end, m["start_token"], m["end_token"])
                n = ov[1] - ov[0]
                stats["cold_tokens_materialized"] += n
                stats["reconstructed_tokens"] += n
                stats["cold_chunk_decodes"] += 1
                stats["cold_chunks_touched"] += 1
                cold.append((m, ov, got))
        if self._recency:
            order = [("cold", c) for c in cold] + [("warm", wov), ("hot", hov)]
        else:
            order = [("hot", hov), ("warm", wov)] + [("cold", c) for c in cold]
        return [(kind, x) for kind, x in order if x is not None]

    # ------------------------------------------------------------------ materialize
    def materialize_window(self, query_positions=None, context_window: Optional[int] = None,
                           router: Optional[AsyncHierarchicalRouterMLX] = None,
                           current_position: Optional[int] = None, cold_chunks: Optional[Sequence[int]] = None):
        """(keys [W, H, D], values [W, H, D], adjusted positions) (cache.py:344-393)."""
        if self.quantizer is None:
            raise RuntimeError("Cache cannot materialize values before update() provides a quantizer")
        start, end, adjusted = self._window_bounds(query_positions, context_window, current_position)
        stats = self._empty_access_stats()
        stats["window_start"], stats["window_end"] = start, end
        stats["window_tokens"] = max(0, end - start)
        stats["context_window"] = -1 if context_window is None else context_window
        stats["used_router"] = int(router is not None)
        plan = self._plan(start, end, stats, router, current_position, context_window, cold_chunks)
        spans = self._tier_spans()
        ks, vs = [], []
        for kind, x in plan:
            if kind == "hot":
                a, b = x[0] - spans["hot"][0], x[1] - spans["hot"][0]
                h = self._hot_head
                ks.append(self._hot_k[:, h + a:h + b].permute(1, 0, 2))
                vs.append(self._hot_v[:, h + a:h + b].permute(1, 0, 2))
            elif kind == "warm":
                a, b = x[0] - spans["warm"][0], x[1] - spans["warm"][0]
                ks.append(_decode_compressed_tensor(_slice_compressed_tensor(self.warm_keys, a, b), self._kq))
                vs.append(_decode_compressed_tensor(_slice_compressed_tensor(self.warm_values, a, b), self._vq))
            else:
                meta, ov, got = x
                if got is None or self.config.cold_medium == "pinned":
                    loaded = self.load_cold_chunk(meta["chunk_id"])
                else:
                    loaded = got
                a, b = ov[0] - meta["start_token"], ov[1] - meta["start_token"]
                kst = _slice_compressed_tensor(self._chunk_store(loaded, "key"), a, b)
                vst = _slice_compressed_tensor(self._chunk_store(loaded, "value"), a, b)
                ks.append(_decode_compressed_tensor(kst, self._kq))
                vs.append(_decode_compressed_tensor(vst, self._vq))
        self.last_access_stats = dict(stats)
        if not ks:
            empty = torch.zeros((0, self.H, self.D), dtype=torch.float16, device=self.device)
            return empty, empty, adjusted
        keys = ks[0] if len(ks) == 1 else torch.cat(ks, 0)
        values = vs[0] if len(vs) == 1 else torch.cat(vs, 0)
        return keys.contiguous(), values.contiguous(), adjusted

    # ------------------------------------------------------------------ attention
    def _fused_ok(self, q_heads: Optional[int] = None) -> bool:
        """The fused kernel serves the long-context warm format, and the
        reference format while no warm vector carries an RVQ correction (the
        reference's pq_only mode, threshold = inf).  K codes laid out as
        score-table rows serve at most 4 query heads per KV head."""
        if self._kq is None or not self._fmt().fused_ok or self._kq.warm_format() != self._vq.warm_format():
            return False
        if q_heads is not None and self._k_layout and not K.score_layout_ok(self._fmt(), q_heads, self.H):
            return False
        if self.num_warm and self._warm_tiled is None:
            return False
        if self._subspace:
            return self.num_cold == 0 or self.config.cold_medium == "pinned"
        no_rvq = int(self.warm_keys.rvq_codes.shape[0]) == 0 and int(self.warm_values.rvq_codes.shape[0]) == 0
        return no_rvq and self.num_cold == 0

    def attention_forward(self, q: torch.Tensor, pq_codebook=None, rvq_codebook=None, causal: bool = True,
                          query_positions=None, router: Optional[AsyncHierarchicalRouterMLX] = None,
                          current_position: Optional[int] = None, context_window: Optional[int] = None,
                          cold_chunks: Optional[Sequence[int]] = None) -> torch.Tensor:
        """cache.py:395-428.  Subspace-format caches run the fused kernel."""
        del pq_codebook, rvq_codebook
        if self.quantizer is None:
            raise RuntimeError("Cache cannot run attention before update() provides a quantizer")
        if q.shape[-1] != self.D or q.dim() != 3 or q.shape[1] % self.H:
            raise ValueError("q must be [B, Hq, D] with Hq a multiple of the cache's KV heads")
        if not self._fused_ok(int(q.shape[1])):
            if self._ref_ok(int(q.shape[1])):
                return self._ref_forward(q, causal, query_positions, router, current_position, context_window,
                                         cold_chunks)
            keys, values, adjusted = self.materialize_window(query_positions, context_window, router,
                                                             current_position, cold_chunks)
            self.last_access_stats["query_tokens"] = int(q.shape[0])
            if int(keys.shape[0]) == 0:
                return torch.zeros_like(q)
            return _blockwise_exact_attention(q=q, keys=keys, values=values, scale=self.D ** -0.5,
                                              block_size=self.config.block_size_seq, causal=causal,
                                              query_positions=adjusted)
        return self._fused_forward(q, causal, query_positions, router, current_position, context_window, cold_chunks)

    def _ref_ok(self, q_heads: int) -> bool:
        """The reference-format kernel (PQ + gated full-dimension RVQ decoded
        on the fly) serves this cache's codebooks and head grouping."""
        if self._kq is None:
            return False
        kq, vq = self._kq, self._vq
        M, C, _ = kq.pq.codebooks.shape
        if tuple(vq.pq.codebooks.shape) != tuple(kq.pq.codebooks.shape):
            return False
        kr, vr = kq.rvq_codebooks, vq.rvq_codebooks
        if (kr is None) != (vr is None) or (kr is not None and tuple(kr.shape) != tuple(vr.shape)):
            return False
        if self._subspace and kq.warm_format() != vq.warm_format():
            return False
        shared = kq.pq.codebooks.data_ptr() == vq.pq.codebooks.data_ptr()
        if not self._subspace:
            return K.ref_attention_ok(self.D, int(M), int(C), q_heads, self.H, shared)
        f = self._fmt()
        return K.ref_attention_ok(self.D, int(M), int(C), q_heads, self.H, shared, f.rvq_subspaces,
                                  f.rvq_centroids, f.sparse_k)

    def _ref_forward(self, q, causal, query_positions, router, current_position, context_window, cold_chunks):
        """attention_forward over tiers the tiled fused kernel does not serve
        (the reference format with active RVQ rows or cold chunks, formats
        outside the tiled kernel's head_dim 64 / M 8 or 16) without decoding
        the window into HBM: the plan of materialize_window (cache.py:344-393)
        becomes a segment table in window order -- the hot tier as exact rows
        of its ring, warm and cold stores as their codes -- and one launch
        attends it, rebuilding each K/V vector in registers with the decode's
        rounding (quantization.py:310-319)."""
        start, end, adjusted = self._window_bounds(query_positions, context_window, current_position)
        stats = self._empty_access_stats()
        stats["window_start"], stats["window_end"] = start, end
        stats["window_tokens"] = max(0, end - start)
        stats["context_window"] = -1 if context_window is None else context_window
        stats["used_router"] = int(router is not None)
        plan = self._plan(start, end, stats, router, current_position, context_window, cold_chunks)
        spans = self._tier_spans()
        B, Hq = int(q.shape[0]), int(q.shape[1])
        sub = self._fmt() if self._subspace else None
        # decode steps of the reference format: score tables with their drift
        # guard (config.score_table_tolerance), as the tiled path uses them;
        # they read the warm tier's codes from a head-major copy of its stores
        # (kept until a demotion or eviction replaces them), for windows with
        # enough coded tokens for the tables to beat the exact decode
        tol = self.config.score_table_tolerance
        coded = sum(x[1] - x[0] if kind == "warm" else x[1][1] - x[1][0] for kind, x in plan if kind != "hot")
        use_tables = (tol is not None and sub is None and B * Hq <= REF_TABLES_MAX_QUERY_HEADS
                      and coded >= K.ref_tables_min_tokens(Hq // self.H, B))
        segs, pos = [], 0
        for kind, x in plan:
            if kind == "hot":
                a, b = x[0] - spans["hot"][0], x[1] - spans["hot"][0]
                hk, hv = self._hot_k, self._hot_v
                segs.append(K.ref_exact_segment(hk, hv, hk.stride(1), hk.stride(0), self._hot_head + a, b - a, pos))
            elif kind == "warm":
                a, b = x[0] - spans["warm"][0], x[1] - spans["warm"][0]
                segs.append(K.ref_store_segment(self.warm_keys, self.warm_values, a, b - a, pos,
                                                head_major=use_tables))
            else:
                meta, ov, got = x
                if got is None or self.config.cold_medium == "pinned":
                    loaded = self.load_cold_chunk(meta["chunk_id"])
                else:
                    loaded = got
                a, b = ov[0] - meta["start_token"], ov[1] - meta["start_token"]
                kst = _to_device_store(self._chunk_store(loaded, "key"), self.device)
                vst = _to_device_store(self._chunk_store(loaded, "value"), self.device)
                segs.append(K.ref_store_segment(kst, vst, a, b - a, pos))
            pos += segs[-1]["len"]
        stats["query_tokens"] = int(q.shape[0])
        self.last_access_stats = dict(stats)
        if pos == 0:
            return torch.zeros_like(q)
        qpos = _normalize_query_positions(adjusted, B, Hq, pos - 1, self.device) if causal else None
        kq, vq = self._kq, self._vq
        tables = {}
        self.last_ref_drift = None
        if use_tables:
            self.last_ref_drift = torch.empty((B, Hq), dtype=torch.float32, device=self.device)
            tables = dict(score_tables=float(tol), table_stats=self._ref_table_stats(), drift=self.last_ref_drift)
        info = {}
        out = K.ref_attention(q.to(torch.float16), kv_heads=self.H, scale=self.D ** -0.5, causal=causal, qpos=qpos,
                              segments=segs, k_pq_cb=kq.pq.codebooks, v_pq_cb=vq.pq.codebooks,
                              k_rvq_cb=kq.rvq_codebooks, v_rvq_cb=vq.rvq_codebooks,
                              rvq_subspaces=sub.rvq_subspaces if sub else 0, sparse_k=sub.sparse_k if sub else 0,
                              info=info, **tables)
        self.last_ref_tables = bool(info.get("score_tables"))
        if not self.last_ref_tables:
            self.last_ref_drift = None
        return out.to(q.dtype)

    def prepare(self, q: torch.Tensor, causal: bool = True, query_positions=None,
                router: Optional[AsyncHierarchicalRouterMLX] = None, current_position: Optional[int] = None,
                context_window: Optional[int] = None, cold_chunks: Optional[Sequence[int]] = None,
                splits: int = 0, out: Optional[torch.Tensor] = None) -> "K.PrefetchedStep":
        """A reusable fused decode step over this window (``q`` is read at
        launch time, so a decode loop refills it in place).  Cold chunks not
        resident in device slots are copied in by every call of the step,
        overlapped with the attention over the resident part; with all of
        them resident the step is one launch.  The step stays valid until
        another call changes the cache or its device slots."""
        if not self._fused_ok(int(q.shape[1])):
            raise ValueError("prepare() needs a cache format the fused kernel serves")
        step = self._fused_forward(q, causal, query_positions, router, current_position, context_window,
                                   cold_chunks, launch=False, splits=splits, out=out)
        if step is None:
            raise ValueError("the window is empty")
        return step

    def _fused_forward(self, q, causal, query_positions, router, current_position, context_window, cold_chunks,
                       launch: bool = True, splits: int = 0, out: Optional[torch.Tensor] = None):
        start, end, adjusted = self._window_bounds(query_positions, context_window, current_position)
        stats = self._empty_access_stats()
        stats["window_start"], stats["window_end"] = start, end
        stats["window_tokens"] = max(0, end - start)
        stats["context_window"] = -1 if context_window is None else context_window
        stats["used_router"] = int(router is not None)
        plan = self._plan(start, end, stats, router, current_position, context_window, cold_chunks)
        stats["query_tokens"] = int(q.shape[0])
        self.last_access_stats = dict(stats)
        B, Hq, D = q.shape
        if not plan:
            return torch.zeros_like(q) if launch else None
        qh = q if (q.device == self.device and q.dtype == torch.float16) else q.to(self.device, torch.float16)
        spans = self._tier_spans()
        fmt = self._fmt()
        # the resident part of the window (hot, warm, cold chunks already in
        # device slots) and the chunks still to copy in
        resident, incoming = K.SegmentTable(B), K.SegmentTable(B)
        hot_len, hot_pos0, hot_off = 0, 0, 0
        res_tokens, in_tokens = 0, 0
        cold_ids = [x[0]["chunk_id"] for kind, x in plan if kind == "cold"]
        slots, fetched, copies, targets = self._stage_cold(cold_ids) if cold_ids else ({}, [], [], [])
        fetched = set(fetched)
        read_slots = [slots[c]["slot"] for c in cold_ids]
        self._order_after_copies()  # resident chunks may still be arriving from a prefetch
        # the warm tier is segment 0 (the kernel keeps segment 0's bases in
        # registers, and a decode session grows it in place by its length);
        # the cold chunks follow in position order
        for kind, x in sorted(plan, key=lambda e: e[0] != "warm"):
            if kind == "hot":
                hot_off = self._hot_head + x[0] - spans["hot"][0]
                hot_len = x[1] - x[0]
                hot_pos0 = x[0] - start
                res_tokens += hot_len
            elif kind == "warm":
                a, b = x[0] - spans["warm"][0], x[1] - spans["warm"][0]
                skip = a // K.TILE
                kt, vt = self._warm_tiled
                (kc, kk, avail), (vc, vk, _) = kt.seg(skip), vt.seg(skip)
                for bi in range(B):
                    resident.add_codes(bi, kc, vc, kk + vk, kt.cap, b - skip * K.TILE,
                                       spans["warm"][0] + skip * K.TILE - start, avail, kt.plane_bytes())
                res_tokens += b - skip * K.TILE
            else:
                meta, ov, _ = x
                dev = slots[meta["chunk_id"]]
                a, b = ov[0] - meta["start_token"], ov[1] - meta["start_token"]
                skip = a // K.TILE
                table = incoming if meta["chunk_id"] in fetched else resident
                (kc, kk, avail), (vc, vk, _) = dev["key"].seg(skip), dev["value"].seg(skip)
                for bi in range(B):
                    table.add_codes(bi, kc, vc, kk + vk, dev["key"].cap, b - skip * K.TILE,
                                    meta["start_token"] + skip * K.TILE - start, avail, dev["key"].plane_bytes())
                if meta["chunk_id"] in fetched:
                    in_tokens += b - skip * K.TILE
                else:
                    res_tokens += b - skip * K.TILE
        qpos = adjusted
        if causal:
            qpos = _normalize_query_positions(adjusted, B, Hq, stats["window_tokens"] - 1, self.device)
        hk = self._hot_k[:, hot_off:] if hot_len else None
        hv = self._hot_v[:, hot_off:] if hot_len else None
        if out is None:
            out = torch.empty((B, Hq, D), dtype=torch.float16, device=self.device)
        common = dict(kv_heads=self.H, scale=self.D ** -0.5, causal=causal, qpos=qpos if causal else None,
                      hot_seq_stride=0, k_pq_cb=self._kq.pq.codebooks, v_pq_cb=self._vq.pq.codebooks,
                      k_rvq_cb=self._kq.rvq.codebooks if fmt.rvq_subspaces else None,
                      v_rvq_cb=self._vq.rvq.codebooks if fmt.rvq_subspaces else None,
                      cb_batch_stride=False, hot_cap=int(self._hot_k.shape[1]), out=out, launch=False,
                      k_layout=self._k_layout, tables=self._entry_tables(bool(fmt.rvq_subspaces)))
        guard = None
        if self._guarded:
            guard = self._guard_tensor()
            common.update(guard=guard, guard_tol=float(self.config.score_table_tolerance))
        has_resident = hot_len > 0 or not resident.empty
        if not fetched or not has_resident:
            # one launch; with chunks to copy it waits for them (nothing to overlap)
            table = resident if not fetched else incoming
            fl = K.fused_attention(qh, fmt, hot_k=hk, hot_v=hv, hot_len=hot_len, hot_pos0=hot_pos0,
                                   segments=table, max_tokens=max(res_tokens + in_tokens, 1), splits=splits,
                                   **common)
            step = K.PrefetchedStep(self._side_stream(), copies, [fl], wait_at=0) if copies else fl
            self.last_drift = fl.drift
        else:
            # attend the resident part while the side stream copies the
            # missing chunks, then the copied chunks; partials merge at the end
            sa = K.fused_splits(B, Hq, self.H, hot_len, max(res_tokens, 1), resident.max_rows, splits)
            sb = K.fused_splits(B, Hq, self.H, 0, max(in_tokens, 1), incoming.max_rows, splits)
            ws = torch.empty(B * Hq * (sa + sb) * (D + 2) * 4, dtype=torch.uint8, device=self.device)
            if guard is not None:
                common["drift"] = torch.empty(B * Hq * (sa + sb), dtype=torch.float32, device=self.device)
            fa = K.fused_attention(qh, fmt, hot_k=hk, hot_v=hv, hot_len=hot_len, hot_pos0=hot_pos0,
                                   segments=resident, max_tokens=max(res_tokens, 1), splits=sa, workspace=ws,
                                   part=(0, sa + sb, False), **common)
            fb = K.fused_attention(qh, fmt, hot_k=None, hot_v=None, hot_len=0, hot_pos0=0, segments=incoming,
                                   max_tokens=max(in_tokens, 1), splits=sb, workspace=ws,
                                   part=(sa, sa + sb, True), **common)
            step = K.PrefetchedStep(self._side_stream(), copies, [fa, fb], wait_at=1)
            self.last_drift = fb.drift
        if not launch:
            if copies:
                # the staged slots count as resident from now on: fill them
                # before any other call reads them (a prepared step re-issues
                # its copies after draining the launch stream)
                self._wait_readers(targets)
                step.issue_copies(drain=False)
                self._side_stream().make_current_wait(self.device)
            self._record_reads(read_slots, prepared=True)
            return step
        if copies:
            self._wait_readers(targets)
            step(drain=False)
        else:
            step()
        self._record_reads(read_slots)
        return out.to(q.dtype)

    def memory_usage_bytes(self) -> Dict[str, int]:
        """cache.py:430-440.  Subspace format: warm_rvq_bytes counts the RVQ
        and sparse bytes actually stored (every vector carries them)."""
        hot_bytes = self.num_hot * self.H * self.D * 2 * 2
        warm_pq_bytes = self.num_warm * self.H * self.config.num_subspaces * 2
        if self._subspace:
            k = self.config.sparse_topk
            warm_rvq_bytes = self.num_warm * self.H * (self.config.rvq_subspaces + 3 * k) * 2
        else:
            rows = int(self.warm_keys.rvq_codes.shape[0] + self.warm_values.rvq_codes.shape[0])
            warm_rvq_bytes = rows * self.config.num_rvq_layers * 2
        return {"hot_bytes": hot_bytes, "warm_pq_bytes": warm_pq_bytes, "warm_rvq_bytes": warm_rvq_bytes,
                "cold_chunks": len(self.cold_chunk_metadata), "cold_tokens": self.num_cold}


class DecodeSession:
    """The decode loop of rfsn_v10_mlx_ane_complete.py:138-158 over one cache:
    each ``step(k, v)`` appends the new token(s) and attends the window with
    the query buffer ``q`` (read at launch time, so the caller refills it in
    place), writing ``out``.

    While a step only adds hot tokens (``_hot_rows``) and the router's chunk
    set stays, the step re-issues one prepared fused launch with its hot
    length grown in place, which appends the new rows itself (attends them
    from the caller's buffers and writes them to their hot slots): the
    attention launch (and its split merge) and no host-side rebuilding.  Any
    other step goes through the cache's general ``update``; when that kept
    the launch's segments in place (a demotion that grows warm at its tail,
    the hot buffers' live range moved to their front) the step patches the
    prepared launch (``_regrow``), and otherwise (a migration to cold,
    another chunk set, new codebooks) it rebuilds the launch.  The
    query is the newest token, so every window token is allowed and the launch
    carries no query positions (cache.py:395-428 with causal masking at the
    newest position).  The split count is pinned at each rebuild, so the
    launch's workspace stays valid as the window grows.  A fast step runs on
    the stream that was current at the last rebuild; a step called with
    another current stream rebuilds on that one.  ``router`` ranks the
    cold chunks (storage.py:203-234); ``cold_attended`` of them are attended,
    made resident in device slots at each rebuild.  A cache whose format the
    tiled kernel does not serve runs ``update`` + ``attention_forward`` (the
    decode-in-register kernel) every step."""

    def __init__(self, cache: RFSNv10KVCacheMLX, q: torch.Tensor, quantizer: QuantizerArg,
                 router: Optional[AsyncHierarchicalRouterMLX] = None, cold_attended: int = 0,
                 out: Optional[torch.Tensor] = None):
        if not cache._recency:
            raise ValueError("a decode session needs tier_policy='recency' (the newest tokens stay hot)")
        self.cache = cache
        self.q = q
        self.quantizer = quantizer
        self.router = router
        self.cold_attended = int(cold_attended)
        self.out = torch.empty_like(q) if out is None else out
        self._launch: Optional[K.FusedLaunch] = None
        self._ids: Optional[List[int]] = None
        self._hot_args: Optional[Tuple[Optional[int], int]] = None  # the fast step's hot-append arguments
        self._layout: Optional[tuple] = None  # the cache's segment layout at the last rebuild
        self._rows: Optional[tuple] = None  # the last fast step's new rows (read by its launch)
        self.rebuilds = 0
        self.regrows = 0  # steps whose update kept the segments in place (launch patched, not rebuilt)

    def _chunk_set(self, total: Optional[int] = None) -> Optional[List[int]]:
        """The router's nearest ``cold_attended`` chunks for a window of
        ``total`` tokens (default: the cache's), or None (the cache's own
        choice: every cold chunk of the window) without a router."""
        if self.router is None or not self.cold_attended:
            return None
        if total is None:
            total = self.cache.total_tokens
        return self.router.rank(total - 1, total)[:self.cold_attended]

    def _append_launch(self, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """The fast step: the prepared launch appends the new rows itself
        (attends them from ``k`` / ``v`` and writes them to their hot slots)
        with its hot length grown by them; one launch per step."""
        c = self.cache
        T = int(k.shape[0])
        p = self._launch.params
        p.app_k, p.app_v, p.app_ld, p.app_count = k.data_ptr(), v.data_ptr(), c.H * c.D, T
        p.app_vabs = self._hot_args[0]
        p.hot_len += T
        p.max_tokens += T
        c.num_hot += T
        c.total_tokens += T
        self._rows = (k, v)  # the caller's rows stay alive while the launch may read them
        return self._launch()

    def step(self, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        c = self.cache
        T = int(k.shape[0])
        # the fast step appends and launches on the stream pinned at the last
        # rebuild; a caller that has switched streams since takes the rebuild
        # path, so its conversions and the launches stay on one stream
        same_stream = self._launch is not None and L.stream_handle(c.device) == self._hot_args[1]
        if same_stream:
            rows = c._hot_rows(k, v)  # None unless the hot tier takes the tokens in place
            if rows is not None:
                ids = self._chunk_set(c.total_tokens + T)
                if ids == self._ids:
                    return self._append_launch(*rows)
        before = c._session_layout() if same_stream else None
        c.update(k, v, self.quantizer)
        ids = self._chunk_set()
        if same_stream and ids == self._ids and c._fused_ok(int(self.q.shape[1])) and self._regrow(before, T):
            self.regrows += 1
            return self._launch()
        if not c._fused_ok(int(self.q.shape[1])):
            # a format the tiled kernel does not serve: one decode-in-register
            # launch over the window per step, nothing to grow in place
            self._launch, self._ids = None, None
            self.rebuilds += 1
            self.out.copy_(c.attention_forward(self.q, causal=False, cold_chunks=ids))
            return self.out
        self._rebuild(ids)
        return self.out

    def _rebuild(self, ids: Optional[List[int]]) -> None:
        c = self.cache
        self.rebuilds += 1
        if ids:
            c.prefetch_cold_chunks(ids, wait=True)  # resident: the step is one launch
        step = c.prepare(self.q, causal=False, cold_chunks=ids, out=self.out)
        if isinstance(step, K.FusedLaunch):
            p = step.params
            p.splits = int(L.load().rfsn_fused_splits(C.byref(p)))  # pinned as the window grows
            self._launch, self._ids = step, ids
            # fast steps append on the launch's stream, so the append and the
            # launch that reads it stay ordered
            self._hot_args = c._hot_append_args(step.stream)
            self._layout = c._session_layout()
        else:  # chunks still copying in: no prepared launch to grow until they are resident
            self._launch, self._ids = None, None
        step()

    def _regrow(self, before: tuple, tokens: int) -> bool:
        """After a general ``update`` that kept the launch's segments in place
        -- the same warm arrays, head and cold tier, the same hot buffers --
        point the prepared launch at the new hot range and grow its warm
        segment by the demoted tokens, instead of rebuilding it.  ``before``
        is the cache's ``_session_layout`` before the update."""
        c = self.cache
        after = c._session_layout()
        if after is None or before is None or after[:-1] != before[:-1] or before[:-1] != self._layout[:-1]:
            return False
        grown = after[-1] - before[-1]  # warm tokens added by the update
        if grown and (before[-1] == 0 or self._launch.seg_table is None):
            return False  # no warm segment 0 in the launch to grow
        p = self._launch.params
        D = c.D
        p.app_count = 0  # the update wrote the new tokens to the hot buffers
        p.hot_k = c._hot_k.data_ptr() + c._hot_head * D * 2
        p.hot_v = c._hot_v.data_ptr() + c._hot_head * D * 2
        p.hot_len = c.num_hot
        p.hot_pos0 = c._tier_spans()["hot"][0]
        p.max_tokens += tokens
        if grown:
            # segment 0 of sequence 0 is the warm tier: its length grows on
            # the launch stream, after the launches that read the old one
            off = L.Segment.len.offset
            self._launch.seg_table[off:off + 4].view(torch.int32).add_(grown)
        self._layout = after
        return True


def _to_host_store(s: CompressedTensorMLX) -> CompressedTensorMLX:
    h = lambda t: None if t is None else t.detach().to("cpu")
    return CompressedTensorMLX(h(s.pq_codes), h(s.rvq_codes), h(s.rvq_mask), h(s.rvq_offsets), s.num_heads,
                               h(s.sparse_idx), h(s.sparse_val))


def _to_device_store(s: CompressedTensorMLX, device) -> CompressedTensorMLX:
    d = lambda t: None if t is None else t.to(device)
    return CompressedTensorMLX(d(s.pq_codes), d(s.rvq_codes), d(s.rvq_mask), d(s.rvq_offsets), s.num_heads,
                               d(s.sparse_idx), d(s.sparse_val))
