"""Torch-facing wrappers over the C ABI of ``librfsn_hip.so``.

Every function takes and returns device tensors, launches on the current
torch stream, takes its scratch space from torch's caching allocator (the
library itself never allocates device memory) and raises on failure.
"""

from __future__ import annotations

import ctypes as C
import weakref
from collections import OrderedDict
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib as L

TILE = 32  # tokens per tile of the tiled code layout


def _dev(t: torch.Tensor, what: str) -> torch.Tensor:
    L.require_device(t, what)
    return t


def _contig(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _stream(t: torch.Tensor) -> int:
    return L.stream_handle(t.device)


# --------------------------------------------------------------------------
# warm format description
# --------------------------------------------------------------------------

@dataclass(frozen=True)
class WarmFormat:
    head_dim: int
    pq_subspaces: int
    pq_centroids: int
    rvq_subspaces: int = 0
    rvq_centroids: int = 0
    sparse_k: int = 0

    def c(self) -> L.Format:
        return L.Format(self.head_dim, self.pq_subspaces, self.pq_centroids, self.rvq_subspaces,
                        self.rvq_centroids, self.sparse_k)

    @property
    def bytes_per_vector(self) -> int:
        return self.pq_subspaces + self.rvq_subspaces + 3 * self.sparse_k

    @property
    def fused_ok(self) -> bool:
        return (self.head_dim == 64 and self.pq_subspaces in (8, 16)
                and self.rvq_subspaces in (0, self.pq_subspaces) and self.sparse_k in (0, 4))


def round_up(n: int, m: int) -> int:
    return (n + m - 1) // m * m


# --------------------------------------------------------------------------
# encode
# --------------------------------------------------------------------------

def pq_encode(x: torch.Tensor, codebooks: torch.Tensor, want_residual: bool = True
              ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Canonical nearest-centroid PQ encode (quantization.py:124-144).

    x [N, D] fp16 (row stride >= D), codebooks [M, C, d] fp16.
    """
    _dev(x, "pq_encode")
    if x.dtype != torch.float16 or codebooks.dtype != torch.float16:
        raise ValueError("pq_encode expects fp16 vectors and codebooks")
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("pq_encode expects [N, D] rows with unit column stride")
    n, D = x.shape
    M, Cn, d = codebooks.shape
    if D != M * d:
        raise ValueError(f"Expected vectors with dim {M * d}, got {D}")
    cb = _contig(codebooks)
    codes = torch.empty((n, M), dtype=torch.uint8, device=x.device)
    resid = torch.empty((n, D), dtype=torch.float16, device=x.device) if want_residual else None
    L.call("rfsn_pq_encode", x.data_ptr(), n, D, x.stride(0), 0, cb.data_ptr(), M, Cn, 0,
           codes.data_ptr(), M, 0, L.ptr(resid), D, 0, 1, _stream(x))
    return codes, resid


def pq_encode_grouped(x: torch.Tensor, codebooks: torch.Tensor) -> torch.Tensor:
    """Encode ``groups`` independent sets: x [G, N, D], codebooks [G, M, C, d] -> [G, N, M]."""
    _dev(x, "pq_encode_grouped")
    x = _contig(x)
    cb = _contig(codebooks)
    G, n, D = x.shape
    _, M, Cn, d = cb.shape
    codes = torch.empty((G, n, M), dtype=torch.uint8, device=x.device)
    L.call("rfsn_pq_encode", x.data_ptr(), n, D, D, n * D, cb.data_ptr(), M, Cn, M * Cn * d,
           codes.data_ptr(), M, n * M, None, D, 0, G, _stream(x))
    return codes


def warm_encode(x: torch.Tensor, fmt: WarmFormat, pq_cb: torch.Tensor,
                rvq_cb: Optional[torch.Tensor] = None) -> Dict[str, torch.Tensor]:
    """PQ + optional subspace RVQ + optional top-k sparse residual of x [N, D]."""
    _dev(x, "warm_encode")
    if x.dim() != 2 or (x.shape[0] and x.stride(1) != 1) or x.dtype != torch.float16:
        raise ValueError("warm_encode expects fp16 [N, D] rows")
    n = x.shape[0]
    dev = x.device
    out = {"pq": torch.empty((n, fmt.pq_subspaces), dtype=torch.uint8, device=dev)}
    if fmt.rvq_subspaces:
        out["rvq"] = torch.empty((n, fmt.rvq_subspaces), dtype=torch.uint8, device=dev)
    if fmt.sparse_k:
        out["sparse_idx"] = torch.empty((n, fmt.sparse_k), dtype=torch.uint8, device=dev)
        out["sparse_val"] = torch.empty((n, fmt.sparse_k), dtype=torch.float16, device=dev)
    if n == 0:
        return out
    f = fmt.c()
    ws_bytes = L.load().rfsn_warm_encode_workspace_bytes(C.byref(f), n)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    codes = L.Codes(out["pq"].data_ptr(), L.ptr(out.get("rvq")), L.ptr(out.get("sparse_idx")),
                    L.ptr(out.get("sparse_val")))
    L.call("rfsn_warm_encode", C.byref(f), x.data_ptr(), n, x.stride(0), _contig(pq_cb).data_ptr(),
           L.ptr(None if rvq_cb is None else _contig(rvq_cb)), codes, ws.data_ptr(), ws_bytes, _stream(x))
    return out


def batch_encode_ok(fmt: WarmFormat) -> bool:
    """Whether ``rfsn_warm_encode_batch`` serves the format: head_dim 64, 4-
    or 8-dim PQ subspaces, an RVQ stage of the same split or none, top-k
    sparse residuals with k 0 or 4 (rows from torch's aligned allocations)."""
    return (fmt.head_dim == 64 and fmt.pq_subspaces in (8, 16)
            and fmt.rvq_subspaces in (0, fmt.pq_subspaces) and fmt.sparse_k in (0, 4))


def warm_encode_batch(items: Sequence[Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]],
                      fmt: WarmFormat) -> List[Dict[str, torch.Tensor]]:
    """``warm_encode`` of several (x, pq_cb, rvq_cb) sets of one format in one
    launch (a chunk's K and V); the formats ``rfsn_warm_encode_batch`` serves."""
    if not items:
        return []
    outs, keep = [], []
    jobs = (L.EncodeJob * len(items))()
    for i, (x, pq_cb, rvq_cb) in enumerate(items):
        _dev(x, "warm_encode_batch")
        if x.dim() != 2 or (x.shape[0] and x.stride(1) != 1) or x.dtype != torch.float16:
            raise ValueError("warm_encode_batch expects fp16 [N, D] rows")
        n, dev = x.shape[0], x.device
        out = {"pq": torch.empty((n, fmt.pq_subspaces), dtype=torch.uint8, device=dev)}
        if fmt.rvq_subspaces:
            out["rvq"] = torch.empty((n, fmt.rvq_subspaces), dtype=torch.uint8, device=dev)
        if fmt.sparse_k:
            out["sparse_idx"] = torch.empty((n, fmt.sparse_k), dtype=torch.uint8, device=dev)
            out["sparse_val"] = torch.empty((n, fmt.sparse_k), dtype=torch.float16, device=dev)
        pcb = _contig(pq_cb)
        rcb = None if rvq_cb is None else _contig(rvq_cb)
        keep += [x, pcb, rcb]
        jobs[i] = L.EncodeJob(x.data_ptr(), n, x.stride(0) if n else x.shape[1], pcb.data_ptr(), L.ptr(rcb),
                              L.Codes(out["pq"].data_ptr(), L.ptr(out.get("rvq")), L.ptr(out.get("sparse_idx")),
                                      L.ptr(out.get("sparse_val"))))
        outs.append(out)
    f = fmt.c()
    L.call("rfsn_warm_encode_batch", C.byref(f), jobs, len(items), _stream(items[0][0]))
    return outs


def rvq_encode_full(resid: torch.Tensor, codebooks: torch.Tensor, threshold: float
                    ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gated full-dimension RVQ (quantization.py:206-252) -> (codes u16 [A, L], mask [N], offsets [A])."""
    _dev(resid, "rvq_encode_full")
    resid = _contig(resid)
    if resid.data_ptr() % 16:
        resid = resid.clone()  # the MFMA search loads 16-byte groups of a row
    n, D = resid.shape
    Ls, Cn, Dc = codebooks.shape
    if D != Dc:
        raise ValueError(f"Expected residual dim {Dc}, got {D}")
    dev = resid.device
    s = _stream(resid)
    mask8 = torch.empty(n, dtype=torch.uint8, device=dev)
    L.call("rfsn_rvq_gate", resid.data_ptr(), n, D, D, float(threshold), mask8.data_ptr(), s)
    offsets_all = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    wsb = L.load().rfsn_mask_compact_workspace_bytes(n)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    L.call("rfsn_mask_compact", mask8.data_ptr(), n, offsets_all.data_ptr(), count.data_ptr(), ws.data_ptr(), wsb, s)
    a = int(count.item())  # host sync, as the reference's np.asarray(mask) (quantization.py:217)
    offsets = offsets_all[:a].clone()
    codes = torch.empty((a, Ls), dtype=torch.uint16, device=dev)
    if a:
        wsb = L.load().rfsn_rvq_encode_full_workspace_bytes(a, D, Ls, Cn)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        cb = _contig(codebooks)
        if cb.data_ptr() % 16:
            cb = cb.clone()
        L.call("rfsn_rvq_encode_full", resid.data_ptr(), D, D, offsets.data_ptr(), a, cb.data_ptr(),
               Ls, Cn, codes.data_ptr(), ws.data_ptr() if wsb else None, wsb, s)
    return codes, mask8.bool(), offsets


# --------------------------------------------------------------------------
# decode
# --------------------------------------------------------------------------

def decode(fmt: WarmFormat, pq: torch.Tensor, pq_cb: torch.Tensor, rvq: Optional[torch.Tensor] = None,
           rvq_cb: Optional[torch.Tensor] = None, sparse_idx: Optional[torch.Tensor] = None,
           sparse_val: Optional[torch.Tensor] = None, add_zero: bool = False) -> torch.Tensor:
    """Warm-format decode of pq [N, M] (+ rvq [N, M_r], sparse [N, k]) -> fp16 [N, D]."""
    _dev(pq, "decode")
    pq = _contig(pq)
    n = pq.shape[0]
    out = torch.empty((n, fmt.head_dim), dtype=torch.float16, device=pq.device)
    if n == 0:
        return out
    rvq = None if rvq is None else _contig(rvq)
    sparse_idx = None if sparse_idx is None else _contig(sparse_idx)
    sparse_val = None if sparse_val is None else _contig(sparse_val)
    codes = L.Codes(pq.data_ptr(), L.ptr(rvq), L.ptr(sparse_idx), L.ptr(sparse_val))
    f = fmt.c()
    L.call("rfsn_decode", C.byref(f), C.byref(codes), n, _contig(pq_cb).data_ptr(),
           L.ptr(None if rvq_cb is None else _contig(rvq_cb)), out.data_ptr(), fmt.head_dim, int(add_zero),
           _stream(pq))
    return out


def sparse_fold(fmt: WarmFormat, pq: torch.Tensor, pq_cb: torch.Tensor, rvq: Optional[torch.Tensor],
                rvq_cb: Optional[torch.Tensor], sparse_idx: torch.Tensor, sparse_val: torch.Tensor,
                delta: bool = False) -> torch.Tensor:
    """Corrected coordinates fp16(K[idx] + val) of the sparse stage, [N, k] fp16:
    the sparse values the fused kernel's layout carries (a store per entry
    instead of a read-modify-write).  ``delta``: the score deltas
    fp16(corrected - (base[idx] + rvq[idx])) of the score-table K layout."""
    _dev(pq, "sparse_fold")
    pq = _contig(pq)
    n = pq.shape[0]
    out = torch.empty((n, fmt.sparse_k), dtype=torch.float16, device=pq.device)
    if n == 0:
        return out
    rvq = None if rvq is None else _contig(rvq)
    sidx, sval = _contig(sparse_idx), _contig(sparse_val)
    codes = L.Codes(pq.data_ptr(), L.ptr(rvq), sidx.data_ptr(), sval.data_ptr())
    f = fmt.c()
    L.call("rfsn_sparse_delta" if delta else "rfsn_sparse_fold", C.byref(f), C.byref(codes), n,
           _contig(pq_cb).data_ptr(), L.ptr(None if rvq_cb is None else _contig(rvq_cb)), out.data_ptr(),
           _stream(pq))
    return out


def decode_ref(pq: torch.Tensor, pq_cb: torch.Tensor, rvq_codes: torch.Tensor, offsets: torch.Tensor,
               rvq_cb: torch.Tensor) -> torch.Tensor:
    """Reference-format hybrid decode (quantization.py:310-319) -> fp16 [N, D]."""
    _dev(pq, "decode_ref")
    pq = _contig(pq)
    n, M = pq.shape
    Mc, Cn, d = pq_cb.shape
    D = M * d
    Ls, Cr, _ = rvq_cb.shape
    out = torch.empty((n, D), dtype=torch.float16, device=pq.device)
    a = int(rvq_codes.shape[0])
    L.call("rfsn_decode_ref", pq.data_ptr(), n, D, M, Cn, _contig(pq_cb).data_ptr(),
           _contig(rvq_codes).data_ptr() if a else None, _contig(offsets).data_ptr() if a else None, a, Ls, Cr,
           _contig(rvq_cb).data_ptr(), out.data_ptr(), _stream(pq))
    return out


# --------------------------------------------------------------------------
# attention
# --------------------------------------------------------------------------

def _qpos(qpos: torch.Tensor, B: int, Hq: int, device) -> torch.Tensor:
    """Query positions as the int32 [B, Hq] array the kernels index; [B] is
    broadcast over heads (attention.py:28-33), any other shape is rejected."""
    qp = qpos.to(device=device, dtype=torch.int32)
    if qp.dim() == 1 and qp.shape[0] == B:
        qp = qp[:, None].expand(B, Hq)
    if tuple(qp.shape) != (B, Hq):
        raise ValueError(f"query positions must be [B] or [B, Hq] = [{B}, {Hq}], got {tuple(qpos.shape)}")
    return qp.contiguous()


def blockwise_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, scale: float,
                        causal: bool, qpos: Optional[torch.Tensor]) -> torch.Tensor:
    """Exact attention of q [B, Hq, D] over keys/values [T, Hkv, D] (strided rows)."""
    _dev(q, "blockwise_attention")
    q = _contig(q)
    B, Hq, D = q.shape
    T, Hkv, Dk = keys.shape
    if Dk != D or values.shape != keys.shape:
        raise ValueError("keys/values must be [T, H, D] with the query's head_dim")
    aligned = all(t.data_ptr() % 16 == 0 for t in (keys, values)) and keys.stride(0) % 8 == 0 \
        and keys.stride(1) % 8 == 0
    if keys.stride() != values.stride() or keys.stride(2) != 1 or not aligned:
        keys, values = keys.contiguous(), values.contiguous()
    out = torch.empty_like(q)
    qp = None if qpos is None else _qpos(qpos, B, Hq, q.device)
    lib = L.load()
    splits_max = 1024
    wsb = lib.rfsn_attention_workspace_bytes(B, Hq, D, splits_max)
    ws = torch.empty(wsb, dtype=torch.uint8, device=q.device)
    L.call("rfsn_blockwise_attention", q.data_ptr(), B, Hq, D, keys.data_ptr() if T else None,
           values.data_ptr() if T else None, T, Hkv, keys.stride(0), keys.stride(1), float(scale), int(causal),
           L.ptr(qp), out.data_ptr(), ws.data_ptr(), wsb, _stream(q))
    return out


def pack_codes(src: torch.Tensor, dst: torch.Tensor, t_base: int) -> None:
    """Plain codes src [H, T, M] into the tiled layout dst [H, cap*M] at tokens t_base.."""
    _dev(src, "pack_codes")
    H, T, M = src.shape
    src = _contig(src)
    L.call("rfsn_pack_codes", src.data_ptr(), T * M, T, M, H, dst.data_ptr(), dst.stride(0), t_base, _stream(src))


def score_layout_ok(fmt: WarmFormat, q_heads: int, kv_heads: int) -> bool:
    """Whether the fused kernel can score K codes through q . centroid tables:
    16 PQ and 16 RVQ subspaces, at most 4 query heads per KV head."""
    return (fmt.pq_subspaces == 16 and fmt.rvq_subspaces == 16 and fmt.head_dim == 64
            and kv_heads > 0 and q_heads % kv_heads == 0 and q_heads // kv_heads <= 4)


def score_guard(k_pq_cb: torch.Tensor, k_rvq_cb: torch.Tensor, vmax, out: Optional[torch.Tensor] = None
                ) -> torch.Tensor:
    """Per-sequence inputs of the score tables' drift guard, float32 [..., 65]:
    W_i = mean_c PQ_c,i^2 + mean_c RVQ_c,i^2 + mean_c |PQ_c(s)|^2 +
    mean_c |RVQ_c(s)|^2 for coordinate i of subspace s (the second moment of
    K^_i, whose fp16 rounding the tables skip, and of the table entries'
    centroids per unit query), then ``vmax`` (an upper bound on |V^|).
    Codebooks [M, C, 4] or [B, M, C, 4] (16 + 16 subspaces of head_dim 64);
    ``vmax`` a number or a [B] tensor.  ``out`` receives the result in place."""
    p, r = k_pq_cb.float(), k_rvq_cb.float()
    lead = p.shape[:-3]
    k2 = (p * p).mean(-2) + (r * r).mean(-2)                        # [..., 16, 4]
    cn = (p * p).sum(-1).mean(-1) + (r * r).sum(-1).mean(-1)        # [..., 16]
    w = (k2 + cn[..., None]).reshape(*lead, 64)
    v = torch.as_tensor(vmax, dtype=torch.float32, device=w.device).expand(lead).reshape(*lead, 1)
    g = torch.cat([w, v], -1)
    if out is None:
        return g
    out.copy_(g)
    return out


def pack_score_codes(pq: torch.Tensor, rvq: torch.Tensor, sidx: Optional[torch.Tensor], sval: Optional[torch.Tensor],
                     dst: Dict[str, Optional[torch.Tensor]], t_base: int) -> None:
    """Plain codes pq, rvq [H, T, 16] and sparse entries sidx, sval [H, T, k]
    (sval: score deltas) into the score-table K layout of ``dst`` (``pq``,
    ``rvq`` [H, cap*16]; ``sparse_idx``, ``sparse_val`` [H, cap, k]) at tokens
    t_base..: token t = 32 tau + 16 u + r has code byte 4g + b at
    512 tau + 32 r + 8 g + 4 u + b holding subspace 4g + (b ^ ((r >> 2) & 3)),
    odd tokens with the two stages swapped, and sparse entry e at
    32 k tau + 2 k r + 2 e + u."""
    _dev(pq, "pack_score_codes")
    H, T, M = pq.shape
    if M != 16 or tuple(rvq.shape) != (H, T, 16):
        raise ValueError("pack_score_codes: PQ and RVQ codes must be [H, T, 16]")
    k = 0 if sidx is None else int(sidx.shape[2])
    cap = dst["pq"].shape[1] // 16
    pq, rvq = _contig(pq), _contig(rvq)
    si = None if sidx is None else _contig(sidx)
    sv = None if sval is None else _contig(sval)
    L.call("rfsn_pack_score_codes", pq.data_ptr(), rvq.data_ptr(), L.ptr(si), L.ptr(sv), k, T, H,
           dst["pq"].data_ptr(), dst["rvq"].data_ptr(), L.ptr(dst.get("sparse_idx") if k else None),
           L.ptr(dst.get("sparse_val") if k else None), cap, t_base, _stream(pq))


def _score_positions(T: int, t0: int, k: int, device):
    """(code byte offsets [T, 16], code subspace of each byte [T, 16], sparse
    entry offsets [T, k]) of tokens t0 .. t0+T-1 in the score-table K layout."""
    t = torch.arange(t0, t0 + T, device=device)
    j = torch.arange(16, device=device)
    tau, u, r = t >> 5, (t >> 4) & 1, t & 15
    pos = (512 * tau + 32 * r + 4 * u)[:, None] + (8 * (j >> 2) + (j & 3))[None, :]
    sub = (j & 12)[None, :] | ((j & 3)[None, :] ^ ((r >> 2) & 3)[:, None])
    e = torch.arange(k, device=device)
    spos = (32 * k * tau + 2 * k * r + u)[:, None] + 2 * e[None, :]
    return pos, sub, spos


def unpack_score_codes(dst: Dict[str, Optional[torch.Tensor]], T: int, t0: int = 0):
    """Inverse of ``pack_score_codes`` for tokens t0 .. t0+T-1: plain
    (pq, rvq [H, T, 16], sparse_idx, sparse_val [H, T, k] or None)."""
    p, r_ = dst["pq"], dst["rvq"]
    H = p.shape[0]
    k = 0 if dst.get("sparse_idx") is None else int(dst["sparse_idx"].shape[2])
    pos, sub, spos = _score_positions(T, t0, k, p.device)
    inv = torch.empty_like(sub)
    inv.scatter_(1, sub, torch.arange(16, device=p.device)[None, :].expand(T, 16).contiguous())
    bytes_at = pos.gather(1, inv)                                   # [T, 16]: byte of subspace s
    gp = p[:, bytes_at.reshape(-1)].reshape(H, T, 16)
    gr = r_[:, bytes_at.reshape(-1)].reshape(H, T, 16)
    odd = ((torch.arange(t0, t0 + T, device=p.device) & 1) == 1)[None, :, None]
    pq, rvq = torch.where(odd, gr, gp), torch.where(odd, gp, gr)
    if not k:
        return pq, rvq, None, None
    flat = spos.reshape(-1)
    si = dst["sparse_idx"].reshape(H, -1)[:, flat].reshape(H, T, k)
    sv = dst["sparse_val"].reshape(H, -1)[:, flat].reshape(H, T, k)
    return pq, rvq, si, sv


def entry_tables(pq_cb: torch.Tensor, rvq_cb: Optional[torch.Tensor]) -> torch.Tensor:
    """The fused kernel's entry-major table of one codebook pair: fp16
    [..., 256, 128], entry e = [PQ entries e of the M subspaces | RVQ entries
    e] (the PQ entries again without an RVQ stage), zeros past a codebook's
    size.  pq_cb [..., M, C, d], rvq_cb [..., M, C_r, d] or None, M * d = 64."""
    def arrange(cb: torch.Tensor) -> torch.Tensor:
        *lead, M, C, d = cb.shape
        if M * d != 64 or C > 256:
            raise ValueError("entry tables: head_dim 64 and at most 256 centroids")
        t = cb.to(torch.float16).movedim(-2, -3).reshape(*lead, C, M * d)
        if C < 256:
            t = torch.cat([t, t.new_zeros((*lead, 256 - C, M * d))], dim=-2)
        return t
    pq = arrange(pq_cb)
    return torch.cat([pq, arrange(rvq_cb) if rvq_cb is not None else pq], dim=-1).contiguous()


def _round256(n: int) -> int:
    """n rounded up to a multiple of 256 (device sub-buffer alignment)."""
    return (n + 255) // 256 * 256


_TILE_MAPS: "OrderedDict[tuple, np.ndarray]" = OrderedDict()


class SegmentTable:
    """Host builder of the device ``rfsn_segment`` table of the fused kernel."""

    def __init__(self, batch: int):
        self.rows: List[List[L.Segment]] = [[] for _ in range(batch)]
        self.tiles: List[List[int]] = [[] for _ in range(batch)]  # 32-token tiles of each segment
        self.keep: List[torch.Tensor] = []
        # per segment: bytes from K's sparse values to their corrected-coordinate
        # plane (the drift guard's exact pass reads it), None without such a plane
        self.k_planes: List[List[Optional[int]]] = [[] for _ in range(batch)]

    def add(self, b: int, k: Dict[str, Optional[torch.Tensor]], v: Dict[str, Optional[torch.Tensor]],
            head_stride: int, length: int, pos0: int) -> None:
        """``k`` may carry ``sparse_cc``, the corrected coordinates in the
        plane after ``sparse_val`` (``TiledCodes(exact_plane=True)``)."""
        def codes(c):
            # the kernel reads whole 32-token tiles of the tiled code rows: the
            # segment must fit the views it is given
            tiles = (length + 31) // 32
            for key in ("pq", "rvq"):
                t = c.get(key)
                if t is not None and length > 0:
                    m = t.stride(0) // head_stride if head_stride > 0 else 0
                    if m <= 0 or tiles * 32 * m > t.shape[1]:
                        raise ValueError(f"segment of {length} tokens exceeds its {key} code rows")
            for key in ("sparse_idx", "sparse_val"):
                t = c.get(key)
                if t is not None and length > t.shape[1]:
                    raise ValueError(f"segment of {length} tokens exceeds its {key} rows")
            for t in c.values():
                if t is not None:
                    self.keep.append(t)
            return L.Codes(L.ptr(c.get("pq")), L.ptr(c.get("rvq")), L.ptr(c.get("sparse_idx")),
                           L.ptr(c.get("sparse_val")))
        sv, cc = k.get("sparse_val"), k.get("sparse_cc")
        plane = None
        if sv is not None and cc is not None:
            if cc.dtype != sv.dtype or cc.shape != sv.shape or cc.stride() != sv.stride():
                raise ValueError("sparse_cc must have the shape and strides of sparse_val")
            plane = cc.data_ptr() - sv.data_ptr()
        self.rows[b].append(L.Segment(codes(k), codes(v), head_stride, length, pos0))
        self.tiles[b].append((int(length) + 31) // 32)
        self.k_planes[b].append(plane)

    def add_codes(self, b: int, k: "L.Codes", v: "L.Codes", keep: Sequence[torch.Tensor], head_stride: int,
                  length: int, pos0: int, available: int, k_plane: Optional[int] = None) -> None:
        """Like ``add`` from precomputed addresses (``TiledCodes.seg``);
        ``available`` = tokens of the code rows from the segment's start;
        ``k_plane`` = bytes from K's sparse values to their corrected-coordinate
        plane (``TiledCodes.plane_bytes``), None without one."""
        if length > 0 and (length + 31) // 32 * 32 > available:
            raise ValueError(f"segment of {length} tokens exceeds its {available} available code rows")
        self.keep.extend(keep)
        self.rows[b].append(L.Segment(k, v, head_stride, length, pos0))
        self.tiles[b].append((int(length) + 31) // 32)
        self.k_planes[b].append(k_plane)

    def check_exact_planes(self, kv_heads: int, sparse_k: int) -> None:
        """The drift guard's exact pass reads K's corrected coordinates at
        ``kv_heads * head_stride * sparse_k`` fp16 values past each K sparse
        value pointer: refuse a table with a K segment lacking that plane."""
        for b, row in enumerate(self.rows):
            for s, seg in enumerate(row):
                want = kv_heads * int(seg.head_stride) * sparse_k * 2
                got = self.k_planes[b][s]
                if seg.len > 0 and got != want:
                    raise ValueError(
                        f"drift guard: K segment {s} of sequence {b} has no corrected-coordinate plane "
                        f"{want} bytes after its sparse values (got {got}); build its codes with "
                        "TiledCodes(exact_plane=True) or pass sparse_cc")

    @property
    def max_rows(self) -> int:
        """Segments of the longest row (the table's max_segments, at least 1)."""
        return max(1, max(len(r) for r in self.rows))

    @property
    def empty(self) -> bool:
        return all(not r for r in self.rows)

    def tile_map(self) -> Tuple[List["np.ndarray"], int]:
        """Per row, (segment << 16) | tile within the segment of every encoded
        tile of segments 1..n-1, in order (the kernel's tile -> segment map).
        Rows with the same segment lengths share one map (memoized)."""
        rows = []
        for b, r in enumerate(self.rows):
            key = tuple(self.tiles[b][1:]) if len(self.tiles[b]) == len(r) else \
                tuple((int(seg.len) + 31) // 32 for seg in r[1:])
            hit = _TILE_MAPS.get(key)
            if hit is not None:
                _TILE_MAPS.move_to_end(key)
                rows.append(hit)
                continue
            tiles = np.array(key, dtype=np.int64)
            if len(tiles) > 0xFFFF or (len(tiles) and tiles.max() > 0x10000):
                raise ValueError("tile map: at most 65535 segments of at most 65536 tiles")
            seg = np.repeat(np.arange(1, len(tiles) + 1, dtype=np.int64), tiles)
            within = np.arange(seg.size, dtype=np.int64) - np.repeat(np.cumsum(tiles) - tiles, tiles)
            m = ((seg << 16) | within).astype(np.uint32)
            _TILE_MAPS[key] = m
            while len(_TILE_MAPS) > 64:
                _TILE_MAPS.popitem(last=False)
            rows.append(m)
        return rows, max(1, max(m.size for m in rows))

    def to_device(self, device) -> Tuple[torch.Tensor, torch.Tensor, int, torch.Tensor, torch.Tensor, int]:
        """(segment table, segment counts, max_segments, tile map, tile map
        counts, tile map stride) in device memory.  Everything travels in one
        asynchronous copy from pinned memory, so building a launch never
        waits for the work already queued."""
        maxs = max(1, max(len(r) for r in self.rows))
        size = C.sizeof(L.Segment)
        nb = size * len(self.rows) * maxs
        host = (L.Segment * (len(self.rows) * maxs))()
        for b, r in enumerate(self.rows):
            for s, seg in enumerate(r):
                host[b * maxs + s] = seg
        counts = (C.c_int32 * len(self.rows))(*[len(r) for r in self.rows])
        maps, stride = self.tile_map()
        nrows = len(self.rows)
        o_counts = nb
        o_map = _round256(o_counts + 4 * nrows)
        o_mcounts = o_map + 4 * nrows * stride
        staged = torch.empty(o_mcounts + 4 * nrows, dtype=torch.uint8, pin_memory=True)  # map rows read up to their counts
        C.memmove(staged.data_ptr(), host, nb)
        C.memmove(staged.data_ptr() + o_counts, counts, C.sizeof(counts))
        buf = staged.numpy()
        flat = buf[o_map:o_mcounts].view(np.uint32).reshape(nrows, stride)
        for b, m in enumerate(maps):
            flat[b, :m.size] = m
        buf[o_mcounts:].view(np.int32)[:] = [m.size for m in maps]
        dev = staged.to(device, non_blocking=True)
        return (dev[:nb], dev[o_counts:o_counts + 4 * nrows].view(torch.int32), maxs,
                dev[o_map:o_mcounts].view(torch.int32), dev[o_mcounts:].view(torch.int32), stride)


def fused_attention(q: torch.Tensor, fmt: WarmFormat, *, kv_heads: int, scale: float, causal: bool,
                    qpos: Optional[torch.Tensor], hot_k: Optional[torch.Tensor], hot_v: Optional[torch.Tensor],
                    hot_len: int, hot_pos0: int, hot_seq_stride: int, segments: SegmentTable,
                    k_pq_cb: torch.Tensor, v_pq_cb: torch.Tensor, k_rvq_cb: Optional[torch.Tensor],
                    v_rvq_cb: Optional[torch.Tensor], cb_batch_stride: bool, max_tokens: int,
                    splits: int = 0, table: Optional[Tuple[torch.Tensor, torch.Tensor, int]] = None,
                    workspace: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                    hot_cap: Optional[int] = None, launch: bool = True,
                    part: Optional[Tuple[int, int, bool]] = None, k_layout: int = 0,
                    guard: Optional[torch.Tensor] = None, guard_tol: float = 2e-3,
                    drift: Optional[torch.Tensor] = None,
                    tables: Optional[Tuple[torch.Tensor, torch.Tensor]] = None):
    """Fused dequant + decode attention; q [B, Hq, D] -> [B, Hq, D] fp16.

    ``k_layout`` = 1 when every segment's K codes are ``pack_score_codes``
    rows with ``sparse_fold(delta=True)`` values (``score_layout_ok``).

    ``guard`` (k_layout 1, float32 [B, 65] from ``score_guard``, [1, 65]
    with shared codebooks): a block
    whose estimated output drift exceeds ``guard_tol`` recomputes its output
    exactly, reading the corrected coordinates of K's sparse entries from the
    plane after the score deltas (``TiledCodes(exact_plane=True)``).  The
    estimates land in ``drift`` (float32, at least B * Hq * slots; allocated
    when None) as [B, Hq, slots], slots = the call's splits or part slots.

    hot_k/hot_v: [.., Hkv, hot_cap, D] fp16 (sequence stride ``hot_seq_stride``
    elements, 0 = shared).  Codebooks [B, M, C, d] when ``cb_batch_stride``
    else [M, C, d] shared.  With ``launch=False`` returns a ``FusedLaunch``
    that re-issues the same launch (same buffers) without rebuilding it.

    ``tables`` = (K, V) ``entry_tables`` of the codebooks ([B, 256, 128]
    with ``cb_batch_stride``, else [256, 128]): staged by the kernel with
    contiguous loads instead of gathered from the codebooks.

    ``part = (base, slots, merge)`` attends one part of a window split over
    several calls on one stream: the call's split partials go to slots
    base .. base+splits-1 of ``slots`` in ``workspace`` (shared by the calls,
    which must pass ``splits`` explicitly), and the call with ``merge`` writes
    ``out`` from all slots.
    """
    _dev(q, "fused_attention")
    q = _contig(q)
    B, Hq, D = q.shape
    if out is None:
        out = torch.empty_like(q)
    # the kernel sizes its splits from max_tokens: a row holding more tokens
    # would lose its last tiles without an error
    longest = hot_len + max((sum(int(s.len) for s in r) for r in segments.rows), default=0)
    if longest > max_tokens:
        raise ValueError(f"a sequence attends {longest} tokens, more than max_tokens = {max_tokens}")
    if table is None:
        table = segments.to_device(q.device)
    seg_t, nseg_t, maxs, *tmap = table
    qp = None if qpos is None else _qpos(qpos, B, Hq, q.device)
    if out.shape != q.shape or out.dtype != torch.float16 or not out.is_contiguous():
        raise ValueError("out must be a contiguous fp16 tensor shaped like q")
    cbs = [None if t is None else _contig(t) for t in (k_pq_cb, v_pq_cb, k_rvq_cb, v_rvq_cb)]
    pq_stride = k_pq_cb[0].numel() if cb_batch_stride else 0
    rvq_stride = (k_rvq_cb[0].numel() if (cb_batch_stride and k_rvq_cb is not None) else 0)
    if hot_cap is None:
        hot_cap = hot_k.shape[-2] if hot_k is not None else 0
    p = L.FusedParams()
    p.fmt = fmt.c()
    p.batch, p.q_heads, p.kv_heads = B, Hq, kv_heads
    p.q, p.out = q.data_ptr(), out.data_ptr()
    p.scale, p.causal, p.qpos = float(scale), int(causal), L.ptr(qp)
    p.hot_k, p.hot_v = L.ptr(hot_k), L.ptr(hot_v)
    p.hot_cap, p.hot_seq_stride, p.hot_len, p.hot_pos0 = hot_cap, hot_seq_stride, hot_len, hot_pos0
    p.segments, p.num_segments, p.max_segments = seg_t.data_ptr(), nseg_t.data_ptr(), maxs
    if tmap:
        map_t, map_n, map_stride = tmap
        p.tile_map, p.tile_map_count, p.tile_map_stride = map_t.data_ptr(), map_n.data_ptr(), map_stride
    p.k_pq_cb, p.v_pq_cb, p.k_rvq_cb, p.v_rvq_cb = (L.ptr(t) for t in cbs)
    p.pq_cb_stride, p.rvq_cb_stride = pq_stride, rvq_stride
    p.max_tokens, p.splits = max_tokens, splits
    p.k_layout = int(k_layout)
    if tables is not None:
        kt, vt = tables
        rows = B if cb_batch_stride else 1
        for t in (kt, vt):
            if t.dtype != torch.float16 or not t.is_contiguous() or t.numel() != rows * 256 * 128 \
                    or t.device != q.device:
                raise ValueError(f"entry tables must be contiguous fp16 [{rows}, 256, 128] on the query's device")
        p.k_tab, p.v_tab, p.tab_stride = kt.data_ptr(), vt.data_ptr(), 65536 if cb_batch_stride else 0
    if part is not None:
        if splits <= 0 or workspace is None:
            raise ValueError("partial calls need explicit splits and a shared workspace")
        p.part_base, p.part_slots, p.merge = int(part[0]), int(part[1]), int(bool(part[2]))
    lib = L.load()
    if guard is not None:
        if not k_layout:
            raise ValueError("the drift guard serves the score-table K layout (k_layout=1) only")
        rows = B if cb_batch_stride else 1  # shared codebooks share one guard row
        if guard.dtype != torch.float32 or not guard.is_contiguous() or guard.numel() < rows * 65 \
                or guard.device != q.device:
            raise ValueError(f"guard must be a contiguous float32 [{rows}, 65] tensor on the query's device")
        slots = p.part_slots if part is not None else int(lib.rfsn_fused_splits(C.byref(p)))
        if drift is None:
            drift = torch.empty(B * Hq * slots, dtype=torch.float32, device=q.device)
        elif drift.dtype != torch.float32 or not drift.is_contiguous() or drift.numel() < B * Hq * slots:
            raise ValueError(f"drift must be a contiguous float32 tensor of at least {B * Hq * slots} values")
        if fmt.sparse_k:
            segments.check_exact_planes(kv_heads, fmt.sparse_k)
        p.guard, p.drift, p.guard_tol = guard.data_ptr(), drift.data_ptr(), float(guard_tol)
        drift = drift[:B * Hq * slots].view(B, Hq, slots)
    wsb = lib.rfsn_fused_workspace_bytes(C.byref(p))
    if workspace is None or workspace.numel() < wsb:
        if part is not None:
            raise ValueError(f"partial calls share a workspace of at least {wsb} bytes")
        workspace = torch.empty(max(wsb, 4), dtype=torch.uint8, device=q.device)
    p.workspace, p.workspace_bytes = workspace.data_ptr(), workspace.numel()
    fl = FusedLaunch(p, [q, out, qp, seg_t, nseg_t, *tmap[:2], workspace, segments, *cbs, guard, drift,
                         *(tables or ())], out, _stream(q))
    fl.drift = drift
    fl.seg_table = seg_t
    if not launch:
        return fl
    fl()
    return out


# --------------------------------------------------------------------------
# reference-format attention (PQ + gated full-dimension RVQ, decoded on the fly)
# --------------------------------------------------------------------------

_ACTIVE_MAPS: Dict[int, tuple] = {}  # id(offsets) -> (weakref, (rows, version), map)


def active_map(offsets: torch.Tensor, rows: int) -> torch.Tensor:
    """int32 [rows]: row r's index into the store's RVQ codes, or -1 -- the
    scatter of the reference's decode (quantization.py:273-274: correction row
    offsets[a] = codes row a); memoized per offsets tensor and version."""
    key = id(offsets)
    hit = _ACTIVE_MAPS.get(key)
    if hit is not None and hit[0]() is offsets and hit[1] == (rows, offsets._version):
        return hit[2]
    out = torch.full((rows,), -1, dtype=torch.int32, device=offsets.device)
    a = int(offsets.shape[0])
    if a:
        out[offsets.long()] = torch.arange(a, dtype=torch.int32, device=offsets.device)
    _ACTIVE_MAPS[key] = (weakref.ref(offsets, lambda _r, k=key: _ACTIVE_MAPS.pop(k, None)), (rows, offsets._version), out)
    return out


_HEAD_MAJOR: Dict[int, tuple] = {}  # id(pq_codes) -> (weakref, signature, codes)


def _store_rows(st) -> tuple:
    """A store's per-row code arrays in its own [T][heads] row order: (pq,
    rvq, active, rvq_sub, sparse_idx, sparse_val) as the segment table takes
    them (rvq with active None: dense rows, row r's codes are row r)."""
    pq = _contig(st.pq_codes)
    rows = int(pq.shape[0]) * int(pq.shape[1])
    if st.rvq_codes.dim() == 3:
        rsub = _contig(st.rvq_codes) if st.rvq_codes.shape[-1] else None
        k = 0 if st.sparse_idx is None else int(st.sparse_idx.shape[-1])
        return (pq, None, None, rsub, _contig(st.sparse_idx) if k else None, _contig(st.sparse_val) if k else None)
    # every row active (the offsets, sorted and distinct, are then 0 .. rows-1): the
    # gated codes of row r are row r, and the kernels take no active map
    a = int(st.rvq_codes.shape[0])
    act = active_map(st.rvq_offsets, rows) if 0 < a < rows else None
    return (pq, _contig(st.rvq_codes) if a else None, act, None, None, None)


def _store_rows_head_major(st) -> tuple:
    """``_store_rows`` with every per-row array in [heads][T] order (row h * T
    + t; active entries still index the store's rvq codes), memoized per store
    until its code tensors change (data pointer, version or shape).  A head's
    consecutive tokens then have consecutive codes, which the decode kernels
    read in whole lines instead of a few bytes of each."""
    pq = st.pq_codes
    sig = tuple(None if t is None else (t.data_ptr(), t._version, tuple(t.shape))
                for t in (pq, st.rvq_codes, st.rvq_offsets, st.sparse_idx, st.sparse_val))
    key = id(pq)
    hit = _HEAD_MAJOR.get(key)
    if hit is not None and hit[0]() is pq and hit[1] == sig:
        return hit[2]
    codes = copy_head_major(st)
    _HEAD_MAJOR[key] = (weakref.ref(pq, lambda _r, k=key: _HEAD_MAJOR.pop(k, None)), sig, codes)
    return codes


def copy_head_major(st) -> tuple:
    """A new [heads][T] copy of a store's per-row code arrays (what
    ``ref_store_segment(..., head_major=True)`` keeps per store version)."""
    pq = st.pq_codes
    T, H = int(pq.shape[0]), int(pq.shape[1])
    base = _store_rows(st)
    gated = st.rvq_codes.dim() != 3

    def hm(t, width):  # [T * H, width] or [T, H, width] rows -> [H, T, width]
        return None if t is None else t.reshape(T, H, width).transpose(0, 1).contiguous()

    pqb, rvq, act, rsub, sidx, sval = base
    if gated:
        dense = rvq is not None and act is None
        codes = (hm(pqb, pqb.shape[-1]), hm(rvq, rvq.shape[-1]) if dense else rvq,
                 None if act is None else act.view(T, H).t().contiguous().view(-1), None, None, None)
    else:
        codes = (hm(pqb, pqb.shape[-1]), None, None, None if rsub is None else hm(rsub, rsub.shape[-1]),
                 None if sidx is None else hm(sidx, sidx.shape[-1]), None if sval is None else hm(sval, sval.shape[-1]))
    return codes


def ref_store_segment(key_store, value_store, token0: int, length: int, pos0: int,
                      head_major: bool = False) -> dict:
    """A coded segment of tokens token0 .. token0+length-1 of two stores in
    CompressedTensorMLX's layout: reference format (pq_codes [T, H, M] u8,
    rvq_codes [A, L] u16 placed by rvq_offsets [A] over the T*H rows) or the
    long-context format (rvq_codes [T, H, M_r] u8, sparse_idx / sparse_val
    [T, H, k]).

    ``head_major`` attends a copy of the codes in [heads][T] order instead,
    kept per store until its code tensors change (so for stores that outlive
    the call: a decode loop's warm tier); stores of unequal lengths keep their
    own order."""
    seg = {"len": int(length), "pos0": int(pos0), "token0": int(token0), "exact": None}
    if token0 < 0 or length < 0 or token0 + length > min(key_store.num_tokens, value_store.num_tokens):
        raise ValueError("segment tokens outside the stores")
    if head_major and key_store.num_tokens == value_store.num_tokens:
        seg["k"] = _store_rows_head_major(key_store)
        seg["v"] = _store_rows_head_major(value_store)
        seg["rows"] = (1, int(key_store.num_tokens))  # row of (t, h) = t * 1 + h * T
        return seg
    for name, st in (("k", key_store), ("v", value_store)):
        seg[name] = _store_rows(st)
    return seg


def ref_exact_segment(k: torch.Tensor, v: torch.Tensor, token_stride: int, head_stride: int, token0: int,
                      length: int, pos0: int) -> dict:
    """An exact segment of [heads, ..., D] fp16 buffers: (t, h, d) at base +
    t * token_stride + h * head_stride + d (elements)."""
    for t in (k, v):
        if t.dtype != torch.float16 or t.stride(-1) != 1:
            raise ValueError("exact rows must be fp16 with unit stride over head_dim")
        hi = (token0 + length - 1) * token_stride + (t.shape[0] - 1) * head_stride + t.shape[-1] if length else 0
        if token0 < 0 or length < 0 or hi > t.numel():
            raise ValueError("exact segment outside its buffer")
    return {"len": int(length), "pos0": int(pos0), "token0": int(token0),
            "exact": (k, v, int(token_stride), int(head_stride)), "k": None, "v": None}


_REF_TABLES: "OrderedDict[Tuple[bytes, str], torch.Tensor]" = OrderedDict()


def _ref_table(raw: bytes, device) -> torch.Tensor:
    """The segment table on the device.  Equal bytes give an equal table, so
    the last few uploads are reused by content; a new one is copied from
    pinned memory without blocking the host (torch keeps the pinned block
    until the copy has run)."""
    key = (raw, str(device))
    hit = _REF_TABLES.get(key)
    if hit is not None:
        _REF_TABLES.move_to_end(key)
        return hit
    host = torch.frombuffer(bytearray(raw), dtype=torch.uint8).pin_memory()
    dev = host.to(device, non_blocking=True)
    _REF_TABLES[key] = dev
    while len(_REF_TABLES) > 16:
        _REF_TABLES.popitem(last=False)
    return dev


def ref_attention_ok(head_dim: int, M: int, C: int, q_heads: int, kv_heads: int, shared_cb: bool,
                     rvq_subspaces: int = 0, rvq_centroids: int = 0, sparse_k: int = 0) -> bool:
    """Whether ``rfsn_ref_attention`` serves the shape."""
    tab = head_dim * C * 2 * (1 if shared_cb else 2)
    sub_ok = rvq_subspaces == 0 or (head_dim % rvq_subspaces == 0 and 1 <= rvq_centroids <= 256)
    return (head_dim in (64, 128, 256) and M in (4, 8, 16, 32) and head_dim % M == 0 and 1 <= C <= 256
            and kv_heads > 0 and q_heads % kv_heads == 0 and q_heads // kv_heads <= 8 and tab <= 160 * 1024
            and sub_ok and 0 <= sparse_k <= 8)


REF_TABLES_MIN_TOKENS = 4096  # coded tokens below which the score tables do not pay off (one q head per KV head)


def ref_tables_min_tokens(group: int, queries: int = 1) -> int:
    """Coded tokens from which the score tables beat the exact decode for
    ``group`` query heads per KV head and ``queries`` query tokens.  The
    tables' histograms cost grows with the query heads while the exact
    decode of a token is shared by its group, so the break-even moves out
    with the group: measured near 3.3k, 4.7k, 8.2k and 10.3k coded tokens for
    groups of 1, 2, 4 and 8 at one query (32 query heads, D 128, 4 gated
    layers of 4,096), which ``(group + 2) / 3`` times
    ``REF_TABLES_MIN_TOKENS``, at most 2.5 times, follows.  The exact decode
    repeats per query token while the tables' launches are shared, so it
    moves in with the queries: at 2, 4 and 8 the measured break-evens were
    0.73, 0.60 and 0.57 times those of one query (groups of 1 and 4), which
    ``(queries + 1) / (2 queries)`` follows."""
    q = max(queries, 1)
    base = min(REF_TABLES_MIN_TOKENS * (max(group, 1) + 2) // 3, REF_TABLES_MIN_TOKENS * 5 // 2)
    return base * (q + 1) // (2 * q)


def _ref_format_params(k_pq_cb: torch.Tensor, k_rvq_cb: Optional[torch.Tensor], rvq_subspaces: int,
                       sparse_k: int) -> "L.RefParams":
    M, Cn, d = k_pq_cb.shape
    p = L.RefParams()
    p.head_dim, p.pq_subspaces, p.pq_centroids = M * d, M, Cn
    if k_rvq_cb is not None and rvq_subspaces:
        p.rvq_subspaces, p.rvq_centroids = int(rvq_subspaces), int(k_rvq_cb.shape[1])
    elif k_rvq_cb is not None:
        p.rvq_layers, p.rvq_centroids = int(k_rvq_cb.shape[0]), int(k_rvq_cb.shape[1])
    p.sparse_k = int(sparse_k)
    return p


def ref_table_stats(k_pq_cb: torch.Tensor, v_pq_cb: torch.Tensor, k_rvq_cb: Optional[torch.Tensor],
                    v_rvq_cb: Optional[torch.Tensor]) -> torch.Tensor:
    """The score tables' drift-guard statistics of a codebook set, float32
    [3, D] (``rfsn_ref_table_stats``): per coordinate i, the second moments
    mean_c PQ(c, i)^2 + 2 sum_l mean_c RVQ(l, c, i)^2 of K and of V, then
    max_c |PQ_V(c, i)| + sum_l max_c |RVQ_V(l, c, i)|."""
    _dev(k_pq_cb, "ref_table_stats")
    cbs = [_contig(t) if t is not None else None for t in (k_pq_cb, v_pq_cb, k_rvq_cb, v_rvq_cb)]
    p = _ref_format_params(cbs[0], cbs[2], 0, 0)
    p.k_pq_cb, p.v_pq_cb, p.k_rvq_cb, p.v_rvq_cb = (L.ptr(t) for t in cbs)
    out = torch.empty((3, p.head_dim), dtype=torch.float32, device=k_pq_cb.device)
    L.call("rfsn_ref_table_stats", C.byref(p), out.data_ptr(), _stream(k_pq_cb))
    return out


class RefLaunch:
    """A prepared ``rfsn_ref_attention`` call: its parameter block, segment
    table and workspace, with the tensors they point to kept alive;
    ``__call__`` re-issues it on the stream it was prepared on (q is read at
    launch time, so a decode loop refills it in place)."""

    def __init__(self, params: "L.RefParams", keep: list, out: torch.Tensor, stream: int, tables: bool):
        self.params = params
        self._keep = keep
        self.out = out
        self.stream = stream
        self.score_tables = tables  # whether the launch attends the coded segments through score tables
        self._fn = L.load().rfsn_ref_attention
        self._ref = C.byref(self.params)

    def __call__(self) -> torch.Tensor:
        st = self._fn(self._ref, self.stream)
        if st:
            L.check(st, "rfsn_ref_attention")
        return self.out


def ref_prepare(q: torch.Tensor, *, kv_heads: int, scale: float, causal: bool, qpos: Optional[torch.Tensor],
                segments: Sequence[dict], k_pq_cb: torch.Tensor, v_pq_cb: torch.Tensor,
                k_rvq_cb: Optional[torch.Tensor], v_rvq_cb: Optional[torch.Tensor],
                rvq_subspaces: int = 0, sparse_k: int = 0,
                out: Optional[torch.Tensor] = None, splits: int = 0,
                score_tables: Optional[float] = None, table_stats: Optional[torch.Tensor] = None,
                drift: Optional[torch.Tensor] = None) -> Optional[RefLaunch]:
    """The launch of ``ref_attention`` for these arguments, or None for an
    empty window (``out`` is then zeroed)."""
    _dev(q, "ref_attention")
    q = _contig(q)
    B, Hq, D = q.shape
    out = torch.empty_like(q) if out is None else out
    total = sum(s["len"] for s in segments)
    if total == 0:
        out.zero_()
        return None
    keep = [q, out]
    arr = (L.RefSegment * len(segments))()
    for i, sd in enumerate(segments):
        seg = arr[i]
        seg.token0, seg.len, seg.pos0 = sd["token0"], sd["len"], sd["pos0"]
        seg.code_token_stride, seg.code_head_stride = sd.get("rows", (0, 0))
        if sd["exact"] is not None:
            ek, ev, ts, hs = sd["exact"]
            seg.exact_k, seg.exact_v = ek.data_ptr(), ev.data_ptr()
            seg.exact_token_stride, seg.exact_head_stride = ts, hs
            keep += [ek, ev]
        else:
            for name, codes in (("k", seg.k), ("v", seg.v)):
                pq, rvq, act, rsub, sidx, sval = sd[name]
                gated_mismatch = rvq is not None and (k_rvq_cb is None or rvq_subspaces)
                if ((0 if rsub is None else rsub.shape[-1]) != rvq_subspaces
                        or (0 if sidx is None else sidx.shape[-1]) != sparse_k or gated_mismatch):
                    raise ValueError("segment codes do not match the format's RVQ / sparse stages")
                codes.pq, codes.rvq, codes.active = pq.data_ptr(), L.ptr(rvq), L.ptr(act)
                codes.rvq_sub, codes.sparse_idx, codes.sparse_val = L.ptr(rsub), L.ptr(sidx), L.ptr(sval)
                keep += [pq, rvq, act, rsub, sidx, sval]
    dev_segs = _ref_table(C.string_at(C.addressof(arr), C.sizeof(arr)), q.device)
    p = _ref_format_params(k_pq_cb, k_rvq_cb, rvq_subspaces, sparse_k)
    p.head_dim = D
    p.batch, p.q_heads, p.kv_heads = B, Hq, kv_heads
    p.q, p.out, p.scale, p.causal = q.data_ptr(), out.data_ptr(), float(scale), int(causal)
    qp = None if qpos is None else _qpos(qpos, B, Hq, q.device)
    p.qpos = L.ptr(qp)
    p.segments, p.num_segments, p.total_tokens = dev_segs.data_ptr(), len(segments), total
    cbs = [_contig(t) if t is not None else None for t in (k_pq_cb, v_pq_cb, k_rvq_cb, v_rvq_cb)]
    p.k_pq_cb, p.v_pq_cb, p.k_rvq_cb, p.v_rvq_cb = (L.ptr(t) for t in cbs)
    p.splits = splits
    coded = sum(sd["len"] for sd in segments if sd["exact"] is None)
    group = Hq // kv_heads if kv_heads > 0 else 1
    use_tables = (score_tables is not None and coded >= ref_tables_min_tokens(group, B)
                  and bool(L.load().rfsn_ref_tables_ok(C.byref(p))))
    if use_tables:
        if table_stats is None:
            table_stats = ref_table_stats(*cbs)
        if (table_stats.dtype != torch.float32 or tuple(table_stats.shape) != (3, D) or not table_stats.is_contiguous()
                or table_stats.device != q.device):
            raise ValueError("ref_attention: table_stats must be a contiguous float32 [3, head_dim] device tensor")
        if drift is not None and (drift.dtype != torch.float32 or drift.numel() != B * Hq or not drift.is_contiguous()
                                  or drift.device != q.device):
            raise ValueError("ref_attention: drift must be a contiguous float32 [B, Hq] device tensor")
        p.score_tables, p.table_tol = 1, float(score_tables)
        p.table_stats, p.drift = table_stats.data_ptr(), L.ptr(drift)
        keep += [table_stats, drift]
    wsb = L.load().rfsn_ref_attention_workspace_bytes(C.byref(p))
    ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device=q.device)
    p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
    keep += [dev_segs, qp, ws, *cbs]
    return RefLaunch(p, keep, out, _stream(q), use_tables)


def ref_attention(q: torch.Tensor, *, kv_heads: int, scale: float, causal: bool, qpos: Optional[torch.Tensor],
                  segments: Sequence[dict], k_pq_cb: torch.Tensor, v_pq_cb: torch.Tensor,
                  k_rvq_cb: Optional[torch.Tensor], v_rvq_cb: Optional[torch.Tensor],
                  rvq_subspaces: int = 0, sparse_k: int = 0,
                  out: Optional[torch.Tensor] = None, splits: int = 0,
                  score_tables: Optional[float] = None, table_stats: Optional[torch.Tensor] = None,
                  drift: Optional[torch.Tensor] = None, info: Optional[dict] = None) -> torch.Tensor:
    """Attention of q [B, Hq, D] over the window of ``segments`` (window
    order; ``ref_store_segment`` / ``ref_exact_segment``), decoding the coded
    ones on the fly (``rfsn_ref_attention``).  RVQ codebooks are [L, C_r, D]
    (gated full-dimension layers) or, with ``rvq_subspaces``, [M_r, C_r, D/M_r].

    ``score_tables`` (a tolerance) attends the coded segments through q .
    codeword tables and per-codeword sums of the weights where the format and
    shape allow it (``rfsn_ref_tables_ok``) and the window holds at least
    ``ref_tables_min_tokens(Hq // kv_heads, B)`` coded tokens, with the drift guard sending a
    group whose estimate exceeds the tolerance back to the exact decode;
    ``table_stats`` (``ref_table_stats`` of the codebooks, computed here when
    None), ``drift`` [B, Hq] float32 receives the estimates.  ``info`` (a
    dict) receives ``score_tables``: whether the launch used them."""
    launch = ref_prepare(q, kv_heads=kv_heads, scale=scale, causal=causal, qpos=qpos, segments=segments,
                         k_pq_cb=k_pq_cb, v_pq_cb=v_pq_cb, k_rvq_cb=k_rvq_cb, v_rvq_cb=v_rvq_cb,
                         rvq_subspaces=rvq_subspaces, sparse_k=sparse_k, out=out, splits=splits,
                         score_tables=score_tables, table_stats=table_stats, drift=drift)
    if info is not None:
        info["score_tables"] = launch is not None and launch.score_tables
    if launch is None:
        return out if out is not None else torch.zeros_like(q)
    return launch()


def fused_splits(batch: int, q_heads: int, kv_heads: int, hot_len: int, max_tokens: int, max_segments: int,
                 splits: int = 0) -> int:
    """Token splits per (sequence, KV head) the fused kernel uses for a call
    of this shape (``splits`` if positive, else its automatic choice)."""
    p = L.FusedParams()
    p.batch, p.q_heads, p.kv_heads = batch, q_heads, kv_heads
    p.hot_len, p.max_tokens, p.max_segments, p.splits = hot_len, max_tokens, max_segments, splits
    return int(L.load().rfsn_fused_splits(C.byref(p)))


class FusedLaunch:
    """A prepared fused launch: the parameter block and the tensors it points
    to, re-issued on the same stream by ``__call__`` (a decode loop's inner
    step, no host-side rebuilding)."""

    def __init__(self, params: L.FusedParams, keep: list, out: torch.Tensor, stream: int):
        self.params = params
        self._keep = keep
        self.out = out
        self.stream = stream
        self.drift: Optional[torch.Tensor] = None  # [B, Hq, slots] drift estimates of the guard, if any
        self.seg_table: Optional[torch.Tensor] = None  # the device rfsn_segment table the launch reads
        self._fn = L.load().rfsn_fused_decode_attention
        self._ref = C.byref(self.params)

    def __call__(self) -> torch.Tensor:
        st = self._fn(self._ref, self.stream)
        if st:
            L.check(st, "rfsn_fused_decode_attention")
        return self.out

    K_SCORING = {0: "codebook K^ rows", 1: "fp16 q.centroid tables", 2: "codebook K^ over score-table rows"}

    @property
    def k_scoring(self) -> str:
        """How the launch scores K: the codebook rows (k_layout 0), the score
        tables (drift guard recomputing where it fires), or the guard's exact
        pass alone (a guarded launch of several short splits)."""
        return self.K_SCORING[int(L.load().rfsn_fused_k_scoring(self._ref))]


class PrefetchedStep:
    """A decode step whose window includes chunks still in pinned host memory.

    ``__call__`` waits (on the host) for the work already on the launch stream,
    which may read the destination slots, queues the host-to-device ``copies``
    (dst, src, bytes) on the side stream, runs ``launches[:wait_at]`` (the
    resident part of the window) while they are in flight, makes the launch
    stream wait for the copies, then runs ``launches[wait_at:]`` (the copied
    chunks, ending with the merge).  Every call re-issues the copies it was
    built with."""

    def __init__(self, side: SideStream, copies: Sequence[Tuple[int, int, int]], launches: Sequence[FusedLaunch],
                 wait_at: int, keep: Optional[list] = None):
        if not launches:
            raise ValueError("a decode step needs at least one launch")
        self.side = side
        self.launches = list(launches)
        self.wait_at = wait_at
        self.stream = self.launches[0].stream
        self.out = self.launches[-1].out
        self.ncopies = len(copies)
        self._copies = (L.Copy * max(1, self.ncopies))()
        for i, (dst, src, nbytes) in enumerate(copies):
            self._copies[i] = L.Copy(dst, src, nbytes)
        self.copy_bytes = sum(int(c[2]) for c in copies)
        self._keep = keep

    def issue_copies(self, drain: bool = True) -> None:
        """The copies alone and their event.  With ``drain`` the host first
        waits for the work already on the launch stream, which may read the
        destination slots (the previous call of this step does); a caller
        that has ordered the copies otherwise passes False."""
        if drain:
            self.side.drain(self.stream)
        L.call("rfsn_prefetch_h2d", self._copies, self.ncopies, self.side.stream)
        L.call("rfsn_event_record", self.side.event, self.side.stream)

    def __call__(self, drain: bool = True) -> torch.Tensor:
        if self.ncopies:
            self.issue_copies(drain)
        for i, fl in enumerate(self.launches):
            if i == self.wait_at and self.ncopies:
                L.call("rfsn_stream_wait_event", self.stream, self.side.event)
            fl()
        if self.wait_at >= len(self.launches) and self.ncopies:
            L.call("rfsn_stream_wait_event", self.stream, self.side.event)
        return self.out


# --------------------------------------------------------------------------
# k-means (rfsn_v10_mlx_ane_complete.py:197-207)
# --------------------------------------------------------------------------

def kmeans_update(x: torch.Tensor, codes: torch.Tensor, codebooks: torch.Tensor) -> None:
    """In-place Lloyd update of codebooks [M, C, d] from x [N, D] and codes [N, M]."""
    _dev(x, "kmeans_update")
    x = _contig(x)
    n, D = x.shape
    M, Cn, d = codebooks.shape
    if not codebooks.is_contiguous():
        raise ValueError("kmeans_update needs contiguous codebooks")
    wsb = L.load().rfsn_kmeans_workspace_bytes(M, Cn, d)
    ws = torch.empty(wsb, dtype=torch.uint8, device=x.device)
    L.call("rfsn_kmeans_update", x.data_ptr(), n, D, D, _contig(codes).data_ptr(), M, Cn, codebooks.data_ptr(),
           ws.data_ptr(), wsb, _stream(x))


# --------------------------------------------------------------------------
# cold tier host API
# --------------------------------------------------------------------------

class SideStream:
    """A default-priority non-blocking HIP stream plus an event, for prefetch."""

    def __init__(self):
        h = C.c_void_p()
        L.call("rfsn_stream_create", C.byref(h))
        self.stream = h.value
        e = C.c_void_p()
        L.call("rfsn_event_create", C.byref(e))
        self.event = e.value
        e2 = C.c_void_p()
        L.call("rfsn_event_create", C.byref(e2))
        self.main_event = e2.value

    def drain(self, stream: int) -> None:
        """Block the host until the work queued so far on ``stream`` is done.

        Copies into device buffers that queued kernels may still read are
        ordered this way, on the host, rather than by making the side stream
        wait on an event of ``stream``: on MI355X a copy-engine transfer
        that waits on a compute-queue event costs about 130 us more than the
        2.9 MB transfer itself (60 us), while the launch stream waiting on the
        copy's event costs a few."""
        L.call("rfsn_event_record", self.main_event, stream)
        L.call("rfsn_event_synchronize", self.main_event)

    def wait_for_current(self, device=None) -> None:
        """Order later side-stream copies after the work queued on the current stream."""
        self.drain(L.stream_handle(device))

    def prefetch(self, copies: Sequence[Tuple[int, int, int]]) -> None:
        arr = (L.Copy * max(1, len(copies)))()
        for i, (dst, src, nbytes) in enumerate(copies):
            arr[i] = L.Copy(dst, src, nbytes)
        L.call("rfsn_prefetch_h2d", arr, len(copies), self.stream)
        L.call("rfsn_event_record", self.event, self.stream)

    def make_current_wait(self, device=None) -> None:
        L.call("rfsn_stream_wait_event", L.stream_handle(device), self.event)

    def synchronize(self) -> None:
        """Block the host until the copies recorded so far have finished."""
        L.call("rfsn_event_synchronize", self.event)

    def close(self) -> None:
        for name in ("event", "main_event"):
            ev = getattr(self, name)
            if ev:
                L.call("rfsn_event_destroy", ev)
                setattr(self, name, None)
        if self.stream:
            L.call("rfsn_stream_destroy", self.stream)
            self.stream = None
