"""Batched warm-tier KV cache: B independent sequences decoded by one fused
launch.

The reference keeps one ``RFSNv10KVCacheMLX`` per sequence
(cache.py:33-57) and its ``attention_forward`` serves queries over that one
cache.  Here the HBM image of B sequences lives in shared device buffers:

* hot tier: ``hot_k / hot_v`` fp16 ``[B, Hkv, hot_cap, D]`` (newest tokens);
* warm tier: PQ / RVQ codes in the tiled layout ``[B, Hkv, cap*M]`` and the
  sparse residual ``[B, Hkv, cap, k]`` (u8 index, fp16 value), plus the
  corrected coordinates fp16(K[idx] + val) the fused kernel streams in place
  of the residual values.  When the kernel can score K through q . centroid
  tables (16 + 16 subspaces, at most 4 query heads per KV head), K codes are
  score-table rows instead and K's streamed sparse values the score deltas;
* codebooks per sequence, K and V separately: ``[B, M, C, d]``.

Window order per sequence is warm (positions 0..W-1) then hot, the recency
tier policy.  ``sequence_window(b)`` materializes one sequence's window with
the decode kernel for parity checks (cache.py:344-393 semantics).
"""

from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import torch

from . import kernels as K
from .quantization import HybridQuantizerMLX
from .storage import RFSNConfig


class RFSNBatchedKVCache:
    def __init__(self, config: RFSNConfig, batch: int, device=None):
        self.config = config
        self.batch = batch
        self.H = config.kv_heads
        self.D = config.head_dim
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.hot_cap = config.hot_capacity
        self.warm_cap = K.round_up(config.warm_capacity, K.TILE)
        self.fmt: Optional[K.WarmFormat] = None
        self.num_hot = [0] * batch
        self.num_warm = [0] * batch
        self._table = None
        self._ws = None
        self._guard: Optional[torch.Tensor] = None  # [B, 65] drift-guard rows (score tables)
        self._vmax = [0.0] * batch                  # per sequence: max |V| of its values and V codebooks
        self.last_drift: Optional[torch.Tensor] = None
        self.quantizers: List[Optional[Tuple[HybridQuantizerMLX, HybridQuantizerMLX]]] = [None] * batch

    def _alloc(self, fmt: K.WarmFormat) -> None:
        B, H, D, dev = self.batch, self.H, self.D, self.device
        self.fmt = fmt
        tables = self.config.fused_score_tables and K.score_layout_ok(fmt, self.config.num_heads, H)
        self.k_layout = 1 if tables else 0
        self.guarded = bool(tables) and self.config.score_table_tolerance is not None
        self.hot_k = torch.zeros((B, H, self.hot_cap, D), dtype=torch.float16, device=dev)
        self.hot_v = torch.zeros_like(self.hot_k)
        cap = self.warm_cap
        self.codes = {}
        for kv in ("k", "v"):
            c = {"pq": torch.zeros((B, H, cap * fmt.pq_subspaces), dtype=torch.uint8, device=dev)}
            c["rvq"] = (torch.zeros((B, H, cap * fmt.rvq_subspaces), dtype=torch.uint8, device=dev)
                        if fmt.rvq_subspaces else None)
            c["sparse_idx"] = (torch.zeros((B, H, cap, fmt.sparse_k), dtype=torch.uint8, device=dev)
                               if fmt.sparse_k else None)
            c["sparse_val"] = (torch.zeros((B, H, cap, fmt.sparse_k), dtype=torch.float16, device=dev)
                               if fmt.sparse_k else None)
            # corrected coordinates fp16(K[idx] + val): the sparse values the fused kernel streams
            # (score deltas for K in the score-table layout, with the indices in that layout; under
            # the drift guard a second plane [B, 2, H, cap, k] holds the corrected coordinates in
            # the same positions for the exact pass)
            c["sparse_fold"], c["sparse_cc"] = None, None
            if fmt.sparse_k and kv == "k" and self.guarded:
                planes = torch.zeros((B, 2, H, cap, fmt.sparse_k), dtype=torch.float16, device=dev)
                c["sparse_fold"], c["sparse_cc"] = planes[:, 0], planes[:, 1]
            elif fmt.sparse_k:
                c["sparse_fold"] = torch.zeros_like(c["sparse_val"])
            c["sparse_idx_s"] = (torch.zeros_like(c["sparse_idx"])
                                 if fmt.sparse_k and kv == "k" and self.k_layout == 1 else None)
            self.codes[kv] = c
        M, Cn, d = fmt.pq_subspaces, fmt.pq_centroids, D // fmt.pq_subspaces
        self.cb = {"k_pq": torch.zeros((B, M, Cn, d), dtype=torch.float16, device=dev)}
        self.cb["v_pq"] = torch.zeros_like(self.cb["k_pq"])
        if fmt.rvq_subspaces:
            Mr, Cr = fmt.rvq_subspaces, fmt.rvq_centroids
            self.cb["k_rvq"] = torch.zeros((B, Mr, Cr, D // Mr), dtype=torch.float16, device=dev)
            self.cb["v_rvq"] = torch.zeros_like(self.cb["k_rvq"])

    def prefill(self, b: int, keys: torch.Tensor, values: torch.Tensor, key_quantizer: HybridQuantizerMLX,
                value_quantizer: HybridQuantizerMLX) -> None:
        """Load sequence b: the newest ``hot_capacity`` tokens stay exact, the
        older ones are encoded into the warm tier."""
        if keys.shape != values.shape or keys.dim() != 3 or keys.shape[1:] != (self.H, self.D):
            raise ValueError(f"keys/values must be [T, {self.H}, {self.D}]")
        fmt = key_quantizer.warm_format()
        if value_quantizer.warm_format() != fmt:
            raise ValueError("key and value quantizers must share one format")
        if self.fmt is None:
            self._alloc(fmt)
        elif fmt != self.fmt:
            raise ValueError("every sequence must use the same warm format")
        T = int(keys.shape[0])
        nh = min(T, self.hot_cap)
        nw = T - nh
        if nw > self.warm_cap:
            raise ValueError(f"{nw} warm tokens exceed the warm capacity {self.warm_cap}")
        keys = keys.to(self.device, torch.float16)
        values = values.to(self.device, torch.float16)
        self.hot_k[b, :, :nh] = keys[nw:].permute(1, 0, 2)
        self.hot_v[b, :, :nh] = values[nw:].permute(1, 0, 2)
        for kv, x, qz in (("k", keys, key_quantizer), ("v", values, value_quantizer)):
            self.cb[f"{kv}_pq"][b] = qz.pq.codebooks
            if fmt.rvq_subspaces:
                self.cb[f"{kv}_rvq"][b] = qz.rvq.codebooks
            if nw == 0:
                continue
            flat = x[:nw].permute(1, 0, 2).reshape(self.H * nw, self.D).contiguous()
            out = K.warm_encode(flat, fmt, qz.pq.codebooks, qz.rvq.codebooks if fmt.rvq_subspaces else None)
            c = self.codes[kv]
            score_rows = kv == "k" and self.k_layout == 1
            fold = None
            if fmt.sparse_k:
                c["sparse_idx"][b, :, :nw] = out["sparse_idx"].view(self.H, nw, -1)
                c["sparse_val"][b, :, :nw] = out["sparse_val"].view(self.H, nw, -1)
                fold = K.sparse_fold(fmt, out["pq"], qz.pq.codebooks, out.get("rvq"),
                                     qz.rvq.codebooks if fmt.rvq_subspaces else None, out["sparse_idx"],
                                     out["sparse_val"], delta=score_rows).view(self.H, nw, -1)
            view3 = lambda t: None if t is None else t.view(self.H, nw, -1)
            if score_rows:
                dst = {"pq": c["pq"][b], "rvq": c["rvq"][b],
                       "sparse_idx": c["sparse_idx_s"][b] if fmt.sparse_k else None,
                       "sparse_val": c["sparse_fold"][b] if fmt.sparse_k else None}
                K.pack_score_codes(view3(out["pq"]), view3(out["rvq"]), view3(out.get("sparse_idx")), fold, dst, 0)
                if c["sparse_cc"] is not None:
                    cc = K.sparse_fold(fmt, out["pq"], qz.pq.codebooks, out["rvq"], qz.rvq.codebooks,
                                       out["sparse_idx"], out["sparse_val"]).view(self.H, nw, -1)
                    K.pack_score_codes(view3(out["pq"]), view3(out["rvq"]), view3(out["sparse_idx"]), cc,
                                       dict(dst, sparse_val=c["sparse_cc"][b]), 0)
            else:
                K.pack_codes(view3(out["pq"]), c["pq"][b], 0)
                if fmt.rvq_subspaces:
                    K.pack_codes(view3(out["rvq"]), c["rvq"][b], 0)
                if fmt.sparse_k:
                    c["sparse_fold"][b, :, :nw] = fold
        self.num_hot[b] = nh
        self.num_warm[b] = nw
        self.quantizers[b] = (key_quantizer, value_quantizer)
        self._table = None
        if self.guarded:
            vp, vr = value_quantizer.pq.codebooks.float(), value_quantizer.rvq.codebooks.float()
            vcb = (vp.abs().amax(-2) + vr.abs().amax(-2)).amax()
            self._vmax[b] = float(torch.maximum(values.abs().amax().float(), vcb))
            self._guard = None

    def _segment_table(self):
        if self._table is None:
            t = K.SegmentTable(self.batch)
            for b in range(self.batch):
                if self.num_warm[b]:
                    kc = {k: (None if v is None else v[b]) for k, v in _kernel_view(self.codes["k"]).items()}
                    vc = {k: (None if v is None else v[b]) for k, v in _kernel_view(self.codes["v"]).items()}
                    t.add(b, kc, vc, self.warm_cap, self.num_warm[b], 0)
            self._table = (t, t.to_device(self.device))
        return self._table

    def _entry_tables(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """Per-sequence entry-major K and V tables ([B, 256, 128],
        ``kernels.entry_tables``), rebuilt when a codebook tensor changes."""
        cbs = [self.cb["k_pq"], self.cb.get("k_rvq"), self.cb["v_pq"], self.cb.get("v_rvq")]
        key = tuple((t.data_ptr(), t._version) if t is not None else None for t in cbs)
        if getattr(self, "_tables_key", None) != key:
            self._tables = (K.entry_tables(cbs[0], cbs[1]), K.entry_tables(cbs[2], cbs[3]))
            self._tables_key = key
        return self._tables

    def prepare(self, q: torch.Tensor, causal: bool = False, query_positions=None, splits: int = 0,
                out: Optional[torch.Tensor] = None) -> "K.FusedLaunch":
        """A reusable launch of ``attention_forward`` on these buffers (q is
        read at launch time, so a decode loop refills q in place)."""
        return self.attention_forward(q, causal, query_positions, splits, out, launch=False)

    def attention_forward(self, q: torch.Tensor, causal: bool = False, query_positions=None, splits: int = 0,
                          out: Optional[torch.Tensor] = None, launch: bool = True):
        """q [B, Hq, D] (one decode query per sequence) -> [B, Hq, D] fp16."""
        if q.shape[0] != self.batch or q.shape[2] != self.D or q.shape[1] % self.H:
            raise ValueError("q must be [B, Hq, D] with Hq a multiple of the KV heads")
        if len(set(self.num_hot)) != 1 or (causal and len(set(self.num_warm)) != 1):
            raise ValueError("every sequence must hold the same hot length (and warm length when causal)")
        if self.k_layout == 1 and not K.score_layout_ok(self.fmt, q.shape[1], self.H):
            raise ValueError(f"K codes are laid out for {self.config.num_heads} query heads; "
                             f"got {q.shape[1]} (more than 4 per KV head)")
        table, dev_table = self._segment_table()
        f = self.fmt
        qpos = None
        if causal:
            total = self.num_hot[0] + self.num_warm[0]
            if query_positions is None:
                qpos = torch.full((self.batch, q.shape[1]), total - 1, dtype=torch.int32, device=self.device)
            else:
                qpos = torch.as_tensor(query_positions, device=self.device).to(torch.int32)
                if qpos.dim() == 1:
                    qpos = qpos[:, None].expand(self.batch, q.shape[1]).contiguous()
        if self._ws is None:
            self._ws = torch.empty(4 << 20, dtype=torch.uint8, device=self.device)
        guard = {}
        if self.guarded:
            if self._guard is None:
                vmax = torch.tensor(self._vmax, dtype=torch.float32, device=self.device)
                self._guard = K.score_guard(self.cb["k_pq"], self.cb["k_rvq"], vmax).contiguous()
            guard = dict(guard=self._guard, guard_tol=float(self.config.score_table_tolerance))
        fl = K.fused_attention(
            q, f, kv_heads=self.H, scale=self.D ** -0.5, causal=causal, qpos=qpos, hot_k=self.hot_k,
            hot_v=self.hot_v, hot_len=self.num_hot[0], hot_pos0=self.num_warm[0],
            hot_seq_stride=self.H * self.hot_cap * self.D, segments=table, table=dev_table,
            k_pq_cb=self.cb["k_pq"], v_pq_cb=self.cb["v_pq"], k_rvq_cb=self.cb.get("k_rvq"),
            v_rvq_cb=self.cb.get("v_rvq"), cb_batch_stride=True, tables=self._entry_tables(),
            max_tokens=max(h + w for h, w in zip(self.num_hot, self.num_warm)), splits=splits,
            workspace=self._ws, out=out, hot_cap=self.hot_cap, launch=False, k_layout=self.k_layout, **guard)
        self.last_drift = fl.drift
        return fl() if launch else fl

    def sequence_window(self, b: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """Materialized (keys, values) [W, Hkv, D] of sequence b, warm then hot."""
        kq, vq = self.quantizers[b]
        nw, nh = self.num_warm[b], self.num_hot[b]
        outs = []
        for kv, qz, hot in (("k", kq, self.hot_k), ("v", vq, self.hot_v)):
            parts = []
            if nw:
                parts.append(self._decode_warm(kv, b, qz).view(self.H, nw, self.D).permute(1, 0, 2))
            parts.append(hot[b, :, :nh].permute(1, 0, 2))
            outs.append(torch.cat(parts, 0).contiguous())
        return outs[0], outs[1]

    def plain_codes(self, kv: str, b: int) -> Dict[str, Optional[torch.Tensor]]:
        """Warm codes of sequence b in the reference layout: pq / rvq [H, W, M]
        and the sparse residual [H, W, k] (device tensors)."""
        f = self.fmt
        nw = self.num_warm[b]
        c = self.codes[kv]
        if kv == "k" and self.k_layout == 1:
            pq, rvq, _, _ = K.unpack_score_codes({"pq": c["pq"][b], "rvq": c["rvq"][b]}, nw)
        else:
            pq = untile(c["pq"][b], f.pq_subspaces, nw)
            rvq = untile(c["rvq"][b], f.rvq_subspaces, nw) if f.rvq_subspaces else None
        return {"pq": pq, "rvq": rvq,
                "sparse_idx": c["sparse_idx"][b, :, :nw] if f.sparse_k else None,
                "sparse_val": c["sparse_val"][b, :, :nw] if f.sparse_k else None}

    def _decode_warm(self, kv: str, b: int, qz: HybridQuantizerMLX) -> torch.Tensor:
        """Decode the warm codes of sequence b (head-major rows)."""
        f = self.fmt
        nw = self.num_warm[b]
        c = self.plain_codes(kv, b)
        flat = lambda t: None if t is None else t.reshape(self.H * nw, -1)
        return K.decode(f, flat(c["pq"]), qz.pq.codebooks, flat(c["rvq"]),
                        qz.rvq.codebooks if f.rvq_subspaces else None, flat(c["sparse_idx"]),
                        flat(c["sparse_val"]))


def _kernel_view(c: Dict[str, Optional[torch.Tensor]]) -> Dict[str, Optional[torch.Tensor]]:
    """The arrays the fused kernel streams: tiled codes, sparse indices and
    the corrected coordinates as its sparse values."""
    si = c["sparse_idx_s"] if c.get("sparse_idx_s") is not None else c["sparse_idx"]
    return {"pq": c["pq"], "rvq": c["rvq"], "sparse_idx": si, "sparse_val": c["sparse_fold"],
            "sparse_cc": c.get("sparse_cc")}


def untile(tiled: torch.Tensor, M: int, T: int) -> torch.Tensor:
    """Inverse of the tiled code layout: [H, cap*M] -> plain [H, T, M]."""
    H = tiled.shape[0]
    tpi = 64 // M
    ipt = 32 // tpi
    t = torch.arange(T, device=tiled.device)
    m = torch.arange(M, device=tiled.device)
    off = ((t // 32) * 32 * M)[:, None] + ((t % tpi)[:, None] * M + m[None, :]) * ipt + ((t % 32) // tpi)[:, None]
    return tiled[:, off.reshape(-1)].reshape(H, T, M)
