"""Timed CPU baselines of the warm-tier decode and encode paths (test
infrastructure only; ``bench.py`` times them beside the GPU kernels, they are
never the thing measured on the GPU).

Encode: the reference's PyTorch form of the nearest-centroid search
(rfsn_v10_unified_mac_launcher.py:358-373), fp32 ``torch.cdist ** 2`` and
``argmin`` per subspace, applied to both stages and followed by the top-k.

Decode (long-context format):

Restates the reference's PyTorch form (rfsn_v10_unified_mac_launcher.py:
217-273): per-subspace ``F.embedding`` decode of the PQ codes, the same for
the RVQ stage, ``fp16(base + rvq)`` (quantization.py:317-319), the sparse
residual ``K[idx] = fp16(K[idx] + val)``, then the blockwise online-softmax
recurrence of attention.py:53-105 in fp32 with ``block`` tokens per step.
GQA: query head h reads KV head h // (Hq // Hkv).

Decode (reference format): ``ref_decode`` / ``ref_decode_step``, the gated
full-dimension correction of quantization.py:254-275 on the PQ base, then
the same attention.

Encode (reference format): ``ref_encode``, the PQ search above, the norm
gate and the chunked full-dimension RVQ search of quantization.py:206-252.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

MASK_FILL_VALUE = -1e30


def decode_codes(codes: torch.Tensor, codebooks: torch.Tensor) -> torch.Tensor:
    """codes [N, M] -> fp16 [N, M*d] (launcher:217-224, in fp16 storage)."""
    M, C, d = codebooks.shape
    out = torch.empty((codes.shape[0], M * d), dtype=torch.float16)
    for m in range(M):
        out[:, m * d:(m + 1) * d] = F.embedding(codes[:, m].long(), codebooks[m])
    return out


def warm_decode(pq: torch.Tensor, pq_cb: torch.Tensor, rvq: Optional[torch.Tensor] = None,
                rvq_cb: Optional[torch.Tensor] = None, sidx: Optional[torch.Tensor] = None,
                sval: Optional[torch.Tensor] = None) -> torch.Tensor:
    x = decode_codes(pq, pq_cb)
    if rvq is not None:
        x = (x.float() + decode_codes(rvq, rvq_cb).float()).half()
    if sidx is not None and sidx.shape[1]:
        idx = sidx.long()
        cur = torch.gather(x, 1, idx).float()
        x.scatter_(1, idx, (cur + sval.float()).half())
    return x


def blockwise_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, scale: float,
                        block: int) -> torch.Tensor:
    """q [B, Hq, D]; keys/values [T, Hkv, D]; non-causal decode (the query is
    the newest position, so every window token is allowed)."""
    B, Hq, D = q.shape
    T, Hkv, _ = keys.shape
    rep = Hq // Hkv
    qf = q.float()
    run_max = torch.full((B, Hq), MASK_FILL_VALUE)
    run_sum = torch.zeros((B, Hq))
    acc = torch.zeros((B, Hq, D))
    for s in range(0, T, block):
        kb = keys[s:s + block].float().repeat_interleave(rep, dim=1).permute(1, 0, 2)  # [Hq, n, D]
        vb = values[s:s + block].float().repeat_interleave(rep, dim=1).permute(1, 0, 2)
        scores = torch.einsum("bhd,hnd->bhn", qf, kb) * scale
        new_max = torch.maximum(run_max, scores.max(dim=-1).values)
        rescale = torch.exp(run_max - new_max)
        run_sum = run_sum * rescale
        acc = acc * rescale[..., None]
        e = torch.exp(scores - new_max[..., None])
        run_sum = run_sum + e.sum(dim=-1)
        acc = acc + torch.einsum("bhn,hnd->bhd", e, vb)
        run_max = new_max
    safe = torch.where(run_sum > 0, run_sum, torch.ones_like(run_sum))
    return (acc / safe[..., None]).half()


def decode_step(q: torch.Tensor, hot_k: torch.Tensor, hot_v: torch.Tensor, warm_k: dict, warm_v: dict,
                cbs: dict, scale: float, block: int) -> torch.Tensor:
    """One decode step of one sequence: decode the warm tier, concatenate
    [warm | hot] and attend.  warm_* hold plain codes [Hkv, T, *]."""
    Hkv, T, _ = warm_k["pq"].shape
    D = hot_k.shape[-1]
    parts_k, parts_v = [], []
    for codes, p, r, parts in ((warm_k, cbs["k_pq"], cbs.get("k_rvq"), parts_k),
                               (warm_v, cbs["v_pq"], cbs.get("v_rvq"), parts_v)):
        n = Hkv * T
        x = warm_decode(codes["pq"].reshape(n, -1), p,
                        None if codes.get("rvq") is None else codes["rvq"].reshape(n, -1), r,
                        None if codes.get("sparse_idx") is None else codes["sparse_idx"].reshape(n, -1),
                        None if codes.get("sparse_val") is None else codes["sparse_val"].reshape(n, -1))
        parts.append(x.reshape(Hkv, T, D).permute(1, 0, 2))
    keys = torch.cat([parts_k[0], hot_k.permute(1, 0, 2)], 0)
    values = torch.cat([parts_v[0], hot_v.permute(1, 0, 2)], 0)
    return blockwise_attention(q, keys, values, scale, block)


def ref_decode(pq: torch.Tensor, pq_cb: torch.Tensor, rvq: torch.Tensor, offsets: torch.Tensor,
               rvq_cb: torch.Tensor) -> torch.Tensor:
    """Reference-format decode (quantization.py:254-275, 310-319): PQ base,
    the gated correction fp16(sum_l fl32(C_l[code_l])) on the rows named by
    ``offsets``, then fp16(base + corr).  pq [N, M]; rvq [A, L]."""
    base = decode_codes(pq, pq_cb)
    corr = torch.zeros_like(base)
    if rvq.shape[0]:
        tot = torch.zeros((rvq.shape[0], base.shape[1]), dtype=torch.float32)
        for layer in range(rvq.shape[1]):
            tot += F.embedding(rvq[:, layer].long(), rvq_cb[layer]).float()
        corr[offsets.long()] = tot.half()
    return (base.float() + corr.float()).half()


def ref_decode_step(q: torch.Tensor, hot_k: torch.Tensor, hot_v: torch.Tensor, warm_k: dict, warm_v: dict,
                    cbs: dict, scale: float, block: int) -> torch.Tensor:
    """One reference-format decode step (cache.py:395-428 with arrival
    tiers): decode the warm stores, concatenate [hot | warm] and attend.
    hot_* [T_hot, H, D]; warm_* hold pq [T, H, M], rvq [A, L], offsets [A]."""
    T, H, M = warm_k["pq"].shape
    D = hot_k.shape[-1]
    dec = [ref_decode(w["pq"].reshape(T * H, M), cbs["pq"], w["rvq"], w["offsets"], cbs["rvq"]).reshape(T, H, D)
           for w in (warm_k, warm_v)]
    keys = torch.cat([hot_k, dec[0]], 0)
    values = torch.cat([hot_v, dec[1]], 0)
    return blockwise_attention(q, keys, values, scale, block)


def pq_encode_cdist(x: torch.Tensor, codebooks: torch.Tensor):
    """Nearest centroid per subspace the way the reference's PyTorch backend
    does it (rfsn_v10_unified_mac_launcher.py:358-373): fp32
    ``torch.cdist(sub, centroids) ** 2`` and ``argmin``; returns the codes
    [N, M] and the fp16 residual fp16(x - c)."""
    M, C, d = codebooks.shape
    codes = torch.empty((x.shape[0], M), dtype=torch.uint8)
    resid = torch.empty_like(x)
    xf = x.float()
    for m in range(M):
        sub = xf[:, m * d:(m + 1) * d]
        cents = codebooks[m].float()
        idx = (torch.cdist(sub, cents) ** 2).argmin(dim=1)
        codes[:, m] = idx.to(torch.uint8)
        resid[:, m * d:(m + 1) * d] = (sub - F.embedding(idx, cents)).half()
    return codes, resid


def ref_encode(x: torch.Tensor, pq_cb: torch.Tensor, rvq_cb: torch.Tensor, threshold: float):
    """Reference-format encode (HybridQuantizerMLX.encode, quantization.py:
    305-308) in torch-CPU fp32: PQ by ``cdist ** 2`` + ``argmin`` per subspace
    (launcher:358-373); the gate ``|fp32(r)| > threshold`` on the fp16 PQ
    residual (quantization.py:216-218); then per stage the distance form of
    ``_squared_l2_distance`` (quantization.py:92-96), ``(|x|^2 - 2 x c^T) +
    |c|^2``, over the reference's 512-centroid chunks merged with a strict <
    (quantization.py:233-246), and ``running -= c`` (249-250).  Returns
    (pq codes [N, M] u8, rvq codes [A, L] int64, mask [N] bool, offsets [A] int32)."""
    pq, r1 = pq_encode_cdist(x, pq_cb)
    r = r1.float()
    mask = torch.sqrt((r * r).sum(dim=1)) > threshold
    offsets = torch.nonzero(mask).flatten().to(torch.int32)
    run = r[offsets.long()]
    L, C, _ = rvq_cb.shape
    codes = torch.zeros((run.shape[0], L), dtype=torch.int64)
    chunk = min(512, C)
    for layer in range(L):
        cb = rvq_cb[layer].float()
        x2 = (run * run).sum(dim=1, keepdim=True)
        best = torch.full((run.shape[0],), float("inf"))
        idx = torch.zeros((run.shape[0],), dtype=torch.int64)
        for s in range(0, C, chunk):
            c = cb[s:s + chunk]
            d = (x2 - 2.0 * run @ c.T) + (c * c).sum(dim=1)[None, :]
            lb, li = d.min(dim=1)
            upd = lb < best
            best = torch.where(upd, lb, best)
            idx = torch.where(upd, li + s, idx)
        codes[:, layer] = idx
        run = run - cb[idx]
    return pq, codes, mask, offsets


def warm_encode(x: torch.Tensor, pq_cb: torch.Tensor, rvq_cb: Optional[torch.Tensor], k: int) -> dict:
    """Warm-format encode of fp16 vectors [N, D] in torch-CPU: PQ by cdist^2 +
    argmin, the subspace RVQ stage on the fp16 PQ residual, then the top-k
    |x - fp16(base + rvq)| coordinates (values fp16)."""
    pq, r1 = pq_encode_cdist(x, pq_cb)
    out = {"pq": pq}
    recon = decode_codes(pq, pq_cb)
    if rvq_cb is not None:
        rvq, _ = pq_encode_cdist(r1, rvq_cb)
        recon = (recon.float() + decode_codes(rvq, rvq_cb).float()).half()
        out["rvq"] = rvq
    if k:
        r2 = x.float() - recon.float()
        # |r2| descending, ties to the lower coordinate (a stable sort keeps index order)
        idx = torch.sort(r2.abs(), dim=1, descending=True, stable=True).indices[:, :k]
        out["sparse_idx"] = idx.to(torch.uint8)
        out["sparse_val"] = torch.gather(r2, 1, idx).half()
    return out
