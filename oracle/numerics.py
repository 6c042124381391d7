"""Oracle numerics: PQ / RVQ / sparse-residual encode-decode and blockwise
exact attention, restated in numpy from the reference (test infrastructure
only; see ``oracle/__init__.py``).

Canonical rounding chain (the contract the HIP kernels match bit-for-bit):

* Squared distance (quantization.py:92-96):
  ``dist_j = fl32(fl32(L - 2*X_j) + R_j)`` with ``L = fl32(S(x*x))``,
  ``X_j = fl32(S(x*c_j))``, ``R_j = fl32(S(c_j*c_j))`` where ``S`` is a
  float64 sum taken sequentially in coordinate order starting from +0.0.
  Every product of an fp16 value with an fp16 or fp32 value is exact in
  float64, so ``S`` is fully specified and reproducible with ``v_fma_f64``.
  The reference evaluates the sums inside MLX with an unknowable order; this
  fixes one.
* Nearest centroid: first index of the minimum (``mx.argmin``,
  quantization.py:139; chunked strict-< merge, quantization.py:238-246).
* PQ residual: ``fp16(fl32(x) - fl32(c))`` (quantization.py:141-142).
* RVQ gate: ``fl32(sqrt(fl32(S(r*r)))) > fl32(thr)`` (quantization.py:216-218).
* RVQ running residual: ``fl32(run - c)`` per stage (quantization.py:249-250).
* RVQ correction: ``fp16(sum_l fl32(C_l[code_l]))`` summed in stage order
  from +0.0 (quantization.py:266-272); hybrid decode ``fp16(base + corr)``
  (quantization.py:317-319).
* Subspace RVQ stage and top-k sparse residual (the warm-tier format of the
  long-context configurations; no reference symbol): the RVQ stage is a PQ
  encode of the fp16 PQ residual with its own ``[M_r, C_r, d_r]`` codebooks;
  ``K_pr = fp16(base + c_rvq)``; ``r2 = fl32(x - K_pr)``; keep the k largest
  ``|r2|`` (descending, ties to the lower coordinate), store ``u8`` index and
  ``fp16(r2)``; decode applies ``K[idx] = fp16(K[idx] + val)``.
* Attention (attention.py:39-105): fp32 scores ``sum(q*k)*scale``, causal
  mask ``pos <= qpos`` filled with -1e30 (storage.py:16), online softmax in
  fp32, output ``fp16(out / safe_sum)``.  GQA maps query head ``h`` to KV head
  ``h // (Hq // Hkv)`` (llama32_adapter.py:384-386).

Parity status: every function here is pinned by ``tests/test_oracle.py``
(float64 brute force, closed forms, known answers, invariants).
"""

from __future__ import annotations

from typing import Optional, Sequence, Tuple

import numpy as np

F16 = np.float16
F32 = np.float32
F64 = np.float64

MASK_FILL_VALUE = F32(-1e30)  # storage.py:16


# --------------------------------------------------------------------------
# distances and nearest centroid
# --------------------------------------------------------------------------

def seq_sum_products(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Sequential float64 sum over the last axis of ``a*b`` (coordinate order).

    ``a`` [..., d] and ``b`` [..., d] broadcast; returns float64 [...].
    """
    a64 = np.asarray(a).astype(F64)
    b64 = np.asarray(b).astype(F64)
    d = a64.shape[-1]
    acc = np.zeros(np.broadcast_shapes(a64.shape[:-1], b64.shape[:-1]), dtype=F64)
    for i in range(d):
        acc = acc + a64[..., i] * b64[..., i]
    return acc


def canonical_sqdist(x: np.ndarray, c: np.ndarray) -> np.ndarray:
    """``_squared_l2_distance`` (quantization.py:92-96) in the canonical chain.

    x: [N, d] fp16 or fp32 values; c: [C, d] fp16 values.  Returns fp32 [N, C].
    """
    x = np.asarray(x)
    c = np.asarray(c)
    L = seq_sum_products(x, x).astype(F32)                       # [N]
    R = seq_sum_products(c, c).astype(F32)                       # [C]
    X = seq_sum_products(x[:, None, :], c[None, :, :]).astype(F32)  # [N, C]
    two_x = F32(2.0) * X                                         # exact
    return (L[:, None] - two_x) + R[None, :]


def nearest(x: np.ndarray, c: np.ndarray, chunk: int = 4096) -> np.ndarray:
    """First-min nearest centroid index for each row of ``x`` (int64 [N])."""
    n = x.shape[0]
    out = np.empty(n, dtype=np.int64)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        out[s:e] = np.argmin(canonical_sqdist(x[s:e], c), axis=1)
    return out


# --------------------------------------------------------------------------
# product quantizer (quantization.py:99-157)
# --------------------------------------------------------------------------

def pq_encode(x16: np.ndarray, codebooks: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """``ProductQuantizerMLX.quantize`` (quantization.py:124-144).

    x16: [N, D] fp16; codebooks: [M, C, d] fp16.  Returns (codes u8 [N, M],
    residual fp16 [N, D]).  Codes are stored as uint8 exactly like
    quantization.py:130,140 (so C must be <= 256).
    """
    x16 = np.asarray(x16)
    M, C, d = codebooks.shape
    n, D = x16.shape
    if D != M * d:
        raise ValueError(f"Expected vectors with dim {M * d}, got {D}")
    codes = np.zeros((n, M), dtype=np.uint8)
    resid = np.zeros_like(x16)
    for m in range(M):
        xs = x16[:, m * d:(m + 1) * d]
        idx = nearest(xs, codebooks[m])
        codes[:, m] = idx.astype(np.uint8)
        recon = codebooks[m][idx].astype(F32)
        resid[:, m * d:(m + 1) * d] = (xs.astype(F32) - recon).astype(x16.dtype)
    return codes, resid


def pq_decode(codes: np.ndarray, codebooks: np.ndarray) -> np.ndarray:
    """``ProductQuantizerMLX.decode`` (quantization.py:146-157): fp16 gather."""
    M, C, d = codebooks.shape
    n = codes.shape[0]
    out = np.zeros((n, M * d), dtype=F16)
    for m in range(M):
        out[:, m * d:(m + 1) * d] = codebooks[m][codes[:, m].astype(np.int64)]
    return out


# --------------------------------------------------------------------------
# gated full-dimension residual VQ (quantization.py:178-275)
# --------------------------------------------------------------------------

def rvq_norms(resid16: np.ndarray) -> np.ndarray:
    """fp32 L2 norm of each residual row (quantization.py:216)."""
    s = seq_sum_products(resid16, resid16).astype(F32)
    return np.sqrt(s).astype(F32)


def rvq_encode_full(resid16: np.ndarray, codebooks: np.ndarray, threshold: float
                    ) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """``ResidualVQMLX.encode`` (quantization.py:206-252).

    resid16 [N, D]; codebooks [L, C, D] fp16.  Returns (codes u16 [A, L],
    mask bool [N], offsets int32 [A]).
    """
    resid16 = np.asarray(resid16)
    L, C, D = codebooks.shape
    n, dim = resid16.shape
    if dim != D:
        raise ValueError(f"Expected residual dim {D}, got {dim}")
    mask = rvq_norms(resid16) > F32(threshold)
    active = np.flatnonzero(mask)
    if active.size == 0:
        return (np.zeros((0, L), dtype=np.uint16), mask, np.zeros((0,), dtype=np.int32))
    running = resid16[active].astype(F32)
    codes = np.zeros((active.size, L), dtype=np.uint16)
    for layer in range(L):
        idx = nearest(running, codebooks[layer])
        codes[:, layer] = idx.astype(np.uint16)
        running = running - codebooks[layer][idx].astype(F32)
    return codes, mask, active.astype(np.int32)


def rvq_decode_correction(codes: np.ndarray, mask: np.ndarray, offsets: np.ndarray,
                          codebooks: np.ndarray) -> np.ndarray:
    """``ResidualVQMLX.decode_correction`` (quantization.py:254-275)."""
    L, C, D = codebooks.shape
    n = int(mask.shape[0])
    corr = np.zeros((n, D), dtype=F16)
    a = int(codes.shape[0])
    if a == 0:
        return corr
    total = np.zeros((a, D), dtype=F32)
    for layer in range(L):
        total = total + codebooks[layer][codes[:, layer].astype(np.int64)].astype(F32)
    corr[np.asarray(offsets, dtype=np.int64)] = total.astype(F16)
    return corr


def hybrid_add(base16: np.ndarray, corr16: np.ndarray) -> np.ndarray:
    """``base + correction`` in fp16 (quantization.py:319): fp16(f32 + f32)."""
    return (base16.astype(F32) + corr16.astype(F32)).astype(F16)


def hybrid_encode(x16, pq_cb, rvq_cb, threshold):
    """``HybridQuantizerMLX.encode`` (quantization.py:305-308)."""
    pq_codes, resid = pq_encode(x16, pq_cb)
    rvq_codes, mask, offsets = rvq_encode_full(resid, rvq_cb, threshold)
    return pq_codes, rvq_codes, mask, offsets


def hybrid_decode(pq_codes, rvq_codes, mask, offsets, pq_cb, rvq_cb):
    """``HybridQuantizerMLX.decode`` (quantization.py:310-319)."""
    base = pq_decode(pq_codes, pq_cb)
    corr = rvq_decode_correction(rvq_codes, mask, offsets, rvq_cb)
    return hybrid_add(base, corr)


# --------------------------------------------------------------------------
# subspace RVQ stage + top-k sparse residual (long-context warm format)
# --------------------------------------------------------------------------

def sparse_topk(x16: np.ndarray, recon16: np.ndarray, k: int) -> Tuple[np.ndarray, np.ndarray]:
    """Top-k |r2| coordinates of ``r2 = fl32(x - recon)``.

    Order: descending |r2|, ties to the lower coordinate index.  Returns
    (idx u8 [N, k], val fp16 [N, k]).
    """
    r2 = x16.astype(F32) - recon16.astype(F32)
    n, D = r2.shape
    if k == 0:
        return np.zeros((n, 0), np.uint8), np.zeros((n, 0), F16)
    a = np.abs(r2)
    # stable sort on -|r2| keeps the lower index first among equal magnitudes
    order = np.argsort(-a, axis=1, kind="stable")[:, :k]
    idx = order.astype(np.uint8)
    val = np.take_along_axis(r2, order, axis=1).astype(F16)
    return idx, val


def apply_sparse(recon16: np.ndarray, idx: np.ndarray, val: np.ndarray) -> np.ndarray:
    """``K[idx] = fp16(K[idx] + val)`` per row (indices are distinct)."""
    out = recon16.copy()
    if idx.shape[1] == 0:
        return out
    rows = np.arange(out.shape[0])[:, None]
    cur = out[rows, idx.astype(np.int64)].astype(F32)
    out[rows, idx.astype(np.int64)] = (cur + val.astype(F32)).astype(F16)
    return out


def ext_encode(x16: np.ndarray, pq_cb: np.ndarray, rvq_cb: Optional[np.ndarray], k: int) -> dict:
    """PQ + optional subspace-RVQ stage + optional top-k sparse residual."""
    pq_codes, r1 = pq_encode(x16, pq_cb)
    base = pq_decode(pq_codes, pq_cb)
    out = {"pq_codes": pq_codes}
    if rvq_cb is not None:
        rvq_codes, _ = pq_encode(r1, rvq_cb)
        recon = hybrid_add(base, pq_decode(rvq_codes, rvq_cb))
        out["rvq_codes"] = rvq_codes
    else:
        recon = base
    if k > 0:
        idx, val = sparse_topk(x16, recon, k)
        out["sparse_idx"] = idx
        out["sparse_val"] = val
    return out


def ext_decode(pq_codes, pq_cb, rvq_codes=None, rvq_cb=None, sparse_idx=None, sparse_val=None):
    recon = pq_decode(pq_codes, pq_cb)
    if rvq_codes is not None:
        recon = hybrid_add(recon, pq_decode(rvq_codes, rvq_cb))
    if sparse_idx is not None and sparse_idx.shape[1] > 0:
        recon = apply_sparse(recon, sparse_idx, sparse_val)
    return recon


def score_delta(pq_codes, pq_cb, rvq_codes, rvq_cb, sparse_idx, sparse_val) -> np.ndarray:
    """Sparse entries as score deltas: ``fp16(c - (fl32(base[idx]) + fl32(rvq[idx])))``
    in fp32, c = the decoded (corrected) coordinate ``ext_decode`` leaves at idx.

    A scorer that sums q . base + q . rvq unrounded adds q[idx] * delta to
    reach q . K of the decoded key at the sparse coordinates.  The decoded
    coordinate follows quantization.py:317-319 (fp16(base + rvq)) and the
    sparse stage of ``apply_sparse``.
    """
    base = pq_decode(pq_codes, pq_cb)
    corr = pq_decode(rvq_codes, rvq_cb) if rvq_codes is not None else np.zeros_like(base)
    dec = ext_decode(pq_codes, pq_cb, rvq_codes, rvq_cb, sparse_idx, sparse_val)
    ix = sparse_idx.astype(np.int64)
    c = np.take_along_axis(dec, ix, axis=1).astype(F32)
    exact = np.take_along_axis(base, ix, axis=1).astype(F32) + np.take_along_axis(corr, ix, axis=1).astype(F32)
    return (c - exact).astype(F16)


# --------------------------------------------------------------------------
# compressed-tensor helpers (quantization.py:330-403), numpy containers
# --------------------------------------------------------------------------

def compress_tensor_sequence(t16: np.ndarray, pq_cb, rvq_cb, threshold) -> dict:
    """``_compress_tensor_sequence`` (quantization.py:330-343)."""
    T, H, D = t16.shape
    pq, rvq, mask, offs = hybrid_encode(t16.reshape(T * H, D), pq_cb, rvq_cb, threshold)
    return {"pq_codes": pq.reshape(T, H, pq_cb.shape[0]), "rvq_codes": rvq,
            "rvq_mask": mask.reshape(T, H), "rvq_offsets": offs.astype(np.int32), "num_heads": H}


def append_compressed(a: dict, b: dict) -> dict:
    """``_append_compressed_tensor`` (quantization.py:346-361)."""
    if a["num_heads"] != b["num_heads"]:
        raise ValueError("Compressed tensors must have the same number of heads")
    shift = a["pq_codes"].shape[0] * a["num_heads"]
    return {"pq_codes": np.concatenate([a["pq_codes"], b["pq_codes"]]),
            "rvq_codes": np.concatenate([a["rvq_codes"], b["rvq_codes"]]),
            "rvq_mask": np.concatenate([a["rvq_mask"], b["rvq_mask"]]),
            "rvq_offsets": np.concatenate([a["rvq_offsets"], b["rvq_offsets"] + shift]).astype(np.int32),
            "num_heads": a["num_heads"]}


def slice_compressed(t: dict, start: int, end: int) -> dict:
    """``_slice_compressed_tensor`` (quantization.py:364-391)."""
    T = t["pq_codes"].shape[0]
    if start < 0 or end < start or end > T:
        raise ValueError("Invalid slice for compressed tensor")
    H = t["num_heads"]
    offs = t["rvq_offsets"].astype(np.int64)
    sel = np.where((offs >= start * H) & (offs < end * H))[0]
    return {"pq_codes": t["pq_codes"][start:end], "rvq_codes": t["rvq_codes"][sel],
            "rvq_mask": t["rvq_mask"][start:end],
            "rvq_offsets": (offs[sel] - start * H).astype(np.int32), "num_heads": H}


def decode_compressed(t: dict, pq_cb, rvq_cb) -> np.ndarray:
    """``_decode_compressed_tensor`` (quantization.py:394-403)."""
    T = t["pq_codes"].shape[0]
    H = t["num_heads"]
    D = pq_cb.shape[0] * pq_cb.shape[2]
    if T == 0:
        return np.zeros((0, H, D), dtype=F16)
    out = hybrid_decode(t["pq_codes"].reshape(T * H, -1), t["rvq_codes"], t["rvq_mask"].reshape(-1),
                        t["rvq_offsets"], pq_cb, rvq_cb)
    return out.reshape(T, H, D)


# --------------------------------------------------------------------------
# attention (attention.py:16-105)
# --------------------------------------------------------------------------

def normalize_query_positions(query_positions, batch: int, heads: int, default: int) -> np.ndarray:
    """``_normalize_query_positions`` (attention.py:16-36)."""
    if query_positions is None:
        return np.full((batch, heads), default, dtype=np.int32)
    pos = np.asarray(query_positions)
    if pos.ndim == 1:
        if pos.shape[0] != batch:
            raise ValueError("query_positions length must equal batch size")
        return np.broadcast_to(pos.reshape(batch, 1).astype(np.int32), (batch, heads)).copy()
    if tuple(pos.shape) == (batch, heads):
        return pos.astype(np.int32)
    raise ValueError("query_positions must have shape [B] or [B, H]")


def kv_head_map(num_q_heads: int, num_kv_heads: int) -> np.ndarray:
    """Query head -> KV head (``_repeat_kv`` index map, llama32_adapter.py:384-386)."""
    if num_q_heads % num_kv_heads:
        raise ValueError("num_q_heads must be a multiple of num_kv_heads")
    return np.arange(num_q_heads) // (num_q_heads // num_kv_heads)


def blockwise_attention(q: np.ndarray, keys: np.ndarray, values: np.ndarray, scale: float,
                        block_size: int, causal: bool = False,
                        query_positions=None) -> np.ndarray:
    """``_blockwise_exact_attention`` (attention.py:39-105), fp32 recurrence.

    q [B, Hq, D]; keys/values [T, Hkv, D] with Hq a multiple of Hkv.
    """
    B, Hq, D = q.shape
    T = int(keys.shape[0])
    if T == 0:
        return np.zeros((B, Hq, D), dtype=q.dtype)
    kvmap = kv_head_map(Hq, keys.shape[1])
    q32 = q.astype(F32)
    run_max = np.full((B, Hq), MASK_FILL_VALUE, dtype=F32)
    run_sum = np.zeros((B, Hq), dtype=F32)
    acc = np.zeros((B, Hq, D), dtype=F32)
    pos = normalize_query_positions(query_positions, B, Hq, T - 1)
    sc = F32(scale)
    for s in range(0, T, block_size):
        e = min(s + block_size, T)
        kb = keys[s:e].astype(F32)[:, kvmap, :].transpose(1, 0, 2)     # [Hq, n, D]
        vb = values[s:e].astype(F32)[:, kvmap, :].transpose(1, 0, 2)
        scores = np.sum(q32[:, :, None, :] * kb[None], axis=-1) * sc    # [B, Hq, n]
        if causal:
            allowed = np.arange(s, e)[None, None, :] <= pos[:, :, None]
            scores = np.where(allowed, scores, MASK_FILL_VALUE).astype(F32)
        else:
            allowed = None
        new_max = np.maximum(run_max, scores.max(axis=-1))
        rescale = np.exp(run_max - new_max).astype(F32)
        run_sum = run_sum * rescale
        acc = acc * rescale[:, :, None]
        ex = np.exp(scores - new_max[:, :, None]).astype(F32)
        if allowed is not None:
            ex = ex * allowed.astype(F32)
        run_sum = run_sum + ex.sum(axis=-1)
        acc = acc + np.sum(ex[:, :, :, None] * vb[None], axis=2)
        run_max = new_max
    safe = np.where(run_sum > 0, run_sum, F32(1.0)).astype(F32)
    return (acc / safe[:, :, None]).astype(q.dtype)


def dense_attention_f64(q, keys, values, scale, causal=False, query_positions=None) -> np.ndarray:
    """Textbook softmax attention in float64 (pins ``blockwise_attention``)."""
    B, Hq, D = q.shape
    T = keys.shape[0]
    kvmap = kv_head_map(Hq, keys.shape[1])
    k = keys.astype(F64)[:, kvmap, :]
    v = values.astype(F64)[:, kvmap, :]
    s = np.einsum("bhd,thd->bht", q.astype(F64), k) * scale
    out = np.zeros((B, Hq, D))
    pos = normalize_query_positions(query_positions, B, Hq, T - 1)
    for b in range(B):
        for h in range(Hq):
            allowed = np.arange(T) <= pos[b, h] if causal else np.ones(T, bool)
            if not allowed.any():
                continue
            z = s[b, h][allowed]
            w = np.exp(z - z.max())
            out[b, h] = (w[:, None] * v[allowed, h, :]).sum(0) / w.sum()
    return out
