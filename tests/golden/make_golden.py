"""Writes the golden fixtures of this directory from the oracle.

The reference path cannot be imported here (it needs MLX, absent from the
image, at quantization.py:6 / attention.py:6 / cache.py:7), and its own tests
hold no golden vectors, so the fixtures come from the pinned CPU oracle
(``oracle/numerics.py``; pins in ``tests/test_oracle.py``).  Each fixture is
a small ``.npz`` of seeded inputs and expected outputs:

* ``pq_m16.npz``     PQ encode, M=16 C=256 d=4 (codes, fp16 residual)
* ``pq_m8.npz``      PQ encode, M=8 C=256 d=8 (the 1,024-token smoke format)
* ``ext_m16.npz``    PQ + subspace RVQ + top-4 sparse encode and decode
* ``rvq_ref.npz``    reference-format gated RVQ, L=3 C=256 D=128, threshold 0.25
* ``attn.npz``       blockwise attention, GQA 32q/8kv, causal rows incl. -1

Run ``python tests/golden/make_golden.py`` to regenerate (deterministic).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import numerics as nx  # noqa: E402


def randn16(g, *shape, scale=1.0):
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float16)


def codebooks(g, M, C, d, scale=1.0):
    return (g.standard_normal((M, C, d), dtype=np.float32) * np.float32((2.0 / d) ** 0.5 * scale)).astype(np.float16)


def main() -> None:
    g = np.random.default_rng(20260)
    x = randn16(g, 512, 64)
    cb = codebooks(g, 16, 256, 4)
    codes, resid = nx.pq_encode(x, cb)
    np.savez_compressed(HERE / "pq_m16.npz", x=x, codebooks=cb, codes=codes, residual=resid)

    x8 = randn16(g, 256, 64)
    cb8 = codebooks(g, 8, 256, 8)
    c8, r8 = nx.pq_encode(x8, cb8)
    np.savez_compressed(HERE / "pq_m8.npz", x=x8, codebooks=cb8, codes=c8, residual=r8)

    xe = randn16(g, 512, 64)
    pq = codebooks(g, 16, 256, 4)
    rv = codebooks(g, 16, 256, 4, scale=0.35)
    e = nx.ext_encode(xe, pq, rv, 4)
    dec = nx.ext_decode(e["pq_codes"], pq, e["rvq_codes"], rv, e["sparse_idx"], e["sparse_val"])
    np.savez_compressed(HERE / "ext_m16.npz", x=xe, pq_codebooks=pq, rvq_codebooks=rv, pq_codes=e["pq_codes"],
                        rvq_codes=e["rvq_codes"], sparse_idx=e["sparse_idx"], sparse_val=e["sparse_val"],
                        decoded=dec)

    xr = randn16(g, 128, 128)
    pqr = codebooks(g, 8, 256, 16)
    # every fifth row is a concatenation of PQ centroids: its residual is zero
    # and the RVQ gate leaves it inactive
    pick = g.integers(0, 256, (len(xr[::5]), 8))
    xr[::5] = np.concatenate([pqr[m][pick[:, m]] for m in range(8)], axis=1)
    rvr = codebooks(g, 3, 256, 128)
    rvr[:, 0] = 0
    pc, rc, mask, offs = nx.hybrid_encode(xr, pqr, rvr, 0.25)
    _, res = nx.pq_encode(xr, pqr)
    np.savez_compressed(HERE / "rvq_ref.npz", x=xr, pq_codebooks=pqr, rvq_codebooks=rvr, threshold=np.float32(0.25),
                        pq_codes=pc, pq_residual=res, rvq_codes=rc, rvq_mask=mask, rvq_offsets=offs,
                        decoded=nx.hybrid_decode(pc, rc, mask, offs, pqr, rvr))

    q = randn16(g, 4, 32, 64)
    k = randn16(g, 160, 8, 64)
    v = randn16(g, 160, 8, 64)
    qpos = np.array([159, 70, 0, -1], np.int32)
    out = nx.blockwise_attention(q, k, v, 0.125, 64, True, qpos)
    out_nc = nx.blockwise_attention(q, k, v, 0.125, 64, False, None)
    np.savez_compressed(HERE / "attn.npz", q=q, keys=k, values=v, qpos=qpos, scale=np.float32(0.125),
                        out_causal=out, out_full=out_nc)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
