"""Golden fixtures (tests/golden/*.npz, written by make_golden.py).

CPU: the oracle reproduces every fixture bit-for-bit.
GPU: the HIP path reproduces them through the C ABI -- codes, residuals,
sparse entries and reconstructions bit-exact, attention within 2e-3.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import numerics as nx

GOLD = Path(__file__).resolve().parent / "golden"
TOL = 2e-3


def load(name):
    with np.load(GOLD / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float16:
        return a.shape == b.shape and np.array_equal(a.view(np.uint16), b.view(np.uint16))
    return np.array_equal(a, b)


def T(a, dev):
    if a.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.uint16).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def H(t):
    t = t.detach().cpu()
    if t.dtype == torch.uint16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


# ---------------------------------------------------------------- oracle (CPU)

@pytest.mark.parametrize("name", ["pq_m16.npz", "pq_m8.npz"])
def test_oracle_pq_golden(name):
    z = load(name)
    c, r = nx.pq_encode(z["x"], z["codebooks"])
    assert same(c, z["codes"]) and same(r, z["residual"])


def test_oracle_ext_golden():
    z = load("ext_m16.npz")
    e = nx.ext_encode(z["x"], z["pq_codebooks"], z["rvq_codebooks"], 4)
    for k in ("pq_codes", "rvq_codes", "sparse_idx", "sparse_val"):
        assert same(e[k], z[k]), k
    d = nx.ext_decode(z["pq_codes"], z["pq_codebooks"], z["rvq_codes"], z["rvq_codebooks"], z["sparse_idx"],
                      z["sparse_val"])
    assert same(d, z["decoded"])


def test_oracle_rvq_ref_golden():
    z = load("rvq_ref.npz")
    pc, rc, mask, offs = nx.hybrid_encode(z["x"], z["pq_codebooks"], z["rvq_codebooks"], float(z["threshold"]))
    assert same(pc, z["pq_codes"]) and same(rc, z["rvq_codes"]) and same(mask, z["rvq_mask"])
    assert same(offs, z["rvq_offsets"])
    assert 0 < mask.sum() < mask.size  # the fixture exercises both gate outcomes
    assert same(nx.hybrid_decode(pc, rc, mask, offs, z["pq_codebooks"], z["rvq_codebooks"]), z["decoded"])


def test_oracle_attention_golden():
    z = load("attn.npz")
    out = nx.blockwise_attention(z["q"], z["keys"], z["values"], float(z["scale"]), 64, True, z["qpos"])
    assert same(out, z["out_causal"])
    assert not z["out_causal"][3].any()  # query position -1 sees nothing
    full = nx.blockwise_attention(z["q"], z["keys"], z["values"], float(z["scale"]), 64)
    assert same(full, z["out_full"])


# ---------------------------------------------------------------- HIP path (GPU)

@pytest.mark.gpu
@pytest.mark.parametrize("name", ["pq_m16.npz", "pq_m8.npz"])
def test_gpu_pq_golden(device, name):
    from apple_amd import kernels as K

    z = load(name)
    c, r = K.pq_encode(T(z["x"], device), T(z["codebooks"], device))
    assert same(H(c), z["codes"]) and same(H(r), z["residual"])


@pytest.mark.gpu
def test_gpu_ext_golden(device):
    from apple_amd import kernels as K

    z = load("ext_m16.npz")
    fmt = K.WarmFormat(64, 16, 256, 16, 256, 4)
    pq, rv = T(z["pq_codebooks"], device), T(z["rvq_codebooks"], device)
    out = K.warm_encode(T(z["x"], device), fmt, pq, rv)
    assert same(H(out["pq"]), z["pq_codes"]) and same(H(out["rvq"]), z["rvq_codes"])
    assert same(H(out["sparse_idx"]), z["sparse_idx"]) and same(H(out["sparse_val"]), z["sparse_val"])
    dec = K.decode(fmt, T(z["pq_codes"], device), pq, T(z["rvq_codes"], device), rv, T(z["sparse_idx"], device),
                   T(z["sparse_val"], device))
    assert same(H(dec), z["decoded"])


@pytest.mark.gpu
def test_gpu_rvq_ref_golden(device):
    from apple_amd import kernels as K

    z = load("rvq_ref.npz")
    c, r = K.pq_encode(T(z["x"], device), T(z["pq_codebooks"], device))
    assert same(H(c), z["pq_codes"]) and same(H(r), z["pq_residual"])
    codes, mask, offs = K.rvq_encode_full(r, T(z["rvq_codebooks"], device), float(z["threshold"]))
    assert same(H(codes), z["rvq_codes"]) and same(H(mask), z["rvq_mask"]) and same(H(offs), z["rvq_offsets"])
    dec = K.decode_ref(c, T(z["pq_codebooks"], device), codes, offs, T(z["rvq_codebooks"], device))
    assert same(H(dec), z["decoded"])


@pytest.mark.gpu
def test_gpu_attention_golden(device):
    from apple_amd import kernels as K

    z = load("attn.npz")
    args = (T(z["q"], device), T(z["keys"], device), T(z["values"], device), float(z["scale"]))
    out = H(K.blockwise_attention(*args, True, T(z["qpos"], device)))
    assert np.abs(out.astype(np.float32) - z["out_causal"].astype(np.float32)).max() <= TOL
    assert not out[3].any()
    full = H(K.blockwise_attention(*args, False, None))
    assert np.abs(full.astype(np.float32) - z["out_full"].astype(np.float32)).max() <= TOL
