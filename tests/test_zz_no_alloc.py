"""The allocation-free fused entry point against the workspace one, through
the C ABI: the same parameter block (split partials in the library's own
device scratch instead of a caller workspace) gives bit-identical outputs on
two calls in a row, the second over a smaller window with fewer splits, and
a call whose partials exceed the scratch is refused without launching."""

import ctypes

import numpy as np
import pytest
import torch

from tests.conftest import randn16
from tests.test_gpu_fused import T, _setup

pytestmark = pytest.mark.gpu


def _prepared(device, seed, Hq, Hkv, nw, nh, B, splits):
    from apple_amd.cache import RFSNv10KVCacheMLX

    g, cfg, keys, values, cbs, kq, vq = _setup(seed, Hq, Hkv, 16, 16, 4, nw, nh)
    cache = RFSNv10KVCacheMLX(cfg, device=device)
    cache.update(T(keys, device), T(values, device), (kq, vq))
    q = T(randn16(g, B, Hq, 64), device)
    out = torch.empty_like(q)
    fl = cache.prepare(q, causal=True, splits=splits, out=out)
    return cache, q, fl


def _noalloc(fl, out):
    from apple_amd import _lib as L

    p = L.FusedParams.from_buffer_copy(fl.params)
    p.out = out.data_ptr()
    p.workspace, p.workspace_bytes = None, 0  # ignored by the entry point
    lib = L.load()
    st = lib.rfsn_fused_decode_attention_noalloc(ctypes.byref(p), fl.stream)
    L.check(st, "rfsn_fused_decode_attention_noalloc")


def test_noalloc_matches_workspace_entry_point(device):
    from apple_amd import _lib as L

    lib = L.load()
    # first call: 2 queries x 32 heads over 4,096 tokens in 24 splits (405 KB
    # of partials); second: 1 query x 8 heads over 1,000 tokens in 6 splits
    for seed, Hq, Hkv, nw, nh, B, splits in ((31, 32, 8, 4000, 96, 2, 24), (32, 8, 8, 960, 40, 1, 6)):
        print(f"noalloc case seed={seed} Hq={Hq} Hkv={Hkv} tokens={nw + nh} B={B} splits={splits}", flush=True)
        cache, q, fl = _prepared(device, seed, Hq, Hkv, nw, nh, B, splits)
        assert lib.rfsn_fused_splits(ctypes.byref(fl.params)) == splits
        assert lib.rfsn_fused_workspace_bytes(ctypes.byref(fl.params)) == B * Hq * splits * 66 * 4
        ref = fl().clone()
        got = torch.full_like(ref, float("nan"))
        _noalloc(fl, got)
        torch.cuda.synchronize()
        assert np.array_equal(ref.cpu().numpy().view(np.uint16), got.cpu().numpy().view(np.uint16))
        # the workspace entry point is unchanged by the scratch's use
        again = fl().clone()
        torch.cuda.synchronize()
        assert torch.equal(again, ref)


def test_noalloc_refuses_oversized_partials(device):
    from apple_amd import _lib as L

    cache, q, fl = _prepared(device, 33, 32, 8, 2000, 64, 4, 150)
    need = L.load().rfsn_fused_workspace_bytes(ctypes.byref(fl.params))
    assert need > (4 << 20)
    out = torch.zeros_like(q)
    with pytest.raises(ValueError, match="scratch"):
        _noalloc(fl, out)
    torch.cuda.synchronize()
    assert not out.any()  # nothing launched
