"""The C-ABI library without a GPU: it loads, exports every function that
include/rfsn_abi.h declares, its structs have the layout the ctypes mirror
assumes, and host-side argument validation reports errors through the
status codes and rfsn_last_error (no kernel is launched)."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "rfsn_abi.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(rfsn_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from apple_amd import _lib

    return _lib.load()


def test_header_declares_the_entry_points():
    names = declared_functions()
    for must in ("rfsn_pq_encode", "rfsn_warm_encode", "rfsn_rvq_encode_full", "rfsn_decode",
                 "rfsn_blockwise_attention", "rfsn_fused_decode_attention", "rfsn_prefetch_h2d",
                 "rfsn_host_alloc", "rfsn_stream_wait_event", "rfsn_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", str(ROOT / "apple_amd" / "librfsn_hip.so")],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (rfsn_[a-z0-9_]+)$", out, flags=re.M))
    assert set(declared_functions()) <= exported


def test_ctypes_signatures_cover_the_header():
    from apple_amd import _lib

    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_struct_layout_matches_c(tmp_path):
    """sizeof / offsetof from gcc on the real header against the ctypes mirror."""
    from apple_amd import _lib

    src = tmp_path / "layout.c"
    fields = {
        "rfsn_format": ["head_dim", "pq_subspaces", "pq_centroids", "rvq_subspaces", "rvq_centroids", "sparse_k"],
        "rfsn_codes": ["pq", "rvq", "sparse_idx", "sparse_val"],
        "rfsn_segment": ["k", "v", "head_stride", "len", "pos0"],
        "rfsn_fused_params": [f for f, _ in _lib.FusedParams._fields_],
        "rfsn_copy": ["dst_dev", "src_host", "bytes"],
        "rfsn_ref_store_codes": [f for f, _ in _lib.RefStoreCodes._fields_],
        "rfsn_ref_segment": [f for f, _ in _lib.RefSegment._fields_],
        "rfsn_ref_params": [f for f, _ in _lib.RefParams._fields_],
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "rfsn_abi.h"', "int main(void) {"]
    for s, fs in fields.items():
        lines.append(f'printf("{s} %zu\\n", sizeof({s}));')
        for f in fs:
            lines.append(f'printf("{s}.{f} %zu\\n", offsetof({s}, {f}));')
    lines.append("return 0; }")
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                  check=True).stdout.splitlines())
    py = {"rfsn_format": _lib.Format, "rfsn_codes": _lib.Codes, "rfsn_segment": _lib.Segment,
          "rfsn_fused_params": _lib.FusedParams, "rfsn_copy": _lib.Copy, "rfsn_ref_store_codes": _lib.RefStoreCodes,
          "rfsn_ref_segment": _lib.RefSegment, "rfsn_ref_params": _lib.RefParams}
    for s, cls in py.items():
        assert int(got[s]) == ctypes.sizeof(cls), s
        for f in fields[s]:
            assert int(got[f"{s}.{f}"]) == getattr(cls, f).offset, (s, f)


def test_version_and_validation_errors(lib):
    from apple_amd import _lib

    assert lib.rfsn_abi_version() >= 1
    # null parameter block: rejected on the host, no kernel launched
    assert lib.rfsn_fused_decode_attention(None, None) == -1
    assert b"null" in lib.rfsn_last_error()
    p = _lib.FusedParams()
    p.fmt.head_dim = 128
    assert lib.rfsn_fused_decode_attention(ctypes.byref(p), None) == -1
    assert b"head_dim" in lib.rfsn_last_error()
    p.fmt.head_dim = 64
    p.fmt.pq_subspaces = 12
    assert lib.rfsn_fused_decode_attention(ctypes.byref(p), None) == -1
    assert lib.rfsn_fused_workspace_bytes(None) == 0
    with pytest.raises(ValueError):
        _lib.check(-1, "probe")


def test_noalloc_rejects_oversized_partials_on_the_host(lib):
    """The allocation-free entry point refuses a call whose split partials
    exceed its fixed scratch before touching the device (no launch, no
    symbol lookup), and reports the size it would have needed."""
    from apple_amd import _lib

    p = _lib.FusedParams()
    p.fmt = _lib.Format(64, 16, 256, 16, 256, 4)
    p.batch, p.q_heads, p.kv_heads = 64, 32, 8
    p.hot_len, p.max_tokens, p.max_segments, p.splits = 0, 1 << 20, 1, 100
    need = lib.rfsn_fused_workspace_bytes(ctypes.byref(p))
    assert need == 64 * 32 * 100 * 66 * 4 > (4 << 20)
    assert lib.rfsn_fused_decode_attention_noalloc(ctypes.byref(p), None) == -1
    msg = lib.rfsn_last_error()
    assert str(need).encode() in msg and b"scratch" in msg
    assert lib.rfsn_fused_decode_attention_noalloc(None, None) == -1


def test_fused_k_scoring_route(lib):
    """The K route a fused call takes, decided on the host: the codebook rows
    for k_layout 0, the score tables for k_layout 1, and with the drift guard
    on the guard's exact pass alone when the call runs several splits of
    fewer than 256 tiles (32 tokens each) per block."""
    from apple_amd import _lib

    def route(batch, hot, tokens, k_layout=1, guard=True, splits=0):
        p = _lib.FusedParams()
        p.fmt = _lib.Format(64, 16, 256, 16, 256, 4)
        p.batch, p.q_heads, p.kv_heads = batch, 32, 8
        p.hot_len, p.max_tokens, p.max_segments, p.splits = hot, tokens, 1, splits
        p.k_layout = k_layout
        if guard:
            p.guard = 256  # never dereferenced on the host
        return lib.rfsn_fused_k_scoring(ctypes.byref(p)), lib.rfsn_fused_splits(ctypes.byref(p))

    # one sequence, 8,192 tokens: 257 tiles over 17 splits, 16 tiles per block
    assert route(1, 512, 8192) == (2, 17)
    assert route(1, 512, 8192, guard=False) == (1, 17)
    assert route(1, 512, 8192, splits=1) == (1, 1)  # one split: the estimate covers the window
    assert route(1, 512, 8192, k_layout=0) == (0, 17)
    # 32,768 tokens: 1,025 tiles; batch 4 -> 8 splits of 129 tiles, batch 8 -> 4 of 257, batch 32 -> 1
    assert route(4, 1024, 32768) == (2, 8)
    assert route(8, 1024, 32768) == (1, 4)
    assert route(32, 1024, 32768) == (1, 1)
    assert lib.rfsn_fused_k_scoring(None) == -1


def test_ref_attention_validation(lib):
    """rfsn_ref_attention rejects shapes outside its kernels on the host."""
    from apple_amd import _lib

    assert lib.rfsn_ref_attention(None, None) == -1
    p = _lib.RefParams()
    p.head_dim, p.pq_subspaces, p.pq_centroids = 96, 8, 256
    assert lib.rfsn_ref_attention(ctypes.byref(p), None) == -1
    assert b"head_dim" in lib.rfsn_last_error()
    p.head_dim, p.pq_subspaces = 128, 2
    assert lib.rfsn_ref_attention(ctypes.byref(p), None) == -1
    assert b"num_subspaces" in lib.rfsn_last_error()
    p.pq_subspaces, p.batch, p.q_heads, p.kv_heads = 8, 1, 12, 1
    assert lib.rfsn_ref_attention(ctypes.byref(p), None) == -1
    assert b"at most 8" in lib.rfsn_last_error()
    p.q_heads, p.kv_heads = 4, 4
    p.q = p.out = p.k_pq_cb = p.v_pq_cb = 16
    p.head_dim, p.pq_centroids = 256, 256  # 2 x 128 KB of PQ tables (K and V differ)
    p.v_pq_cb = 32
    assert lib.rfsn_ref_attention(ctypes.byref(p), None) == -1
    assert b"LDS" in lib.rfsn_last_error()
    p.head_dim, p.total_tokens = 128, 0
    assert lib.rfsn_ref_attention(ctypes.byref(p), None) == -1
    assert b"empty window" in lib.rfsn_last_error()
    p.total_tokens, p.num_segments, p.segments = 4096, 1, 64
    assert lib.rfsn_ref_attention_workspace_bytes(ctypes.byref(p)) > 0  # 4 units: split
    assert lib.rfsn_ref_attention(ctypes.byref(p), None) == -1
    assert b"workspace" in lib.rfsn_last_error()


def test_ref_tables_shape_checks(lib):
    """rfsn_ref_tables_ok and score_tables' host checks: the gated reference
    format (or PQ only) with its tables and histograms in LDS and a window
    within the histogram blocks' token limit; anything else is refused before
    a launch (and rfsn_ref_attention_workspace_bytes reports 0)."""
    from apple_amd import _lib

    assert lib.rfsn_ref_tables_ok(None) == 0
    p = _lib.RefParams()
    p.head_dim, p.pq_subspaces, p.pq_centroids, p.rvq_layers, p.rvq_centroids = 128, 8, 256, 4, 4096
    p.batch, p.q_heads, p.kv_heads, p.total_tokens = 1, 32, 32, 32768
    assert lib.rfsn_ref_tables_ok(ctypes.byref(p)) == 1          # the reference default: 18,432 entries
    p.rvq_centroids = 8192                                        # 34,816 entries: no room in LDS
    assert lib.rfsn_ref_tables_ok(ctypes.byref(p)) == 0
    p.rvq_centroids, p.rvq_layers = 4096, 0                       # PQ only
    assert lib.rfsn_ref_tables_ok(ctypes.byref(p)) == 1
    p.rvq_layers, p.total_tokens = 4, 1 << 20                     # 256 blocks x 4,096 tokens per query head
    assert lib.rfsn_ref_tables_ok(ctypes.byref(p)) == 1
    p.total_tokens = (1 << 20) + 1
    assert lib.rfsn_ref_tables_ok(ctypes.byref(p)) == 0
    p.total_tokens, p.pq_subspaces = 1 << 19, 32                  # M = 32: 1,024 tokens per block
    assert lib.rfsn_ref_tables_ok(ctypes.byref(p)) == 0
    p.pq_subspaces, p.rvq_layers, p.rvq_subspaces, p.rvq_centroids = 8, 0, 8, 256   # long-context format
    assert lib.rfsn_ref_tables_ok(ctypes.byref(p)) == 0
    p.rvq_subspaces, p.rvq_layers, p.rvq_centroids, p.total_tokens = 0, 4, 4096, 32768
    p.q = p.out = p.k_pq_cb = p.v_pq_cb = p.k_rvq_cb = p.v_rvq_cb = 16
    p.num_segments, p.segments = 1, 64
    p.score_tables, p.table_tol = 1, 2e-3
    assert lib.rfsn_ref_attention_workspace_bytes(ctypes.byref(p)) > 0
    assert lib.rfsn_ref_attention(ctypes.byref(p), None) == -1
    assert b"table_stats" in lib.rfsn_last_error()
    p.table_stats, p.table_tol = 16, -1.0
    assert lib.rfsn_ref_attention(ctypes.byref(p), None) == -1
    assert b"table_tol" in lib.rfsn_last_error()
    p.table_tol, p.rvq_centroids = 2e-3, 8192
    assert lib.rfsn_ref_attention_workspace_bytes(ctypes.byref(p)) == 0
    assert lib.rfsn_ref_attention(ctypes.byref(p), None) == -1
    assert b"score tables need" in lib.rfsn_last_error()
    p.rvq_centroids, p.score_tables = 4096, 2
    assert lib.rfsn_ref_attention(ctypes.byref(p), None) == -1
    assert b"score_tables must be 0 or 1" in lib.rfsn_last_error()
