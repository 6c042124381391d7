"""ctypes binding of ``librfsn_hip.so`` (the C ABI in ``include/rfsn_abi.h``).

The library is loaded after ``torch`` so that both share torch's HIP runtime
(same SONAME, ``libamdhip64.so.7``).  Every call is checked: a nonzero status
raises ``ValueError`` (contract violations, as the reference raises) or
``RuntimeError`` (HIP failures, unsupported shapes).  There is no fallback:
if the library is missing, importing the product path raises.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path
from typing import Optional

import torch  # noqa: F401  (loads the HIP runtime first)

LIB_PATH = Path(__file__).resolve().parent / "librfsn_hip.so"

RFSN_OK = 0
RFSN_ERR_INVALID = -1
RFSN_ERR_STATE = -2
RFSN_ERR_HIP = -3
RFSN_ERR_UNSUPPORTED = -4

vp = C.c_void_p
i32 = C.c_int32
i64 = C.c_int64
f32 = C.c_float
sz = C.c_size_t


class Format(C.Structure):
    _fields_ = [("head_dim", i32), ("pq_subspaces", i32), ("pq_centroids", i32),
                ("rvq_subspaces", i32), ("rvq_centroids", i32), ("sparse_k", i32)]


class Codes(C.Structure):
    _fields_ = [("pq", vp), ("rvq", vp), ("sparse_idx", vp), ("sparse_val", vp)]


class Segment(C.Structure):
    _fields_ = [("k", Codes), ("v", Codes), ("head_stride", i64), ("len", i32), ("pos0", i32)]


class FusedParams(C.Structure):
    _fields_ = [("fmt", Format), ("batch", i32), ("q_heads", i32), ("kv_heads", i32),
                ("q", vp), ("out", vp), ("scale", f32), ("causal", i32), ("qpos", vp),
                ("hot_k", vp), ("hot_v", vp), ("hot_cap", i64), ("hot_seq_stride", i64),
                ("hot_len", i32), ("hot_pos0", i32),
                ("segments", vp), ("num_segments", vp), ("max_segments", i32),
                ("k_pq_cb", vp), ("k_rvq_cb", vp), ("v_pq_cb", vp), ("v_rvq_cb", vp),
                ("pq_cb_stride", i64), ("rvq_cb_stride", i64),
                ("max_tokens", i32), ("splits", i32), ("workspace", vp), ("workspace_bytes", sz),
                ("part_base", i32), ("part_slots", i32), ("merge", i32), ("k_layout", i32),
                ("guard", vp), ("drift", vp), ("guard_tol", f32),
                ("tile_map", vp), ("tile_map_count", vp), ("tile_map_stride", i64),
                ("k_tab", vp), ("v_tab", vp), ("tab_stride", i64),
                ("app_k", vp), ("app_v", vp), ("app_ld", i64), ("app_vabs", vp), ("app_count", i32)]


class RefStoreCodes(C.Structure):
    _fields_ = [("pq", vp), ("rvq", vp), ("active", vp), ("rvq_sub", vp), ("sparse_idx", vp), ("sparse_val", vp)]


class RefSegment(C.Structure):
    _fields_ = [("k", RefStoreCodes), ("v", RefStoreCodes), ("exact_k", vp), ("exact_v", vp),
                ("exact_token_stride", i64), ("exact_head_stride", i64), ("token0", i64), ("len", i32),
                ("pos0", i32), ("code_token_stride", i64), ("code_head_stride", i64)]


class RefParams(C.Structure):
    _fields_ = [("head_dim", i32), ("pq_subspaces", i32), ("pq_centroids", i32), ("rvq_layers", i32),
                ("rvq_centroids", i32), ("rvq_subspaces", i32), ("sparse_k", i32), ("batch", i32), ("q_heads", i32), ("kv_heads", i32),
                ("q", vp), ("out", vp), ("scale", f32), ("causal", i32), ("qpos", vp),
                ("segments", vp), ("num_segments", i32), ("total_tokens", i32),
                ("k_pq_cb", vp), ("v_pq_cb", vp), ("k_rvq_cb", vp), ("v_rvq_cb", vp),
                ("splits", i32), ("workspace", vp), ("workspace_bytes", sz),
                ("score_tables", i32), ("table_tol", f32), ("table_stats", vp), ("drift", vp)]


class EncodeJob(C.Structure):
    _fields_ = [("x", vp), ("n", i64), ("ldx", i64), ("pq_cb", vp), ("rvq_cb", vp), ("out", Codes)]


class Copy(C.Structure):
    _fields_ = [("dst_dev", vp), ("src_host", vp), ("bytes", sz)]


# name -> (restype, argtypes); every symbol declared in include/rfsn_abi.h
SIGNATURES = {
    "rfsn_abi_version": (i32, []),
    "rfsn_last_error": (C.c_char_p, []),
    "rfsn_pq_encode": (i32, [vp, i64, i32, i64, i64, vp, i32, i32, i64, vp, i64, i64, vp, i64, i64, i32, vp]),
    "rfsn_warm_encode_workspace_bytes": (sz, [C.POINTER(Format), i64]),
    "rfsn_warm_encode": (i32, [C.POINTER(Format), vp, i64, i64, vp, vp, Codes, vp, sz, vp]),
    "rfsn_warm_encode_batch": (i32, [C.POINTER(Format), C.POINTER(EncodeJob), i32, vp]),
    "rfsn_hot_append": (i32, [vp, vp, i64, i32, i32, i32, vp, vp, i64, i64, vp, vp]),
    "rfsn_ref_attention_workspace_bytes": (sz, [C.POINTER(RefParams)]),
    "rfsn_ref_attention": (i32, [C.POINTER(RefParams), vp]),
    "rfsn_ref_tables_ok": (i32, [C.POINTER(RefParams)]),
    "rfsn_ref_table_stats": (i32, [C.POINTER(RefParams), vp, vp]),
    "rfsn_read_stream": (i32, [vp, i64, vp, i32, vp]),
    "rfsn_rvq_gate": (i32, [vp, i64, i32, i64, f32, vp, vp]),
    "rfsn_mask_compact_workspace_bytes": (sz, [i64]),
    "rfsn_mask_compact": (i32, [vp, i64, vp, vp, vp, sz, vp]),
    "rfsn_rvq_encode_full_workspace_bytes": (sz, [i64, i32, i32, i32]),
    "rfsn_rvq_encode_full": (i32, [vp, i64, i32, vp, i64, vp, i32, i32, vp, vp, sz, vp]),
    "rfsn_decode": (i32, [C.POINTER(Format), C.POINTER(Codes), i64, vp, vp, vp, i64, i32, vp]),
    "rfsn_sparse_fold": (i32, [C.POINTER(Format), C.POINTER(Codes), i64, vp, vp, vp, vp]),
    "rfsn_sparse_delta": (i32, [C.POINTER(Format), C.POINTER(Codes), i64, vp, vp, vp, vp]),
    "rfsn_decode_ref": (i32, [vp, i64, i32, i32, i32, vp, vp, vp, i64, i32, i32, vp, vp, vp]),
    "rfsn_attention_workspace_bytes": (sz, [i32, i32, i32, i32]),
    "rfsn_blockwise_attention": (i32, [vp, i32, i32, i32, vp, vp, i64, i32, i64, i64, f32, i32, vp, vp, vp, sz, vp]),
    "rfsn_pack_codes": (i32, [vp, i64, i64, i32, i32, vp, i64, i64, vp]),
    "rfsn_pack_score_codes": (i32, [vp, vp, vp, vp, i32, i64, i32, vp, vp, vp, vp, i64, i64, vp]),
    "rfsn_warm_append_pair": (i32, [C.POINTER(Format), C.POINTER(Codes), C.POINTER(Codes), i64, i32, vp, vp, vp,
                                    vp, C.POINTER(Codes), i32, vp, C.POINTER(Codes), i64, i64, C.POINTER(Codes),
                                    vp, C.POINTER(Codes), vp, i64, vp]),
    "rfsn_fused_splits": (i32, [C.POINTER(FusedParams)]),
    "rfsn_fused_k_scoring": (i32, [C.POINTER(FusedParams)]),
    "rfsn_fused_workspace_bytes": (sz, [C.POINTER(FusedParams)]),
    "rfsn_fused_decode_attention": (i32, [C.POINTER(FusedParams), vp]),
    "rfsn_fused_decode_attention_noalloc": (i32, [C.POINTER(FusedParams), vp]),
    "rfsn_kmeans_workspace_bytes": (sz, [i32, i32, i32]),
    "rfsn_kmeans_update": (i32, [vp, i64, i32, i64, vp, i32, i32, vp, vp, sz, vp]),
    "rfsn_host_alloc": (i32, [sz, C.POINTER(vp)]),
    "rfsn_host_free": (i32, [vp]),
    "rfsn_prefetch_h2d": (i32, [C.POINTER(Copy), i32, vp]),
    "rfsn_stream_create": (i32, [C.POINTER(vp)]),
    "rfsn_stream_destroy": (i32, [vp]),
    "rfsn_event_create": (i32, [C.POINTER(vp)]),
    "rfsn_event_destroy": (i32, [vp]),
    "rfsn_event_record": (i32, [vp, vp]),
    "rfsn_stream_wait_event": (i32, [vp, vp]),
    "rfsn_event_synchronize": (i32, [vp]),
    "rfsn_event_query": (i32, [vp]),
    "rfsn_stream_query": (i32, [vp]),
}

_lib: Optional[C.CDLL] = None


def load(path: Optional[os.PathLike] = None) -> C.CDLL:
    """Load the library (once) and bind every ABI symbol."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"RFSN HIP library not built: {p} is missing (run `python -m apple_amd.build`)")
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.rfsn_abi_version() != 8:
        raise RuntimeError("librfsn_hip.so ABI version mismatch")
    if path is None:
        _lib = lib
    return lib


def check(status: int, what: str = "") -> None:
    if status == RFSN_OK:
        return
    msg = (load().rfsn_last_error() or b"").decode(errors="replace")
    text = f"{what}: {msg}" if what else msg
    if status == RFSN_ERR_INVALID:
        raise ValueError(text)
    raise RuntimeError(text)


def call(name: str, *args) -> int:
    fn = getattr(load(), name)
    st = fn(*args)
    check(st, name)
    return st


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_handle(device: Optional[torch.device] = None) -> int:
    """The current torch stream of ``device`` as a hipStream_t."""
    if isinstance(device, torch.device) and device.index is not None:
        return torch._C._cuda_getCurrentRawStream(device.index)  # no Stream object built
    return torch.cuda.current_stream(device).cuda_stream


def require_device(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{what}: the RFSN path runs on the GPU only (got a CPU tensor); "
                           "move inputs to a ROCm device")
