"""MI355X-native warm-tier quantized-KV decode path of RFSN (dawsonblock/apple).

Drop-in counterparts of the reference's Python API (``storage.py``,
``quantization.py``, ``attention.py``, ``cache.py`` and
``calibrate_quantizer``) running on hand-written gfx950 HIP kernels through
the C ABI of ``librfsn_hip.so`` (``include/rfsn_abi.h``).
"""

from .storage import (  # noqa: F401
    MASK_FILL_VALUE,
    AsyncHierarchicalRouterMLX,
    CompressedTensorMLX,
    RFSNConfig,
    chunk_file_path,
    compressed_tensor_from_loaded,
    load_compressed_chunk,
    save_compressed_chunk,
)

__all__ = [
    "MASK_FILL_VALUE", "AsyncHierarchicalRouterMLX", "CompressedTensorMLX", "RFSNConfig", "chunk_file_path",
    "compressed_tensor_from_loaded", "load_compressed_chunk", "save_compressed_chunk",
]


def __getattr__(name):
    # GPU-backed modules load lazily so that host-only code (config, NPZ I/O)
    # imports without the HIP library.
    import importlib

    mods = ("quantization", "attention", "cache", "batched", "calibrate", "kernels", "workloads")
    if name in mods or name.startswith("_"):
        return importlib.import_module(f".{name}", __name__)
    for mod in mods:
        m = importlib.import_module(f".{mod}", __name__)
        if hasattr(m, name):
            return getattr(m, name)
    raise AttributeError(name)
