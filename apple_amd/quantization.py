"""PQ / RVQ quantizers and compressed-tensor helpers on MI355X -- the
counterpart of the reference's ``quantization.py``.

Names, signatures, shapes, dtypes and exceptions follow quantization.py:92-403;
arrays are torch tensors on a ROCm device and every encode/decode runs a HIP
kernel of ``librfsn_hip.so`` (no CPU path).

Codebook initialisation follows quantization.py:108-115 and 188-197
(N(0,1) * sqrt(2/dim), stored fp16, RVQ row 0 zeroed) with a seeded torch
generator.  The Apple ANE 6-bit codebook path (quantization.py:36-89,
159-175, 277-293) is not part of this build and raises NotImplementedError.

Long-context warm format (``config.ext_format``: ``rvq_subspaces > 0`` or
``sparse_topk > 0``; no reference symbol): the optional RVQ stage is a
product quantizer of the fp16 PQ residual with ``rvq_subspaces`` subspaces
and ``rvq_codebook_size`` centroids, applied to every vector, and
``config.sparse_topk`` coordinates of the remaining residual are kept.
``HybridQuantizerMLX.encode`` then returns ``(pq_codes, rvq_codes,
sparse_idx, sparse_val)`` (empty arrays for absent stages) and ``decode``
takes the same four arrays.
"""

from __future__ import annotations

import logging
from typing import Dict, Optional, Tuple

import torch

from . import kernels as K
from .storage import CompressedTensorMLX, RFSNConfig, _concat0, _index0

logger = logging.getLogger("RFSN_QUANT")


def _default_device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("the RFSN MI355X path needs a ROCm GPU; none is visible")
    return torch.device("cuda", torch.cuda.current_device())


def _random_codebooks(shape, dim: int, generator: Optional[torch.Generator], device) -> torch.Tensor:
    scale = (2.0 / dim) ** 0.5
    cb = torch.randn(shape, generator=generator, dtype=torch.float32) * scale
    return cb.to(torch.float16).to(device)


class ProductQuantizerMLX:
    """Product quantizer (quantization.py:99-175)."""

    def __init__(self, config: RFSNConfig, device=None, generator: Optional[torch.Generator] = None,
                 codebooks: Optional[torch.Tensor] = None):
        self.config = config
        self.num_subspaces = config.num_subspaces
        self.subspace_dim = config.subspace_dim
        self.codebook_size = 1 << config.pq_bits
        if self.codebook_size > 256:
            raise ValueError("pq_bits > 8 is not representable in uint8 codes")
        self.device = torch.device(device) if device is not None else _default_device()
        if codebooks is None:
            codebooks = _random_codebooks((self.num_subspaces, self.codebook_size, self.subspace_dim),
                                          self.subspace_dim, generator, self.device)
        self.codebooks = codebooks.to(device=self.device, dtype=torch.float16).contiguous()

    def _codebook(self, subspace: int, dtype=torch.float32) -> torch.Tensor:
        return self.codebooks[subspace].to(dtype)

    def quantize(self, vectors: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """(codes u8 [N, M], residuals [N, D] in the input dtype) (quantization.py:124-144)."""
        num_tokens, dim = vectors.shape
        expected_dim = self.num_subspaces * self.subspace_dim
        if dim != expected_dim:
            raise ValueError(f"Expected vectors with dim {expected_dim}, got {dim}")
        x = vectors.to(device=self.device, dtype=torch.float16)
        codes, resid = K.pq_encode(x, self.codebooks)
        return codes, resid

    def decode(self, codes: torch.Tensor) -> torch.Tensor:
        """fp16 [N, D] gather (quantization.py:146-157)."""
        fmt = K.WarmFormat(self.config.head_dim, self.num_subspaces, self.codebook_size)
        return K.decode(fmt, codes.to(self.device), self.codebooks)

    def quantize_codebooks_for_ane(self) -> Dict[str, int]:
        raise NotImplementedError("the Apple ANE codebook path is not part of the MI355X build")


class ResidualVQMLX:
    """Gated full-dimension residual VQ (quantization.py:178-293)."""

    def __init__(self, config: RFSNConfig, device=None, generator: Optional[torch.Generator] = None,
                 codebooks: Optional[torch.Tensor] = None):
        self.config = config
        self.num_layers = config.num_rvq_layers
        self.codebook_size = config.rvq_codebook_size
        self.head_dim = config.head_dim
        self.sparsity_threshold = config.rvq_sparsity_threshold
        self.device = torch.device(device) if device is not None else _default_device()
        if codebooks is None:
            codebooks = _random_codebooks((self.num_layers, self.codebook_size, self.head_dim), self.head_dim,
                                          generator, self.device)
            codebooks[:, 0] = 0  # quantization.py:196-197
        self.codebooks = codebooks.to(device=self.device, dtype=torch.float16).contiguous()

    def _codebook(self, layer_idx: int, dtype=torch.float32) -> torch.Tensor:
        return self.codebooks[layer_idx].to(dtype)

    def encode(self, residuals: torch.Tensor, base_codes: Optional[torch.Tensor] = None
               ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(codes u16 [A, L], mask bool [N], offsets int32 [A]) (quantization.py:206-252)."""
        del base_codes
        num_tokens, dim = residuals.shape
        if dim != self.head_dim:
            raise ValueError(f"Expected residual dim {self.head_dim}, got {dim}")
        r = residuals.to(device=self.device, dtype=torch.float16)
        return K.rvq_encode_full(r, self.codebooks, self.sparsity_threshold)

    def decode_correction(self, rvq_codes: torch.Tensor, rvq_mask: torch.Tensor,
                          rvq_offsets: torch.Tensor) -> torch.Tensor:
        """fp16 [N, D] correction, zero on inactive rows (quantization.py:254-275)."""
        n = int(rvq_mask.shape[0])
        a = int(rvq_codes.shape[0])
        zeros_pq = torch.zeros((n, 1), dtype=torch.uint8, device=self.device)
        zero_cb = torch.zeros((1, 1, self.head_dim), dtype=torch.float16, device=self.device)
        if a == 0:
            return torch.zeros((n, self.head_dim), dtype=torch.float16, device=self.device)
        # base = 0 (a one-entry zero codebook), so fp16(0 + corr) = corr exactly
        return K.decode_ref(zeros_pq, zero_cb, rvq_codes.to(self.device), rvq_offsets.to(self.device),
                            self.codebooks)

    def quantize_codebooks_for_ane(self) -> Dict[str, int]:
        raise NotImplementedError("the Apple ANE codebook path is not part of the MI355X build")


class SubspaceRVQ:
    """Subspace RVQ stage on the PQ residual (extension; see module docstring)."""

    def __init__(self, config: RFSNConfig, device=None, generator: Optional[torch.Generator] = None,
                 codebooks: Optional[torch.Tensor] = None):
        self.config = config
        self.num_subspaces = config.rvq_subspaces
        self.subspace_dim = config.head_dim // config.rvq_subspaces
        self.codebook_size = config.rvq_codebook_size
        if self.codebook_size > 256:
            raise ValueError("subspace RVQ codes are uint8: rvq_codebook_size must be <= 256")
        self.device = torch.device(device) if device is not None else _default_device()
        if codebooks is None:
            codebooks = _random_codebooks((self.num_subspaces, self.codebook_size, self.subspace_dim),
                                          self.subspace_dim, generator, self.device)
        self.codebooks = codebooks.to(device=self.device, dtype=torch.float16).contiguous()


class HybridQuantizerMLX:
    """PQ base plus RVQ refinement (quantization.py:296-327)."""

    def __init__(self, config: RFSNConfig, device=None, generator: Optional[torch.Generator] = None,
                 pq_codebooks: Optional[torch.Tensor] = None, rvq_codebooks: Optional[torch.Tensor] = None):
        self.config = config
        self.pq = ProductQuantizerMLX(config, device, generator, pq_codebooks)
        self.device = self.pq.device
        if config.ext_format:
            self.rvq = SubspaceRVQ(config, self.device, generator, rvq_codebooks) if config.subspace_rvq else None
        else:
            self.rvq = ResidualVQMLX(config, self.device, generator, rvq_codebooks)

    @property
    def subspace(self) -> bool:
        """True for the long-context warm format (subspace RVQ and/or sparse residual)."""
        return self.config.ext_format

    def warm_format(self) -> K.WarmFormat:
        """Format of the fused kernel; for the reference format, its PQ part."""
        c = self.config
        if not self.subspace:
            return K.WarmFormat(c.head_dim, c.num_subspaces, self.pq.codebook_size)
        has_rvq = self.rvq is not None
        return K.WarmFormat(c.head_dim, c.num_subspaces, self.pq.codebook_size, c.rvq_subspaces if has_rvq else 0,
                            self.rvq.codebook_size if has_rvq else 0, c.sparse_topk)

    @property
    def rvq_codebooks(self) -> Optional[torch.Tensor]:
        return None if self.rvq is None else self.rvq.codebooks

    def encode(self, vectors: torch.Tensor):
        """Reference mode: (pq, rvq u16 [A, L], mask, offsets) (quantization.py:305-308).
        Subspace mode: (pq, rvq u8 [N, M_r], sparse_idx u8 [N, k], sparse_val fp16 [N, k])."""
        if not self.subspace:
            pq_codes, residuals = self.pq.quantize(vectors)
            rvq_codes, rvq_mask, rvq_offsets = self.rvq.encode(residuals, pq_codes)
            return pq_codes, rvq_codes, rvq_mask, rvq_offsets
        num_tokens, dim = vectors.shape
        if dim != self.config.head_dim:
            raise ValueError(f"Expected vectors with dim {self.config.head_dim}, got {dim}")
        x = vectors.to(device=self.device, dtype=torch.float16)
        out = K.warm_encode(x, self.warm_format(), self.pq.codebooks, self.rvq_codebooks)
        empty_i = torch.zeros((num_tokens, 0), dtype=torch.uint8, device=self.device)
        empty_v = torch.zeros((num_tokens, 0), dtype=torch.float16, device=self.device)
        return (out["pq"], out.get("rvq", empty_i), out.get("sparse_idx", empty_i),
                out.get("sparse_val", empty_v))

    def decode(self, pq_codes: torch.Tensor, rvq_codes: torch.Tensor, third: torch.Tensor,
               fourth: torch.Tensor) -> torch.Tensor:
        """fp16(base + correction) (quantization.py:310-319)."""
        if not self.subspace:
            return K.decode_ref(pq_codes.to(self.device), self.pq.codebooks, rvq_codes.to(self.device),
                                fourth.to(self.device), self.rvq.codebooks)
        fmt = self.warm_format()
        k = fmt.sparse_k
        return K.decode(fmt, pq_codes.to(self.device), self.pq.codebooks,
                        rvq_codes.to(self.device) if fmt.rvq_subspaces else None, self.rvq_codebooks,
                        third.to(self.device) if k else None, fourth.to(self.device) if k else None)

    def quantize_codebooks_for_ane(self) -> Dict[str, int]:
        raise NotImplementedError("the Apple ANE codebook path is not part of the MI355X build")


def _compress_tensor_sequence(tensor: torch.Tensor, quantizer: HybridQuantizerMLX) -> CompressedTensorMLX:
    """[T, H, D] -> CompressedTensorMLX, token-major / head-minor (quantization.py:330-343)."""
    num_tokens, num_heads, head_dim = tensor.shape
    flat = tensor.reshape(num_tokens * num_heads, head_dim)
    if not quantizer.subspace:
        pq_codes, rvq_codes, rvq_mask, rvq_offsets = quantizer.encode(flat)
        return CompressedTensorMLX(
            pq_codes=pq_codes.reshape(num_tokens, num_heads, quantizer.config.num_subspaces),
            rvq_codes=rvq_codes,
            rvq_mask=rvq_mask.reshape(num_tokens, num_heads),
            rvq_offsets=rvq_offsets.to(torch.int32),
            num_heads=num_heads,
        )
    pq, rvq, sidx, sval = quantizer.encode(flat)
    dev = quantizer.device
    return CompressedTensorMLX(
        pq_codes=pq.reshape(num_tokens, num_heads, -1),
        rvq_codes=rvq.reshape(num_tokens, num_heads, -1),
        rvq_mask=torch.ones((num_tokens, num_heads), dtype=torch.bool, device=dev),
        rvq_offsets=torch.zeros((0,), dtype=torch.int32, device=dev),
        num_heads=num_heads,
        sparse_idx=sidx.reshape(num_tokens, num_heads, -1),
        sparse_val=sval.reshape(num_tokens, num_heads, -1),
    )


def _encode_pair_head_major(keys: torch.Tensor, values: torch.Tensor, kq: HybridQuantizerMLX,
                            vq: HybridQuantizerMLX):
    """K and V [T, H, D] of one subspace format in one ``warm_encode_batch``
    launch, with head-major codes: per tensor (pq, rvq, sparse_idx,
    sparse_val), each [H, T, *] (None for a stage the format lacks).  The
    codes are those of ``_compress_tensor_sequence`` (each vector is encoded
    on its own), laid out for the tiled store.  None when that launch does
    not serve the pair (the reference format, two formats, or one the
    one-launch encode does not cover)."""
    if not (kq.subspace and vq.subspace):
        return None
    fmt = kq.warm_format()
    if fmt != vq.warm_format() or not K.batch_encode_ok(fmt):
        return None
    T, H, D = keys.shape
    if T == 0:
        return None
    hm = [(t if t.dtype is torch.float16 and t.device == kq.device else t.to(device=kq.device, dtype=torch.float16))
          .permute(1, 0, 2).contiguous().view(H * T, D) for t in (keys, values)]
    outs = K.warm_encode_batch([(hm[0], kq.pq.codebooks, kq.rvq_codebooks),
                                (hm[1], vq.pq.codebooks, vq.rvq_codebooks)], fmt)
    shape = lambda t: None if t is None else t.view(H, T, -1)
    return [tuple(shape(o.get(f)) for f in ("pq", "rvq", "sparse_idx", "sparse_val")) for o in outs]


def _head_major_store(codes, contiguous: bool = False) -> CompressedTensorMLX:
    """A token-major CompressedTensorMLX of head-major subspace codes (pq,
    rvq, sparse_idx, sparse_val) [H, T, *]: views, or copies with
    ``contiguous``."""
    pq, rvq, sidx, sval = codes
    H, T, _ = pq.shape
    dev = pq.device
    pm = (lambda t: t.permute(1, 0, 2).contiguous()) if contiguous else (lambda t: t.permute(1, 0, 2))
    tm = lambda t, dt: pm(t) if t is not None else torch.zeros((T, H, 0), dtype=dt, device=dev)
    return CompressedTensorMLX(pq_codes=pm(pq), rvq_codes=tm(rvq, torch.uint8),
                               rvq_mask=torch.ones((T, H), dtype=torch.bool, device=dev),
                               rvq_offsets=torch.zeros((0,), dtype=torch.int32, device=dev), num_heads=H,
                               sparse_idx=tm(sidx, torch.uint8), sparse_val=tm(sval, torch.float16))


def _append_compressed_tensor(base: CompressedTensorMLX, addition: CompressedTensorMLX) -> CompressedTensorMLX:
    """quantization.py:346-361."""
    if base.num_heads != addition.num_heads:
        raise ValueError("Compressed tensors must have the same number of heads")
    if base.subspace:
        return CompressedTensorMLX(
            pq_codes=_concat0(base.pq_codes, addition.pq_codes),
            rvq_codes=_concat0(base.rvq_codes, addition.rvq_codes),
            rvq_mask=_concat0(base.rvq_mask, addition.rvq_mask),
            rvq_offsets=base.rvq_offsets,
            num_heads=base.num_heads,
            sparse_idx=_concat0(base.sparse_idx, addition.sparse_idx),
            sparse_val=_concat0(base.sparse_val, addition.sparse_val),
        )
    offset_shift = base.num_tokens * base.num_heads
    shifted = addition.rvq_offsets + offset_shift if addition.rvq_offsets.shape[0] else addition.rvq_offsets
    return CompressedTensorMLX(
        pq_codes=_concat0(base.pq_codes, addition.pq_codes),
        rvq_codes=_concat0(base.rvq_codes, addition.rvq_codes),
        rvq_mask=_concat0(base.rvq_mask, addition.rvq_mask),
        rvq_offsets=_concat0(base.rvq_offsets, shifted.to(torch.int32)),
        num_heads=base.num_heads,
    )


def _slice_compressed_tensor(tensor: CompressedTensorMLX, start: int, end: int) -> CompressedTensorMLX:
    """Token-range slice with re-based offsets (quantization.py:364-391)."""
    if start < 0 or end < start or end > tensor.num_tokens:
        raise ValueError("Invalid slice for compressed tensor")
    if tensor.subspace:
        return CompressedTensorMLX(
            pq_codes=tensor.pq_codes[start:end], rvq_codes=tensor.rvq_codes[start:end],
            rvq_mask=tensor.rvq_mask[start:end], rvq_offsets=tensor.rvq_offsets, num_heads=tensor.num_heads,
            sparse_idx=tensor.sparse_idx[start:end], sparse_val=tensor.sparse_val[start:end])
    flat_start = start * tensor.num_heads
    flat_end = end * tensor.num_heads
    offs = tensor.rvq_offsets
    select = (offs >= flat_start) & (offs < flat_end)
    rvq_codes = _index0(tensor.rvq_codes, select)
    rvq_offsets = (offs[select] - flat_start).to(torch.int32)
    return CompressedTensorMLX(
        pq_codes=tensor.pq_codes[start:end],
        rvq_codes=rvq_codes,
        rvq_mask=tensor.rvq_mask[start:end],
        rvq_offsets=rvq_offsets,
        num_heads=tensor.num_heads,
    )


def _decode_compressed_tensor(tensor: CompressedTensorMLX, quantizer: HybridQuantizerMLX) -> torch.Tensor:
    """-> fp16 [T, H, D] (quantization.py:394-403)."""
    D = quantizer.config.head_dim
    if tensor.num_tokens == 0:
        return torch.zeros((0, tensor.num_heads, D), dtype=torch.float16, device=quantizer.device)
    n = tensor.num_tokens * tensor.num_heads
    flat_codes = tensor.pq_codes.reshape(n, -1)
    if tensor.subspace:
        decoded = quantizer.decode(flat_codes, tensor.rvq_codes.reshape(n, -1), tensor.sparse_idx.reshape(n, -1),
                                   tensor.sparse_val.reshape(n, -1))
    else:
        flat_mask = tensor.rvq_mask.reshape(n)
        decoded = quantizer.decode(flat_codes, tensor.rvq_codes, flat_mask, tensor.rvq_offsets)
    return decoded.reshape(tensor.num_tokens, tensor.num_heads, D)
