"""Decoder layers over the MI355X cache: the caller one step up from the
decode path.

* ``RFSNDecoderLayerMLX`` -- the reference's layer
  (rfsn_v10_mlx_ane_complete.py:55-172): RMSNorm, q/k/v projections into the
  tiered cache, cache-backed single-token decode, o_proj and a GELU FFN.
* ``Llama32DecoderLayerMLX`` -- the Llama layer of llama32_adapter.py
  (375-662): RMSNorm with weights, rotary position embeddings on q and k,
  grouped KV heads and a SwiGLU MLP.  The cache stores the KV heads as they
  are (``num_kv_heads``); the reference repeats them to the query heads
  first (llama32_adapter.py:380-386, 578-579).

Norms, projections, activations and the dense prompt attention are torch
ops on the GPU, computed in fp32 from fp16 activations with fp16 results at
the reference's cast points.  Cache-backed decode goes through the cache's
fused dequant-attention kernel.  Weights are module parameters: the
reference's initialisation or a local state dict; nothing is downloaded.
"""

from __future__ import annotations

import itertools
import math
import shutil
from pathlib import Path
from typing import Dict, Optional, Tuple

import torch

from .cache import RFSNv10KVCacheMLX
from .quantization import HybridQuantizerMLX
from .storage import AsyncHierarchicalRouterMLX, RFSNConfig

MASK_FILL_VALUE = -1e30


def _gelu(x: torch.Tensor) -> torch.Tensor:
    """attention.py:137-138 (tanh form)."""
    return 0.5 * x * (1.0 + torch.tanh(0.7978845608 * (x + 0.044715 * (x ** 3))))


def _dense_exact_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, scale: float,
                           causal: bool = True) -> torch.Tensor:
    """attention.py:108-134: q [B, S, H, D], keys/values [B, T, H, D] ->
    [B, S, H, D] in q's dtype; fp32 scores, mask k_pos <= q_pos."""
    qf = q.float().permute(0, 2, 1, 3).contiguous()          # [B, H, S, D]
    kf = keys.float().permute(0, 2, 3, 1).contiguous()       # [B, H, D, T]
    vf = values.float().permute(0, 2, 1, 3).contiguous()     # [B, H, T, D]
    scores = torch.matmul(qf, kf) * scale
    if causal:
        qp = torch.arange(q.shape[1], device=q.device)
        kp = torch.arange(keys.shape[1], device=q.device)
        allowed = kp[None, :] <= qp[:, None]
        scores = torch.where(allowed[None, None], scores, torch.full_like(scores, MASK_FILL_VALUE))
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs, vf).permute(0, 2, 1, 3).to(q.dtype)


def _repeat_kv(x: torch.Tensor, repeats: int) -> torch.Tensor:
    """llama32_adapter.py:380-386: [B, T, Hkv, D] -> [B, T, Hkv * repeats, D]."""
    if repeats == 1:
        return x
    B, T, H, D = x.shape
    return x[:, :, :, None, :].expand(B, T, H, repeats, D).reshape(B, T, H * repeats, D)


def _linear_weight(out_features: int, in_features: int, generator, device) -> torch.nn.Parameter:
    """fp32 weights drawn U(-1/sqrt(in), 1/sqrt(in)), the initialisation of the reference's nn.Linear."""
    bound = 1.0 / math.sqrt(in_features)
    w = (torch.rand((out_features, in_features), generator=generator, dtype=torch.float32) * 2 - 1) * bound
    return torch.nn.Parameter(w.to(device), requires_grad=False)


def _project(x16: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """fp16 activations times fp32 weights in fp32, result fp16."""
    return (x16.float() @ weight.t()).to(torch.float16)


def _rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor], eps: float) -> torch.Tensor:
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    if weight is not None:
        y = y * weight.float()
    return y.to(torch.float16)


class RFSNDecoderLayerMLX(torch.nn.Module):
    """Decoder layer that owns its projections, quantizer and cache-backed
    decode path (rfsn_v10_mlx_ane_complete.py:55-172).  With
    ``config.num_kv_heads`` below ``num_heads`` the K/V projections produce
    only the KV heads and the cache serves the query heads grouped."""

    def __init__(self, config: RFSNConfig, layer_idx: int = 0, ffn_multiplier: int = 2, device=None,
                 generator: Optional[torch.Generator] = None, quantizer=None):
        super().__init__()
        if device is None:
            if not torch.cuda.is_available():
                raise RuntimeError("the RFSN MI355X decoder layer needs a ROCm GPU; none is visible")
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = torch.device(device)
        self.config = config
        self.layer_idx = layer_idx
        self.num_heads = config.num_heads
        self.num_kv_heads = config.kv_heads
        self.head_dim = config.head_dim
        self.model_dim = config.hidden_dim
        self.ffn_hidden_dim = max(config.hidden_dim * ffn_multiplier, config.hidden_dim)
        self.scale = config.head_dim ** -0.5
        self.eps = 1e-5
        g = generator if generator is not None else torch.Generator().manual_seed(1234 + layer_idx)
        D, H, Hkv = config.hidden_dim, config.num_heads, self.num_kv_heads
        self.attn_norm_weight = torch.nn.Parameter(torch.ones(D, device=self.device), requires_grad=False)
        self.ffn_norm_weight = torch.nn.Parameter(torch.ones(D, device=self.device), requires_grad=False)
        self.q_proj = _linear_weight(H * self.head_dim, D, g, self.device)
        self.k_proj = _linear_weight(Hkv * self.head_dim, D, g, self.device)
        self.v_proj = _linear_weight(Hkv * self.head_dim, D, g, self.device)
        self.o_proj = _linear_weight(D, H * self.head_dim, g, self.device)
        self.ffn_up = _linear_weight(self.ffn_hidden_dim, D, g, self.device)
        self.ffn_down = _linear_weight(D, self.ffn_hidden_dim, g, self.device)
        self.quantizer = quantizer if quantizer is not None else HybridQuantizerMLX(config, device=self.device)
        self.disk_cache_dir = Path(config.disk_cache_dir) / f"decoder_layer_{layer_idx}"
        self.cache = RFSNv10KVCacheMLX(config, layer_idx=layer_idx, device=self.device)

    @property
    def cache_tokens(self) -> int:
        return self.cache.total_tokens

    def reset_cache(self, remove_disk: bool = True) -> None:
        if remove_disk and self.disk_cache_dir.exists():
            shutil.rmtree(self.disk_cache_dir)
        self.cache = RFSNv10KVCacheMLX(self.config, layer_idx=self.layer_idx, device=self.device)

    def _heads(self, projected: torch.Tensor, heads: int) -> torch.Tensor:
        B, S, _ = projected.shape
        return projected.reshape(B, S, heads, self.head_dim).to(torch.float16)

    def _qkv(self, x16: torch.Tensor):
        a = _rms_norm(x16, self.attn_norm_weight, self.eps)
        return (self._heads(_project(a, self.q_proj), self.num_heads),
                self._heads(_project(a, self.k_proj), self.num_kv_heads),
                self._heads(_project(a, self.v_proj), self.num_kv_heads))

    def prefill_cache(self, x: torch.Tensor, reset: bool = True) -> None:
        """rfsn_v10_mlx_ane_complete.py:90-104: the prompt's K/V into the cache."""
        if x.dim() != 3 or int(x.shape[0]) != 1:
            raise ValueError("prefill_cache expects input shape [1, seq_len, hidden_dim]")
        if reset:
            self.reset_cache(remove_disk=True)
        _, keys, values = self._qkv(x.to(self.device, torch.float16))
        self.cache.update(keys[0], values[0], self.quantizer, disk_dir=self.disk_cache_dir)

    def forward(self, x: torch.Tensor, use_cache: bool = False,
                router: Optional[AsyncHierarchicalRouterMLX] = None,
                context_window: Optional[int] = None) -> torch.Tensor:
        """rfsn_v10_mlx_ane_complete.py:114-172."""
        if x.dim() != 3:
            raise ValueError("Decoder layer expects input shape [batch, seq_len, hidden_dim]")
        if int(x.shape[-1]) != self.model_dim:
            raise ValueError(f"Expected hidden_dim {self.model_dim}, got {int(x.shape[-1])}")
        residual = x.to(self.device, torch.float16)
        q, k, v = self._qkv(residual)
        if use_cache:
            if tuple(int(d) for d in x.shape[:2]) != (1, 1):
                raise ValueError("cache-backed decoding currently supports input shape [1, 1, hidden_dim]; "
                                 "use prefill_cache() for longer prompts")
            self.cache.update(k[0], v[0], self.quantizer, disk_dir=self.disk_cache_dir)
            pos = self.cache.total_tokens - 1
            window = context_window
            if window is None:
                window = max(self.config.block_size_seq, min(self.cache.total_tokens, self.config.warm_capacity))
            attended = self.cache.attention_forward(
                q[:, 0], causal=True, query_positions=torch.tensor([pos], dtype=torch.int32, device=self.device),
                router=router, current_position=pos, context_window=window,
            ).reshape(1, 1, self.num_heads, self.head_dim)
        else:
            rep = self.num_heads // self.num_kv_heads
            attended = _dense_exact_attention(q, _repeat_kv(k, rep), _repeat_kv(v, rep), self.scale, causal=True)
        B, S = attended.shape[:2]
        attn_out = _project(attended.reshape(B, S, self.num_heads * self.head_dim), self.o_proj)
        hidden = residual + attn_out
        f = _rms_norm(hidden, self.ffn_norm_weight, self.eps)
        ffn_out = (_gelu(f.float() @ self.ffn_up.t()) @ self.ffn_down.t()).to(torch.float16)  # fp32 until the end
        return hidden + ffn_out


# Rotary frequency scaling of the Llama 3.1 / 3.2 checkpoints (their
# config.json "rope_scaling"; Llama-3.2-1B: factor 32, low / high frequency
# factors 1 / 4, original context 8192).
LLAMA3_ROPE_SCALING = {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                       "original_max_position_embeddings": 8192}


def rope_inv_freq(head_dim: int, theta: float = 500000.0, rope_scaling: Optional[Dict] = None,
                  device=None) -> torch.Tensor:
    """Rotary inverse frequencies [head_dim / 2] (float64): theta^(-2i/D),
    then, for ``rope_scaling`` of type "llama3", Meta's published Llama 3.1
    frequency scaling: components whose wavelength 2*pi/f is shorter than
    original / high_freq_factor keep f, longer than original /
    low_freq_factor become f / factor, and those between interpolate
    linearly in original / wavelength between the two."""
    inv = theta ** (-torch.arange(0, head_dim, 2, dtype=torch.float64, device=device) / head_dim)
    if not rope_scaling:
        return inv
    kind = rope_scaling.get("rope_type", rope_scaling.get("type"))
    if kind != "llama3":
        raise ValueError(f"unsupported rope_scaling type {kind!r} (only 'llama3')")
    factor = float(rope_scaling["factor"])
    lo, hi = float(rope_scaling["low_freq_factor"]), float(rope_scaling["high_freq_factor"])
    orig = float(rope_scaling["original_max_position_embeddings"])
    ratio = orig * inv / (2 * math.pi)           # periods of each component within the original context
    smooth = ((ratio - lo) / (hi - lo)).clamp(0.0, 1.0)
    return inv / factor * (1.0 - smooth) + inv * smooth


def rope_cos_sin(positions: torch.Tensor, head_dim: int, theta: float = 500000.0,
                 rope_scaling: Optional[Dict] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Rotary tables [S, head_dim] (fp32): angle p * f_i (``rope_inv_freq``),
    the two halves repeated, as the rotary module the adapter calls returns
    them (llama32_adapter.py:528-553)."""
    inv = rope_inv_freq(head_dim, theta, rope_scaling, positions.device)
    ang = positions.to(torch.float64)[:, None] * inv[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().float(), ang.sin().float()


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    """llama32_adapter.py:375-377."""
    half = x.shape[-1] // 2
    return torch.cat([-x[..., half:], x[..., :half]], dim=-1)


class Llama32DecoderLayerMLX(torch.nn.Module):
    """The Llama decoder layer of llama32_adapter.py on the MI355X cache.

    ``weights`` (optional) maps ``input_layernorm``, ``post_attention_layernorm``,
    ``q_proj``, ``k_proj``, ``v_proj``, ``o_proj``, ``gate_proj``, ``up_proj``,
    ``down_proj`` to tensors of the Hugging Face layer's shapes (a local state
    dict); otherwise weights are drawn as an untrained layer's would be.

    Rotary tables come, in this order, from the call's ``position_embeddings``
    (cos, sin), from ``rotary_module`` (the reference's argument: called as
    ``module(hidden, position_ids)``, else ``module(position_ids)``), or from
    ``rope_cos_sin`` with ``rope_theta`` and ``rope_scaling`` (default: the
    Llama-3.2 checkpoints' llama3 scaling).  Without ``position_ids`` a call's
    positions continue after the cached tokens (the reference's adapter
    defaults to 0 .. seq_len-1 and leaves positions to its caller)."""

    WEIGHTS = ("input_layernorm", "post_attention_layernorm", "q_proj", "k_proj", "v_proj", "o_proj",
               "gate_proj", "up_proj", "down_proj")

    def __init__(self, config: RFSNConfig, intermediate_size: int, layer_idx: int = 0, rms_norm_eps: float = 1e-5,
                 rope_theta: float = 500000.0, weights: Optional[Dict[str, torch.Tensor]] = None, device=None,
                 generator: Optional[torch.Generator] = None, quantizer=None,
                 rope_scaling: Optional[Dict] = LLAMA3_ROPE_SCALING, rotary_module=None):
        super().__init__()
        if device is None:
            if not torch.cuda.is_available():
                raise RuntimeError("the RFSN MI355X decoder layer needs a ROCm GPU; none is visible")
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = torch.device(device)
        self.config = config
        self.layer_idx = layer_idx
        self.num_heads = config.num_heads
        self.num_kv_heads = config.kv_heads
        self.num_key_value_groups = self.num_heads // self.num_kv_heads
        self.head_dim = config.head_dim
        self.hidden_dim = config.hidden_dim
        self.scale = config.head_dim ** -0.5
        self.rms_norm_eps = rms_norm_eps
        self.rope_theta = rope_theta
        self.rope_scaling = dict(rope_scaling) if rope_scaling else None
        if self.rope_scaling:
            rope_inv_freq(config.head_dim, rope_theta, self.rope_scaling)  # rejects unsupported types now
        self.rotary_module = rotary_module
        D, H, Hkv, I = config.hidden_dim, config.num_heads, self.num_kv_heads, intermediate_size
        shapes = {"input_layernorm": (D,), "post_attention_layernorm": (D,), "q_proj": (H * self.head_dim, D),
                  "k_proj": (Hkv * self.head_dim, D), "v_proj": (Hkv * self.head_dim, D),
                  "o_proj": (D, H * self.head_dim), "gate_proj": (I, D), "up_proj": (I, D), "down_proj": (D, I)}
        g = generator if generator is not None else torch.Generator().manual_seed(4321 + layer_idx)
        for name in self.WEIGHTS:
            if weights is not None:
                w = torch.as_tensor(weights[name]).float()
                if tuple(w.shape) != shapes[name]:
                    raise ValueError(f"{name}: expected shape {shapes[name]}, got {tuple(w.shape)}")
                p = torch.nn.Parameter(w.to(self.device), requires_grad=False)
            elif len(shapes[name]) == 1:
                p = torch.nn.Parameter(torch.ones(shapes[name], device=self.device), requires_grad=False)
            else:
                p = _linear_weight(shapes[name][0], shapes[name][1], g, self.device)
            setattr(self, name, p)
        self.quantizer = quantizer if quantizer is not None else HybridQuantizerMLX(config, device=self.device)
        self.disk_cache_dir = Path(config.disk_cache_dir) / f"llama_layer_{layer_idx}"
        self.cache = RFSNv10KVCacheMLX(config, layer_idx=layer_idx, device=self.device)

    @property
    def cache_tokens(self) -> int:
        return self.cache.total_tokens

    def reset_cache(self, remove_disk: bool = True) -> None:
        if remove_disk and self.disk_cache_dir.exists():
            shutil.rmtree(self.disk_cache_dir)
        self.cache = RFSNv10KVCacheMLX(self.config, layer_idx=self.layer_idx, device=self.device)

    def _positions(self, seq_len: int, position_embeddings, position_ids) -> Tuple[torch.Tensor, torch.Tensor]:
        if position_embeddings is not None:
            cos, sin = (torch.as_tensor(t, device=self.device).float().reshape(-1, self.head_dim)[-seq_len:]
                        for t in position_embeddings)
            return cos, sin
        if position_ids is None:
            start = self.cache.total_tokens
            position_ids = torch.arange(start, start + seq_len, device=self.device)
        pid = torch.as_tensor(position_ids, device=self.device).reshape(-1)
        if self.rotary_module is not None:
            # llama32_adapter.py:535-553: HF rotary modules take (hidden, position_ids)
            # on the device of their own buffers or parameters
            first = next(itertools.chain(self.rotary_module.buffers(), self.rotary_module.parameters()), None)
            rdev = self.device if first is None else first.device
            ids = pid.reshape(1, -1).to(rdev)
            hidden = torch.zeros((1, seq_len, self.hidden_dim), dtype=torch.float32, device=rdev)
            try:
                cos, sin = self.rotary_module(hidden, ids)
            except TypeError:
                cos, sin = self.rotary_module(ids)
            return tuple(torch.as_tensor(t, device=self.device).float().reshape(-1, self.head_dim)[-seq_len:]
                         for t in (cos, sin))
        return rope_cos_sin(pid, self.head_dim, self.rope_theta, self.rope_scaling)

    def _project_qkv(self, h16: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
        """llama32_adapter.py:570-580 without the KV repeat (the cache groups heads)."""
        n = _rms_norm(h16, self.input_layernorm, self.rms_norm_eps)
        B, S, _ = h16.shape
        q = _project(n, self.q_proj).reshape(B, S, self.num_heads, self.head_dim)
        k = _project(n, self.k_proj).reshape(B, S, self.num_kv_heads, self.head_dim)
        v = _project(n, self.v_proj).reshape(B, S, self.num_kv_heads, self.head_dim)
        c, s = cos[None, :, None, :], sin[None, :, None, :]
        qf, kf = q.float(), k.float()
        q = (qf * c + _rotate_half(qf) * s).to(torch.float16)       # llama32_adapter.py:555-568
        k = (kf * c + _rotate_half(kf) * s).to(torch.float16)
        return q, k, v

    def _mlp(self, h16: torch.Tensor) -> torch.Tensor:
        """llama32_adapter.py:582-587."""
        m = _rms_norm(h16, self.post_attention_layernorm, self.rms_norm_eps)
        gate = _project(m, self.gate_proj).float()
        up = _project(m, self.up_proj)
        act = (gate * torch.sigmoid(gate)).to(torch.float16)
        return _project((act.float() * up.float()).to(torch.float16), self.down_proj)

    def prefill_cache(self, hidden_states: torch.Tensor, position_embeddings=None, position_ids=None,
                      reset: bool = True) -> None:
        """llama32_adapter.py:589-614."""
        if int(hidden_states.shape[0]) != 1:
            raise ValueError("prefill_cache currently supports batch size 1 only")
        if reset:
            self.reset_cache(remove_disk=True)
        S = int(hidden_states.shape[1])
        if S == 0:
            return
        cos, sin = self._positions(S, position_embeddings, position_ids)
        _, k, v = self._project_qkv(hidden_states.to(self.device, torch.float16), cos, sin)
        self.cache.update(k[0], v[0], self.quantizer, disk_dir=self.disk_cache_dir)

    def forward(self, hidden_states: torch.Tensor, position_embeddings=None, position_ids=None,
                use_cache: bool = False, router: Optional[AsyncHierarchicalRouterMLX] = None,
                context_window: Optional[int] = None) -> torch.Tensor:
        """llama32_adapter.py:616-662."""
        if int(hidden_states.shape[0]) != 1:
            raise ValueError("The Llama adapter currently supports batch size 1 only")
        S = int(hidden_states.shape[1])
        cos, sin = self._positions(S, position_embeddings, position_ids)
        residual = hidden_states.to(self.device, torch.float16)
        q, k, v = self._project_qkv(residual, cos, sin)
        if use_cache:
            if S != 1:
                raise ValueError("cache-backed decode expects input shape [1, 1, hidden_dim]")
            self.cache.update(k[0], v[0], self.quantizer, disk_dir=self.disk_cache_dir)
            pos = self.cache.total_tokens - 1
            attended = self.cache.attention_forward(
                q[:, 0], causal=True, query_positions=torch.tensor([pos], dtype=torch.int32, device=self.device),
                router=router, current_position=pos, context_window=context_window,
            ).reshape(1, 1, self.num_heads, self.head_dim)
        else:
            g = self.num_key_value_groups
            attended = _dense_exact_attention(q, _repeat_kv(k, g), _repeat_kv(v, g), self.scale, causal=True)
        attn = _project(attended.reshape(1, S, self.num_heads * self.head_dim), self.o_proj)
        hidden = residual + attn
        return hidden + self._mlp(hidden)
