"""Decoder layers over the MI355X cache (rfsn_v10_mlx_ane_complete.py:55-172,
llama32_adapter.py:375-662): the reference suite's layer test, and each
layer's cache-backed decode step against a float64 restatement of the layer
around the oracle's blockwise attention over the window the cache holds."""

import numpy as np
import pytest
import torch

from oracle import numerics as nx
from tests.conftest import randn16, rng

pytestmark = pytest.mark.gpu


def H(t):
    return t.detach().float().cpu().numpy()


def f16(a):
    return np.asarray(a, dtype=np.float64).astype(np.float16)


def _rms(x, w, eps):
    x = x.astype(np.float64)
    return f16(x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w)


def _gelu(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))


def test_decoder_layer_api(device, tmp_path):
    """rfsn_v10_mlx_ane_complete.py:556-574 (the reference suite's config)."""
    from apple_amd.layer import RFSNDecoderLayerMLX
    from apple_amd.storage import RFSNConfig

    cfg = RFSNConfig(hidden_dim=512, num_heads=4, head_dim=128, num_layers=2, num_subspaces=8, subspace_dim=16,
                     num_rvq_layers=3, rvq_codebook_size=256, rvq_sparsity_threshold=0.25, hot_capacity=16,
                     warm_capacity=24, cold_capacity=128, block_size_seq=16, disk_cache_dir=str(tmp_path),
                     prefetch_throttle_s=0.0)
    layer = RFSNDecoderLayerMLX(cfg, layer_idx=0, device=device)
    g = rng(31)
    out = layer(torch.from_numpy(randn16(g, 2, 6, 512)).to(device), use_cache=False)
    assert out.shape == (2, 6, 512) and out.dtype == torch.float16
    layer.prefill_cache(torch.from_numpy(randn16(g, 1, 4, 512)).to(device))
    assert layer.cache_tokens == 4
    dec = layer(torch.from_numpy(randn16(g, 1, 1, 512)).to(device), use_cache=True, context_window=8)
    assert dec.shape == (1, 1, 512) and layer.cache_tokens == 5
    layer.reset_cache(remove_disk=True)
    assert layer.cache_tokens == 0
    with pytest.raises(ValueError):
        layer(torch.zeros((1, 2, 512), dtype=torch.float16, device=device), use_cache=True)


def _ext_config(tmp_path, **kw):
    from apple_amd.storage import RFSNConfig

    base = dict(hidden_dim=512, num_heads=8, head_dim=64, num_subspaces=16, subspace_dim=4, num_rvq_layers=1,
                rvq_codebook_size=256, rvq_sparsity_threshold=0.0, hot_capacity=64, warm_capacity=256,
                block_size_seq=64, num_kv_heads=4, rvq_subspaces=16, sparse_topk=4, tier_policy="recency",
                cold_medium="pinned", cold_chunk_tokens=64, disk_cache_dir=str(tmp_path))
    base.update(kw)
    return RFSNConfig(**base)


def _ext_quantizer(cfg, device, seed):
    from apple_amd.quantization import HybridQuantizerMLX
    from tests.conftest import rand_codebooks

    g = rng(seed)
    return HybridQuantizerMLX(cfg, device=device, pq_codebooks=torch.from_numpy(rand_codebooks(g, 16, 256, 4)),
                              rvq_codebooks=torch.from_numpy(rand_codebooks(g, 16, 256, 4) * np.float16(0.35)))


def test_rfsn_layer_decode_matches_restatement(device, tmp_path):
    """Prompt prefill, then three cache-backed decode steps of the reference
    layer on the long-context format (grouped KV heads, pinned cold chunks):
    each step equals RMSNorm -> o_proj(attention over the cache's window) ->
    residual -> GELU FFN restated in float64, the attention by the oracle
    over the window the cache materializes, within 2e-2."""
    from apple_amd.layer import RFSNDecoderLayerMLX

    cfg = _ext_config(tmp_path)
    layer = RFSNDecoderLayerMLX(cfg, device=device, quantizer=_ext_quantizer(cfg, device, 7))
    g = rng(32)
    layer.prefill_cache(torch.from_numpy(randn16(g, 1, 500, 512)).to(device))
    assert layer.cache.num_cold > 0 and layer.cache._fused_ok()
    W = {n: H(getattr(layer, n)).astype(np.float64) for n in ("q_proj", "o_proj", "ffn_up", "ffn_down")}
    for step in range(3):
        x = randn16(g, 1, 1, 512)
        out = H(layer(torch.from_numpy(x).to(device), use_cache=True))
        pos = layer.cache.total_tokens - 1
        window = max(cfg.block_size_seq, min(layer.cache.total_tokens, cfg.warm_capacity))
        mk, mv, adj = layer.cache.materialize_window(query_positions=torch.tensor([pos], device=device),
                                                     context_window=window)
        a = _rms(x[0], 1.0, 1e-5)
        q = f16(a.astype(np.float64) @ W["q_proj"].T).reshape(1, 8, 64)
        att = nx.blockwise_attention(q, H(mk).astype(np.float16), H(mv).astype(np.float16), 64 ** -0.5,
                                     cfg.block_size_seq, True, H(adj).astype(np.int32))
        hidden = f16(x[0].astype(np.float64) + f16(att.reshape(1, 512).astype(np.float64) @ W["o_proj"].T))
        ffn = f16(_gelu(_rms(hidden, 1.0, 1e-5).astype(np.float64) @ W["ffn_up"].T) @ W["ffn_down"].T)
        ref = f16(hidden.astype(np.float64) + ffn)
        assert np.abs(out[0] - ref.astype(np.float32)).max() <= 2e-2, step
    assert layer.cache_tokens == 503


def test_llama_layer_decode_matches_restatement(device, tmp_path):
    """The Llama layer: rotary embeddings on q and k (positions continue
    after the prompt), grouped KV heads stored as they are, SwiGLU MLP; a
    decode step against a float64 restatement around the oracle attention,
    and the prompt path (dense attention over repeated KV heads) against the
    same restatement."""
    from apple_amd.layer import LLAMA3_ROPE_SCALING, Llama32DecoderLayerMLX, rope_cos_sin

    cfg = _ext_config(tmp_path)
    layer = Llama32DecoderLayerMLX(cfg, intermediate_size=1024, device=device, quantizer=_ext_quantizer(cfg, device, 8))
    W = {n: H(getattr(layer, n)).astype(np.float64) for n in Llama32DecoderLayerMLX.WEIGHTS}
    g = rng(33)
    S = 400
    prompt = randn16(g, 1, S, 512)
    layer.prefill_cache(torch.from_numpy(prompt).to(device))

    def rope(x, pos):                      # x [S, h, 64] fp16 -> fp16
        cos, sin = (t.double().cpu().numpy() for t in rope_cos_sin(torch.tensor(pos), 64, 500000.0,
                                                                      LLAMA3_ROPE_SCALING))
        xf = x.astype(np.float64)
        rot = np.concatenate([-xf[..., 32:], xf[..., :32]], -1)
        return f16(xf * cos[:, None, :] + rot * sin[:, None, :])

    def mlp(h):
        m = _rms(h, W["post_attention_layernorm"], 1e-5).astype(np.float64)
        gate = f16(m @ W["gate_proj"].T).astype(np.float64)
        up = f16(m @ W["up_proj"].T).astype(np.float64)
        act = f16(gate / (1.0 + np.exp(-gate))).astype(np.float64)
        return f16(f16(act * up).astype(np.float64) @ W["down_proj"].T)

    x = randn16(g, 1, 1, 512)
    out = H(layer(torch.from_numpy(x).to(device), use_cache=True))
    n = _rms(x[0], W["input_layernorm"], 1e-5).astype(np.float64)
    q = rope(f16(n @ W["q_proj"].T).reshape(1, 8, 64), [S])
    mk, mv, _ = layer.cache.materialize_window()
    att = nx.blockwise_attention(q, H(mk).astype(np.float16), H(mv).astype(np.float16), 0.125, 64, False, None)
    hidden = f16(x[0].astype(np.float64) + f16(att.reshape(1, 512).astype(np.float64) @ W["o_proj"].T))
    ref = f16(hidden.astype(np.float64) + mlp(hidden))
    assert np.abs(out[0] - ref.astype(np.float32)).max() <= 2e-2
    # the newest key in the cache is the rotated projection of the decode token
    k_new = rope(f16(n @ W["k_proj"].T).reshape(1, 4, 64), [S])
    assert np.abs(H(layer.cache.hot_keys[-1]) - k_new[0].astype(np.float32)).max() <= 4e-3  # one fp16 ulp
    # prompt path: dense causal attention over the KV heads repeated to the query heads
    xs = randn16(g, 1, 24, 512)
    layer.reset_cache()
    dense = H(layer(torch.from_numpy(xs).to(device), use_cache=False))
    n = _rms(xs[0], W["input_layernorm"], 1e-5).astype(np.float64)
    pos = list(range(24))
    qs = rope(f16(n @ W["q_proj"].T).reshape(24, 8, 64), pos)
    ks = np.repeat(rope(f16(n @ W["k_proj"].T).reshape(24, 4, 64), pos), 2, axis=1)
    vs = np.repeat(f16(n @ W["v_proj"].T).reshape(24, 4, 64), 2, axis=1)
    ctx = np.zeros((24, 8, 64))
    for t in range(24):
        s = np.einsum("hd,thd->ht", qs[t].astype(np.float64), ks[:t + 1].astype(np.float64)) * 0.125
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        ctx[t] = np.einsum("ht,thd->hd", p, vs[:t + 1].astype(np.float64))
    hidden = f16(xs[0].astype(np.float64) + f16(f16(ctx).reshape(24, 512).astype(np.float64) @ W["o_proj"].T))
    ref = f16(hidden.astype(np.float64) + mlp(hidden))
    assert np.abs(dense[0] - ref.astype(np.float32)).max() <= 2e-2


def test_llama_layer_cpu_rotary_module(device, tmp_path):
    """A rotary module whose buffers live on the CPU is called on the CPU
    (llama32_adapter.py:535-553 resolves the device from the module) and its
    tables give the same decode step as the layer's own rope_cos_sin."""
    from apple_amd.layer import LLAMA3_ROPE_SCALING, Llama32DecoderLayerMLX, rope_cos_sin

    class CpuRotary(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.register_buffer("anchor", torch.zeros(1))
            self.calls = 0

        def forward(self, hidden, position_ids):
            assert hidden.device.type == "cpu" and position_ids.device.type == "cpu"
            self.calls += 1
            cos, sin = rope_cos_sin(position_ids.reshape(-1), 64, 500000.0, LLAMA3_ROPE_SCALING)
            return cos[None], sin[None]

    cfg = _ext_config(tmp_path)
    base = Llama32DecoderLayerMLX(cfg, intermediate_size=256, device=device, quantizer=_ext_quantizer(cfg, device, 8),
                                  generator=torch.Generator().manual_seed(4))
    weights = {n: getattr(base, n).detach().clone() for n in Llama32DecoderLayerMLX.WEIGHTS}
    rot = CpuRotary()
    other = Llama32DecoderLayerMLX(_ext_config(tmp_path / "b"), intermediate_size=256, device=device,
                                   quantizer=_ext_quantizer(cfg, device, 8), weights=weights, rotary_module=rot)
    g = rng(34)
    prompt = torch.from_numpy(randn16(g, 1, 40, 512)).to(device)
    x = torch.from_numpy(randn16(g, 1, 1, 512)).to(device)
    outs = []
    for layer in (base, other):
        layer.prefill_cache(prompt)
        outs.append(H(layer(x, use_cache=True)))
    assert rot.calls >= 2
    np.testing.assert_array_equal(outs[0], outs[1])
