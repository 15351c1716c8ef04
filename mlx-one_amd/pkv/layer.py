"""A Llama-3-shaped GQA attention layer whose KV path is the paged cache.

The caller side of ``PagedBatchCache.attend``, restated from the reference's
attention block (``src/mlx_one/models/shared/transformer.py:140-209``):
``q/k/v = x @ W`` reshaped to ``[B, heads, T, D]``, RoPE on queries and keys at
their logical positions (``transformer.py:32-90``: rotate-half, ``theta``,
optional ``llama3`` frequency scaling), ``cache.attend(q, k, v, scale=,
position_ids=)`` (append-and-quantize + paged attention in libpkv), then the
output projection.  Projections and RoPE run as torch-ROCm ops (hipBLASLt
GEMMs) in the activation dtype; weights are random (synthetic), the shapes
are the model's.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field


@dataclass(frozen=True)
class LayerLayout:
    """One attention layer's cache-relevant shape (``engine/cache_specs.py`` layer specs)."""

    layer_id: int
    query_heads: int
    kv_heads: int
    key_dim: int
    kind: str = "full_kv"

    @property
    def num_kv_heads(self):
        return self.kv_heads

    @property
    def key_head_dim(self):
        return self.key_dim

    @property
    def value_head_dim(self):
        return self.key_dim


@dataclass(frozen=True)
class ModelSpec:
    """Llama-3-8B attention shape by default: hidden 4096, 32 query / 8 KV heads, D 128."""

    hidden: int = 4096
    query_heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    num_layers: int = 1
    rope_theta: float = 500000.0
    rope_scaling: dict | None = field(default=None)
    dtype: str = "bfloat16"
    vocab_size: int = 128256

    @property
    def layers(self):
        return tuple(LayerLayout(i, self.query_heads, self.kv_heads, self.head_dim)
                     for i in range(self.num_layers))

    def bytes_per_token(self):
        """Float K+V bytes per token over all layers (2 bytes per element)."""
        return self.num_layers * 2 * self.kv_heads * self.head_dim * 2


def rope_inverse_frequencies(head_dim, theta, rope_scaling=None):
    """float32 ``[head_dim / 2]`` inverse frequencies (``transformer.py:50-66``)."""
    import torch

    half = head_dim // 2
    inv = theta ** (-torch.arange(half, dtype=torch.float64) / half)
    if rope_scaling and rope_scaling.get("rope_type", rope_scaling.get("type")) == "llama3":
        factor = rope_scaling["factor"]
        low, high = rope_scaling["low_freq_factor"], rope_scaling["high_freq_factor"]
        original = rope_scaling["original_max_position_embeddings"]
        denom = 1.0 / inv
        wavelengths = 2 * math.pi * denom
        smooth = (original / wavelengths - low) / (high - low)
        mixed = denom / (smooth + (1 - smooth) / factor)
        denom = torch.where(wavelengths < original / high, denom,
                            torch.where(wavelengths > original / low, denom * factor, mixed))
        inv = 1.0 / denom
    return inv.to(torch.float32)


def apply_rope(x, positions, inv_freq):
    """Rotate-half RoPE of ``x [B, heads, T, D]`` at ``positions [B, T]`` (float32 math)."""
    import torch

    angles = positions.to(torch.float32)[:, None, :, None] * inv_freq.to(x.device)[None, None, None, :]
    cos, sin = torch.cos(angles), torch.sin(angles)
    xf = x.float()
    half = x.shape[-1] // 2
    a, b = xf[..., :half], xf[..., half:]
    return torch.cat([a * cos - b * sin, b * cos + a * sin], dim=-1).to(x.dtype)


class AttentionLayer:
    """Projection weights of one layer on the device (random, seeded)."""

    def __init__(self, spec: ModelSpec, layer_id: int, *, device="cuda", seed=0):
        import torch

        self.spec, self.layer_id = spec, layer_id
        dtype = getattr(torch, spec.dtype)
        gen = torch.Generator(device="cpu")
        gen.manual_seed(1000 * seed + layer_id)
        h, hq, hk, d = spec.hidden, spec.query_heads, spec.kv_heads, spec.head_dim

        def weight(rows, cols):
            w = torch.randn((rows, cols), generator=gen, dtype=torch.float32) / math.sqrt(rows)
            return w.to(device=device, dtype=dtype)

        wq, wk, wv = weight(h, hq * d), weight(h, hk * d), weight(h, hk * d)
        # one fused q|k|v projection; wq/wk/wv are column views of it
        self.wqkv = torch.cat([wq, wk, wv], dim=1)
        self.wq = self.wqkv[:, :hq * d]
        self.wk = self.wqkv[:, hq * d:(hq + hk) * d]
        self.wv = self.wqkv[:, (hq + hk) * d:]
        self.wo = weight(hq * d, h)
        self.scale = 1.0 / math.sqrt(d)
        self.inv_freq = rope_inverse_frequencies(d, spec.rope_theta, spec.rope_scaling).to(device)

    def project(self, x, positions):
        """``x [B, T, hidden]`` -> RoPE'd ``q [B, H, T, D]``, ``k, v [B, HK, T, D]``:
        one GEMM over the fused weight, then libpkv's RoPE kernel, which also
        writes the head-major layouts (``transformer.py:146-184``)."""
        from pkv import ops

        s = self.spec
        return ops.rope_qkv(x @ self.wqkv, positions, self.inv_freq, s.query_heads, s.kv_heads)

    def project_reference(self, x, positions):
        """The same projection as separate GEMMs and torch element-wise RoPE
        (``apply_rope``): the comparison path of the tests."""
        s = self.spec
        batch, width, _ = x.shape
        q = (x @ self.wq).view(batch, width, s.query_heads, s.head_dim).transpose(1, 2)
        k = (x @ self.wk).view(batch, width, s.kv_heads, s.head_dim).transpose(1, 2)
        v = (x @ self.wv).view(batch, width, s.kv_heads, s.head_dim).transpose(1, 2)
        return apply_rope(q, positions, self.inv_freq), apply_rope(k, positions, self.inv_freq), v

    def __call__(self, x, cache, position_ids):
        """One layer through ``cache.attend`` (``transformer.py:202-209``).  Host
        ``position_ids`` stay on the host for the cache's position check (no
        device sync); RoPE reads a device copy."""
        q, k, v = self.project(x, position_ids.to(x.device, non_blocking=True))
        out = cache.attend(q, k, v, scale=self.scale, position_ids=position_ids)
        batch, _, width, _ = out.shape
        return out.transpose(1, 2).reshape(batch, width, -1) @ self.wo


class AttentionStack:
    """``num_layers`` attention layers applied in sequence: the model the runner drives."""

    def __init__(self, spec: ModelSpec = ModelSpec(), *, device="cuda", seed=0):
        self.spec = spec
        self.device, self.seed = device, seed
        self.layers = tuple(AttentionLayer(spec, i, device=device, seed=seed)
                            for i in range(spec.num_layers))
        self.activation_dtype = spec.dtype
        self._embedding = None

    def embed(self, token_ids):
        """``[T, hidden]`` inputs of the first layer for token ids: rows of a
        random (seeded) embedding table, built on first use."""
        import torch

        ids = torch.as_tensor(list(token_ids), dtype=torch.int64)
        if ids.numel() < 1 or int(ids.min()) < 0 or int(ids.max()) >= self.spec.vocab_size:
            raise ValueError(f"token ids must lie in [0, {self.spec.vocab_size})")
        if self._embedding is None:
            gen = torch.Generator(device=self.device)
            gen.manual_seed(1000 * self.seed + 999)
            table = torch.randn((self.spec.vocab_size, self.spec.hidden), generator=gen,
                                device=self.device)
            self._embedding = table.to(getattr(torch, self.spec.dtype))
        return self._embedding[ids.to(self._embedding.device)]

    def forward(self, x, *, cache, position_ids):
        for layer, layer_cache in zip(self.layers, cache, strict=True):
            x = layer(x, layer_cache, position_ids)
        return x
