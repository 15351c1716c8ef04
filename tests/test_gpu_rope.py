"""GPU: libpkv's RoPE kernel (``pkv_rope_qkv``) against float64 and the torch composite.

The kernel rotates q and k of a fused projection at their positions and writes
head-major q, k, v (``models/shared/transformer.py:32-90``, :146-184).  Checks:
- against a float64 NumPy rotate-half of the same inputs, within the output
  dtype's rounding (the float32 math differs from float64 by far less than one
  output ulp, so the bound is one ulp plus the float32 cos/sin error);
- against the torch float32 composite ``apply_rope`` (the element-wise path it
  replaces), within one output ulp;
- v is a bit-exact copy, the layouts are head-major, and position 0 is the identity.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

CASES = [
    # (batch, tokens, heads, kv_heads, dim, dtype, max position, llama3 scaling)
    (32, 1, 32, 8, 128, "float16", 8192, False),        # decode, Llama-3-8B shape
    (2, 37, 4, 1, 64, "bfloat16", 600, False),          # ragged prefill chunk
    (3, 5, 8, 2, 256, "float16", 131072, True),         # long positions, llama3 frequencies
    (1, 2, 2, 2, 2, "bfloat16", 10, False),             # smallest head
    (2, 3, 3, 1, 48, "float16", 1000, False),           # dim/2 not a multiple of 8
    (2, 4, 2, 1, 16, "bfloat16", 50, False),            # one lane per head
]


def _inputs(batch, tokens, heads, kv_heads, dim, dtype, max_pos, llama3, seed=0):
    from pkv.layer import rope_inverse_frequencies

    gen = torch.Generator().manual_seed(seed)
    width = (heads + 2 * kv_heads) * dim
    qkv = torch.randn((batch, tokens, width), generator=gen).to(getattr(torch, dtype))
    pos = torch.randint(0, max_pos, (batch, tokens), generator=gen, dtype=torch.int64)
    scaling = dict(rope_type="llama3", factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
                   original_max_position_embeddings=8192) if llama3 else None
    inv = rope_inverse_frequencies(dim, 500000.0, scaling)
    return qkv, pos, inv


def _split(qkv, heads, kv_heads, dim):
    b, t, _ = qkv.shape
    x = qkv.view(b, t, heads + 2 * kv_heads, dim).transpose(1, 2)
    return x[:, :heads], x[:, heads:heads + kv_heads], x[:, heads + kv_heads:]


def _rope64(x, pos, inv):
    """float64 rotate-half of x [B, h, T, D] at pos [B, T]."""
    x = x.double().numpy()
    ang = pos.double().numpy()[:, None, :, None] * inv.double().numpy()[None, None, None, :]
    c, s = np.cos(ang), np.sin(ang)
    half = x.shape[-1] // 2
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


def _ulp(dtype):
    return 2.0 ** -10 if dtype == "float16" else 2.0 ** -7


@pytest.mark.parametrize("case", CASES)
def test_rope_matches_float64_and_the_torch_composite(case):
    from pkv import ops
    from pkv.layer import apply_rope

    batch, tokens, heads, kv_heads, dim, dtype, max_pos, llama3 = case
    qkv, pos, inv = _inputs(*case)
    print(f"rope case {case}", flush=True)
    q, k, v = ops.rope_qkv(qkv.cuda(), pos.cuda(), inv.cuda(), heads, kv_heads)
    torch.cuda.synchronize()
    assert q.shape == (batch, heads, tokens, dim) and k.shape == v.shape == (
        batch, kv_heads, tokens, dim)
    assert q.is_contiguous() and k.is_contiguous() and v.is_contiguous()
    xq, xk, xv = _split(qkv, heads, kv_heads, dim)
    assert torch.equal(v.cpu(), xv.contiguous())                     # v: bit-exact copy
    ulp = _ulp(dtype)
    for got, x in ((q, xq), (k, xk)):
        want = _rope64(x, pos, inv)
        err = np.abs(got.cpu().double().numpy() - want)
        # one output ulp (half an ulp of rounding each side) plus float32 trig error
        # at angles up to max_pos (|angle| * 2^-23 relative)
        bound = ulp * np.maximum(np.abs(want), 2.0 ** -14) + 4 * max_pos * 2.0 ** -24 * np.abs(
            x.double().numpy()).max()
        assert (err <= bound).all(), f"max err {err.max()} (ulp {ulp})"
        composite = apply_rope(x.cuda(), pos.cuda(), inv.cuda()).cpu()
        diff = (got.cpu().float() - composite.float()).abs()
        assert (diff <= ulp * composite.float().abs().clamp_min(2.0 ** -14)).all()


def test_position_zero_is_the_identity_and_layer_projection_matches():
    from pkv import ops
    from pkv.layer import AttentionLayer, ModelSpec

    qkv, _, inv = _inputs(2, 3, 4, 2, 64, "float16", 1, False)
    zero = torch.zeros((2, 3), dtype=torch.int64)
    q, k, v = ops.rope_qkv(qkv.cuda(), zero.cuda(), inv.cuda(), 4, 2)
    xq, xk, _ = _split(qkv, 4, 2, 64)
    assert torch.equal(q.cpu(), xq.contiguous()) and torch.equal(k.cpu(), xk.contiguous())

    spec = ModelSpec(hidden=256, query_heads=4, kv_heads=2, head_dim=64, dtype="float16")
    layer = AttentionLayer(spec, 0, device="cuda", seed=3)
    x = torch.randn((3, 4, 256), generator=torch.Generator().manual_seed(1)).half().cuda()
    pos = torch.arange(12).view(3, 4).cuda() + 100
    fused = layer.project(x, pos)
    split = layer.project_reference(x, pos)
    for a, b in zip(fused, split):
        # fused and split GEMMs may sum in different orders: a few output ulps
        torch.testing.assert_close(a, b.contiguous(), rtol=4e-3, atol=4e-3)
