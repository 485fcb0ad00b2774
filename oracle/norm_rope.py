"""Fused q/k RMSNorm + NeoX RoPE + paged KV write on the CPU (test infrastructure only).

Restates ``qk_norm_rope_store_reference`` and ``_sum_squares_reference``
(oxr_runtime/kernels.py:133-165) in numpy float32 with explicit bf16 rounding:

    h   = f32(x)
    var = (S(h[:64]) + S(h[64:])) / 128        S: kernels.py:158-165 tree
    h   = h * rsqrt(var + eps)                  rsqrt = 1 / sqrt, both fp32 IEEE
    y   = f32(bf16(w * bf16(h)))                kernels.py:146
    out = bf16(cat(y1*c - y2*s, y1*s + y2*c))   kernels.py:147-149, c, s = f32(bf16 table)

then ``k_cache.view(-1, KV, D)[slots] = k`` and ``v_cache...[slots] = v``
(kernels.py:152-154).  torch's CPU ``rsqrt`` equals float32 ``1 / sqrt`` bit for
bit (tests/test_oracle_norm_rope.py checks it), and the whole chain is pinned
against vectors written by the reference function itself
(tests/golden/make_golden.py).
"""

from __future__ import annotations

import numpy as np

from . import bf16


def sum_squares(x: np.ndarray) -> np.ndarray:
    """Sum of squares over the last axis (64 values) in the order of kernels.py:158-165:
    split into two chunks of 32, pairwise adds at strides 16, 8, 4, 2, 1 inside each,
    then chunk 0 + chunk 1."""
    assert x.shape[-1] == 64
    y = (x * x).astype(np.float32).reshape(*x.shape[:-1], 2, 32)
    while y.shape[-1] > 1:
        half = y.shape[-1] // 2
        y = (y[..., :half] + y[..., half:]).astype(np.float32)
    y = y[..., 0]
    return (y[..., 0] + y[..., 1]).astype(np.float32)


def norm_rope(x_bits: np.ndarray, w_bits: np.ndarray, cos_bits: np.ndarray, sin_bits: np.ndarray, eps: float) -> np.ndarray:
    """x_bits uint16 [n, heads, 128]; w_bits [128]; cos/sin [n, 64].  Returns uint16 [n, heads, 128]."""
    d = x_bits.shape[-1]
    assert d == 128
    half = d // 2
    h = bf16.to_f32(x_bits)
    var = ((sum_squares(h[..., :half]) + sum_squares(h[..., half:])) / np.float32(d)).astype(np.float32)
    r = (np.float32(1.0) / np.sqrt((var + np.float32(eps)).astype(np.float32))).astype(np.float32)
    h = (h * r[..., None]).astype(np.float32)
    y = bf16.round_f32(bf16.to_f32(w_bits) * bf16.round_f32(h))
    c = bf16.to_f32(cos_bits)[:, None, :]
    s = bf16.to_f32(sin_bits)[:, None, :]
    y1, y2 = y[..., :half], y[..., half:]
    out = np.concatenate(((y1 * c - y2 * s).astype(np.float32), (y1 * s + y2 * c).astype(np.float32)), axis=-1)
    return bf16.from_f32(out)


def qk_norm_rope_store(
    qkv_bits: np.ndarray, q_weight_bits: np.ndarray, k_weight_bits: np.ndarray, cos_bits: np.ndarray,
    sin_bits: np.ndarray, eps: float, k_cache_bits: np.ndarray, v_cache_bits: np.ndarray, slots: np.ndarray,
    num_heads: int, num_kv_heads: int, head_dim: int, *, need_kv: bool,
):
    """kernels.py:133-155.  Caches are uint16 arrays whose flat view is [slots, KV, D]; they are
    written in place.  Returns (q, k | None, v | None) as uint16 arrays."""
    n = qkv_bits.shape[0]
    heads = qkv_bits.reshape(n, num_heads + 2 * num_kv_heads, head_dim)
    q = heads[:, :num_heads]
    k = heads[:, num_heads : num_heads + num_kv_heads]
    v = heads[:, num_heads + num_kv_heads :]
    q_out = norm_rope(q, q_weight_bits, cos_bits, sin_bits, eps)
    k_out = norm_rope(k, k_weight_bits, cos_bits, sin_bits, eps)
    flat = (-1, num_kv_heads, head_dim)
    k_cache_bits.reshape(flat)[slots] = k_out
    v_cache_bits.reshape(flat)[slots] = v
    if need_kv:
        return q_out, k_out, np.ascontiguousarray(v)
    return q_out, None, None


def rope_tables(max_positions: int, head_dim: int = 128, theta: float = 1e6) -> tuple[np.ndarray, np.ndarray]:
    """language.py:160-170: fp32 ``outer(arange, 1/theta^(arange(0, D, 2)/D))`` cos/sin, stored as bf16.

    Computed with torch on the CPU, as the reference does, so the fp32 angles and
    their cos/sin round the same way; returns uint16 bf16 bits [max_positions, D/2]."""
    import torch

    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    freqs = torch.outer(torch.arange(max_positions, dtype=torch.float), inv_freq)
    cos = freqs.cos().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    sin = freqs.sin().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return cos, sin
