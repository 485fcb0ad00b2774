"""Fused q/k RMSNorm + RoPE + paged KV write: the drop-in for oxr_runtime/kernels.py.

``qk_norm_rope_store`` keeps the reference signature (kernels.py:102-113) and runs the
hand-written gfx950 kernel ``oxr_qk_norm_rope_store`` (csrc/qk_norm_rope.hip).  The
reference dispatches CPU tensors to a torch restatement (kernels.py:111-112); this build
has no CPU path and raises for CPU tensors instead.
"""

from __future__ import annotations

import torch

from . import _lib


def qk_norm_rope_store(
    qkv: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
    eps: float, k_cache: torch.Tensor, v_cache: torch.Tensor, slots: torch.Tensor,
    num_heads: int, num_kv_heads: int, head_dim: int, *, need_kv: bool,
    q_out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor | None]:
    """``qkv`` is the ``[n, (H + 2*KV) * D]`` projection (bf16, contiguous); ``cos``/``sin`` are
    ``[n, D/2]`` bf16; ``k_cache``/``v_cache`` are one layer's paged caches
    (``[blocks, block_size, KV, D]``), token i is written to slot ``slots[i]``.  Returns ``q``
    (``[n, H, D]``) and, when ``need_kv``, contiguous ``k``/``v`` (``[n, KV, D]``).

    ``q_out`` (optional, this build only) receives q instead of a new tensor."""
    device = _lib.require_gpu(qkv, q_weight, k_weight, cos, sin, k_cache, v_cache, slots, name="qk_norm_rope_store")
    n = qkv.shape[0]
    width = (num_heads + 2 * num_kv_heads) * head_dim
    _lib.require(head_dim == 128, f"head_dim must be 128 (got {head_dim}), as the reference's kernel")
    for name, t in (("qkv", qkv), ("q_weight", q_weight), ("k_weight", k_weight), ("cos", cos), ("sin", sin),
                    ("k_cache", k_cache), ("v_cache", v_cache)):
        _lib.require(t.dtype == torch.bfloat16, f"{name} must be bfloat16 (got {t.dtype})")
        _lib.require(t.is_contiguous(), f"{name} must be contiguous")
    _lib.require(qkv.dim() == 2 and qkv.shape[1] == width, f"qkv must be [n, {width}] (got {list(qkv.shape)})")
    _lib.require(q_weight.numel() == head_dim and k_weight.numel() == head_dim, "norm weights must have head_dim values")
    _lib.require(tuple(cos.shape) == (n, head_dim // 2) and cos.shape == sin.shape, "cos/sin must be [n, head_dim/2]")
    _lib.require(k_cache.shape == v_cache.shape, "k_cache and v_cache shapes differ")
    _lib.require(k_cache.shape[-2:] == (num_kv_heads, head_dim), "caches must end in [KV, head_dim]")
    _lib.require(slots.dim() == 1 and slots.shape[0] == n, "slots must be [n]")
    if slots.dtype != torch.int64 or not slots.is_contiguous():
        slots = slots.to(torch.int64).contiguous()
    num_slots = k_cache.numel() // (num_kv_heads * head_dim)

    if q_out is None:
        q = qkv.new_empty(n, num_heads, head_dim)
    else:
        _lib.require(q_out.shape == (n, num_heads, head_dim) and q_out.dtype == torch.bfloat16 and q_out.is_contiguous(),
                     "q_out must be contiguous bf16 [n, H, D]")
        q = q_out
    k = qkv.new_empty(n, num_kv_heads, head_dim) if need_kv else None
    v = qkv.new_empty(n, num_kv_heads, head_dim) if need_kv else None
    _lib.call(
        "oxr_qk_norm_rope_store", qkv.data_ptr(), q_weight.data_ptr(), k_weight.data_ptr(), cos.data_ptr(),
        sin.data_ptr(), float(eps), k_cache.data_ptr(), v_cache.data_ptr(), slots.data_ptr(), num_slots, n,
        num_heads, num_kv_heads, head_dim, q.data_ptr(), _lib.ptr(k), _lib.ptr(v), _lib.stream(device),
    )
    return q, k, v
