"""Paged verify attention and variable-length (prefill) attention on the CPU (test
infrastructure only).

attention.paged_extend (oxr_runtime/attention.py:96-109) calls flash-attn, which is not in
the reference tree; its math is the reference's test stub ``_attend`` / ``_paged_extend``
(tests/test_language_fused.py:19-28, 50-57): gather the sequence's keys through the block
table, repeat kv heads to the q heads (GQA), fp32 scores ``q.k * scale``, a causal mask
aligned to the end (new token i of n sees keys <= i + m - n), fp32 softmax, fp32 PV, then
rounding to q's dtype.  Computed here in float64 before the final bf16 rounding, so the
oracle is the exact value the kernel's fp32/bf16 arithmetic approximates.
"""

from __future__ import annotations

import numpy as np

from . import bf16


def attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, causal: bool = True) -> np.ndarray:
    """q [n, H, D], k/v [m, KV, D] as float arrays -> float64 [n, H, D] (causal: end-aligned mask)."""
    n, h, _ = q.shape
    m, kv, _ = k.shape
    rep = h // kv
    k = np.repeat(k.astype(np.float64), rep, axis=1)
    v = np.repeat(v.astype(np.float64), rep, axis=1)
    scores = np.einsum("nhd,mhd->hnm", q.astype(np.float64), k) * scale
    if causal:
        mask = np.arange(m)[None, :] > (np.arange(n)[:, None] + m - n)
        scores = np.where(mask[None], -np.inf, scores)
    scores -= scores.max(-1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("hnm,mhd->nhd", p, v)


def paged_extend(q_bits: np.ndarray, k_rows: list[np.ndarray], v_rows: list[np.ndarray], scale: float) -> tuple[np.ndarray, np.ndarray]:
    """q_bits uint16 [B, S, H, D]; k_rows[b] / v_rows[b] uint16 [L_b, KV, D] (the sequence's keys in
    order, already gathered through the block table).  Returns (exact float64 [B, S, H, D],
    bf16-rounded uint16 [B, S, H, D])."""
    q = bf16.to_f32(q_bits)
    exact = np.stack([attend(q[b], bf16.to_f32(k_rows[b]), bf16.to_f32(v_rows[b]), scale) for b in range(q.shape[0])])
    return exact, bf16.from_f32(exact.astype(np.float32))


def varlen(q_bits: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray, cu_seqlens: np.ndarray, scale: float,
           causal: bool) -> np.ndarray:
    """attention.varlen (oxr_runtime/attention.py:47-59; flash-attn's varlen call with equal query
    and key lengths per sequence): sequences concatenated along the tokens, q uint16 [T, H, D],
    k/v uint16 [T, KV, D], cu_seqlens [n + 1]; attention within each sequence, causal (token i
    sees tokens <= i of its sequence) or not.  Returns exact float64 [T, H, D]."""
    q, k, v = bf16.to_f32(q_bits), bf16.to_f32(k_bits), bf16.to_f32(v_bits)
    out = np.zeros(q.shape, dtype=np.float64)
    for a, b in zip(cu_seqlens[:-1], cu_seqlens[1:]):
        if b > a:
            out[a:b] = attend(q[a:b], k[a:b], v[a:b], scale, causal)
    return out
