"""The verify forward of the decoder on the CPU with torch (test infrastructure only).

Restates ``LanguageModel.extend`` / ``logits`` and the step around them
(oxr_runtime/language.py:69-104, 201-214, 247-269, 301-317; decode_graph.py:161-167),
with attention as the reference test stub (tests/test_language_fused.py:19-57) and the
fused q/k norm + RoPE + KV write as ``qk_norm_rope_store_reference`` (kernels.py:181-203,
through ``oracle.norm_rope``).  Rounding points are the reference's: bf16 activations,
bf16 ``nn.Linear`` outputs (fp32 accumulation), fp32 norms, residual stored in bf16 before
it is normalised, fp32 softmax.

It is also the CPU baseline ``bench.py`` times (torch on the host's cores).
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import ngram, norm_rope


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _from_bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """language.py:69-72."""
    h = x.float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return weight * h.to(x.dtype)


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """language.py:102-104."""
    gate, up = gate_up.chunk(2, dim=-1)
    return F.silu(gate) * up


def paged_extend(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, seq_lens: torch.Tensor,
                 block_table: torch.Tensor, scale: float) -> torch.Tensor:
    """The test stub's ``_paged_extend`` (tests/test_language_fused.py:19-28, 50-57)."""
    out = []
    for b, length in enumerate(seq_lens.tolist()):
        pages = -(-length // k_cache.shape[1])
        k = k_cache[block_table[b, :pages].long()].flatten(0, 1)[:length]
        v = v_cache[block_table[b, :pages].long()].flatten(0, 1)[:length]
        qb = q[b]
        rep = qb.shape[1] // k.shape[1]
        kk, vv = k.repeat_interleave(rep, dim=1), v.repeat_interleave(rep, dim=1)
        scores = torch.einsum("nhd,mhd->hnm", qb.float(), kk.float()) * scale
        n, m = qb.shape[0], kk.shape[0]
        mask = torch.arange(m)[None, :] > (torch.arange(n)[:, None] + m - n)
        scores = scores.masked_fill(mask, float("-inf"))
        out.append(torch.einsum("hnm,mhd->nhd", scores.softmax(-1), vv.float()).to(q.dtype))
    return torch.stack(out)


def qk_norm_rope_store(qkv, q_weight, k_weight, cos, sin, eps, k_cache, v_cache, slots, H, KV, D):
    """kernels.py:181-203: q/k through ``oracle.norm_rope.norm_rope`` (bit-identical to the
    reference function), then the cache rows at ``slots`` are written (kernels.py:200-202)."""
    n = qkv.shape[0]
    heads = _bits(qkv).reshape(n, H + 2 * KV, D)
    c, s_ = _bits(cos), _bits(sin)
    q = norm_rope.norm_rope(heads[:, :H], _bits(q_weight), c, s_, eps)
    k = norm_rope.norm_rope(heads[:, H : H + KV], _bits(k_weight), c, s_, eps)
    flat = (-1, KV, D)
    k_cache.view(flat)[slots] = _from_bits(k)
    v_cache.view(flat)[slots] = _from_bits(np.ascontiguousarray(heads[:, H + KV :]))
    return _from_bits(q)


def extend(config, weights, ids, positions, slots, seq_lens, block_table, tokens_per_seq, cache_k, cache_v,
           trace: list | None = None, mid: list | None = None):
    """``LanguageModel.extend`` (language.py:201-211) on CPU tensors; caches [L, blocks, bs, KV, D]
    are updated in place.  Returns the final-norm hidden states [B * S, hidden] (bf16).

    ``trace`` (a list) receives the residual stream entering each layer (after the previous
    layer's MLP add) and, last, the one entering the final norm; ``mid`` receives each layer's
    residual after its attention add."""
    c, w = config, weights
    x = w.embed[ids]
    cos, sin = w.rope_cos[positions], w.rope_sin[positions]
    b, s = block_table.shape[0], tokens_per_seq
    residual = None
    for index, layer in enumerate(w.layers):
        if residual is None:
            residual, h = x, rms_norm(x, layer.input_norm, c.rms_norm_eps)
        else:
            residual = x + residual
            h = rms_norm(residual, layer.input_norm, c.rms_norm_eps)
        if trace is not None:
            trace.append(residual.clone())
        qkv = F.linear(h, layer.qkv)
        q = qk_norm_rope_store(qkv, layer.q_norm, layer.k_norm, cos, sin, c.rms_norm_eps, cache_k[index],
                               cache_v[index], slots, c.num_heads, c.num_kv_heads, c.head_dim)
        attn = paged_extend(q.view(b, s, c.num_heads, c.head_dim), cache_k[index], cache_v[index], seq_lens,
                            block_table, c.head_dim ** -0.5)
        residual = F.linear(attn.reshape(b * s, -1), layer.o) + residual
        if mid is not None:
            mid.append(residual.clone())
        h = rms_norm(residual, layer.post_norm, c.rms_norm_eps)
        x = F.linear(silu_mul(F.linear(h, layer.gate_up)), layer.down)
    residual = x + residual
    if trace is not None:
        trace.append(residual.clone())
    return rms_norm(residual, w.final_norm, c.rms_norm_eps)


def logits(weights, hidden: torch.Tensor) -> torch.Tensor:
    """language.py:213-214."""
    return F.linear(hidden, weights.lm_head)


def verify_step(config, weights, histories, seq_lens, block_table, k, max_n, cache_k, cache_v, block_size):
    """One speculative step as Engine._speculate performs it (engine.py:674-737) with graph width
    S = k + 1: draft per sequence, assemble rows, extend, greedy ids, accept.  Returns
    (drafts, predicted [B, S], taken per sequence, new seq_lens)."""
    s = k + 1
    drafts = [ngram.NgramIndex(h, max_n).propose(list(h), k) for h in histories]
    ids, positions, slots = [], [], []
    for b, (h, draft) in enumerate(zip(histories, drafts)):
        row = [h[-1], *draft] + [0] * (s - 1 - len(draft))
        for j, token in enumerate(row):
            pos = int(seq_lens[b]) + j
            ids.append(int(token))
            positions.append(pos)
            slots.append(int(block_table[b, pos // block_size]) * block_size + pos % block_size)
    attn_lens = torch.tensor([int(x) + s for x in seq_lens], dtype=torch.int32)
    hidden = extend(config, weights, torch.tensor(ids), torch.tensor(positions), torch.tensor(slots), attn_lens,
                    torch.from_numpy(np.asarray(block_table)), s, cache_k, cache_v)
    predicted = logits(weights, hidden).argmax(-1).view(len(histories), s)
    taken = [ngram.accept(d, predicted[b, : len(d) + 1].tolist()) for b, d in enumerate(drafts)]
    new_lens = [int(seq_lens[b]) + len(t) for b, t in enumerate(taken)]
    return drafts, predicted, taken, new_lens
