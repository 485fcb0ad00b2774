"""The verify forward of the decoder on the CPU with torch (test infrastructure only).

Restates ``LanguageModel.extend`` / ``logits`` and the step around them
(oxr_runtime/language.py:69-104, 201-214, 247-269, 301-317; decode_graph.py:161-167),
with attention as the reference test stub (tests/test_language_fused.py:19-57) and the
fused q/k norm + RoPE + KV write as ``qk_norm_rope_store_reference`` (kernels.py:133-155,
through ``oracle.norm_rope``).  Rounding points are the reference's: bf16 activations,
bf16 ``nn.Linear`` outputs (fp32 accumulation), fp32 norms, residual stored in bf16 before
it is normalised, fp32 softmax.

Pinned (tests/test_oracle_decoder.py) by golden vectors the reference's own
``LanguageModel.extend`` wrote (tests/golden/make_golden_decoder.py): hidden states, cache rows,
logits and argmax bit for bit, at GQA 4/2 with S=4 and GQA 16/8 with S=9; by the same forward
computed from the equations without rounding; and by the reference's extend == full-sequence
invariant.

It is also the CPU baseline ``bench.py`` times (torch on the host's cores).
"""

from __future__ import annotations

from typing import NamedTuple

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
    """kernels.py:133-155: q/k through ``oracle.norm_rope.norm_rope`` (bit-identical to the
    reference function), then the cache rows at ``slots`` are written (kernels.py:152-154)."""
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


class VerifyStep(NamedTuple):
    drafts: list[list[int]]  # per sequence, as propose() returns them
    predicted: torch.Tensor  # int64 [B, S]: the oracle's greedy ids
    taken: list[list[int]]   # per sequence: accept(draft, predicted row)
    new_lens: list[int]      # seq.length after the step
    logits: torch.Tensor     # bf16 [B * S, vocab]


def drafts_for(histories, seq_lens, k, max_n, *, max_tokens=None, max_positions=None) -> list[list[int]]:
    """engine.py:675-684: each sequence's draft from the ids it generated, at most
    ``min(k, max(room, 0))`` long with room = min(max_tokens - len(output) - 1,
    max_positions - length - 1) (a limit left out is no limit)."""
    out = []
    for b, h in enumerate(histories):
        room = k
        if max_tokens is not None:
            room = min(room, int(max_tokens[b]) - len(h) - 1)
        if max_positions is not None:
            room = min(room, int(max_positions) - int(seq_lens[b]) - 1)
        out.append(ngram.NgramIndex(h, max_n).propose(list(h), min(k, max(room, 0))))
    return out


def verify_rows(histories, drafts, seq_lens, block_table, s, block_size):
    """engine.py:700-710: row b is [output[-1], *draft, 0 ...] of width S at positions length + j,
    slots through the block table (language.py:320-322); seq_lens length + S."""
    ids, positions, slots = [], [], []
    for b, (h, draft) in enumerate(zip(histories, drafts)):
        row = [h[-1], *draft] + [0] * (s - 1 - len(draft))
        for j, token in enumerate(row):
            pos = int(seq_lens[b]) + j
            ids.append(int(token))
            positions.append(pos)
            slots.append(int(block_table[b, pos // block_size]) * block_size + pos % block_size)
    attn_lens = torch.tensor([int(x) + s for x in seq_lens], dtype=torch.int32)
    return torch.tensor(ids), torch.tensor(positions), torch.tensor(slots), attn_lens


def accept_step(drafts, predicted, seq_lens) -> tuple[list[list[int]], list[int]]:
    """engine.py:729-734: taken = accept(draft, row[:len(draft) + 1]); length += len(taken)."""
    rows = predicted.tolist() if isinstance(predicted, torch.Tensor) else [list(r) for r in predicted]
    taken = [ngram.accept(d, rows[b][: len(d) + 1]) for b, d in enumerate(drafts)]
    return taken, [int(seq_lens[b]) + len(t) for b, t in enumerate(taken)]


def verify_step(config, weights, histories, seq_lens, block_table, k, max_n, cache_k, cache_v, block_size, *,
                max_tokens=None, max_positions=None) -> VerifyStep:
    """One speculative step as Engine._speculate performs it (engine.py:674-737) with graph width
    S = k + 1: draft per sequence, assemble rows, extend, greedy ids, accept."""
    s = k + 1
    drafts = drafts_for(histories, seq_lens, k, max_n, max_tokens=max_tokens, max_positions=max_positions)
    ids, positions, slots, attn_lens = verify_rows(histories, drafts, seq_lens, block_table, s, block_size)
    hidden = extend(config, weights, ids, positions, slots, attn_lens, torch.from_numpy(np.asarray(block_table)), s,
                    cache_k, cache_v)
    out = logits(weights, hidden)
    predicted = out.argmax(-1).view(len(histories), s)
    taken, new_lens = accept_step(drafts, predicted, seq_lens)
    return VerifyStep(drafts, predicted, taken, new_lens, out)
