"""The verify forward from the Qwen3 equations with no intermediate rounding (test helper).

Used to measure how far a bf16 implementation sits from exact arithmetic: the oracle (the
reference's rounding points) and the gfx950 path are both compared with it.  Written from the
equations, not from either implementation: RMSNorm x / sqrt(mean(x^2) + eps) * w; per-head q/k
RMSNorm, then NeoX RoPE at each token's position with the model's (bf16) cos/sin tables; causal
attention of the S new tokens of each sequence over its keys [0, seq_len) -- the cached context
through the block table, then the step's own new K/V -- with q head h reading kv head
``kv_head_of(h)``; SwiGLU MLP; residual adds; final RMSNorm; LM head.

``dtype`` is the arithmetic type (float64, or float32 whose rounding is ~1e-7 relative, three
orders of magnitude below bf16's).  Weights use the fused layout (``qkv`` = q|k|v rows,
``gate_up`` = gate|up rows, language.py:234-245).
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def extend(config, weights, ids, positions, seq_lens, block_table, s, k_cache, v_cache, block_size, *,
           dtype=torch.float64, kv_head_of=None, with_logits=False, new_kv: list | None = None):
    """Final-norm hidden states [B * S, hidden] (and logits [B * S, vocab] with ``with_logits``).
    ``k_cache``/``v_cache`` are bf16 [layers, blocks, block_size, KV, D]; only positions below
    ``seq_len - S`` are read from them (the step's own K/V are computed here; ``new_kv``, a list,
    receives each layer's (K, V) rows of the new tokens)."""
    c = config
    g = c.num_heads // c.num_kv_heads
    kv_of = torch.tensor([(kv_head_of or (lambda h: h // g))(h) for h in range(c.num_heads)])
    up = lambda t: t.to(dtype)
    rms = lambda x, w: x / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + c.rms_norm_eps) * up(w)
    pos = torch.as_tensor(np.asarray(positions))
    cos, sin = up(weights.rope_cos[pos])[:, None, :], up(weights.rope_sin[pos])[:, None, :]
    half, d = c.head_dim // 2, c.head_dim

    def rope(x):
        x1, x2 = x[..., :half], x[..., half:]
        return torch.cat((x1 * cos - x2 * sin, x1 * sin + x2 * cos), dim=-1)

    lens = [int(x) for x in np.asarray(seq_lens)]
    table = np.asarray(block_table)
    b_count = len(lens)
    ctx_slots = []
    for b, length in enumerate(lens):
        keys = np.arange(length - s)
        ctx_slots.append(torch.from_numpy(table[b, keys // block_size].astype(np.int64) * block_size
                                          + keys % block_size))
    x = up(weights.embed[torch.as_tensor(np.asarray(ids))])
    n = x.shape[0]
    for i, layer in enumerate(weights.layers):
        h = rms(x, layer.input_norm)
        qkv = h @ up(layer.qkv).T
        q = rope(rms(qkv[:, : c.num_heads * d].view(n, c.num_heads, d), layer.q_norm))
        k = rope(rms(qkv[:, c.num_heads * d : (c.num_heads + c.num_kv_heads) * d].view(n, c.num_kv_heads, d),
                     layer.k_norm))
        v = qkv[:, (c.num_heads + c.num_kv_heads) * d :].view(n, c.num_kv_heads, d)
        if new_kv is not None:
            new_kv.append((k, v))
        kf = k_cache[i].view(-1, c.num_kv_heads, d)
        vf = v_cache[i].view(-1, c.num_kv_heads, d)
        out = torch.empty(n, c.num_heads, d, dtype=dtype)
        for b in range(b_count):
            rows = slice(b * s, (b + 1) * s)
            kk = torch.cat([up(kf[ctx_slots[b]]), k[rows]])[:, kv_of]  # [L, H, D]
            vv = torch.cat([up(vf[ctx_slots[b]]), v[rows]])[:, kv_of]
            scores = torch.einsum("nhd,mhd->hnm", q[rows], kk) * d ** -0.5
            length = kk.shape[0]
            mask = torch.arange(length)[None, :] > (torch.arange(s)[:, None] + length - s)
            scores = scores.masked_fill(mask, float("-inf"))
            out[rows] = torch.einsum("hnm,mhd->nhd", scores.softmax(-1), vv)
        x = x + out.reshape(n, -1) @ up(layer.o).T
        h = rms(x, layer.post_norm)
        gu = h @ up(layer.gate_up).T
        gate, upv = gu.chunk(2, dim=-1)
        x = x + (F.silu(gate) * upv) @ up(layer.down).T
    hidden = rms(x, weights.final_norm)
    if not with_logits:
        return hidden
    head = weights.lm_head
    logits = torch.cat([hidden @ up(head[r : r + 16384]).T for r in range(0, head.shape[0], 16384)], dim=1)
    return hidden, logits
