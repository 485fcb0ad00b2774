"""Seeded inputs of the decoder golden cases (``decoder_extend.npz``).

Shared by ``make_golden_decoder.py``, which runs the reference's ``LanguageModel.extend`` on them
in the build container, and by ``tests/test_oracle_decoder.py``, which runs the oracle on the
same inputs.  Everything is drawn from ``numpy.random.default_rng(seed)`` in float32 and rounded
to bf16 once; a SHA-256 of the rounded bits is stored with the vectors, so a generator that drew
different numbers fails loudly instead of comparing other inputs.

Names follow the reference's parameter names (oxr_runtime/language.py:149-158, 221-231, with
the unfused q/k/v and gate/up projections that ``fuse_projections``, language.py:234-245,
concatenates).  The KV block size is the reference's fixed 256 (kv_cache.py:19).
"""

from __future__ import annotations

import hashlib
from types import SimpleNamespace

import numpy as np
import torch

BLOCK_SIZE = 256

# batch B sequences of S new tokens each; seq_lens include the S tokens (engine.py:710).
CASES = {
    # GQA 4/2, two pages per sequence at most, contexts straddling a page boundary.
    "gqa4_s4": dict(hidden=256, intermediate=384, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=384,
                    tokens_per_seq=4, seq_lens=(300, 517), num_blocks=8, max_positions=1024, seed=11),
    # The reference's default verify width (1 + speculative_tokens = 9, engine.py:121) at the
    # benchmark's 16/8 heads; one sequence holds only its 9 new tokens.
    "gqa16_s9": dict(hidden=512, intermediate=768, layers=2, heads=16, kv_heads=8, head_dim=128, vocab=1000,
                     tokens_per_seq=9, seq_lens=(9, 270, 700), num_blocks=10, max_positions=1024, seed=12),
}


def config(case: dict) -> SimpleNamespace:
    """The shapes of ``LanguageConfig`` (config.py:38-50)."""
    return SimpleNamespace(hidden_size=case["hidden"], intermediate_size=case["intermediate"],
                           num_layers=case["layers"], num_heads=case["heads"], num_kv_heads=case["kv_heads"],
                           head_dim=case["head_dim"], rms_norm_eps=1e-6, rope_theta=1e6, vocab_size=case["vocab"])


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)


def parameters(case: dict) -> dict[str, torch.Tensor]:
    """bf16 parameters by reference name (unfused projections), in a fixed order."""
    c = config(case)
    rng = np.random.default_rng(case["seed"])
    h, d, i = c.hidden_size, c.head_dim, c.intermediate_size
    mat = lambda rows, cols, std: _bf16(rng.standard_normal((rows, cols), dtype=np.float32) * std)
    norm = lambda n: _bf16(1.0 + 0.1 * rng.standard_normal(n, dtype=np.float32))
    p = {"embed_tokens.weight": mat(c.vocab_size, h, 1.0)}
    for layer in range(c.num_layers):
        pre = f"layers.{layer}."
        p[pre + "input_layernorm.weight"] = norm(h)
        p[pre + "q_proj.weight"] = mat(c.num_heads * d, h, h ** -0.5)
        p[pre + "k_proj.weight"] = mat(c.num_kv_heads * d, h, h ** -0.5)
        p[pre + "v_proj.weight"] = mat(c.num_kv_heads * d, h, h ** -0.5)
        p[pre + "q_norm.weight"] = norm(d)
        p[pre + "k_norm.weight"] = norm(d)
        p[pre + "o_proj.weight"] = mat(h, c.num_heads * d, (c.num_heads * d) ** -0.5)
        p[pre + "post_attention_layernorm.weight"] = norm(h)
        p[pre + "gate_proj.weight"] = mat(i, h, h ** -0.5)
        p[pre + "up_proj.weight"] = mat(i, h, h ** -0.5)
        p[pre + "down_proj.weight"] = mat(h, i, i ** -0.5)
    p["norm.weight"] = norm(h)
    p["lm_head.weight"] = mat(c.vocab_size, h, h ** -0.5)
    return p


def step_inputs(case: dict) -> dict[str, np.ndarray]:
    """Block table, token ids, positions, slots, seq_lens and the pre-filled caches of the step."""
    c = config(case)
    rng = np.random.default_rng(case["seed"] + 1000)
    s, seq_lens = case["tokens_per_seq"], np.asarray(case["seq_lens"], dtype=np.int32)
    b = len(seq_lens)
    pages = -(-seq_lens // BLOCK_SIZE)
    width = int(pages.max())
    perm = rng.permutation(case["num_blocks"]).astype(np.int32)
    table = np.zeros((b, width), dtype=np.int32)
    offset = 0
    for i in range(b):
        table[i, : pages[i]] = perm[offset : offset + pages[i]]
        offset += int(pages[i])
    positions = np.concatenate([np.arange(n - s, n) for n in seq_lens]).astype(np.int64)
    rows = np.repeat(np.arange(b), s)
    slots = (table[rows, positions // BLOCK_SIZE].astype(np.int64) * BLOCK_SIZE + positions % BLOCK_SIZE)
    ids = rng.integers(0, c.vocab_size, size=b * s).astype(np.int64)
    shape = (c.num_layers, case["num_blocks"], BLOCK_SIZE, c.num_kv_heads, c.head_dim)
    k_cache = rng.standard_normal(shape, dtype=np.float32)
    v_cache = rng.standard_normal(shape, dtype=np.float32)
    return dict(table=table, positions=positions, slots=slots, ids=ids, seq_lens=seq_lens, k_cache=k_cache,
                v_cache=v_cache)


def caches(inputs: dict[str, np.ndarray]) -> tuple[torch.Tensor, torch.Tensor]:
    return _bf16(inputs["k_cache"]), _bf16(inputs["v_cache"])


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def checksum(params: dict[str, torch.Tensor], k_cache: torch.Tensor, v_cache: torch.Tensor) -> str:
    """SHA-256 over every parameter's and both caches' bf16 bits, in order."""
    digest = hashlib.sha256()
    for name, t in params.items():
        digest.update(name.encode())
        digest.update(bits(t).tobytes())
    digest.update(bits(k_cache).tobytes())
    digest.update(bits(v_cache).tobytes())
    return digest.hexdigest()
