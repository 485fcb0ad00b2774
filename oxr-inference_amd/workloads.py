"""Seeded synthetic inputs for the verify-step configurations (numpy, host side).

Shapes and distributions follow the five workloads the benchmarks and parity tests use:

1. drafting + acceptance: B=4 int32 histories of 512 ids from a 151,936-id vocabulary,
   ~70% of positions overwritten by repeated fragments (period 8-24, 2-5 repeats), fp32
   verify logits [4, 4, V] ~N(0, 1) with each draft token planted as the row argmax with
   probability 0.6;
2. fused q/k norm + RoPE + KV write: 32 sequences x 4 tokens, 16/8 heads, D=128, contexts
   U{256..4096}, block size 16, block tables from a permutation of 65,536 blocks;
3. paged verify attention: B=8, S=4, contexts U{2048..8192}, same pool;
4. LM head + acceptance: hidden [256, 2048] ~N(0, 1), weight [151936, 2048] ~N(0, 0.02);
5. the full verify step of a random-init 28-layer decoder.

Nothing here computes a result; it only builds inputs.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

VOCAB = 151_936


def repetitive_history(
    rng: np.random.Generator, length: int, vocab: int = VOCAB, *, fill: float = 0.7,
    period: tuple[int, int] = (8, 24), repeats: tuple[int, int] = (2, 5), repetitive_tail: bool = False,
) -> np.ndarray:
    """Uniform random ids with at least ``fill`` of the positions overwritten by repeated fragments."""
    h = rng.integers(0, vocab, size=length, dtype=np.int64)
    covered = np.zeros(length, dtype=bool)
    while covered.mean() < fill:
        p = int(rng.integers(period[0], period[1] + 1))
        r = int(rng.integers(repeats[0], repeats[1] + 1))
        span = min(p * r, length)
        start = int(rng.integers(0, length - span + 1))
        h[start : start + span] = np.tile(rng.integers(0, vocab, size=p), r)[:span]
        covered[start : start + span] = True
    if repetitive_tail:
        p = int(rng.integers(period[0], period[1] + 1))
        span = min(p * int(rng.integers(repeats[0], repeats[1] + 1)), length)
        h[length - span :] = np.tile(rng.integers(0, vocab, size=p), span // p + 1)[:span]
    return h.astype(np.int32)


def unmatched_history(rng: np.random.Generator, length: int, vocab: int = VOCAB) -> np.ndarray:
    """All-distinct ids: the last id never occurred before, so no n-gram matches."""
    return rng.permutation(vocab)[:length].astype(np.int32)


@dataclass
class DraftingWorkload:
    histories: np.ndarray  # int32 [B, L]
    logits: np.ndarray     # float32 [B, S, V], planted after drafting
    k: int
    max_n: int


def drafting_histories(seed: int = 0, batch: int = 4, length: int = 512, vocab: int = VOCAB) -> np.ndarray:
    """Workload 1's histories: sequence 0 has a repetitive tail, the last one matches nothing."""
    rng = np.random.default_rng(seed)
    rows = []
    for b in range(batch):
        if b == batch - 1 and batch > 1:
            rows.append(unmatched_history(rng, length, vocab))
        else:
            rows.append(repetitive_history(rng, length, vocab, repetitive_tail=(b == 0)))
    return np.stack(rows)


def plant_logits(
    rng: np.random.Generator, draft: np.ndarray, draft_len: np.ndarray, tokens_per_seq: int,
    vocab: int = VOCAB, p: float = 0.6,
) -> np.ndarray:
    """fp32 [B, S, V] ~N(0, 1); for j < draft_len[b], with probability p the draft id is made the
    row's strict maximum (row max + 1)."""
    b = draft.shape[0]
    logits = rng.standard_normal((b, tokens_per_seq, vocab), dtype=np.float32)
    for i in range(b):
        for j in range(int(draft_len[i])):
            if rng.random() < p:
                logits[i, j, draft[i, j]] = logits[i, j].max() + 1.0
    return logits


@dataclass
class PagedBatch:
    seq_lens: np.ndarray     # int32 [B], includes the S new tokens
    block_table: np.ndarray  # int32 [B, W]
    slots: np.ndarray        # int64 [B * S], slots of the S new tokens
    positions: np.ndarray    # int64 [B * S]
    num_blocks: int
    block_size: int


def paged_batch(
    rng: np.random.Generator, batch: int, tokens_per_seq: int, ctx_range: tuple[int, int], *,
    block_size: int = 16, num_blocks: int = 65_536, table_width: int | None = None,
) -> PagedBatch:
    """Context lengths U{lo..hi} (each includes the S new tokens at its end); every sequence gets
    disjoint pages drawn from one random permutation of the pool."""
    lo, hi = ctx_range
    seq_lens = rng.integers(lo, hi + 1, size=batch).astype(np.int32)
    blocks_needed = (seq_lens + block_size - 1) // block_size
    if table_width is None:
        table_width = int(blocks_needed.max())
    if int(blocks_needed.sum()) > num_blocks:
        raise ValueError("pool too small for the batch")
    perm = rng.permutation(num_blocks).astype(np.int32)
    table = np.zeros((batch, table_width), dtype=np.int32)
    offset = 0
    for b in range(batch):
        n = int(blocks_needed[b])
        table[b, :n] = perm[offset : offset + n]
        offset += n
    positions = np.concatenate([np.arange(L - tokens_per_seq, L) for L in seq_lens]).astype(np.int64)
    rows = np.repeat(np.arange(batch), tokens_per_seq)
    slots = table[rows, positions // block_size].astype(np.int64) * block_size + positions % block_size
    return PagedBatch(seq_lens, table, slots, positions, num_blocks, block_size)
