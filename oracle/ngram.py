"""n-gram drafting and greedy acceptance on the CPU (test infrastructure only).

Follows oxr_runtime/speculative.py:12-48 of the reference.

Two independent restatements of ``NgramProposer.propose`` are kept so that each
checks the other (tests/test_oracle_ngram.py):

- ``NgramIndex``: the reference's own data structure, a dict from every n-gram
  (n = 1..max_n) that ends just before position p to the latest such p
  (speculative.py:15-31), looked up longest-suffix first (speculative.py:33-39).
- ``propose_closed_form``: brute force over candidates p in [1, L-1]: m(p) is
  the number of tokens before p that match the history's suffix (capped at
  min(max_n, p)); the answer maximises (m(p), p).
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np

MAX_N = 4  # speculative.py:12


class NgramIndex:
    """speculative.py:15-39 with the n-gram cap as a parameter."""

    def __init__(self, tokens: Sequence[int], max_n: int = MAX_N):
        self.max_n = max_n
        self._index: dict[tuple[int, ...], int] = {}
        for position in range(1, len(tokens)):
            self._add(tokens, position)

    def _add(self, tokens: Sequence[int], position: int) -> None:
        for n in range(1, min(self.max_n, position) + 1):
            self._index[tuple(tokens[position - n : position])] = position

    def extend(self, tokens: Sequence[int], old_length: int) -> None:
        for position in range(max(old_length, 1), len(tokens)):
            self._add(tokens, position)

    def propose(self, tokens: Sequence[int], k: int) -> list[int]:
        for n in range(min(self.max_n, len(tokens)), 0, -1):
            start = self._index.get(tuple(tokens[-n:]))
            if start is not None:
                return list(tokens[start : start + k])
        return []


def propose_closed_form(tokens: Sequence[int], k: int, max_n: int = MAX_N, index_len: int | None = None) -> list[int]:
    """Largest (m(p), p) over candidates p in [1, min(L, index_len) - 1]."""
    h = np.asarray(tokens, dtype=np.int64)
    length = len(h)
    nmax = min(max_n, length)
    last = length - 1 if index_len is None else min(length, index_len) - 1
    best_m, best_p = 0, -1
    for p in range(last, 0, -1):
        m = 0
        while m < min(nmax, p) and h[p - 1 - m] == h[length - 1 - m]:
            m += 1
        if m > best_m:
            best_m, best_p = m, p
            if m == nmax:
                break
    if best_m == 0:
        return []
    return [int(t) for t in h[best_p : best_p + k]]


def accept(draft: Sequence[int], predicted: Sequence[int]) -> list[int]:
    """speculative.py:42-48: longest matching prefix of ``draft`` plus the model's next token."""
    accepted = 0
    while accepted < len(draft) and draft[accepted] == predicted[accepted]:
        accepted += 1
    return list(draft[:accepted]) + [predicted[accepted]]


def propose_batch(
    histories: Sequence[Sequence[int]], k: int, max_n: int = MAX_N, k_limit: Sequence[int] | None = None
) -> tuple[np.ndarray, np.ndarray]:
    """Drafts for a batch, padded: (draft int32 [B, k] zero-filled, draft_len int32 [B]).

    The per-sequence cap mirrors engine.py:683-684, ``propose(output, min(k, max(room, 0)))``."""
    b = len(histories)
    draft = np.zeros((b, k), dtype=np.int32)
    lens = np.zeros(b, dtype=np.int32)
    for i, tokens in enumerate(histories):
        kb = k if k_limit is None else max(0, min(k, int(k_limit[i])))
        d = NgramIndex(tokens, max_n).propose(list(tokens), kb)
        draft[i, : len(d)] = d
        lens[i] = len(d)
    return draft, lens
