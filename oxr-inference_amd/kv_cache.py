"""Paged KV cache with a runtime block size: the drop-in for oxr_runtime/kv_cache.py.

The layout is the reference's (kv_cache.py:27): per K and V one tensor
``[layers, blocks, block_size, KV, D]``, one page table shared by all layers, a thread-safe
free list.  The reference fixes ``BLOCK_SIZE = 256`` (flash-attn's paging granularity); the
gfx950 attention kernel takes any power-of-two page size, so it is a constructor argument
here (the verify benchmark uses 16).
"""

from __future__ import annotations

import threading

import numpy as np
import torch

BLOCK_SIZE = 256  # kv_cache.py:19 default


def _shape_args(first, rest: tuple, what: str) -> tuple[int, int, int, tuple]:
    """(layers, kv heads, head dim, remaining args) from either call form: the reference's
    ``(config, ...)`` or explicit ``(num_layers, num_kv_heads, head_dim, ...)``."""
    if hasattr(first, "num_kv_heads"):
        return first.num_layers, first.num_kv_heads, first.head_dim, rest
    if len(rest) < 2:
        raise TypeError(f"{what}: pass a config, or num_layers, num_kv_heads and head_dim")
    return int(first), int(rest[0]), int(rest[1]), rest[2:]


class KVCache:
    """Pages of ``block_size`` tokens; ``allocate``/``release`` may be called from several threads.

    ``KVCache(config, num_blocks, *, dtype, device)`` is the reference's call (kv_cache.py:26-32);
    ``KVCache(num_layers, num_kv_heads, head_dim, num_blocks, ...)`` names the shape directly.
    ``block_size`` (default 256, the reference's) and ``fill`` (initial contents; default
    uninitialised) are keywords of both."""

    def __init__(self, config_or_layers, *args, dtype: torch.dtype = torch.bfloat16,
                 device: torch.device | str = "cuda", block_size: int = BLOCK_SIZE, fill: float | None = None):
        num_layers, num_kv_heads, head_dim, rest = _shape_args(config_or_layers, args, "KVCache")
        if len(rest) != 1:
            raise TypeError("KVCache: num_blocks is required (and the only other positional argument)")
        num_blocks = int(rest[0])
        shape = (num_layers, num_blocks, block_size, num_kv_heads, head_dim)
        make = torch.empty if fill is None else (lambda s, **kw: torch.full(s, fill, **kw))
        self.k = make(shape, dtype=dtype, device=device)
        self.v = make(shape, dtype=dtype, device=device)
        self.num_blocks = num_blocks
        self.block_size = block_size
        self._free = list(range(num_blocks - 1, -1, -1))
        self._lock = threading.Lock()

    @staticmethod
    def bytes_per_block(config_or_layers, *args, dtype: torch.dtype | None = None,
                        block_size: int = BLOCK_SIZE) -> int:
        """K + V bytes of one page over all layers: ``bytes_per_block(config, dtype)`` as in the
        reference (kv_cache.py:34-37), or ``bytes_per_block(num_layers, num_kv_heads, head_dim[, dtype])``."""
        num_layers, num_kv_heads, head_dim, rest = _shape_args(config_or_layers, args, "bytes_per_block")
        if rest:
            dtype = rest[0]
        element = torch.empty((), dtype=dtype or torch.bfloat16).element_size()
        return 2 * num_layers * block_size * num_kv_heads * head_dim * element

    @property
    def free_blocks(self) -> int:
        return len(self._free)

    def allocate(self, count: int) -> list[int] | None:
        """``count`` pages, or None (and nothing taken) when fewer are free."""
        with self._lock:
            if count > len(self._free):
                return None
            return [self._free.pop() for _ in range(count)]

    def release(self, blocks: list[int]) -> None:
        with self._lock:
            self._free.extend(reversed(blocks))


def blocks_for(tokens: int, block_size: int = BLOCK_SIZE) -> int:
    """Pages needed for ``tokens`` tokens (kv_cache.py:55-57)."""
    return -(-tokens // block_size)


def slot_of(blocks: list[int], position: int, block_size: int = BLOCK_SIZE) -> int:
    """Flat cache row of token ``position`` (language.py:320-322)."""
    page, offset = divmod(position, block_size)
    return blocks[page] * block_size + offset


def pack_page_table(out: np.ndarray, tables: list[list[int]], fill: int) -> None:
    """Write each sequence's pages at the start of its row of ``out`` and ``fill`` everywhere else,
    including rows past ``len(tables)`` (kv_cache.py:60-72), in one vectorised scatter."""
    out.fill(fill)
    if not tables:
        return
    lengths = np.array([len(t) for t in tables], dtype=np.int64)
    total = int(lengths.sum())
    if total == 0:
        return
    flat = np.fromiter((p for t in tables for p in t), dtype=out.dtype, count=total)
    starts = np.concatenate(([0], np.cumsum(lengths)[:-1]))
    row = np.repeat(np.arange(len(tables)), lengths)
    col = np.arange(total) - np.repeat(starts, lengths)
    out[row, col] = flat
