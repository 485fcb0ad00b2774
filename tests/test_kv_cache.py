"""Host side of the paged KV cache (kv_cache.py, the drop-in for oxr_runtime/kv_cache.py).

- ``pack_page_table`` against the reference's own cases (tests/test_kv_cache.py:13-41): the
  known answer for three sequences of 2, 0 and 3 pages, and a thousand random sequences against a
  row-by-row fill.
- ``blocks_for`` / ``slot_of`` against their closed forms.
- ``KVCache``: the reference's constructor call, the page arithmetic of ``bytes_per_block``,
  all-or-nothing ``allocate``, pages coming back through ``release``, and no page handed out
  twice when several threads allocate at once.  CPU tensors: the cache is bookkeeping here.
"""

from __future__ import annotations

import threading

import numpy as np
import pytest
import torch

from conftest import pkg

kv_cache = pkg("kv_cache")
language = pkg("language")


def test_pack_page_table_rows_and_padding() -> None:
    """tests/test_kv_cache.py:13-26: rows start with each sequence's pages in order; every other
    cell, the row without a sequence included, is the fill value; old contents do not survive."""
    out = np.full((4, 5), -7, dtype=np.int32)
    kv_cache.pack_page_table(out, [[3, 8], [], [5, 1, 4]], fill=99)
    assert out.tolist() == [
        [3, 8, 99, 99, 99],
        [99, 99, 99, 99, 99],
        [5, 1, 4, 99, 99],
        [99, 99, 99, 99, 99],
    ]


def test_pack_page_table_matches_row_by_row() -> None:
    """tests/test_kv_cache.py:29-41: a thousand sequences of 0-6 random pages."""
    rng = np.random.default_rng(0)
    tables = [rng.integers(0, 5000, size=rng.integers(0, 7)).tolist() for _ in range(1000)]
    expected = np.full((1024, 8), 7, dtype=np.int32)
    for i, pages in enumerate(tables):
        expected[i, : len(pages)] = pages
    out = np.zeros((1024, 8), dtype=np.int32)
    kv_cache.pack_page_table(out, tables, fill=7)
    assert np.array_equal(out, expected)


def test_pack_page_table_no_sequences() -> None:
    out = np.zeros((3, 4), dtype=np.int32)
    kv_cache.pack_page_table(out, [], fill=5)
    assert (out == 5).all()
    kv_cache.pack_page_table(out, [[], []], fill=6)
    assert (out == 6).all()


@pytest.mark.parametrize("block_size", [16, 256])
def test_blocks_for_and_slot_of(block_size) -> None:
    for tokens in (0, 1, block_size - 1, block_size, block_size + 1, 10 * block_size + 3):
        assert kv_cache.blocks_for(tokens, block_size) == (tokens + block_size - 1) // block_size
    blocks = [7, 2, 9]
    for pos in range(3 * block_size):
        assert kv_cache.slot_of(blocks, pos, block_size) == blocks[pos // block_size] * block_size + pos % block_size
    assert kv_cache.blocks_for(257) == 2  # the reference's default page of 256 tokens


def test_reference_constructor_and_page_bytes() -> None:
    c = language.LanguageConfig(512, 768, 3, 4, 2, 128, 1e-6, 1e6, 1000)
    cache = kv_cache.KVCache(c, 5, dtype=torch.bfloat16, device="cpu")
    assert cache.k.shape == cache.v.shape == (3, 5, 256, 2, 128)
    assert cache.block_size == 256 and cache.num_blocks == 5 and cache.free_blocks == 5
    per_block = 2 * 3 * 256 * 2 * 128 * 2
    assert kv_cache.KVCache.bytes_per_block(c, torch.bfloat16) == per_block
    assert kv_cache.KVCache.bytes_per_block(3, 2, 128, torch.float32) == 2 * per_block
    same = kv_cache.KVCache(3, 2, 128, 5, device="cpu", block_size=16, fill=0.5)
    assert same.k.shape == (3, 5, 16, 2, 128) and bool((same.v == 0.5).all())
    with pytest.raises(TypeError):
        kv_cache.KVCache(3, 2, device="cpu")


def test_allocate_is_all_or_nothing_and_release_returns_pages() -> None:
    cache = kv_cache.KVCache(1, 1, 128, 6, device="cpu", block_size=16)
    a = cache.allocate(4)
    assert a == [0, 1, 2, 3] and cache.free_blocks == 2
    assert cache.allocate(3) is None and cache.free_blocks == 2  # nothing taken
    b = cache.allocate(2)
    assert sorted(a + b) == list(range(6)) and cache.allocate(1) is None
    cache.release(a[1:3])
    assert cache.free_blocks == 2
    assert sorted(cache.allocate(2)) == sorted(a[1:3])


def test_concurrent_allocation_hands_out_each_page_once() -> None:
    cache = kv_cache.KVCache(1, 1, 128, 4000, device="cpu", block_size=16)
    got: list[list[int]] = []
    lock = threading.Lock()

    def worker(seed: int) -> None:
        rng = np.random.default_rng(seed)
        mine = []
        for _ in range(200):
            pages = cache.allocate(int(rng.integers(1, 4)))
            if pages is None:
                break
            mine.extend(pages)
            if rng.random() < 0.3:
                cache.release([mine.pop()])
        with lock:
            got.append(mine)

    threads = [threading.Thread(target=worker, args=(s,)) for s in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    held = [p for mine in got for p in mine]
    assert len(held) == len(set(held)), "a page was handed out twice"
    assert cache.free_blocks + len(held) == 4000
