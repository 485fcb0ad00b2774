"""The one-token decode step (decode_graph.py:33-119, attention.py:76-93) on the gfx950 kernels.

- ``attention.paged_decode`` (the drop-in for attention.py:76-93) against the oracle's attention
  with one query per sequence, including contexts shorter than one key tile and block size 256.
- The reference's decode test (tests/test_language_fused.py:144-160): prefill a few tokens per
  sequence, then decode one more; the decode result equals a causal forward over the whole
  sequence (the oracle), within the tolerance of the end-to-end forward.
- ``DecodeGraphs`` (decode_graph.py:33-119): graph replay gives exactly the eager decode's logits
  and ids, padded bucket rows touch only the scratch page, and batches past the largest bucket
  return None; up to the engine's 256 running sequences (engine.py:111).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, pkg
from oracle import attention as oracle_attention
from oracle import decoder as oracle_decoder

pytestmark = pytest.mark.gpu
attention = pkg("attention")
language = pkg("language")
kv_cache = pkg("kv_cache")
decode_graph = pkg("decode_graph")
lm_head = pkg("lm_head")

ATOL, RTOL = 2e-2, 1e-2
SMALL = language.LanguageConfig(512, 768, 2, 4, 2, 128, 1e-6, 1e6, 1000)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("seq_lens,block_size", [([1, 7, 16, 33, 300, 2049, 4100, 5], 16), ([1, 257, 900], 256),
                                                 (np.random.default_rng(256).integers(1, 2000, size=256).tolist(), 16)])
def test_paged_decode_matches_oracle(seq_lens, block_size) -> None:
    rng = np.random.default_rng(len(seq_lens))
    B, H, KV = len(seq_lens), 16, 8
    lens = np.asarray(seq_lens, dtype=np.int32)
    need = (lens + block_size - 1) // block_size
    num_blocks = int(need.sum()) + 4
    perm = rng.permutation(num_blocks).astype(np.int32)
    table = np.zeros((B, int(need.max())), dtype=np.int32)
    off = 0
    for b in range(B):
        table[b, : need[b]] = perm[off : off + need[b]]
        off += need[b]
    g = torch.Generator(device="cuda").manual_seed(int(lens.sum()))
    kc = torch.randn(num_blocks, block_size, KV, 128, generator=g, device="cuda").to(torch.bfloat16)
    vc = torch.randn(num_blocks, block_size, KV, 128, generator=g, device="cuda").to(torch.bfloat16)
    q = torch.randn(B, H, 128, generator=g, device="cuda").to(torch.bfloat16)
    announce("paged_decode", seq_lens, block_size)
    out = attention.paged_decode(q, kc, vc, torch.from_numpy(lens).cuda(), torch.from_numpy(table).cuda())
    torch.cuda.synchronize()
    assert out.shape == (B, H, 128)
    k_rows, v_rows = [], []
    for b in range(B):
        blocks = torch.from_numpy(table[b, : need[b]].astype(np.int64)).cuda()
        k_rows.append(_bits(kc[blocks].flatten(0, 1)[: lens[b]]))
        v_rows.append(_bits(vc[blocks].flatten(0, 1)[: lens[b]]))
    exact, _ = oracle_attention.paged_extend(_bits(q.view(B, 1, H, 128)), k_rows, v_rows, 128 ** -0.5)
    got = out.float().cpu().numpy()
    err = np.abs(got - exact.reshape(B, H, 128))
    assert (err <= ATOL + RTOL * np.abs(exact.reshape(B, H, 128))).all(), err.max()


def _model(seed=0):
    w = language.random_weights(SMALL, 1024, seed=seed, std=0.05)
    return language.LanguageModel(SMALL, w), w.to("cpu")


def test_decode_after_prefill_equals_full_sequence() -> None:
    """tests/test_language_fused.py:144-160 on this path: two sequences prefilled with 5 and 3
    tokens (one extend each), then one decode step for both, against one causal forward over each
    whole sequence."""
    model, cpu_w = _model(seed=21)
    rng = np.random.default_rng(21)
    bs, num_blocks = 16, 8
    cache = kv_cache.KVCache(SMALL.num_layers, SMALL.num_kv_heads, SMALL.head_dim, num_blocks, block_size=bs, fill=0.0)
    table = np.array([[2, 0], [5, 7]], dtype=np.int32)
    lens = [5, 3]
    toks = [rng.integers(0, SMALL.vocab_size, size=n + 1) for n in lens]
    d = lambda a, dt: torch.from_numpy(np.asarray(a)).to(dt).cuda()
    slot = lambda b, p: int(table[b, p // bs]) * bs + p % bs
    announce("prefill then decode")
    for b, n in enumerate(lens):  # prefill sequence b alone: an extend of n tokens at positions 0..n-1
        eb = language.ExtendBatch(None, d(np.arange(n), torch.int64),
                                  d([slot(b, p) for p in range(n)], torch.int64), d([n], torch.int32),
                                  d(table[b : b + 1], torch.int32), n, ids=d(toks[b][:n], torch.int64))
        model.extend(eb, cache)
    db = language.DecodeBatch(None, d(lens, torch.int64),
                              d([slot(b, n) for b, n in enumerate(lens)], torch.int64),
                              d([n + 1 for n in lens], torch.int32), d(table, torch.int32),
                              ids=d([t[-1] for t in toks], torch.int64))
    hidden = model.decode(db, cache)
    torch.cuda.synchronize()
    for b, n in enumerate(lens):
        ck = torch.zeros(SMALL.num_layers, num_blocks, bs, SMALL.num_kv_heads, SMALL.head_dim, dtype=torch.bfloat16)
        cv = torch.zeros_like(ck)
        full = oracle_decoder.extend(
            SMALL, cpu_w, torch.from_numpy(toks[b]), torch.arange(n + 1),
            torch.tensor([slot(b, p) for p in range(n + 1)]), torch.tensor([n + 1], dtype=torch.int32),
            torch.from_numpy(table[b : b + 1]), n + 1, ck, cv)
        want = full[-1].float()
        err = (hidden[b].float().cpu() - want).abs()
        assert bool((err <= (SMALL.num_layers + 1) * (ATOL + RTOL * want.abs())).all()), err.max().item()
        assert (err.pow(2).sum() / want.pow(2).sum()).sqrt().item() < 2e-2


@pytest.mark.parametrize("max_batch,n,buckets", [(6, 3, [1, 2, 4, 6]),
                                                  (256, 200, [1, 2, 4, 8, 16, 32, 64, 128, 192, 256])])
def test_decode_graphs_match_eager_and_keep_padding_on_scratch(max_batch, n, buckets) -> None:
    """n sequences replayed in the next bucket up (3 in the bucket of 4; 200 of the engine's up to
    256 running sequences, engine.py:111, in the bucket of 256, 200 token rows through the
    GEMMs)."""
    model, _ = _model(seed=22)
    rng = np.random.default_rng(22)
    bs, width = 16, 8
    num_blocks = 8 * n + 16
    cache = kv_cache.KVCache(SMALL.num_layers, SMALL.num_kv_heads, SMALL.head_dim, num_blocks, block_size=bs)
    g = torch.Generator(device="cuda").manual_seed(22)
    cache.k.copy_(torch.randn(cache.k.shape, generator=g, device="cuda").to(torch.bfloat16))
    cache.v.copy_(torch.randn(cache.v.shape, generator=g, device="cuda").to(torch.bfloat16))
    announce("DecodeGraphs", max_batch, n)
    graphs = decode_graph.DecodeGraphs(model, cache, max_batch=max_batch, max_positions=width * bs)
    assert graphs.buckets == buckets
    pages = [p for p in range(num_blocks) if p != graphs.scratch_block]
    lens = rng.integers(20, width * bs - 1, size=n)
    tables = [pages[8 * b : 8 * b + int(-(-(lens[b] + 1) // bs))] for b in range(n)]
    ids = rng.integers(0, SMALL.vocab_size, size=n).tolist()
    positions = lens.tolist()
    slots = [tables[b][positions[b] // bs] * bs + positions[b] % bs for b in range(n)]
    seq_lens = (lens + 1).tolist()
    before_k, before_v = cache.k.clone(), cache.v.clone()

    logits, tokens = graphs.run(ids, positions, slots, seq_lens, tables)
    logits, tokens = logits.clone(), tokens.clone()
    torch.cuda.synchronize()
    after_k, after_v = cache.k.clone(), cache.v.clone()

    # Only the real rows' slots and the scratch page's first slot were written.
    written = torch.zeros(num_blocks * bs, dtype=torch.bool)
    written[torch.tensor(slots)] = True
    written[graphs.scratch_block * bs] = True
    for before, after in ((before_k, after_k), (before_v, after_v)):
        changed = (before != after).flatten(0, 0).view(SMALL.num_layers, num_blocks * bs, -1).any(-1).any(0).cpu()
        assert not bool((changed & ~written).any())

    # Eager decode from the same cache state gives the same bits.
    cache.k.copy_(before_k)
    cache.v.copy_(before_v)
    d = lambda a, dt: torch.tensor(a, dtype=dt, device="cuda")
    table_t = torch.full((n, width), graphs.scratch_block, dtype=torch.int32, device="cuda")
    for b in range(n):
        table_t[b, : len(tables[b])] = torch.tensor(tables[b], dtype=torch.int32)
    hidden = model.decode(language.DecodeBatch(None, d(positions, torch.int64), d(slots, torch.int64),
                                               d(seq_lens, torch.int32), table_t, ids=d(ids, torch.int64)), cache)
    want_tokens, want_logits = lm_head.lm_head_argmax(hidden, model.weights.lm_head, return_logits=True)
    torch.cuda.synchronize()
    assert torch.equal(tokens, want_tokens)
    assert torch.equal(logits.view(torch.int16), want_logits.view(torch.int16))
    assert torch.equal(cache.k, after_k) and torch.equal(cache.v, after_v)

    big = max_batch + 1
    assert graphs.run([0] * big, [0] * big, [0] * big, [1] * big, [[0]] * big) is None  # past the largest bucket


def test_decode_graphs_reject_batches_past_the_kernels() -> None:
    model, _ = _model(seed=23)
    cache = kv_cache.KVCache(SMALL.num_layers, SMALL.num_kv_heads, SMALL.head_dim, 4, block_size=16)
    with pytest.raises(ValueError):
        decode_graph.DecodeGraphs(model, cache, max_batch=257, max_positions=64)
