"""gfx950 paged verify attention vs the oracle (bf16 tolerance: |err| <= 2e-2 + 1e-2 |ref|).

Config 3 of the benchmark (B=8, S=4, 16/8 heads, contexts U{2048..8192}, block 16, block
tables from a permutation of a 65,536-block pool), plus ragged and edge shapes: contexts
shorter than one 32-key step, not multiples of the block or chunk size, block size 256
(the reference's), one kv head per q head, and S=1.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, pkg
from oracle import attention as oracle_attention

pytestmark = pytest.mark.gpu
attention = pkg("attention")
workloads = pkg("workloads")

ATOL, RTOL = 2e-2, 1e-2


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _inputs(seq_lens, S, H, KV, block_size, num_blocks, seed, table_width=None):
    """q, caches, lengths and table on the GPU, and each sequence's visible K/V rows (bits) for the oracle."""
    rng = np.random.default_rng(seed)
    B = len(seq_lens)
    seq_lens = np.asarray(seq_lens, dtype=np.int32)
    need = (seq_lens + block_size - 1) // block_size
    width = table_width or int(need.max())
    perm = rng.permutation(num_blocks).astype(np.int32)
    table = np.full((B, width), -7, dtype=np.int32)
    off = 0
    for b in range(B):
        table[b, : need[b]] = perm[off : off + need[b]]
        off += need[b]
    g = torch.Generator(device="cuda").manual_seed(seed)
    kc = torch.randn(num_blocks, block_size, KV, 128, generator=g, device="cuda").to(torch.bfloat16)
    vc = torch.randn(num_blocks, block_size, KV, 128, generator=g, device="cuda").to(torch.bfloat16)
    q = torch.randn(B, S, H, 128, generator=g, device="cuda").to(torch.bfloat16)
    k_rows, v_rows = [], []
    for b in range(B):
        blocks = torch.from_numpy(table[b, : need[b]].astype(np.int64)).cuda()
        k_rows.append(_bits(kc[blocks].flatten(0, 1)[: seq_lens[b]]))
        v_rows.append(_bits(vc[blocks].flatten(0, 1)[: seq_lens[b]]))
    return q, kc, vc, torch.from_numpy(seq_lens).cuda(), torch.from_numpy(table).cuda(), k_rows, v_rows


def _run(seq_lens, S, H, KV, block_size, num_blocks, seed, table_width=None, max_seq_len=None, planned=False):
    rng = np.random.default_rng(seed)
    B = len(seq_lens)
    seq_lens = np.asarray(seq_lens, dtype=np.int32)
    need = (seq_lens + block_size - 1) // block_size
    width = table_width or int(need.max())
    perm = rng.permutation(num_blocks).astype(np.int32)
    table = np.full((B, width), -7, dtype=np.int32)  # unused entries are garbage on purpose
    off = 0
    for b in range(B):
        table[b, : need[b]] = perm[off : off + need[b]]
        off += need[b]
    g = torch.Generator(device="cuda").manual_seed(seed)
    kc = torch.randn(num_blocks, block_size, KV, 128, generator=g, device="cuda").to(torch.bfloat16)
    vc = torch.randn(num_blocks, block_size, KV, 128, generator=g, device="cuda").to(torch.bfloat16)
    q = torch.randn(B, S, H, 128, generator=g, device="cuda").to(torch.bfloat16)
    table_t = torch.from_numpy(table).cuda()
    lens_t = torch.from_numpy(seq_lens).cuda()
    plan = None
    if planned:
        mx = max_seq_len or width * block_size
        plan = attention.build_plan(lens_t, S, H, KV, mx)
    out = attention.paged_extend(q, kc, vc, lens_t, table_t, max_seq_len=max_seq_len, plan=plan)
    torch.cuda.synchronize()
    k_rows, v_rows = [], []
    for b in range(B):
        blocks = torch.from_numpy(table[b, : need[b]].astype(np.int64)).cuda()
        k_rows.append(_bits(kc[blocks].flatten(0, 1)[: seq_lens[b]]))
        v_rows.append(_bits(vc[blocks].flatten(0, 1)[: seq_lens[b]]))
    exact, _ = oracle_attention.paged_extend(_bits(q), k_rows, v_rows, 128 ** -0.5)
    got = out.float().cpu().numpy()
    err = np.abs(got - exact)
    bound = ATOL + RTOL * np.abs(exact)
    assert (err <= bound).all(), f"max err {err.max():.3g}, worst excess {(err - bound).max():.3g}"
    return err.max()


def test_config3_bit_budget() -> None:
    rng = np.random.default_rng(30)
    seq_lens = rng.integers(2048, 8193, size=8)
    announce("attention config3", seq_lens.tolist())
    err = _run(seq_lens, 4, 16, 8, 16, 65_536, seed=31)
    print("max abs err", err)


@pytest.mark.parametrize("seq_lens", [[4, 5, 17, 31], [32, 33, 255, 256, 257, 300], [1000, 4097, 511, 7]])
def test_ragged_contexts(seq_lens) -> None:
    announce("attention ragged", seq_lens)
    _run(seq_lens, 4, 16, 8, 16, 4096, seed=32)


@pytest.mark.parametrize("planned", [False, True])
@pytest.mark.parametrize("seq_lens", [[5, 33, 16000, 700, 4096, 12000, 64, 2048], [16000, 40], [20000]])
def test_widely_mixed_contexts(seq_lens, planned) -> None:
    """Contexts of very different lengths in one launch, cut into the launch's split count or by a
    plan (long contexts taking the workgroups short ones leave): contexts of one piece, stored
    directly, beside others that are merged; a batch of two with 32 splits each; and one 20,000-key
    context over 64 splits."""
    announce("attention mixed contexts", seq_lens, "planned" if planned else "even")
    _run(seq_lens, 4, 16, 8, 16, 4096, seed=37, planned=planned)


def test_config3_planned() -> None:
    rng = np.random.default_rng(30)
    seq_lens = rng.integers(2048, 8193, size=8)
    announce("attention config3 planned", seq_lens.tolist())
    _run(seq_lens, 4, 16, 8, 16, 65_536, seed=31, planned=True)


@pytest.mark.parametrize("seq_lens,S,H,KV", [
    ([5, 33, 16000, 700, 4096, 12000, 64, 2048], 4, 16, 8),
    ([7800, 3218, 5262, 4413, 7985, 5358, 3562, 2106], 4, 16, 8),
    ([4100] * 8, 4, 16, 8),
    ([100, 30000, 1, 0, 2500, 9999, 17, 4096, 300, 12, 8000, 64, 640, 4097, 33, 1024], 4, 16, 8),
    ([3000, 20], 1, 8, 8),
])
def test_plan_covers_every_piece_once(seq_lens, S, H, KV) -> None:
    """The device-built plan, read back: each context's pieces 0 .. n-1 are taken by exactly one
    workgroup slot (its own first `splits` slots, then spare slots of other sequences), no slot takes
    two, n is at most 2 x splits, the piece table names each piece's slot, and equal contexts give
    the even split."""
    lens = torch.tensor(seq_lens, dtype=torch.int32, device="cuda")
    B = len(seq_lens)
    max_len = max(seq_lens) + 64
    announce("attention plan", seq_lens)
    plan = attention.build_plan(lens, S, H, KV, max_len)
    torch.cuda.synchronize()
    assert plan is not None
    p = plan.cpu().numpy()
    splits = int(p[1])
    assert p[0] == B and splits > 1 and p.size == 2 + B + 3 * B * splits
    pieces = p[2 : 2 + B]
    slots = p[2 + B : 2 + B + B * splits].reshape(B, splits)
    piece_slots = p[2 + B + B * splits :].reshape(B, 2 * splits)
    assert (pieces >= 1).all() and (pieces <= 2 * splits).all()
    taken = {}
    for z in range(B):
        for x in range(splits):
            e = int(slots[z, x])
            if e < 0:
                continue
            b, j = e >> 8, e & 255
            assert (b, j) not in taken, f"piece {(b, j)} taken twice"
            taken[(b, j)] = (z, x)
            if x < pieces[z]:
                assert (b, j) == (z, x)
    assert set(taken) == {(b, j) for b in range(B) for j in range(int(pieces[b]))}
    for b in range(B):  # the merge's view: the slot that holds each piece, -1 past the pieces
        for j in range(2 * splits):
            want = (taken[(b, j)][0] << 8) | taken[(b, j)][1] if j < pieces[b] else -1
            assert piece_slots[b, j] == want, (b, j)
    assert int(pieces.sum()) <= B * splits
    if len(set(seq_lens)) == 1:
        assert (pieces == splits).all() or (pieces == pieces[0]).all()


def test_reference_block_size_256_and_table_slack() -> None:
    announce("attention block 256")
    _run([300, 700, 40], 4, 16, 8, 256, 64, seed=33, table_width=8)


def test_single_token_and_mha() -> None:
    announce("attention S=1, H=KV")
    _run([100, 1, 65], 1, 8, 8, 16, 256, seed=34)
    _run([70, 90], 2, 8, 8, 16, 256, seed=35)


def test_max_seq_len_bounds_chunks() -> None:
    announce("attention max_seq_len")
    _run([600, 1200], 4, 16, 8, 16, 1024, seed=36, table_width=200, max_seq_len=1300)


def test_workspace_sized_for_a_batch_serves_smaller_batches() -> None:
    """One workspace, sized for the largest batch, serves calls of smaller batches (which split
    their contexts further) and different contexts in a row; each output equals the output with a
    fresh workspace of its own, bit for bit."""
    rng = np.random.default_rng(5)
    H, KV, S, bs, num_blocks = 16, 8, 4, 16, 4096
    kc = torch.randn(num_blocks, bs, KV, 128, device="cuda").to(torch.bfloat16)
    vc = torch.randn(num_blocks, bs, KV, 128, device="cuda").to(torch.bfloat16)
    max_len = 4096
    shared = torch.empty(attention.workspace_bytes(16, KV, max_len), dtype=torch.uint8, device="cuda")
    for batch in (8, 3, 16, 1, 8, 16):
        seq = rng.integers(S, max_len, size=batch).astype(np.int32)
        seq[0] = max_len  # the longest context uses every split
        table = rng.integers(0, num_blocks, size=(batch, max_len // bs)).astype(np.int32)
        q = torch.randn(batch, S, H, 128, device="cuda").to(torch.bfloat16)
        seq_t, table_t = torch.from_numpy(seq).cuda(), torch.from_numpy(table).cuda()
        announce("shared workspace", batch)
        got = attention.paged_extend(q, kc, vc, seq_t, table_t, max_seq_len=max_len, workspace=shared)
        fresh = attention.paged_extend(q, kc, vc, seq_t, table_t, max_seq_len=max_len)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), fresh.view(torch.int16)), f"batch {batch}"


def test_reference_default_width_s9() -> None:
    """The reference's default verify width: 1 + speculative_tokens = 9 tokens per sequence
    (engine.py:121, 242-246) at 16/8 heads, so 18 query rows per kv head (two 16-row MFMA tiles),
    config 3's contexts and pool, and the reference's block size 256."""
    rng = np.random.default_rng(37)
    seq_lens = rng.integers(2048, 8193, size=8)
    announce("attention S=9, 16/8 heads", seq_lens.tolist())
    _run(seq_lens, 9, 16, 8, 16, 65_536, seed=37)
    announce("attention S=9, block 256")
    _run([300, 9, 1000, 2600], 9, 16, 8, 256, 64, seed=38)


@pytest.mark.parametrize("S,H,KV", [(16, 16, 8), (12, 8, 8), (5, 32, 8), (16, 16, 16), (2, 16, 8), (3, 16, 8),
                                    (7, 8, 8)])
def test_query_row_tiles(S, H, KV) -> None:
    """Up to 32 query rows per kv head: 16 tokens x 2 heads (both tiles full), 12 x 1, 5 x 4 (20
    rows), 16 tokens of MHA; contexts shorter than S, inside one split, and across splits.  4, 6
    and 7 rows take the split merge in two dim slices (8 and more rows: four; fewer than 4: one)."""
    announce("attention row tiles", S, H, KV)
    _run([S, S + 1, 700, 3000], S, H, KV, 16, 1024, seed=39 + S + H)


def test_plan_for_another_launch_is_ignored() -> None:
    """A plan whose header names another split count (written for a longer max_seq_len) or another
    batch (same split count) is ignored: the launch runs on even pieces, bit-identical to the launch
    without a plan, and reads nothing outside its arrays."""
    # max_seq_len 1024 gives 4 splits (at least 256 keys each); a plan for 4096 has the batch's 8.
    lens = [5, 33, 1000, 700, 1024, 200, 64, 512]
    q, kc, vc, lens_t, table, _, _ = _inputs(lens, 4, 16, 8, 16, 4096, seed=41)
    announce("attention plan of another launch")
    even = attention.paged_extend(q, kc, vc, lens_t, table, max_seq_len=1024)
    other_splits = attention.build_plan(lens_t, 4, 16, 8, 4096)
    own = attention.build_plan(lens_t, 4, 16, 8, 1024)
    torch.cuda.synchronize()
    assert int(other_splits[1]) != int(own[1])
    got = attention.paged_extend(q, kc, vc, lens_t, table, max_seq_len=1024, plan=other_splits)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(got), _bits(even))
    # max_seq_len 512 caps both batches at 2 splits; the plan was written for 16 sequences.
    short = [min(n, 512) for n in lens]
    q, kc, vc, lens_t, table, _, _ = _inputs(short, 4, 16, 8, 16, 4096, seed=42)
    even = attention.paged_extend(q, kc, vc, lens_t, table, max_seq_len=512)
    other_batch = attention.build_plan(torch.cat([lens_t, lens_t.flip(0)]), 4, 16, 8, 512)
    mine = attention.build_plan(lens_t, 4, 16, 8, 512)
    torch.cuda.synchronize()
    assert int(other_batch[0]) == 16 and int(other_batch[1]) == int(mine[1])
    got = attention.paged_extend(q, kc, vc, lens_t, table, max_seq_len=512, plan=other_batch)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(got), _bits(even))


def test_plan_from_shorter_lengths_gives_nan_rows() -> None:
    """A plan written from shorter contexts than the launch's (same batch and split count): the
    sequence whose planned pieces cannot reach its last key gets NaN rows instead of silently
    dropped keys; sequences the plan still covers match the oracle."""
    built_for = [20] * 8  # one piece each: the 4000-key context cannot fit one even piece
    lens = [100] * 7 + [4000]
    q, kc, vc, lens_t, table, k_rows, v_rows = _inputs(lens, 4, 16, 8, 16, 4096, seed=43, table_width=256)
    announce("attention stale plan")
    plan = attention.build_plan(torch.tensor(built_for, dtype=torch.int32, device="cuda"), 4, 16, 8, 4096)
    out = attention.paged_extend(q, kc, vc, lens_t, table, max_seq_len=4096, plan=plan)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isnan(got[7]).all()
    exact, _ = oracle_attention.paged_extend(_bits(q[:7]), k_rows[:7], v_rows[:7], 128 ** -0.5)
    err = np.abs(got[:7] - exact)
    assert (err <= ATOL + RTOL * np.abs(exact)).all(), err.max()
