"""The fused attention block (q/k norm + RoPE + K/V store + paged attention in one launch) against
the two separate calls it replaces: the output and every cache row must be bit-identical.

Contexts are chosen so the S new tokens fall inside one context split, straddle two splits, or
fill a split of their own; S=1, S=4 and S=8 (16 query rows per kv head) and block sizes 16 and
256 are covered, as is a slot outside the cache (not stored by either path; only the sequence
that owns it may then differ, since the fused kernel attends to the token's computed row).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, pkg

pytestmark = pytest.mark.gpu
attention = pkg("attention")
gemm = pkg("gemm")
_lib = pkg("_lib")


def _case(seq_lens, S, H, KV, block_size, seed, bad_slot=False, planned=False):
    rng = np.random.default_rng(seed)
    B = len(seq_lens)
    seq_lens = np.asarray(seq_lens, dtype=np.int32)
    need = (seq_lens + block_size - 1) // block_size
    width = int(need.max()) + 1
    num_blocks = int(need.sum()) + 8
    perm = rng.permutation(num_blocks).astype(np.int32)
    table = np.zeros((B, width), dtype=np.int32)
    off = 0
    for b in range(B):
        table[b, : need[b]] = perm[off : off + need[b]]
        off += need[b]
    positions = np.concatenate([np.arange(L - S, L) for L in seq_lens]).astype(np.int64)
    slots = np.array([table[i // S, p // block_size] * block_size + p % block_size for i, p in enumerate(positions)],
                     dtype=np.int64)
    if bad_slot:
        slots[1] = num_blocks * block_size + 5  # outside the cache: neither path stores it
    g = torch.Generator(device="cuda").manual_seed(seed)
    dev = "cuda"
    kc = torch.randn(num_blocks, block_size, KV, 128, generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn(num_blocks, block_size, KV, 128, generator=g, device=dev).to(torch.bfloat16)
    qkv = torch.randn(B * S, (H + 2 * KV) * 128, generator=g, device=dev).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
    rows = int(seq_lens.max()) + 4
    ang = torch.rand(rows, 64, generator=g, device=dev) * 6.283
    cos, sin = torch.cos(ang).to(torch.bfloat16), torch.sin(ang).to(torch.bfloat16)
    t = lambda a: torch.from_numpy(a).to(dev)
    seq_t, table_t, pos_t, slots_t = t(seq_lens), t(table), t(positions), t(slots)
    eps = 1e-6

    # Separate: oxr_qk_norm_rope_store_at, then oxr_paged_extend.
    k1, v1 = kc.clone(), vc.clone()
    q = torch.empty(B, S, H, 128, dtype=torch.bfloat16, device=dev)
    _lib.call("oxr_qk_norm_rope_store_at", qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), cos.data_ptr(),
              sin.data_ptr(), rows, pos_t.data_ptr(), eps, k1.data_ptr(), v1.data_ptr(), slots_t.data_ptr(),
              num_blocks * block_size, B * S, H, KV, 128, q.data_ptr(), None, None, _lib.stream(torch.device(dev)))
    plan = attention.build_plan(seq_t, S, H, KV, table_t.shape[1] * block_size) if planned else None
    out1 = attention.paged_extend(q, k1, v1, seq_t, table_t, plan=plan)

    # Fused.
    k2, v2 = kc.clone(), vc.clone()
    out2 = attention.qk_norm_rope_paged_extend(qkv, qw, kw, cos, sin, pos_t, eps, k2, v2, slots_t, seq_t, table_t, H,
                                               plan=plan)
    # Fused, output packed for the o_proj GEMM: the same values.
    k3, v3 = kc.clone(), vc.clone()
    out3 = attention.qk_norm_rope_paged_extend(qkv, qw, kw, cos, sin, pos_t, eps, k3, v3, slots_t, seq_t, table_t, H,
                                               out=gemm.packed_rows(B * S, H * 128, dev), plan=plan)
    torch.cuda.synchronize()
    assert torch.equal(out2.view(torch.int16).view(B * S, H * 128), out3.unpack().view(torch.int16)), "packed output"
    assert torch.equal(k2.view(torch.int16), k3.view(torch.int16)) and torch.equal(v2.view(torch.int16), v3.view(torch.int16))
    if bad_slot:
        # The row with no valid slot is not stored by either path; the fused kernel still attends to
        # the token's computed row, the separate calls to whatever the cache held.  Sequence 0 owns
        # that token; every other sequence must match exactly.
        out1, out2 = out1[1:], out2[1:]
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16)), "attention output differs"
    assert torch.equal(k1.view(torch.int16), k2.view(torch.int16)), "K cache differs"
    assert torch.equal(v1.view(torch.int16), v2.view(torch.int16)), "V cache differs"


@pytest.mark.parametrize("S", [1, 4, 8])
def test_small_contexts_straddling_splits(S) -> None:
    lens = [33, 64, 65, 66, 67, 95, 96, 97]
    announce(f"fused attention S={S} lens={lens}")
    _case(lens, S, 16, 8, 16, seed=S)


def test_verify_step_shape_and_ragged() -> None:
    lens = [4100, 4096 + 5, 2051, 8192, 300, 4127, 4128, 4129]
    announce(f"fused attention verify shape lens={lens}")
    _case(lens, 4, 16, 8, 16, seed=11)


@pytest.mark.parametrize("S", [4, 9])
def test_planned_mixed_contexts(S) -> None:
    """With a plan (long contexts taking the workgroups short ones leave, so a new token's K/V row may
    be stored by a workgroup of another sequence's slot), the fused launch still equals the separate
    calls bit for bit, and every new row is stored exactly once."""
    lens = [S, 40, 9000, 300, 4100, 7000, 65, 2051]
    announce(f"fused attention planned S={S} lens={lens}")
    _case(lens, S, 16, 8, 16, seed=30 + S, planned=True)


def test_block_256_and_skipped_slot() -> None:
    announce("fused attention block 256, one slot outside the cache")
    _case([700, 257, 1300, 90], 4, 16, 8, 256, seed=12, bad_slot=True)


def test_eight_new_tokens_long_contexts() -> None:
    """S=8 (one kv head per workgroup) at contexts long enough for every split to hold keys."""
    lens = [4100, 2600, 700, 5000]
    announce(f"fused attention S=8 lens={lens}")
    _case(lens, 8, 16, 8, 16, seed=14)


def test_single_sequence_many_splits() -> None:
    announce("fused attention B=1 (32 splits)")
    _case([5000], 4, 16, 8, 16, seed=13)


@pytest.mark.parametrize("S", [9, 16])
def test_reference_default_width(S) -> None:
    """S=9 (the reference's default 1 + 8, engine.py:121) and S=16: two query-row tiles per kv
    head and the row jobs in two rounds; new tokens inside one split, straddling splits, and
    contexts of only the new tokens."""
    lens = [S, S + 31, 4100, 2600, 97, 700, 5000, 8192]
    announce(f"fused attention S={S} lens={lens}")
    _case(lens, S, 16, 8, 16, seed=20 + S)


def test_s9_block_256_and_skipped_slot() -> None:
    announce("fused attention S=9 block 256, one slot outside the cache")
    _case([700, 257, 1300, 90], 9, 16, 8, 256, seed=15, bad_slot=True)
