"""gfx950 variable-length (prefill) attention vs the oracle (bf16 tolerance: |err| <= 2e-2 + 1e-2 |ref|).

``attention.varlen`` is the drop-in for attention.varlen (oxr_runtime/attention.py:47-59).  Cases:
lengths around the 16-row query and 64-key tile edges, an empty sequence, one-token sequences,
causal and bidirectional, every supported head grouping (1, 2, 4 and 8 q heads per kv head),
prefill-sized sequences, and the persistent causal launch (pairs divisible by 8) over several
rounds of items per workgroup, fewer pairs than XCD groups, replayed from a captured graph and run
on two streams at once; and at the benchmark's prefill shapes, rows at the start, middle and end of
every sequence against the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, pkg
from oracle import attention as oracle_attention
from oracle import bf16

pytestmark = pytest.mark.gpu
attention = pkg("attention")

ATOL, RTOL = 2e-2, 1e-2


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _case(lens, H, KV, causal, seed):
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(T, H, 128, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn(T, KV, 128, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(T, KV, 128, generator=g, device="cuda").to(torch.bfloat16)
    out = torch.full_like(q, float("nan"))
    announce("varlen", lens if len(lens) < 12 else f"{len(lens)} seqs", H, KV, "causal" if causal else "bidir")
    attention.varlen(q, k, v, torch.from_numpy(cu).cuda(), max(lens), causal=causal, out=out)
    torch.cuda.synchronize()
    exact = oracle_attention.varlen(_bits(q), _bits(k), _bits(v), cu, 128 ** -0.5, causal)
    got = out.float().cpu().numpy()
    err = np.abs(got - exact)
    bound = ATOL + RTOL * np.abs(exact)
    assert np.isfinite(got).all(), "rows left unwritten"
    assert (err <= bound).all(), f"max err {err.max():.3g}, worst excess {(err - bound).max():.3g}"


@pytest.mark.parametrize("causal", [True, False])
def test_tile_edges_and_empty(causal) -> None:
    _case([1, 15, 16, 17, 0, 63, 64, 65, 127, 128, 129, 200], 16, 8, causal, seed=1 + causal)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("kv", [16, 8, 4, 2])
def test_head_groupings(kv, causal) -> None:
    _case([97, 300, 1], 16, kv, causal, seed=10 + kv)


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_sizes(causal) -> None:
    _case([1024, 777], 16, 8, causal, seed=20 + causal)


@pytest.mark.parametrize("lens", [[700, 513, 1, 0, 640, 64, 300, 129], [1500, 900, 5]])
def test_persistent_rounds(lens) -> None:
    # 32 q heads over 8 kv heads: pairs divisible by 8 take the persistent causal launch, here with
    # several rounds of items per workgroup, ragged and empty sequences, and (3 sequences: 3 pairs
    # per XCD) a last pair group of one.
    _case(lens, 32, 8, True, seed=30 + len(lens))


@pytest.mark.parametrize("lens,H,KV", [([1000], 8, 1), ([513, 7], 4, 2), ([300, 1, 77], 8, 4)])
def test_causal_few_pairs(lens, H, KV) -> None:
    # Fewer (sequence, kv head) pairs than XCD groups: the empty groups' workgroups take every item
    # from the other groups' lists.
    _case(lens, H, KV, True, seed=50 + len(lens))


@pytest.mark.parametrize("lens", [[4096] * 8, np.random.default_rng(0).integers(1, 4097, 32).tolist()],
                         ids=["8x4096", "32 mixed lengths"])
def test_causal_full_size_rows(lens) -> None:
    # The benchmark's prefill shapes (16 q heads over 8 kv heads, 8 x 4096 and 32 mixed lengths up to
    # 4096): every row is written, and blocks of 8 query rows at the start, middle and end of each
    # sequence match the oracle (the oracle on those rows only: a block of rows [p0, p1) over keys
    # [0, p1) with its end-aligned causal mask is exactly their causal attention).
    H, KV = 16, 8
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    g = torch.Generator(device="cuda").manual_seed(60 + len(lens))
    q = torch.randn(T, H, 128, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn(T, KV, 128, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(T, KV, 128, generator=g, device="cuda").to(torch.bfloat16)
    out = torch.full_like(q, float("nan"))
    announce("varlen full size", f"{len(lens)} seqs, {T} tokens")
    attention.varlen(q, k, v, torch.from_numpy(cu).cuda(), max(lens), causal=True, out=out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all()), "rows left unwritten"
    qb, kb, vb = _bits(q), _bits(k), _bits(v)
    got_all = out.float().cpu().numpy()
    for i, n in enumerate(lens):
        start = int(cu[i])
        for p0 in sorted({0, max(0, n // 2 - 4), max(0, n - 8)}):
            p1 = min(n, p0 + 8)
            exact = oracle_attention.attend(bf16.to_f32(qb[start + p0:start + p1]), bf16.to_f32(kb[start:start + p1]),
                                            bf16.to_f32(vb[start:start + p1]), 128 ** -0.5, causal=True)
            got = got_all[start + p0:start + p1]
            err = np.abs(got - exact)
            bound = ATOL + RTOL * np.abs(exact)
            assert (err <= bound).all(), f"seq {i} rows [{p0}, {p1}): max err {err.max():.3g}"


def _inputs(lens, H, KV, seed):
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    g = torch.Generator(device="cuda").manual_seed(seed)
    q, k, v = (torch.randn(T, n, 128, generator=g, device="cuda").to(torch.bfloat16) for n in (H, KV, KV))
    return q, k, v, torch.from_numpy(cu).cuda()


def test_persistent_graph_replays() -> None:
    # The persistent launch's work counters reset themselves at the end of each launch, so a captured
    # launch replays correctly; eager launches (other inputs) run between the replays.  Items are
    # independent of the workgroup that computes them, so every result is bit-identical.
    lens = [640, 1, 300, 513, 0, 64, 700, 129]
    q, k, v, cu = _inputs(lens, 32, 8, seed=41)
    q2, k2, v2, cu2 = _inputs([97, 1500, 33, 5, 800, 2, 64, 257], 32, 8, seed=42)
    announce("varlen graph replays", lens)
    want = attention.varlen(q, k, v, cu, max(lens), causal=True)
    want2 = attention.varlen(q2, k2, v2, cu2, 1500, causal=True)
    out = torch.full_like(q, float("nan"))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        attention.varlen(q, k, v, cu, max(lens), causal=True, out=out)
    torch.cuda.synchronize()
    for _ in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(_bits_t(out), _bits_t(want))
        got2 = attention.varlen(q2, k2, v2, cu2, 1500, causal=True)
        torch.cuda.synchronize()
        assert torch.equal(_bits_t(got2), _bits_t(want2))


def test_persistent_concurrent_streams() -> None:
    # Two persistent launches in flight at once on two streams use different counter sets.
    a = _inputs([1024, 700, 3, 900, 1024, 0, 512, 64], 32, 8, seed=43)
    b = _inputs([800] * 8, 32, 8, seed=44)
    announce("varlen concurrent streams")
    want_a = attention.varlen(*a[:4], 1024, causal=True)
    want_b = attention.varlen(*b[:4], 800, causal=True)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    outs = []
    for _ in range(4):
        with torch.cuda.stream(s1):
            oa = attention.varlen(*a[:4], 1024, causal=True)
        with torch.cuda.stream(s2):
            ob = attention.varlen(*b[:4], 800, causal=True)
        outs.append((oa, ob))
    torch.cuda.synchronize()
    for oa, ob in outs:
        assert torch.equal(_bits_t(oa), _bits_t(want_a))
        assert torch.equal(_bits_t(ob), _bits_t(want_b))


def _bits_t(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(torch.int16)


def test_rejects_unsupported_grouping() -> None:
    q = torch.zeros(4, 12, 128, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(4, 4, 128, dtype=torch.bfloat16, device="cuda")  # 3 q heads per kv head
    with pytest.raises(RuntimeError):
        attention.varlen(q, k, k, torch.tensor([0, 4], dtype=torch.int32, device="cuda"), 4, causal=True)
