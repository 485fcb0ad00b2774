"""gfx950 drafting, verify-input assembly and acceptance vs the oracle (bit-exact, integer).

Covers the reference's known answers (tests/test_speculative.py:8-41) through the list
API, workload-1 histories, random small-vocabulary histories for every n cap, prefix
indexing, k limits, empty and length-1 histories, 16k-token histories, and the engine's
row assembly (engine.py:700-710) and bookkeeping (engine.py:729-737, 647-664).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, pkg
from oracle import bf16, ngram
from oracle import lm_head as oracle_lm_head

pytestmark = pytest.mark.gpu
spec = pkg("speculative")
workloads = pkg("workloads")


def _gpu_drafts(rows: list[list[int]], k: int, max_n: int, k_limit=None, index_len=None):
    cap = max(1, max((len(r) for r in rows), default=1))
    hist = np.zeros((len(rows), cap), dtype=np.int32)
    for i, r in enumerate(rows):
        hist[i, : len(r)] = r
    lens = torch.tensor([len(r) for r in rows], dtype=torch.int32, device="cuda")
    kl = None if k_limit is None else torch.tensor(k_limit, dtype=torch.int32, device="cuda")
    il = None if index_len is None else torch.tensor(index_len, dtype=torch.int32, device="cuda")
    draft, dlen = spec.propose_batch(torch.from_numpy(hist).cuda(), lens, k, max_n=max_n, k_limit=kl, index_len=il)
    draft, dlen = draft.cpu().numpy(), dlen.cpu().numpy()
    return [draft[i, : dlen[i]].tolist() for i in range(len(rows))], draft, dlen


def test_list_api_known_answers() -> None:
    announce("known answers")
    td, end, one, two = 10, 11, 1, 2
    tokens = [td, one, end, td, two, end, td]
    assert spec.NgramProposer(tokens).propose(tokens, 3) == [two, end, td]
    assert spec.NgramProposer([1, 2, 3, 4]).propose([1, 2, 3, 4], 8) == []
    tokens = [5, 6, 7, 5, 6, 8, 5, 6, 7, 9, 5, 6]
    incremental = spec.NgramProposer(tokens[:5])
    incremental.extend(tokens, 5)
    for k in (1, 2, 4):
        assert incremental.propose(tokens, k) == ngram.NgramIndex(tokens).propose(tokens, k)
    assert spec.accept([7, 8, 9, 10], [7, 8, 3, 0, 0]) == [7, 8, 3]
    assert spec.accept([7, 8], [7, 8, 5]) == [7, 8, 5]
    assert spec.accept([7, 8], [1, 8, 5]) == [1]
    assert spec.accept([], [4]) == [4]


def test_extend_sequences_match_reference_dict() -> None:
    """Random sequences of extend calls, as the engine makes them (old_length = the previous length)
    and re-indexing from an earlier old_length: drafts identical to the reference's dict."""
    rng = np.random.default_rng(6)
    announce("extend sequences")
    for _ in range(10):
        tokens = rng.integers(0, 4, size=int(rng.integers(2, 60))).tolist()
        n0 = int(rng.integers(0, len(tokens)))
        mine, ref = spec.NgramProposer(tokens[:n0]), ngram.NgramIndex(tokens[:n0])
        length = n0
        while length < len(tokens):
            new = min(len(tokens), length + int(rng.integers(1, 6)))
            old = length if rng.random() < 0.7 else int(rng.integers(0, length + 1))
            mine.extend(tokens[:new], old)
            ref.extend(tokens[:new], old)
            length = new
            for k in (1, 3):
                assert mine.propose(tokens[:length], k) == ref.propose(tokens[:length], k)


def test_stale_index_matches_reference_dict() -> None:
    """A proposer built on a prefix and not extended only knows the prefix's positions."""
    rng = np.random.default_rng(5)
    announce("stale index")
    for _ in range(20):
        tokens = rng.integers(0, 4, size=int(rng.integers(2, 40))).tolist()
        prefix = int(rng.integers(0, len(tokens) + 1))
        want = ngram.NgramIndex(tokens[:prefix]).propose(tokens, 3)
        assert spec.NgramProposer(tokens[:prefix]).propose(tokens, 3) == want


@pytest.mark.parametrize("max_n", [1, 2, 3, 4, 8])
def test_random_small_vocab_histories(max_n: int) -> None:
    rng = np.random.default_rng(100 + max_n)
    rows = [rng.integers(0, int(rng.integers(2, 6)), size=int(rng.integers(0, 700))).tolist() for _ in range(64)]
    ks = [0, 1, 3, 8]
    announce("random histories", max_n)
    for k in ks:
        got, _, _ = _gpu_drafts(rows, k, max_n)
        want = [ngram.propose_closed_form(r, k, max_n) for r in rows]
        assert got == want


def test_prefix_index_and_k_limit() -> None:
    rng = np.random.default_rng(7)
    rows = [rng.integers(0, 3, size=int(rng.integers(1, 300))).tolist() for _ in range(32)]
    index_len = [int(rng.integers(0, len(r) + 1)) for r in rows]
    k_limit = [int(x) for x in rng.integers(-2, 6, size=len(rows))]
    announce("prefix index + k_limit")
    got, draft, _ = _gpu_drafts(rows, 4, 4, k_limit=k_limit, index_len=index_len)
    for i, r in enumerate(rows):
        kb = max(0, min(4, k_limit[i]))
        assert got[i] == ngram.NgramIndex(r[: index_len[i]]).propose(r, kb)
        assert (draft[i, len(got[i]) :] == 0).all()


def test_edge_histories() -> None:
    rows = [[], [7], [7, 7], [3, 3, 3, 3, 3], [1, 2, 3], [9, 1, 9], list(range(300)) + [0]]
    announce("edge histories")
    for max_n in (1, 4):
        got, _, _ = _gpu_drafts(rows, 3, max_n)
        assert got == [ngram.NgramIndex(r, max_n).propose(r, 3) for r in rows]


def test_workload1_histories_all_caps() -> None:
    histories = workloads.drafting_histories(seed=0)
    rows = [h.tolist() for h in histories]
    announce("workload1")
    for max_n in (3, 4):
        got, _, dlen = _gpu_drafts(rows, 3, max_n)
        assert got == [ngram.NgramIndex(r, max_n).propose(r, 3) for r in rows]
        assert dlen[0] == 3 and dlen[-1] == 0


def test_long_histories() -> None:
    """16k-token histories: matches far from the end, near the start, and none."""
    rng = np.random.default_rng(9)
    L = 16384
    base = rng.permutation(workloads.VOCAB)[:L].astype(np.int32)
    far = base.copy()
    far[100:104] = far[-4:]  # only match is near the start
    near = workloads.repetitive_history(rng, L, repetitive_tail=True)
    rows = [base.tolist(), far.tolist(), near.tolist()]
    announce("long histories")
    got, _, _ = _gpu_drafts(rows, 3, 4)
    assert got == [ngram.propose_closed_form(r, 3, 4) for r in rows]
    assert got[1] == far[104:107].tolist()


def test_histories_across_scan_chunks() -> None:
    """Histories around the kernel's 4096-candidate LDS chunks: the only, or the longest, match sits
    just before or just after a chunk edge, and a shorter match in a later chunk must not win over
    a longer one in an earlier-scanned (later) chunk or the reverse."""
    rng = np.random.default_rng(17)
    rows = []
    for L in (4095, 4096, 4097, 4105, 8193):
        base = rng.permutation(workloads.VOCAB)[:L].astype(np.int32)
        for p in (L - 4096 - 1, L - 4096, L - 4096 + 1, L - 4096 + 7):  # candidate positions at the edge
            if 4 <= p <= L - 5:
                r = base.copy()
                r[p - 4 : p] = r[-4:]  # a full 4-token match ending just before p
                rows.append(r.tolist())
        r = base.copy()
        r[L - 4096 + 40 - 2 : L - 4096 + 40] = r[-2:]  # 2-token match in the last-scanned chunk
        r[10:13] = r[-3:]  # longer (3-token) match near the start
        rows.append(r.tolist())
    announce("chunk-edge histories", len(rows))
    got, _, _ = _gpu_drafts(rows, 3, 4)
    assert got == [ngram.propose_closed_form(r, 3, 4) for r in rows]


def test_verify_inputs_assembly() -> None:
    rng = np.random.default_rng(11)
    B, k, S, bs = 8, 3, 4, 16
    histories = [workloads.repetitive_history(rng, int(rng.integers(50, 400)), repetitive_tail=bool(i % 2))
                 for i in range(B)]
    cap = 512
    hist = np.zeros((B, cap), dtype=np.int32)
    for i, h in enumerate(histories):
        hist[i, : len(h)] = h
    seq_len = rng.integers(100, 1000, size=B).astype(np.int32)
    width = 80
    table = rng.permutation(4096)[: B * width].reshape(B, width).astype(np.int32)
    announce("verify inputs")
    out = spec.propose_verify_inputs(
        torch.from_numpy(hist).cuda(), torch.tensor([len(h) for h in histories], dtype=torch.int32, device="cuda"), k,
        torch.from_numpy(seq_len).cuda(), torch.from_numpy(table).cuda(), bs, S, max_n=4,
    )
    ids, pos, slots = out.ids.cpu().numpy(), out.positions.cpu().numpy(), out.slots.cpu().numpy()
    for b, h in enumerate(histories):
        tokens = h.tolist()
        draft = ngram.NgramIndex(tokens).propose(tokens, k)
        row = [tokens[-1], *draft] + [0] * (S - 1 - len(draft))  # engine.py:703-709
        assert ids[b * S : (b + 1) * S].tolist() == row
        for j in range(S):
            p = int(seq_len[b]) + j
            assert pos[b * S + j] == p
            assert slots[b * S + j] == table[b, p // bs] * bs + p % bs  # language.py:320-322
    assert out.attn_seq_lens.cpu().numpy().tolist() == (seq_len + S).tolist()


@pytest.mark.parametrize("k", [3, 8, 12])
def test_accept_batch_and_rollback(k: int) -> None:
    """k = 3 (the benchmark), 8 (the engine's default speculative_tokens, engine.py:121) and 12 (past
    the kernel's preloaded drafts and predictions)."""
    rng = np.random.default_rng(13 + k)
    B, S = 64, k + 1
    draft = rng.integers(0, 5, size=(B, k)).astype(np.int32)
    dlen = rng.integers(0, k + 1, size=B).astype(np.int32)
    for b in range(B):
        draft[b, dlen[b] :] = 0
    predicted = rng.integers(0, 5, size=(B, S)).astype(np.int64)
    predicted[::3, :k] = draft[::3]  # some full accepts
    seq_len = rng.integers(10, 100, size=B).astype(np.int32)
    cap = 64
    hist_len = rng.integers(1, 50, size=B).astype(np.int32)
    hist = rng.integers(0, 5, size=(B, cap)).astype(np.int32)
    eos = 4
    max_tokens = rng.integers(2, 60, size=B).astype(np.int32)
    d = lambda a: torch.from_numpy(a).cuda()
    seq_t, hist_t, hlen_t, fin_t = d(seq_len.copy()), d(hist.copy()), d(hist_len.copy()), torch.zeros(B, dtype=torch.int32, device="cuda")
    announce("accept batch")
    res = spec.accept_batch(d(draft), d(dlen), d(predicted), seq_len=seq_t, history=hist_t, history_len=hlen_t,
                            eos_id=eos, max_tokens=d(max_tokens), finished=fin_t)
    acc, com = res.accepted.cpu().numpy(), res.committed.cpu().numpy()
    for b in range(B):
        taken = ngram.accept(draft[b, : dlen[b]].tolist(), predicted[b, : dlen[b] + 1].tolist())
        a = len(taken) - 1
        assert acc[b] == a and com[b, : a + 1].tolist() == taken and (com[b, a + 1 :] == -1).all()
        assert seq_t[b].item() == seq_len[b] + a + 1
        # engine.py:647-664: EOS finishes without appending; max_tokens finishes after appending.
        out = hist[b, : hist_len[b]].tolist()
        reason = 0
        for t in taken:
            if t == eos:
                reason = 1
                break
            out.append(t)
            if len(out) >= max_tokens[b]:
                reason = 2
                break
        assert hlen_t[b].item() == len(out) and hist_t[b, : len(out)].cpu().tolist() == out
        assert fin_t[b].item() == reason
    # Finished sequences take nothing on the next call.
    before = seq_t.clone()
    done = fin_t.cpu().numpy() != 0
    assert done.any() and not done.all()
    spec.accept_batch(d(draft), d(dlen), d(predicted), seq_len=seq_t, history=hist_t, history_len=hlen_t,
                      eos_id=eos, max_tokens=d(max_tokens), finished=fin_t)
    assert np.array_equal(seq_t.cpu().numpy()[done], before.cpu().numpy()[done])


lm_head = pkg("lm_head")


def _torch_argmax(a: np.ndarray) -> np.ndarray:
    """torch.argmax on the CPU: first index of the maximum, NaN counted as the maximum."""
    return torch.from_numpy(a).argmax(-1).numpy()


def test_config1_planted_logits_argmax_and_accept() -> None:
    """Workload 1's acceptance leg: drafts of the four histories (max_n 3, k 3), fp32 verify
    logits [4, 4, 151936] ~N(0, 1) with each draft id planted as the row's strict maximum with
    p = 0.6, argmax on the GPU, then acceptance (engine.py:726-733) -- ids, accepted lengths,
    committed ids and the next tokens bit-exact against the oracle."""
    hist_np = workloads.drafting_histories(seed=0)
    rows = [h.tolist() for h in hist_np]
    k, S = 3, 4
    announce("config 1 drafting")
    draft, dlen = spec.propose_batch(torch.from_numpy(hist_np).cuda(), torch.full((4,), 512, dtype=torch.int32,
                                                                                  device="cuda"), k, max_n=3)
    want_draft, want_len = ngram.propose_batch(rows, k, max_n=3)
    assert np.array_equal(draft.cpu().numpy(), want_draft) and np.array_equal(dlen.cpu().numpy(), want_len)
    logits = workloads.plant_logits(np.random.default_rng(1), want_draft, want_len, S)
    announce("config 1 argmax + accept")
    predicted = lm_head.argmax(torch.from_numpy(logits).cuda())
    res = spec.accept_batch(draft, dlen, predicted)
    want_pred = np.argmax(logits, axis=-1)
    assert np.array_equal(predicted.cpu().numpy(), want_pred)
    acc, com = res.accepted.cpu().numpy(), res.committed.cpu().numpy()
    planted = 0
    for b in range(4):
        taken = ngram.accept(want_draft[b, : want_len[b]].tolist(), want_pred[b, : want_len[b] + 1].tolist())
        assert acc[b] == len(taken) - 1 and com[b, : len(taken)].tolist() == taken
        assert com[b, len(taken) - 1] == taken[-1]  # the next token: the model's own after the accepted prefix
        planted += acc[b]
    assert want_len.max() > 0 and planted > 0, "nothing accepted: the planted path went untested"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_argmax_edge_cases(dtype) -> None:
    """Ties to the lowest index (also across column chunks), NaN as the maximum (first NaN),
    -0 == +0, all -inf rows, odd widths and a row stride that breaks 16-byte alignment."""
    rng = np.random.default_rng(3)
    vocab = 151_936
    a = rng.standard_normal((9, vocab)).astype(np.float32)
    a[1, [70_000, 5, 140_000]] = 50.0            # tie across chunks -> 5
    a[2, [9, 100_000]] = np.nan                    # first NaN
    a[3] = -np.inf                                  # all -inf -> 0
    a[4] = 0.0
    a[4, :1000] = -0.0                              # -0 == +0 -> 0
    a[5, -1] = 1e30                                 # last column
    a[6, 151_935] = np.inf
    a[6, 77] = np.inf                               # first +inf
    a = torch.from_numpy(a).to(dtype)
    announce("argmax edge cases", dtype)
    got = lm_head.argmax(a.cuda()).cpu().numpy()
    assert np.array_equal(got, a.float().argmax(-1).numpy()), got
    odd = a[:, 3 : 3 + 1001].contiguous()
    assert np.array_equal(lm_head.argmax(odd.cuda()).cpu().numpy(), odd.float().argmax(-1).numpy())
    strided = a.cuda()[:, 1:1001]  # rows 16-byte aligned only by chance: the unvectorised form
    assert np.array_equal(lm_head.argmax(strided).cpu().numpy(), a[:, 1:1001].float().argmax(-1).numpy())
    batch = a[:8].reshape(2, 4, vocab)  # leading dims kept
    assert lm_head.argmax(batch.cuda()).shape == (2, 4)


gemm = pkg("gemm")


@pytest.mark.parametrize("B,S,vocab", [(8, 4, 151936), (1, 4, 32768), (8, 9, 32768), (16, 4, 32768),
                                       (12, 20, 32768), (64, 4, 5000)])
def test_greedy_accept_matches_separate_launches(B: int, S: int, vocab: int) -> None:
    """oxr_lm_head_accept_packed against oxr_lm_head_argmax_packed followed by oxr_accept on the
    same inputs: greedy ids, accepted lengths, committed ids, KV lengths, histories and finish
    reasons bit for bit.  Rows 32 and under take the persistent LM head, more the wide one;
    S = 20 needs two rounds of key loads.  Drafts copy the separate path's ids with p = 0.6 per
    position, so runs of every length are accepted; the last sequence starts finished, one id is
    the EOS and max_tokens stops some histories."""
    rng = np.random.default_rng(100 * B + S)
    gen = torch.Generator(device="cuda").manual_seed(B + S)
    hidden = torch.randn(B * S, 2048, device="cuda", generator=gen).to(torch.bfloat16)
    w = gemm.pack_weight((torch.randn(vocab, 2048, device="cuda", generator=gen) * 0.02).to(torch.bfloat16))
    ws = torch.empty(lm_head.workspace_bytes(B * S, vocab), dtype=torch.uint8, device="cuda")
    announce(f"greedy accept B={B} S={S} vocab={vocab}: separate launches")
    pred_ref = lm_head.lm_head_argmax(hidden, w, workspace=ws)[0]
    pr = pred_ref.view(B, S).cpu().numpy()
    k = S - 1
    draft = np.where(rng.random((B, k)) < 0.6, pr[:, :k], rng.integers(0, vocab, (B, k))).astype(np.int32)
    dlen = rng.integers(0, k + 1, size=B).astype(np.int32)
    dlen[0] = k
    draft[0] = pr[0, :k]  # one full accept
    cap = 64
    hist_len = rng.integers(1, 30, size=B).astype(np.int32)
    hist = rng.integers(0, vocab, size=(B, cap)).astype(np.int32)
    max_tokens = (hist_len + rng.integers(1, S + 2, size=B)).astype(np.int32)
    fin = np.zeros(B, dtype=np.int32)
    if B > 1:
        fin[-1] = 2
    eos = int(pr[B // 2, 1])
    seq_len = rng.integers(100, 9000, size=B).astype(np.int32)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()

    def state():
        return dict(seq_len=d(seq_len), history=d(hist), history_len=d(hist_len), max_tokens=d(max_tokens),
                    finished=d(fin), eos_id=eos)

    ref = state()
    res_ref = spec.accept_batch(d(draft), d(dlen), pred_ref.view(B, S), **ref)
    announce(f"greedy accept B={B} S={S} vocab={vocab}: fused")
    got = state()
    pred = torch.full((B, S), -7, dtype=torch.int64, device="cuda")
    ws.fill_(0xAB)
    res = spec.greedy_accept_batch(hidden, w, d(draft), d(dlen), predicted=pred, workspace=ws, **got)
    assert torch.equal(pred.view(-1), pred_ref)
    for name in ("accepted", "committed", "num_committed"):
        assert torch.equal(getattr(res, name), getattr(res_ref, name)), name
    for name in ("seq_len", "history", "history_len", "finished"):
        assert torch.equal(got[name], ref[name]), name
    acc = res.accepted.cpu().numpy()
    assert acc[0] == k
    if B > 2:
        assert (acc[:-1] < k).any()
    if B > 1:
        assert acc[-1] == 0 and res.num_committed[-1].item() == 0  # started finished


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def test_greedy_accept_config4_against_exact_product() -> None:
    """Config 4 through the step's real tail (``greedy_accept_batch``: the wide LM head over 256 token
    rows, its argmax finished inside the acceptance launch): 64 sequences x 4 positions, vocab
    151,936, k = 3, each draft id planted as the reference argmax of its row with p = 0.5.  Greedy
    ids equal the oracle's argmax of the exact product wherever its top-2 margin exceeds 2e-2; the
    acceptance is bit-exact against ``oracle.ngram.accept`` on the kernel's ids, and against the
    oracle's own ids on every sequence whose rows are all decided by a clear margin; KV lengths
    advance by the committed count (engine.py:729-737)."""
    B, S, vocab, k, atol = 64, 4, 151_936, 3, 2e-2
    rng = np.random.default_rng(404)
    gen = torch.Generator(device="cuda").manual_seed(404)
    hidden = torch.randn(B * S, 2048, device="cuda", generator=gen).to(torch.bfloat16)
    weight = (torch.randn(vocab, 2048, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
    announce("greedy accept config4: exact product")
    exact = oracle_lm_head.logits_exact(_u16(hidden), _u16(weight))
    ref_ids = oracle_lm_head.argmax(bf16.from_f32(exact.astype(np.float32))).reshape(B, S)
    sure = (oracle_lm_head.top2_margin(exact) > atol).reshape(B, S)
    draft = ref_ids[:, :k].copy()
    miss = rng.random((B, k)) >= 0.5
    other = rng.integers(0, vocab - 1, size=(B, k))
    draft[miss] = other[miss] + (other[miss] >= ref_ids[:, :k][miss])  # a random id other than the argmax
    draft = draft.astype(np.int32)
    dlen = np.full(B, k, dtype=np.int32)
    seq0 = rng.integers(1000, 9000, size=B).astype(np.int32)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    seq_len = d(seq0)
    packed = gemm.pack_weight(weight)
    ws = torch.empty(lm_head.workspace_bytes(B * S, vocab), dtype=torch.uint8, device="cuda")
    pred = torch.full((B, S), -7, dtype=torch.int64, device="cuda")
    announce("greedy accept config4: launch")
    res = spec.greedy_accept_batch(hidden, packed, d(draft), d(dlen), predicted=pred, workspace=ws, seq_len=seq_len)
    torch.cuda.synchronize()
    got = pred.cpu().numpy()
    assert sure.mean() > 0.8
    assert np.array_equal(got[sure], ref_ids[sure])
    accepted = res.accepted.cpu().numpy()
    committed = res.committed.cpu().numpy()
    num = res.num_committed.cpu().numpy()
    for b in range(B):
        taken = ngram.accept(draft[b].tolist(), got[b].tolist())
        assert accepted[b] == len(taken) - 1 and num[b] == len(taken), b
        assert committed[b, : num[b]].tolist() == taken, b
        if sure[b].all():
            assert taken == ngram.accept(draft[b].tolist(), ref_ids[b].tolist()), b
    assert np.array_equal(seq_len.cpu().numpy(), seq0 + num)
    assert (accepted == k).any() and (accepted == 0).any() and ((accepted > 0) & (accepted < k)).any()

