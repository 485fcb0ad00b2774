"""The whole verify forward on gfx950 kernels vs the CPU oracle (oracle/decoder.py).

- Teacher-forced, layer by layer: each GPU layer starts from the oracle's residual stream; the
  K/V it writes match the oracle within bf16 tolerance, its output residual within 1.5%
  relative RMS (see ``_residual_close``); embedding gather exact; final norm within tolerance.
- ``extend`` end to end on a small random-init decoder (2 layers): rounding differences
  compound through the residual stream (an all-CPU run with fp32-accumulated GEMMs and bf16
  attention probabilities, which is what the kernels compute, diverges from the oracle by the
  same ~1% relative RMS), so the bound is 2% relative RMS; greedy ids identical wherever the
  oracle's top-2 logit margin exceeds the tolerance.
- The reference's invariant (tests/test_language_fused.py:250-278): feeding a sequence
  through successive 4-token extends equals one causal forward over the whole sequence.
- :class:`VerifyLoop` replayed from a HIP graph, step by step against the oracle's
  ``verify_step`` from the same state: drafts, accepted lengths, committed ids, KV lengths
  and histories identical (where the greedy ids are decided by a clear margin).
- :class:`ExtendGraphs` (the reference's list interface) equals eager ``extend``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, pkg
from oracle import decoder as oracle_decoder
from oracle import ngram

pytestmark = pytest.mark.gpu
language = pkg("language")
kv_cache = pkg("kv_cache")
decode_graph = pkg("decode_graph")
workloads = pkg("workloads")

ATOL, RTOL = 2e-2, 1e-2
SMALL = language.LanguageConfig(512, 768, 2, 4, 2, 128, 1e-6, 1e6, 1000)


def _model(config, seed=0, max_positions=1024):
    w = language.random_weights(config, max_positions, seed=seed, std=0.05)
    return language.LanguageModel(config, w), w.to("cpu")


def _cache(config, num_blocks, block_size, seed):
    cache = kv_cache.KVCache(config.num_layers, config.num_kv_heads, config.head_dim, num_blocks, block_size=block_size)
    g = torch.Generator(device="cuda").manual_seed(seed)
    cache.k.copy_(torch.randn(cache.k.shape, generator=g, device="cuda").to(torch.bfloat16))
    cache.v.copy_(torch.randn(cache.v.shape, generator=g, device="cuda").to(torch.bfloat16))
    return cache


def _close(got: torch.Tensor, want: torch.Tensor) -> float:
    got, want = got.float().cpu(), want.float().cpu()
    err = (got - want).abs()
    assert bool((err <= ATOL + RTOL * want.abs()).all()), f"max err {err.max().item():.3g}"
    return err.max().item()


def _residual_close(got: torch.Tensor, want: torch.Tensor) -> None:
    """A layer's output residual.  Its attention and MLP outputs come from GEMMs whose inputs pass
    through RMSNorms, so an input's relative rounding error reappears as an error proportional to
    the row's output scale, not to each element: the check is per layer, 1.5% relative RMS and
    an absolute cap of 0.25.  (An all-CPU run of the same layer with fp32-accumulated GEMMs and
    bf16 attention probabilities -- what the kernels compute -- differs from the oracle by up to
    0.7% relative RMS and 0.05 absolute on this model; wiring mistakes show up as O(1) errors.)"""
    got, want = got.float().cpu(), want.float().cpu()
    err = (got - want).abs()
    rel = (err.pow(2).sum() / want.pow(2).sum()).sqrt().item()
    assert rel < 1.5e-2 and err.max().item() < 0.25, (rel, err.max().item())


def _ids_agree(pred: np.ndarray, cpu_logits: torch.Tensor, margin_floor: float = ATOL) -> None:
    values = cpu_logits.float().numpy()
    part = np.partition(values, -2, axis=-1)
    margin = part[:, -1] - part[:, -2]
    sure = margin > margin_floor
    want = cpu_logits.argmax(-1).numpy()
    assert sure.mean() > 0.5
    assert np.array_equal(pred[sure], want[sure]), (pred, want, margin)


def _small_case(seed):
    rng = np.random.default_rng(seed)
    model, cpu_w = _model(SMALL, seed=seed)
    B, S, bs = 3, 4, 16
    batch = workloads.paged_batch(rng, B, S, (40, 300), block_size=bs, num_blocks=256, table_width=24)
    cache = _cache(SMALL, 256, bs, seed=seed + 1)
    ids = rng.integers(0, SMALL.vocab_size, size=B * S)
    d = lambda a, dt: torch.from_numpy(np.asarray(a)).to(dt).cuda()
    eb = language.ExtendBatch(None, d(batch.positions, torch.int64), d(batch.slots, torch.int64),
                              d(batch.seq_lens, torch.int32), d(batch.block_table, torch.int32), S, ids=d(ids, torch.int64))
    cpu_args = (torch.from_numpy(ids), torch.from_numpy(batch.positions), torch.from_numpy(batch.slots),
                torch.from_numpy(batch.seq_lens), torch.from_numpy(batch.block_table), S)
    return model, cpu_w, cache, eb, cpu_args, batch


def test_each_layer_within_bf16_tolerance() -> None:
    """Teacher-forced: every GPU layer starts from the oracle's residual stream, so its result must
    match the oracle's next residual within bf16 tolerance; the K/V it writes likewise.  Embedding
    gather is exact; final norm + LM head are checked from the oracle's last residual."""
    model, cpu_w, cache, eb, cpu_args, batch = _small_case(1)
    cpu_k, cpu_v = cache.k.cpu(), cache.v.cpu()
    trace = []
    want_hidden = oracle_decoder.extend(SMALL, cpu_w, *cpu_args, cpu_k, cpu_v, trace=trace)
    buffers = language.StepBuffers.allocate(SMALL, 3, 4, 24 * 16, "cuda")
    t = 12
    announce("teacher-forced layers")
    model.embed(eb, buffers)
    torch.cuda.synchronize()
    assert torch.equal(buffers.residual[:t].cpu(), trace[0])
    flat = lambda c: c.view(-1, SMALL.num_kv_heads, SMALL.head_dim)
    slots = torch.from_numpy(batch.slots)
    for i in range(SMALL.num_layers):
        buffers.residual[:t].copy_(trace[i].cuda())
        buffers.pending_splits = 0
        model.run_layers(eb, cache, buffers, i, i + 1)
        model.settle(eb, buffers, cpu_w.final_norm.cuda())  # adds the layer's pending down_proj partials
        torch.cuda.synchronize()
        _residual_close(buffers.residual[:t], trace[i + 1])
        _close(flat(cache.k[i].cpu())[slots], flat(cpu_k[i])[slots])
        _close(flat(cache.v[i].cpu())[slots], flat(cpu_v[i])[slots])
    buffers.residual[:t].copy_(trace[-1].cuda())
    buffers.pending_splits = 0
    hidden = model.final_norm(eb, buffers)
    _close(hidden, want_hidden)
    pred = model.greedy(hidden).cpu().numpy()
    _ids_agree(pred, oracle_decoder.logits(cpu_w, want_hidden))


def test_extend_end_to_end_small_model() -> None:
    """Untied run: bf16 rounding differences compound through the residual stream, so the
    end-to-end bound is the layer tolerance widened by the layer count; greedy ids still agree
    wherever the oracle's top-2 margin is clear."""
    model, cpu_w, cache, eb, cpu_args, _ = _small_case(2)
    cpu_k, cpu_v = cache.k.cpu(), cache.v.cpu()
    announce("extend end to end")
    hidden = model.extend(eb, cache)
    pred = model.greedy(hidden).cpu().numpy()
    torch.cuda.synchronize()
    want = oracle_decoder.extend(SMALL, cpu_w, *cpu_args, cpu_k, cpu_v)
    err = (hidden.float().cpu() - want.float()).abs()
    layers = SMALL.num_layers + 1
    assert bool((err <= layers * (ATOL + RTOL * want.float().abs())).all()), err.max().item()
    rel = (err.pow(2).sum() / want.float().pow(2).sum()).sqrt().item()
    assert rel < 2e-2, rel
    # The untied logits carry the compounded ~1-2% error too: ids must agree where the oracle's
    # top-2 margin is well clear of it (0.1, five times the per-op tolerance).
    _ids_agree(pred, oracle_decoder.logits(cpu_w, want), margin_floor=0.1)


def test_reference_eager_verify_sequence() -> None:
    """The reference's eager verify fallback in its own form (engine.py:716-726): the batch built
    positionally as ``ExtendBatch(language.embed_tokens(ids), positions, slots, seq_lens, table,
    width)``, then ``extend`` -> ``logits`` -> ``argmax(-1).view(B, width)``.  ``embed_tokens`` gives
    the table's rows exactly; the hidden state is bit-identical to the ``ids=`` form (the gather
    fused into the first norm); both are checked against the oracle as the end-to-end test does."""
    model, cpu_w, cache, eb_ids, cpu_args, _ = _small_case(4)
    cpu_k, cpu_v = cache.k.cpu(), cache.v.cpu()
    ids_cpu, positions, slots, seq_lens, table, width = cpu_args
    B = table.shape[0]
    announce("reference eager verify sequence")
    embeds = model.embed_tokens(ids_cpu.cuda())
    torch.cuda.synchronize()
    assert embeds.dtype == torch.bfloat16 and tuple(embeds.shape) == (B * width, SMALL.hidden_size)
    assert torch.equal(embeds.cpu(), cpu_w.embed[ids_cpu])
    batch = language.ExtendBatch(embeds, positions.cuda(), slots.cuda(), seq_lens.cuda(), table.cuda(), width)
    hidden = model.extend(batch, cache)
    tokens = model.logits(hidden).argmax(dim=-1).view(B, width)
    hidden_ids = model.extend(eb_ids, cache)  # same K/V rewritten at the same slots
    torch.cuda.synchronize()
    assert torch.equal(hidden.cpu(), hidden_ids.cpu())
    want = oracle_decoder.extend(SMALL, cpu_w, *cpu_args, cpu_k, cpu_v)
    err = (hidden.float().cpu() - want.float()).abs()
    rel = (err.pow(2).sum() / want.float().pow(2).sum()).sqrt().item()
    assert rel < 2e-2, rel
    _ids_agree(tokens.reshape(-1).cpu().numpy(), oracle_decoder.logits(cpu_w, want), margin_floor=0.1)


def test_chunked_extends_equal_full_sequence() -> None:
    """tests/test_language_fused.py:250-278 of the reference, on the GPU path."""
    rng = np.random.default_rng(3)
    model, cpu_w = _model(SMALL, seed=3)
    B, S, bs, n = 2, 4, 16, 24
    cache = kv_cache.KVCache(SMALL.num_layers, SMALL.num_kv_heads, SMALL.head_dim, 8, block_size=bs, fill=0.0)
    table = np.array([[0, 1], [5, 3]], dtype=np.int32)
    tokens = rng.integers(0, SMALL.vocab_size, size=(B, n))
    announce("chunked extend")
    for start in range(0, n, S):
        pos = np.concatenate([np.arange(start, start + S)] * B)
        rows = np.repeat(np.arange(B), S)
        slots = table[rows, pos // bs] * bs + pos % bs
        eb = language.ExtendBatch(
            None, torch.from_numpy(pos).cuda(),
            torch.from_numpy(slots.astype(np.int64)).cuda(), torch.full((B,), start + S, dtype=torch.int32).cuda(),
            torch.from_numpy(table).cuda(), S, ids=torch.from_numpy(tokens[:, start : start + S].reshape(-1)).cuda(),
        )
        hidden = model.extend(eb, cache)
    torch.cuda.synchronize()
    # One causal forward over all n tokens of each sequence (an extend of n tokens on an empty cache).
    ck = torch.zeros(SMALL.num_layers, 8, bs, SMALL.num_kv_heads, SMALL.head_dim, dtype=torch.bfloat16)
    cv = torch.zeros_like(ck)
    pos = np.concatenate([np.arange(n)] * B)
    rows = np.repeat(np.arange(B), n)
    slots = table[rows, pos // bs] * bs + pos % bs
    full = oracle_decoder.extend(SMALL, cpu_w, torch.from_numpy(tokens.reshape(-1)), torch.from_numpy(pos),
                                 torch.from_numpy(slots.astype(np.int64)), torch.full((B,), n, dtype=torch.int32),
                                 torch.from_numpy(table), n, ck, cv)
    want = full.view(B, n, -1)[:, -S:].reshape(B * S, -1)
    err = (hidden.float().cpu() - want.float()).abs()
    assert bool((err <= (SMALL.num_layers + 1) * (ATOL + RTOL * want.float().abs())).all()), err.max().item()
    assert (err.pow(2).sum() / want.float().pow(2).sum()).sqrt().item() < 2e-2


def _loop_setup(seed, B=4, k=3, bs=16):
    rng = np.random.default_rng(seed)
    model, cpu_w = _model(SMALL, seed=seed)
    width = 40
    num_blocks = max(512, B * width + 16)
    cache = _cache(SMALL, num_blocks, bs, seed=seed + 1)
    ctx = rng.integers(100, 400, size=B).astype(np.int32)
    perm = rng.permutation(num_blocks).astype(np.int32)
    table = perm[: B * width].reshape(B, width)
    histories = [workloads.repetitive_history(rng, int(rng.integers(30, 90)), SMALL.vocab_size,
                                              repetitive_tail=bool(b % 2)) for b in range(B)]
    loop = decode_graph.VerifyLoop(model, cache, batch=B, k=k, max_n=4, history_capacity=256, table_width=width)
    loop.load(histories, ctx, table)
    return loop, model, cpu_w, cache, table, histories, ctx


# Ids of the untied 2-layer model may differ from the oracle's only where the oracle's own top-2
# logit margin is within the end-to-end logit error (the bound of test_extend_end_to_end_small_model).
LOOP_MARGIN = 0.1


def _margins(logits: torch.Tensor) -> np.ndarray:
    values = logits.float().numpy()
    part = np.partition(values, -2, axis=-1)
    return part[:, -1] - part[:, -2]


@pytest.mark.parametrize("B", [4, 16])  # 16 sequences x 4 tokens: the 64-row LM head
def test_verify_loop_graph_matches_oracle_steps(B) -> None:
    """Four graph replays of the device-resident loop, each against the oracle's step from the same
    state: drafts, accepted lengths, committed ids, KV lengths and histories identical.  Where a
    greedy id differs, the oracle's top-2 margin at that row must be within LOOP_MARGIN; the
    comparison then continues from the GPU's ids (the oracle accepts them in the GPU's place), so
    every step's state propagation is checked."""
    loop, model, cpu_w, cache, table, histories, ctx = _loop_setup(5, B=B)
    B, k, s = loop.batch, loop.k, loop.tokens_per_seq
    announce("verify loop capture")
    loop.capture()
    hist = [list(map(int, h)) for h in histories]
    lens = [int(x) for x in ctx]
    compared = drafted = 0
    for step in range(4):
        cpu_k, cpu_v = cache.k.cpu(), cache.v.cpu()
        announce("verify loop step", step)
        loop.replay()
        torch.cuda.synchronize()
        want = oracle_decoder.verify_step(SMALL, cpu_w, hist, np.array(lens), table, k, 4, cpu_k, cpu_v, 16,
                                          max_positions=loop.max_positions)
        got_draft = loop.inputs.draft.cpu().numpy()
        got_len = loop.inputs.draft_len.cpu().numpy()
        assert [got_draft[b, : got_len[b]].tolist() for b in range(B)] == want.drafts
        drafted += sum(1 for d in want.drafts if d)
        got_pred = loop.buffers.predicted[: B * s].view(B, s).cpu().numpy()
        differ = (got_pred != want.predicted.numpy()).reshape(-1)
        margin = _margins(want.logits)
        assert (margin[differ] <= LOOP_MARGIN).all(), (step, margin[differ])
        taken, new_lens = oracle_decoder.accept_step(want.drafts, got_pred, lens)
        assert loop.accepted.accepted.cpu().numpy().tolist() == [len(t) - 1 for t in taken]
        committed = loop.accepted.committed.cpu().numpy()
        assert [committed[b, : len(taken[b])].tolist() for b in range(B)] == taken
        assert all((committed[b, len(taken[b]) :] == -1).all() for b in range(B))
        assert loop.seq_len.cpu().numpy().tolist() == new_lens
        hl = loop.history_len.cpu().numpy()
        hist = [h + t for h, t in zip(hist, taken)]
        assert [loop.history[b, : hl[b]].cpu().tolist() for b in range(B)] == hist
        lens = new_lens
        compared += 1
    assert compared == 4
    assert drafted > 0, "no sequence drafted: the acceptance path went untested"


def test_extend_graphs_list_interface_matches_eager() -> None:
    rng = np.random.default_rng(7)
    model, _ = _model(SMALL, seed=7)
    bs = 16
    cache = _cache(SMALL, 128, bs, seed=8)
    scratch = cache.allocate(1)[0]
    announce("extend graphs capture")
    graphs = decode_graph.ExtendGraphs(model, cache, max_batch=4, tokens_per_seq=4, max_positions=512,
                                       scratch_block=scratch)
    n, s = 3, 4
    tables = [cache.allocate(6) for _ in range(n)]
    seq_lens = [int(x) for x in rng.integers(20, 90, size=n)]
    ids, positions, slots = [], [], []
    for b in range(n):
        for j in range(s):
            pos = seq_lens[b] - s + j
            ids.append(int(rng.integers(0, SMALL.vocab_size)))
            positions.append(pos)
            slots.append(kv_cache.slot_of(tables[b], pos, bs))
    before_k, before_v = cache.k.clone(), cache.v.clone()
    tokens = graphs.run(ids, positions, slots, seq_lens, tables).clone()
    torch.cuda.synchronize()
    # The padded sequence of the bucket (n = 3 in the bucket of 4) wrote only the scratch page's
    # first S slots; the real rows only their own slots.
    written = torch.zeros(128 * bs, dtype=torch.bool)
    written[torch.tensor(slots)] = True
    written[scratch * bs : scratch * bs + s] = True
    for before, after in ((before_k, cache.k), (before_v, cache.v)):
        changed = (before != after).view(SMALL.num_layers, 128 * bs, -1).any(-1).any(0).cpu()
        assert not bool((changed & ~written).any())
    cache.k.copy_(before_k)
    cache.v.copy_(before_v)
    table = np.full((n, 6), scratch, dtype=np.int32)
    for b in range(n):
        table[b] = tables[b]
    eb = language.ExtendBatch(None, torch.tensor(positions).cuda(), torch.tensor(slots).cuda(),
                              torch.tensor(seq_lens, dtype=torch.int32).cuda(), torch.from_numpy(table).cuda(), s,
                              ids=torch.tensor(ids).cuda())
    eager = model.greedy(model.extend(eb, cache)).view(n, s)
    torch.cuda.synchronize()
    assert torch.equal(tokens, eager)


def test_step_record_expands_to_padded_bucket() -> None:
    """The one-copy step record (decode_graph._StepRecord) expanded on the device: the real
    sequences' rows and page lists as given, padded sequences on the scratch page's first S slots
    with seq_len S, table entries past each page list holding the scratch page."""
    capacity, s, width, scratch, bs = 8, 3, 5, 77, 16
    rec = decode_graph._StepRecord(capacity, s, width, torch.device("cuda"))
    rng = np.random.default_rng(9)
    n, bucket = 3, 4
    tables = [[4, 9], [], [1, 2, 3, 5, 6]]
    ids = rng.integers(0, 1000, size=n * s).tolist()
    positions = rng.integers(0, 80, size=n * s).tolist()
    slots = rng.integers(0, 1000, size=n * s).tolist()
    seq_lens = [33, 2, 71]
    rec.write(ids, positions, slots, seq_lens, tables)
    out = [torch.full((capacity * s,), -5, dtype=torch.int64, device="cuda") for _ in range(3)]
    lens = torch.full((capacity,), -5, dtype=torch.int32, device="cuda")
    table = torch.full((capacity, width), -5, dtype=torch.int32, device="cuda")
    announce("step record expansion")
    _lib = pkg("_lib")
    _lib.call("oxr_unpack_step_inputs", rec.device.data_ptr(), capacity, bucket, s, width, scratch, bs,
              out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(), lens.data_ptr(), table.data_ptr(),
              _lib.stream(table.device))
    torch.cuda.synchronize()
    pad = bucket - n
    assert out[0][: bucket * s].tolist() == ids + [0] * (pad * s)
    assert out[1][: bucket * s].tolist() == positions + list(range(s)) * pad
    assert out[2][: bucket * s].tolist() == slots + [scratch * bs + j for j in range(s)] * pad
    assert out[0][bucket * s :].tolist() == [-5] * ((capacity - bucket) * s)  # past the bucket: untouched
    assert lens.tolist() == seq_lens + [s] * pad + [-5] * (capacity - bucket)
    want = [t + [scratch] * (width - len(t)) for t in tables] + [[scratch] * width] * pad
    assert table[:bucket].tolist() == want
    with pytest.raises(ValueError):
        rec.write(ids, positions, slots, seq_lens, [[1] * (width + 1), [], []])  # page list wider than the table


GQA16 = language.LanguageConfig(1024, 1536, 2, 16, 8, 128, 1e-6, 1e6, 1000)


@pytest.mark.parametrize("n", [8, 5])
def test_extend_graphs_reference_defaults(n) -> None:
    """The engine's verify graphs at the reference's defaults (speculative_tokens = 8,
    speculative_max_batch = 8: ExtendGraphs(max_batch=8, tokens_per_seq=9), engine.py:121-123,
    242-246) on a 16/8-head model: 72 token rows through the GEMMs, 18 query rows per kv head.
    The replay equals eager extend bit for bit (n = 5: padded in the bucket of 8), and its greedy
    ids equal the oracle's wherever the oracle's top-2 margin is clear."""
    rng = np.random.default_rng(40 + n)
    model, cpu_w = _model(GQA16, seed=40)
    bs, s = 16, 9
    cache = _cache(GQA16, 512, bs, seed=41)
    scratch = cache.allocate(1)[0]
    announce("extend graphs S=9 capture", n)
    graphs = decode_graph.ExtendGraphs(model, cache, max_batch=8, tokens_per_seq=s, max_positions=1024,
                                       scratch_block=scratch)
    assert graphs.buckets == [1, 2, 4, 8]
    tables = [cache.allocate(int(rng.integers(8, 40))) for _ in range(n)]
    seq_lens = [int(rng.integers(s, len(t) * bs)) for t in tables]
    ids, positions, slots = [], [], []
    for b in range(n):
        for j in range(s):
            pos = seq_lens[b] - s + j
            ids.append(int(rng.integers(0, GQA16.vocab_size)))
            positions.append(pos)
            slots.append(kv_cache.slot_of(tables[b], pos, bs))
    cpu_k, cpu_v = cache.k.cpu(), cache.v.cpu()
    before_k, before_v = cache.k.clone(), cache.v.clone()
    tokens = graphs.run(ids, positions, slots, seq_lens, tables).clone()
    torch.cuda.synchronize()
    after_k, after_v = cache.k.clone(), cache.v.clone()
    # The graphs' table width (max_positions / block size): the same context split, so the same bits.
    table = np.full((n, graphs.width), scratch, dtype=np.int32)
    for b in range(n):
        table[b, : len(tables[b])] = tables[b]
    cache.k.copy_(before_k)
    cache.v.copy_(before_v)
    eb = language.ExtendBatch(None, torch.tensor(positions).cuda(), torch.tensor(slots).cuda(),
                              torch.tensor(seq_lens, dtype=torch.int32).cuda(), torch.from_numpy(table).cuda(), s,
                              ids=torch.tensor(ids).cuda())
    eager = model.greedy(model.extend(eb, cache)).view(n, s)
    torch.cuda.synchronize()
    assert torch.equal(tokens, eager)
    flat = lambda c: c.view(GQA16.num_layers, -1, GQA16.num_kv_heads, GQA16.head_dim)
    assert torch.equal(flat(cache.k)[:, slots], flat(after_k)[:, slots])
    assert torch.equal(flat(cache.v)[:, slots], flat(after_v)[:, slots])
    hidden = oracle_decoder.extend(GQA16, cpu_w, torch.tensor(ids), torch.tensor(positions), torch.tensor(slots),
                                   torch.tensor(seq_lens, dtype=torch.int32), torch.from_numpy(table), s, cpu_k, cpu_v)
    _ids_agree(tokens.reshape(-1).cpu().numpy(), oracle_decoder.logits(cpu_w, hidden), margin_floor=0.1)
